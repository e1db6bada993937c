// Shared device helpers for the muZero codec kernels (gfx950, wave64).
//
// Every kernel in this library is compiled with -ffp-contract=off: the
// reference computes each elementwise torch op separately, so a fused
// multiply-add would change the rounding of codes and dequantized values.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/muzero_hip.h"

namespace mz {

constexpr int kWave = 64;
constexpr int kGroup = 64;  // q_group_size supported by the HIP path

// ---------------------------------------------------------------- per-device host state
// The library's only mutable state: facts fetched from the runtime once per
// device and process.  A slot is written with the same value by whichever
// thread gets there first, so concurrent first calls are harmless.
constexpr int kMaxDevices = 64;

// Compute units of the current device (256 if the runtime cannot tell).
inline int device_cu_count() {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  const bool slot = dev >= 0 && dev < kMaxDevices;
  if (slot) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (slot) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Raise kernel `fn`'s dynamic LDS limit to `bytes` on the current device,
// once per device (`done` holds one bit per device, owned by the caller).
inline hipError_t set_dynamic_lds(const void* fn, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  const uint64_t bit = dev >= 0 && dev < kMaxDevices ? (uint64_t)1 << dev : 0;
  if (bit && (done.load(std::memory_order_relaxed) & bit)) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_relaxed);
  return e;
}

// ---------------------------------------------------------------- rounding
// torch's float -> bfloat16 conversion: round to nearest even, NaN -> 0x7FC0
// (c10/util/BFloat16.h round_to_nearest_even).
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if (f != f) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t f2h(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Value of an op result after ATen stores it in the input dtype DT.
template <int DT> __device__ __forceinline__ float rnd(float x);
template <> __device__ __forceinline__ float rnd<MZ_F32>(float x) { return x; }
// gfx950 converts to bf16 in hardware (v_cvt_pk_bf16_f32, round to nearest
// even, the same as f2bf for every non-NaN input; a NaN stays a NaN but its
// payload is not canonicalised, so stores go through f2bf).
// The value goes to the high half of the converted pair with 0 in the low
// half, so the pair's bits are already the fp32 value: one instruction.
template <> __device__ __forceinline__ float rnd<MZ_BF16>(float x) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(float, __builtin_convertvector(f32x2_t{0.f, x}, bf16x2_t));
}
template <> __device__ __forceinline__ float rnd<MZ_F16>(float x) { return h2f(f2h(x)); }

template <int DT> __device__ __forceinline__ float load_val(const void* p, int64_t i);
template <> __device__ __forceinline__ float load_val<MZ_F32>(const void* p, int64_t i) {
  return ((const float*)p)[i];
}
template <> __device__ __forceinline__ float load_val<MZ_BF16>(const void* p, int64_t i) {
  return bf2f(((const uint16_t*)p)[i]);
}
template <> __device__ __forceinline__ float load_val<MZ_F16>(const void* p, int64_t i) {
  return h2f(((const uint16_t*)p)[i]);
}

// Store a value already representable in DT (or to be rounded to it).
__device__ __forceinline__ void store_val(void* p, int64_t i, float v, int dt) {
  if (dt == MZ_F32) ((float*)p)[i] = v;
  else if (dt == MZ_BF16) ((uint16_t*)p)[i] = f2bf(v);
  else ((uint16_t*)p)[i] = f2h(v);
}
__device__ __forceinline__ float load_any(const void* p, int64_t i, int dt) {
  if (dt == MZ_F32) return ((const float*)p)[i];
  if (dt == MZ_BF16) return bf2f(((const uint16_t*)p)[i]);
  return h2f(((const uint16_t*)p)[i]);
}

// torch.clamp / clamp_min semantics: NaN passes through.
__device__ __forceinline__ float clamp01(float x) { return x < 0.f ? 0.f : (x > 1.f ? 1.f : x); }
__device__ __forceinline__ float clamp_min(float x, float lo) { return x < lo ? lo : x; }

// ------------------------------------------------------------ reductions
// NaN-propagating min/max (torch.amin/amax propagate NaN).
__device__ __forceinline__ float nmin(float a, float b) { return (a != a || a < b) ? a : b; }
__device__ __forceinline__ float nmax(float a, float b) { return (a != a || a > b) ? a : b; }

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nmin(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nmax(v, __shfl_xor(v, o, kWave));
  return v;
}

// Cross-lane reductions on DPP (no LDS round trips).  dpp_sel<CTRL>(v) reads v
// from the lane that the gfx9 DPP control CTRL names.
template <int CTRL>
__device__ __forceinline__ float dpp_sel(float v) {
  // every control used here reads a lane of the same row, so no lane takes the
  // bound value (bound_ctrl set: no register to preload)
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_sel_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
constexpr int DPP_QUAD_XOR1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;  // lane i <- 7 - i within 8
constexpr int DPP_ROW_MIRROR = 0x140;       // lane i <- 15 - i within 16

// Reduction over aligned groups of N lanes (N a power of two <= 64); every
// lane of a group gets the same result (each step combines the lane's value
// with a partner holding the other half, in a fixed order).
template <int N, typename Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
  if constexpr (N >= 2) v = op(v, dpp_sel<DPP_QUAD_XOR1>(v));
  if constexpr (N >= 4) v = op(v, dpp_sel<DPP_QUAD_XOR2>(v));
  if constexpr (N >= 8) v = op(v, dpp_sel<DPP_ROW_HALF_MIRROR>(v));
  if constexpr (N >= 16) v = op(v, dpp_sel<DPP_ROW_MIRROR>(v));
  if constexpr (N >= 32) v = op(v, __shfl_xor(v, 16, 64));
  if constexpr (N >= 64) v = op(v, __shfl_xor(v, 32, 64));
  return v;
}

// ---------------------------------------------------------------- packing
// LSB-first bitstream (muzero/quantizer.py:189-202): stream bit j = bit
// (j mod BITS) of code (j div BITS).  Lane t of the wave assembles byte t of
// the row from the codes of the (at most ceil(8/BITS)+1) lanes overlapping it.
template <int BITS>
__device__ __forceinline__ uint32_t pack_byte(uint32_t code, int lane) {
  const int first = (8 * lane) / BITS;
  constexpr int SPAN = (8 + BITS - 1) / BITS + 1;
  uint32_t acc = 0;
#pragma unroll
  for (int k = 0; k < SPAN; ++k) {
    const int i = first + k;
    const uint32_t c = __shfl(code, i < kWave ? i : kWave - 1, kWave);
    const int sh = i * BITS - 8 * lane;
    const uint32_t part = sh >= 0 ? (c << (sh & 31)) : (c >> ((-sh) & 31));
    if (i < kWave && sh < 8) acc |= part;
  }
  return acc & 0xFFu;
}

// Code i (0..63) of a packed row held as bytes in `row` (any alignment).
template <int BITS>
__device__ __forceinline__ uint32_t unpack_code(const uint8_t* row, int i) {
  const int bit = i * BITS;
  const int byte = bit >> 3;
  uint32_t w = row[byte];
  if ((bit & 7) + BITS > 8) w |= (uint32_t)row[byte + 1] << 8;
  return (w >> (bit & 7)) & ((1u << BITS) - 1u);
}

// ------------------------------------------------------- dequantization
// Row parameters recomputed from the STORED metadata (quantizer.py:241-249).
struct DeqRow {
  float mn, s, za, zl, pb, nb, pe, ne;
  int offp, offn;  // expm1-table row offsets for pb and nb
};

__device__ __forceinline__ int expm1_row(int bins) { return (bins - 1) * (bins + 2) / 2; }

// `guard`: clamp the stored scale to >= 1e-8 before use, as the reference
// CUDA extension does (muzero/kernels/loader.py:201).  An all-zero group is
// stored with scale fp16(1e-8) == 0, which the torch path turns into NaN.
__device__ __forceinline__ DeqRow deq_row(float mn, float s, float qmax, bool guard) {
  const float eps = 1e-8f;
  DeqRow r;
  if (guard && !(s >= eps)) s = eps;
  r.mn = mn;
  r.s = s;
  r.za = clamp01((0.f - mn) / s);
  r.zl = rintf(r.za * qmax);
  r.pb = fmaxf(qmax - r.zl, 1.f);
  r.nb = fmaxf(r.zl, 1.f);
  r.pe = clamp_min(1.f - r.za, eps);
  r.ne = clamp_min(r.za, eps);
  if (!(r.pb == r.pb)) r.pb = 1.f;
  if (!(r.nb == r.nb)) r.nb = 1.f;
  const int ipb = (int)r.pb;
  const int inb = (int)r.nb;
  r.offp = expm1_row(ipb);
  r.offn = expm1_row(inb);
  return r;
}

// Exact fp32 dequantized value of code q (quantizer.py:250-255, no FMA).
__device__ __forceinline__ float deq_value(const DeqRow& r, uint32_t q, const float* E) {
  const float qf = (float)q;
  float norm;
  // d is clamped to the row's 0..bins range so corrupt metadata cannot index
  // outside the table (for valid metadata the clamp never changes d).
  if (qf >= r.zl) {
    const int d = min(max((int)(qf - r.zl), 0), (int)r.pb);
    const float pn = E[r.offp + d];
    const float t = r.pe * pn;
    norm = r.za + t;
  } else {
    const int d = min(max((int)(r.zl - qf), 0), (int)r.nb);
    const float nn = E[r.offn + d];
    const float t = r.ne * nn;
    norm = r.za - t;
  }
  norm = clamp01(norm);
  const float u = norm * r.s;
  return u + r.mn;
}

}  // namespace mz
