// Shared pieces of the decode-attention kernels (gfx950, wave64, MFMA 16x16x32).
#pragma once
#include "common.hpp"

namespace mz {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int IO> struct Mfma;
template <> struct Mfma<MZ_BF16> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                    0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t cvt(float x) { return f2bf(x); }
  static __device__ __forceinline__ float load(uint16_t h) { return bf2f(h); }
};
template <> struct Mfma<MZ_F16> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                   0, 0);
  }
  static __device__ __forceinline__ uint16_t cvt(float x) { return f2h(x); }
  static __device__ __forceinline__ float load(uint16_t h) { return h2f(h); }
};

// Orders LDS writes and reads of one wave (the compiler must not move the
// reads of other lanes' data above the writes).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float meta_load(const void* p, int64_t i, int dt) { return load_any(p, i, dt); }

struct OpMax {
  __device__ __forceinline__ float operator()(float x, float y) const { return fmaxf(x, y); }
};
struct OpAdd {
  __device__ __forceinline__ float operator()(float x, float y) const { return x + y; }
};

// Wave-uniform maximum (NaN operands are ignored, as by fmaxf).
__device__ __forceinline__ float wave_max_fast(float v) {
  v = group_reduce<16>(v, OpMax());
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Upper bounds of the wave-wide maxima of two non-negative floats, reduced
// together: each is cut to its top 16 bits rounded up (at most 2^-8 above the
// value, same or next binade), so both ride one DPP chain as u16 pairs.  NaN
// and overflowing inputs come back as the largest finite bound.
__device__ __forceinline__ void wave_max2_bound(float& x, float& y) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const uint32_t hx = min(__float_as_uint(x) >> 16, 0x7F7Eu) + 1u;
  const uint32_t hy = min(__float_as_uint(y) >> 16, 0x7F7Eu) + 1u;
  u16x2 p = __builtin_bit_cast(u16x2, hx | (hy << 16));
  p = __builtin_elementwise_max(p, __builtin_bit_cast(u16x2, dpp_sel_u<DPP_QUAD_XOR1>(__builtin_bit_cast(uint32_t, p))));
  p = __builtin_elementwise_max(p, __builtin_bit_cast(u16x2, dpp_sel_u<DPP_QUAD_XOR2>(__builtin_bit_cast(uint32_t, p))));
  p = __builtin_elementwise_max(p, __builtin_bit_cast(u16x2, dpp_sel_u<DPP_ROW_HALF_MIRROR>(__builtin_bit_cast(uint32_t, p))));
  p = __builtin_elementwise_max(p, __builtin_bit_cast(u16x2, dpp_sel_u<DPP_ROW_MIRROR>(__builtin_bit_cast(uint32_t, p))));
  const uint32_t b = __builtin_bit_cast(uint32_t, p);
  u16x2 r = __builtin_bit_cast(u16x2, (uint32_t)__builtin_amdgcn_readlane((int)b, 0));
  r = __builtin_elementwise_max(r, __builtin_bit_cast(u16x2, (uint32_t)__builtin_amdgcn_readlane((int)b, 16)));
  r = __builtin_elementwise_max(r, __builtin_bit_cast(u16x2, (uint32_t)__builtin_amdgcn_readlane((int)b, 32)));
  r = __builtin_elementwise_max(r, __builtin_bit_cast(u16x2, (uint32_t)__builtin_amdgcn_readlane((int)b, 48)));
  const uint32_t rb = __builtin_bit_cast(uint32_t, r);
  x = __uint_as_float(rb << 16);
  y = __uint_as_float(rb & 0xFFFF0000u);
}

// Workspace record of one (batch, q-head, split): acc[D], m, l (fp32).
template <int D>
__device__ __forceinline__ float* ws_record(const mz_decode_args& a, int b, int qh, int split, int n_split) {
  const int Hq = a.kv_heads * a.n_rep;
  return (float*)a.workspace + (((int64_t)b * Hq + qh) * n_split + split) * (D + 2);
}

}  // namespace mz
