// Quantize + bit-pack and dequantize kernels (gfx950, wave64).
//
// One wavefront per 64-value group: lane i holds value i.  The group min/max
// is a wave reduction, every per-element op of the reference quantizer
// (muzero/quantizer.py:161-186) is evaluated in its own dtype with IEEE
// rounding and no contraction, and the one transcendental step
// (round(log1p(alpha*p)/lb*bins)) comes from a host-built constant table, so
// codes and metadata are bit-identical to the reference torch path.
#include "common.hpp"

namespace mz {

// Code of one lane's value given the group's min and scale.  DT is the dtype
// every reference op rounds to.  `table` is the fp32 threshold table (DT ==
// F32) or the 16-bit ratio table indexed by the pattern of p (DT == BF16/F16).
template <int DT, int BITS>
__device__ __forceinline__ uint32_t lane_code(float v, float mn, float sc, float eps, const void* table) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  const float norm = clamp01(rnd<DT>(rnd<DT>(v - mn) / sc));
  const float za = clamp01(rnd<DT>(rnd<DT>(0.f - mn) / sc));
  const float zl = rintf(rnd<DT>(za * qmax));
  const float pb = clamp_min(rnd<DT>(qmax - zl), 1.f);
  const float nb = clamp_min(zl, 1.f);
  const float pe = clamp_min(rnd<DT>(1.f - za), eps);
  const float ne = clamp_min(za, eps);
  const bool up = norm >= za;  // torch.where(norm >= za, q_pos, q_neg); false on NaN
  const float p = up ? clamp01(rnd<DT>(rnd<DT>(norm - za) / pe))
                     : clamp01(rnd<DT>(rnd<DT>(za - norm) / ne));
  const float bins = up ? pb : nb;
  float off;
  if constexpr (DT == MZ_F32) {
    // #{k : p >= T[bins][k]} by binary search over the bins thresholds.
    const float* T = (const float*)table;
    const int ib = (bins == bins) ? (int)bins : 1;
    const float* row = T + ib * (ib - 1) / 2;
    int lo = 0, hi = ib;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (row[mid] <= p) lo = mid + 1; else hi = mid;
    }
    off = (p == p) ? (float)lo : __builtin_nanf("");
  } else {
    const uint16_t* Y = (const uint16_t*)table;
    float y;
    if (p == p) {
      const uint32_t pat = (DT == MZ_BF16 ? (uint32_t)f2bf(p) : (uint32_t)f2h(p)) & 0x7FFFu;  // -0 -> 0
      y = DT == MZ_BF16 ? bf2f(Y[pat]) : h2f(Y[pat]);
    } else {
      y = p;
    }
    off = rintf(rnd<DT>(y * bins));
  }
  const float q = up ? rnd<DT>(zl + off) : rnd<DT>(zl - off);
  // clamp(0, qmax).to(uint8); a NaN code converts to 0 (as on the reference CPU)
  if (!(q == q)) return 0u;
  return (uint32_t)fminf(fmaxf(q, 0.f), qmax);
}

// Quantize the wave's group (lane value v) and store packed bytes and metadata.
template <int DT, int BITS>
__device__ __forceinline__ void quantize_group(float v, int lane, uint8_t* prow, void* mn_out, void* sc_out,
                                               int64_t midx, int meta_dtype, float eps_in, const void* table) {
  const float mn = wave_min(v);
  const float mx = wave_max(v);
  const float eps = rnd<DT>(eps_in);
  const float sc = clamp_min(rnd<DT>(mx - mn), eps);
  const uint32_t code = lane_code<DT, BITS>(v, mn, sc, eps, table);
  const uint32_t byte = pack_byte<BITS>(code, lane);
  if (lane < 8 * BITS) prow[lane] = (uint8_t)byte;
  if (lane == 0) {
    store_val(mn_out, midx, mn, meta_dtype);
    store_val(sc_out, midx, sc, meta_dtype);
  }
}

// ------------------------------------------------------------- rows
template <int DT, int BITS>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const void* __restrict__ x, int64_t nrows,
                                                            int64_t xs, uint8_t* __restrict__ packed, int64_t ps,
                                                            void* mn, void* sc, int meta_dtype, int64_t ms,
                                                            float eps, const void* __restrict__ table) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= nrows) return;
  const float v = load_val<DT>(x, row * xs + lane);
  quantize_group<DT, BITS>(v, lane, packed + row * ps, mn, sc, row * ms, meta_dtype, eps, table);
}

// ------------------------------------------------------------- values
// Row (b, h, t, j): channels 64j..64j+63 of token t, zero beyond D.
template <int DT, int BITS>
__global__ __launch_bounds__(256) void quantize_values_kernel(const void* __restrict__ x, int B, int H, int T, int D,
                                                              int64_t sb, int64_t sh, int64_t st,
                                                              uint8_t* __restrict__ packed, int64_t psb, int64_t psh,
                                                              void* mn, void* sc, int meta_dtype, int64_t msb,
                                                              int64_t msh, float eps, const void* __restrict__ table) {
  const int ng = (D + 63) / 64;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)B * H * T * ng;
  if (row >= nrows) return;
  const int j = (int)(row % ng);
  const int64_t r1 = row / ng;
  const int t = (int)(r1 % T);
  const int64_t r2 = r1 / T;
  const int h = (int)(r2 % H);
  const int b = (int)(r2 / H);
  const int c = 64 * j + lane;
  const float v = c < D ? load_val<DT>(x, b * sb + h * sh + t * st + c) : 0.f;
  constexpr int QB = 8 * BITS;
  uint8_t* prow = packed + b * psb + h * psh + ((int64_t)t * ng + j) * QB;
  const int64_t midx = b * msb + h * msh + (int64_t)t * ng + j;
  quantize_group<DT, BITS>(v, lane, prow, mn, sc, midx, meta_dtype, eps, table);
}

// ------------------------------------------------------------- keys
// One workgroup per (b, h, token group): the [64 x D] tile is staged in LDS
// (coalesced along D), and each wave quantizes channels reading the tile's
// columns, so the reference's permute+contiguous copy never touches HBM.
template <int DT, int BITS>
__global__ __launch_bounds__(256) void quantize_keys_kernel(const void* __restrict__ x, int B, int H, int T, int D,
                                                            int64_t sb, int64_t sh, int64_t st,
                                                            uint8_t* __restrict__ packed, int64_t psb, int64_t psh,
                                                            void* mn, void* sc, int meta_dtype, int64_t msb,
                                                            int64_t msh, float eps, const void* __restrict__ table) {
  extern __shared__ float tile[];  // [64][D + 1]
  const int nsg = T / 64;
  const int s = blockIdx.x % nsg;
  const int h = (blockIdx.x / nsg) % H;
  const int b = blockIdx.x / (nsg * H);
  const int ld = D + 1;
  const int64_t base = b * sb + h * sh + (int64_t)(64 * s) * st;
  for (int e = threadIdx.x; e < 64 * D; e += 256) {
    const int t = e / D, c = e - t * D;
    tile[t * ld + c] = load_val<DT>(x, base + t * st + c);
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  constexpr int QB = 8 * BITS;
  uint8_t* gbase = packed + b * psb + h * psh + (int64_t)s * D * QB;
  const int64_t mbase = b * msb + h * msh + (int64_t)s * D;
  for (int c = wave; c < D; c += 4) {
    const float v = tile[lane * ld + c];
    quantize_group<DT, BITS>(v, lane, gbase + (int64_t)c * QB, mn, sc, mbase + c, meta_dtype, eps, table);
  }
}

// ------------------------------------------------------------- dequantize
template <int BITS>
__global__ __launch_bounds__(256) void dequantize_rows_kernel(const uint8_t* __restrict__ packed, int64_t nrows,
                                                              int64_t ps, const void* mn, const void* sc,
                                                              int meta_dtype, int64_t ms, void* out, int out_dtype,
                                                              int64_t os, const float* __restrict__ E) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= nrows) return;
  constexpr float qmax = (float)((1 << BITS) - 1);
  const DeqRow r = deq_row(load_any(mn, row * ms, meta_dtype), load_any(sc, row * ms, meta_dtype), qmax, true);
  const uint32_t q = unpack_code<BITS>(packed + row * ps, lane);
  store_val(out, row * os + lane, deq_value(r, q, E), out_dtype);
}

// ------------------------------------------------------------- dispatch
#define MZ_BITS_SWITCH(BITS, ...)                      \
  switch (BITS) {                                      \
    case 1: { constexpr int B_ = 1; __VA_ARGS__; } break; \
    case 2: { constexpr int B_ = 2; __VA_ARGS__; } break; \
    case 3: { constexpr int B_ = 3; __VA_ARGS__; } break; \
    case 4: { constexpr int B_ = 4; __VA_ARGS__; } break; \
    case 5: { constexpr int B_ = 5; __VA_ARGS__; } break; \
    case 6: { constexpr int B_ = 6; __VA_ARGS__; } break; \
    case 7: { constexpr int B_ = 7; __VA_ARGS__; } break; \
    case 8: { constexpr int B_ = 8; __VA_ARGS__; } break; \
    default: return MZ_EINVAL;                         \
  }

#define MZ_DT_SWITCH(DTV, ...)                                   \
  switch (DTV) {                                                 \
    case MZ_F32: { constexpr int D_ = MZ_F32; __VA_ARGS__; } break;   \
    case MZ_BF16: { constexpr int D_ = MZ_BF16; __VA_ARGS__; } break; \
    case MZ_F16: { constexpr int D_ = MZ_F16; __VA_ARGS__; } break;   \
    default: return MZ_EINVAL;                                   \
  }

static inline bool dtype_ok(int dt) { return dt == MZ_F32 || dt == MZ_BF16 || dt == MZ_F16; }

static inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

}  // namespace mz

using namespace mz;

extern "C" int muzero_quantize_rows(const void* x, int x_dtype, int64_t nrows, int64_t x_row_stride,
                                    uint8_t* packed, int64_t packed_row_stride, void* mn, void* scale,
                                    int meta_dtype, int64_t meta_stride, int bits, float eps, const void* table,
                                    mz_stream_t stream) {
  if (nrows < 0 || !dtype_ok(x_dtype) || !dtype_ok(meta_dtype) || bits < 1 || bits > 8) return MZ_EINVAL;
  if (nrows == 0) return MZ_OK;
  if (!x || !packed || !mn || !scale || !table) return MZ_EINVAL;
  if (x_row_stride < 64 || packed_row_stride < 8 * bits || meta_stride < 1) return MZ_EINVAL;
  const dim3 grid((unsigned)((nrows + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  MZ_DT_SWITCH(x_dtype, MZ_BITS_SWITCH(bits,
      hipLaunchKernelGGL((quantize_rows_kernel<D_, B_>), grid, dim3(256), 0, s, x, nrows, x_row_stride, packed,
                         packed_row_stride, mn, scale, meta_dtype, meta_stride, eps, table)));
  return launch_status();
}

static int check_block(const void* x, int x_dtype, int B, int H, int T, int D, const uint8_t* packed,
                       const void* mn, const void* scale, int meta_dtype, int bits, const void* table) {
  if (!dtype_ok(x_dtype) || !dtype_ok(meta_dtype) || bits < 1 || bits > 8) return MZ_EINVAL;
  if (B < 0 || H < 0 || T < 0 || D <= 0) return MZ_EINVAL;
  if ((int64_t)B * H * T == 0) return 1;  // nothing to do
  if (!x || !packed || !mn || !scale || !table) return MZ_EINVAL;
  return MZ_OK;
}

extern "C" int muzero_quantize_keys(const void* keys, int x_dtype, int B, int H, int T, int D, int64_t x_sb,
                                    int64_t x_sh, int64_t x_st, uint8_t* packed, int64_t p_sb, int64_t p_sh,
                                    void* mn, void* scale, int meta_dtype, int64_t m_sb, int64_t m_sh, int bits,
                                    float eps, const void* table, mz_stream_t stream) {
  int st = check_block(keys, x_dtype, B, H, T, D, packed, mn, scale, meta_dtype, bits, table);
  if (st == 1) return MZ_OK;
  if (st) return st;
  if (T % 64) return MZ_EINVAL;
  const size_t lds = (size_t)64 * (D + 1) * sizeof(float);
  if (lds > 160 * 1024) return MZ_EUNSUPPORTED;
  const dim3 grid((unsigned)((int64_t)B * H * (T / 64)));
  hipStream_t s = (hipStream_t)stream;
  MZ_DT_SWITCH(x_dtype, MZ_BITS_SWITCH(bits,
      if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute((const void*)quantize_keys_kernel<D_, B_>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
      }
      hipLaunchKernelGGL((quantize_keys_kernel<D_, B_>), grid, dim3(256), lds, s, keys, B, H, T, D, x_sb, x_sh, x_st,
                         packed, p_sb, p_sh, mn, scale, meta_dtype, m_sb, m_sh, eps, table)));
  return launch_status();
}

extern "C" int muzero_quantize_values(const void* values, int x_dtype, int B, int H, int T, int D, int64_t x_sb,
                                      int64_t x_sh, int64_t x_st, uint8_t* packed, int64_t p_sb, int64_t p_sh,
                                      void* mn, void* scale, int meta_dtype, int64_t m_sb, int64_t m_sh, int bits,
                                      float eps, const void* table, mz_stream_t stream) {
  int st = check_block(values, x_dtype, B, H, T, D, packed, mn, scale, meta_dtype, bits, table);
  if (st == 1) return MZ_OK;
  if (st) return st;
  const int64_t nrows = (int64_t)B * H * T * ((D + 63) / 64);
  const dim3 grid((unsigned)((nrows + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  MZ_DT_SWITCH(x_dtype, MZ_BITS_SWITCH(bits,
      hipLaunchKernelGGL((quantize_values_kernel<D_, B_>), grid, dim3(256), 0, s, values, B, H, T, D, x_sb, x_sh,
                         x_st, packed, p_sb, p_sh, mn, scale, meta_dtype, m_sb, m_sh, eps, table)));
  return launch_status();
}

extern "C" int muzero_dequantize_rows(const uint8_t* packed, int64_t nrows, int64_t packed_row_stride,
                                      const void* mn, const void* scale, int meta_dtype, int64_t meta_stride,
                                      void* out, int out_dtype, int64_t out_row_stride, int bits,
                                      const float* e_table, mz_stream_t stream) {
  if (nrows < 0 || !dtype_ok(meta_dtype) || !dtype_ok(out_dtype) || bits < 1 || bits > 8) return MZ_EINVAL;
  if (nrows == 0) return MZ_OK;
  if (!packed || !mn || !scale || !out || !e_table) return MZ_EINVAL;
  if (packed_row_stride < 8 * bits || out_row_stride < 64 || meta_stride < 1) return MZ_EINVAL;
  const dim3 grid((unsigned)((nrows + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  MZ_BITS_SWITCH(bits, hipLaunchKernelGGL((dequantize_rows_kernel<B_>), grid, dim3(256), 0, s, packed, nrows,
                                          packed_row_stride, mn, scale, meta_dtype, meta_stride, out, out_dtype,
                                          out_row_stride, e_table));
  return launch_status();
}

extern "C" const char* muzero_version(void) { return "muzero_hip 0.1.0 gfx950"; }

extern "C" const char* muzero_strerror(int status) {
  switch (status) {
    case MZ_OK: return "ok";
    case MZ_EINVAL: return "invalid argument (pointer, size, stride, dtype or bit width)";
    case MZ_EUNSUPPORTED: return "shape not supported by the HIP path";
    case MZ_EWORKSPACE: return "workspace too small";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown error";
  }
}
