// Decode-step prologue of one attention layer (gfx950, wave64): the work the
// model does between its q/k/v projections and the attention for a single
// new token, in one launch instead of about 25 small ones:
//   q, k <- RMSNorm(q), RMSNorm(k) per head (Qwen3's q_norm / k_norm; skipped
//           when no weight is given, as for Llama),
//   q, k <- q*cos + rotate_half(q)*sin (transformers' apply_rotary_pos_emb),
//   k, v -> the cache layer's residual rows for the new token,
//   q    -> the decode-attention query [B, Hq, 1, D].
// Every elementwise op rounds to the io dtype like the torch op it replaces
// (the RoPE products, the sum, the norm's multiply by the weight); the norm's
// mean of squares is an fp32 wave reduction (torch's own reduction order is
// not specified, so the normalized value can differ from torch's in the last
// bit of the io dtype).
// One wave per (batch, row): rows 0..Hq-1 are query heads, then Hkv key heads,
// then Hkv value heads.  Lane l holds elements l and l + D/2, the two halves
// rotate_half pairs, so no lane exchange is needed.
#include "common.hpp"

namespace mz {

template <int IO>
__device__ __forceinline__ float rio(float x) { return rnd<IO>(x); }

template <int IO>
__device__ __forceinline__ float ld(const void* p, int64_t i) { return load_val<IO>(p, i); }

template <int IO>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  ((uint16_t*)p)[i] = IO == MZ_BF16 ? f2bf(v) : f2h(v);
}

template <int D, int IO>
__global__ __launch_bounds__(64) void prologue_kernel(const mz_prologue_args a) {
  constexpr int H2 = D / 2;
  const int lane = threadIdx.x;
  const int row = blockIdx.x;
  const int b = blockIdx.y;
  const bool active = lane < H2;
  const int i0 = lane, i1 = lane + H2;
  if (row >= a.q_heads + a.kv_heads) {
    // value head: copied as it is
    const int h = row - a.q_heads - a.kv_heads;
    if (active) {
      const uint16_t* src = (const uint16_t*)a.v + b * a.v_sb + (int64_t)h * a.v_sh;
      uint16_t* dst = (uint16_t*)a.v_dst + b * a.vd_sb + (int64_t)h * a.vd_sh;
      dst[i0] = src[i0];
      dst[i1] = src[i1];
    }
    return;
  }
  const bool is_q = row < a.q_heads;
  const int h = is_q ? row : row - a.q_heads;
  const void* src = is_q ? a.q : a.k;
  const int64_t base = is_q ? b * a.q_sb + (int64_t)h * a.q_sh : b * a.k_sb + (int64_t)h * a.k_sh;
  float x0 = active ? ld<IO>(src, base + i0) : 0.f;
  float x1 = active ? ld<IO>(src, base + i1) : 0.f;
  const void* w = is_q ? a.q_norm_w : a.k_norm_w;
  if (w) {
    // RMSNorm: x * rsqrt(mean(x^2) + eps) in fp32, rounded to the io dtype, times the weight
    float ss = x0 * x0 + x1 * x1;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float r = rsqrtf(ss / (float)D + a.eps);
    x0 = rio<IO>(ld<IO>(w, i0) * rio<IO>(x0 * r));
    x1 = rio<IO>(ld<IO>(w, i1) * rio<IO>(x1 * r));
  }
  if (!active) return;
  // RoPE: q*cos + rotate_half(q)*sin, rotate_half(q) = cat(-q[D/2:], q[:D/2])
  const int64_t cb = b * a.cs_sb;
  const float c0 = ld<IO>(a.cos, cb + i0), c1 = ld<IO>(a.cos, cb + i1);
  const float s0 = ld<IO>(a.sin, cb + i0), s1 = ld<IO>(a.sin, cb + i1);
  const float y0 = rio<IO>(rio<IO>(x0 * c0) + rio<IO>(-x1 * s0));
  const float y1 = rio<IO>(rio<IO>(x1 * c1) + rio<IO>(x0 * s1));
  void* dst = is_q ? a.q_out : a.k_dst;
  const int64_t ob = is_q ? b * a.qo_sb + (int64_t)h * a.qo_sh : b * a.kd_sb + (int64_t)h * a.kd_sh;
  st<IO>(dst, ob + i0, y0);
  st<IO>(dst, ob + i1, y1);
}

}  // namespace mz

using namespace mz;

extern "C" int muzero_decode_prologue(const mz_prologue_args* a, mz_stream_t stream) {
  if (!a) return MZ_EINVAL;
  if (a->batch < 0 || a->q_heads <= 0 || a->kv_heads <= 0) return MZ_EINVAL;
  if (a->io_dtype != MZ_BF16 && a->io_dtype != MZ_F16) return MZ_EINVAL;
  if (a->head_dim != 64 && a->head_dim != 128) return MZ_EUNSUPPORTED;
  if (a->batch == 0) return MZ_OK;
  if (!a->q || !a->k || !a->v || !a->cos || !a->sin || !a->q_out || !a->k_dst || !a->v_dst) return MZ_EINVAL;
  if ((a->q_norm_w == nullptr) != (a->k_norm_w == nullptr)) return MZ_EINVAL;
  const dim3 grid(a->q_heads + 2 * a->kv_heads, a->batch);
  hipStream_t s = (hipStream_t)stream;
  if (a->head_dim == 128) {
    if (a->io_dtype == MZ_BF16) hipLaunchKernelGGL((prologue_kernel<128, MZ_BF16>), grid, dim3(64), 0, s, *a);
    else hipLaunchKernelGGL((prologue_kernel<128, MZ_F16>), grid, dim3(64), 0, s, *a);
  } else {
    if (a->io_dtype == MZ_BF16) hipLaunchKernelGGL((prologue_kernel<64, MZ_BF16>), grid, dim3(64), 0, s, *a);
    else hipLaunchKernelGGL((prologue_kernel<64, MZ_F16>), grid, dim3(64), 0, s, *a);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}
