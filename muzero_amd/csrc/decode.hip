// Packed-KV decode attention (gfx950, wave64, MFMA 16x16x32).
//
// Work decomposition: one workgroup (4 waves) per (batch, kv-head, token
// split).  A split is a run of 64-token tiles: first the quantized prefix
// groups, then the dense residual window in tiles of up to 64 tokens.  Each
// wave takes every 4th tile of its split and keeps its own online-softmax
// state for the n_rep query heads of the kv-head (GQA grouping: the heads are
// the M rows of the MFMA, padded to 16).  At the end the 4 waves merge in LDS
// and the workgroup writes one (m, l, acc) partial; a second kernel combines
// the splits with a log-sum-exp merge.  No float atomics: results are
// deterministic.
//
// Per tile:
//   K tile -> LDS [64 tokens][D] in the io dtype (dequantized exactly as the
//   reference's _dequantize_rows_torch and rounded to the layer dtype, or
//   copied from the residual), QK^T with MFMA (A = Q rows, B = K tile),
//   online softmax on the MFMA accumulator layout, P -> LDS in fp16,
//   V tile -> LDS [D][64] in fp16 (transposed so an MFMA B operand is 8
//   consecutive tokens of one channel), acc += P V with an fp16 MFMA.
// P V runs in fp16 whatever the io dtype: weights keep 11 mantissa bits (bf16
// weights cost up to 2^-9 relative each, too coarse for peaked softmax rows),
// and every bf16 value in fp16's normal range converts to fp16 exactly.  The
// softmax denominator sums the same rounded weights the numerator uses.
#include "decode_common.hpp"

namespace mz {

constexpr int kTile = 64;
constexpr int kWaves = 4;
constexpr int kPad = 8;  // halfwords of padding per LDS row

template <int D>
struct Lds {
  static constexpr int K_LD = D + kPad;       // K tile row: one token
  static constexpr int V_LD = kTile + kPad;   // V tile row: one channel
  static constexpr int KV_HALVES = (kTile * K_LD > D * V_LD) ? kTile * K_LD : D * V_LD;
  static constexpr int P_LD = kTile + kPad;
  static constexpr int P_HALVES = 16 * P_LD;
  static constexpr int WAVE_HALVES = KV_HALVES + P_HALVES;
  static constexpr int E_FLOATS = 528;  // expm1 table rows for bins <= 31 (bits <= 5)
  static constexpr size_t BYTES = (size_t)kWaves * WAVE_HALVES * 2 + 2 * E_FLOATS * 4;
};

template <int D, int BITS, int IO>
__global__ __launch_bounds__(256) void decode_split_kernel(const mz_decode_args a, int tiles_per_split, int n_split) {
  using L = Lds<D>;
  using M = Mfma<IO>;
  constexpr int QB = 8 * BITS;
  constexpr int NG = (D + 63) / 64;
  constexpr float qmax = (float)((1 << BITS) - 1);
  constexpr bool kLdsE = BITS <= 5;

  extern __shared__ __align__(16) uint16_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int n_rep = a.n_rep;

  uint16_t* kv = lds + wave * L::WAVE_HALVES;
  uint16_t* pb = kv + L::KV_HALVES;
  float* eK = (float*)(lds + kWaves * L::WAVE_HALVES);
  float* eV = eK + L::E_FLOATS;
  const float* EK = a.e_key;
  const float* EV = a.e_value;
  if constexpr (kLdsE) {
    // the expm1 tables exist only when there is a quantized prefix
    if (a.n_groups > 0) {
      for (int i = threadIdx.x; i < L::E_FLOATS; i += 256) {
        eK[i] = a.e_key[i];
        eV[i] = a.e_value[i];
      }
    }
    __syncthreads();
    EK = eK;
    EV = eV;
  }

  // Q rows as the MFMA A operand: lane (m=n, g) holds Q[m][32*ks + 8g .. +7].
  u32x4 qa[D / 32];
  {
    const int m = n;
    const uint16_t* qrow = (const uint16_t*)a.query + b * a.q_sb + (int64_t)(kvh * n_rep + m) * a.q_sh;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      if (m < n_rep) qa[ks] = *(const u32x4*)(qrow + 32 * ks + 8 * g);
      else qa[ks] = u32x4{0, 0, 0, 0};
    }
  }

  // online softmax state for heads 4g+i (replicated over the 16 lanes of a row)
  float m_run[4], l_run[4];
  f32x4 acc[D / 16];
#pragma unroll
  for (int i = 0; i < 4; ++i) { m_run[i] = -INFINITY; l_run[i] = 0.f; }
#pragma unroll
  for (int j = 0; j < D / 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int n_tiles = a.n_groups + (a.n_residual + kTile - 1) / kTile;
  const int t_begin = split * tiles_per_split;
  const int t_end = min(n_tiles, t_begin + tiles_per_split);
  const float scale = a.scaling;

  for (int tile = t_begin + wave; tile < t_end; tile += kWaves) {
    const bool quant = tile < a.n_groups;
    const int r0 = quant ? 0 : (tile - a.n_groups) * kTile;
    const int n_valid = quant ? kTile : min(kTile, a.n_residual - r0);
    const int pos0 = quant ? tile * kTile : a.n_groups * kTile + r0;

    // ---------------- K tile -> kv[t * K_LD + c]
    if (quant) {
      // lane = channel: the channel's packed row holds its 64 tokens' codes
#pragma unroll
      for (int cc = 0; cc < D / 64; ++cc) {
        const int c = lane + 64 * cc;
        const int64_t midx = b * a.km_sb + kvh * a.km_sh + (int64_t)tile * D + c;
        const DeqRow r = deq_row(meta_load(a.k_mn, midx, a.meta_dtype), meta_load(a.k_scale, midx, a.meta_dtype),
                                 qmax, true);
        const uint8_t* prow = a.k_packed + b * a.kp_sb + kvh * a.kp_sh + ((int64_t)tile * D + c) * QB;
        uint32_t w[QB / 4];
#pragma unroll
        for (int i = 0; i < QB / 4; ++i) w[i] = ((const uint32_t*)prow)[i];
        const uint8_t* bytes = (const uint8_t*)w;
#pragma unroll
        for (int t = 0; t < kTile; ++t) {
          const uint32_t q = unpack_code<BITS>(bytes, t);
          kv[t * L::K_LD + c] = M::cvt(deq_value(r, q, EK));
        }
      }
    } else {
      // lane = token: copy the residual row
      const int t = lane;
      if (t < n_valid) {
        const uint16_t* src = (const uint16_t*)a.k_res + b * a.kr_sb + kvh * a.kr_sh + (int64_t)(r0 + t) * a.kr_st;
#pragma unroll
        for (int c = 0; c < D; c += 8) *(u32x4*)(kv + t * L::K_LD + c) = *(const u32x4*)(src + c);
      } else {
#pragma unroll
        for (int c = 0; c < D; c += 8) *(u32x4*)(kv + t * L::K_LD + c) = u32x4{0, 0, 0, 0};
      }
    }
    wave_lds_sync();

    // ---------------- S = Q K^T : lane (n, g) gets heads 4g+i of token 16j+n
    f32x4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) {
        const u32x4 kb = *(const u32x4*)(kv + (16 * j + n) * L::K_LD + 32 * ks + 8 * g);
        s[j] = M::run(qa[ks], kb, s[j]);
      }
    }

    // ---------------- online softmax over this tile
    float tmax[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) tmax[i] = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * j + n;
      const float madd = (a.mask && t < n_valid) ? a.mask[b * a.mask_sb + pos0 + t] : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = s[j][i] * scale + madd;
        if (t >= n_valid) v = -INFINITY;
        s[j][i] = v;
        tmax[i] = fmaxf(tmax[i], v);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) tmax[i] = fmaxf(tmax[i], __shfl_xor(tmax[i], o, 16));
    }
    float corr[4], psum[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mn = fmaxf(m_run[i], tmax[i]);
      corr[i] = (mn == -INFINITY) ? 1.f : __expf(m_run[i] - mn);
      m_run[i] = mn;
      psum[i] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = (s[j][i] == -INFINITY) ? 0.f : __expf(s[j][i] - m_run[i]);
        const uint16_t ph = f2h(p);
        psum[i] += h2f(ph);
        pb[(4 * g + i) * L::P_LD + 16 * j + n] = ph;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) psum[i] += __shfl_xor(psum[i], o, 16);
      l_run[i] = l_run[i] * corr[i] + psum[i];
    }
#pragma unroll
    for (int jn = 0; jn < D / 16; ++jn) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[jn][i] *= corr[i];
    }

    // ---------------- V tile -> kv[c * V_LD + t]  (lane = token)
    {
      const int t = lane;
      if (quant) {
        const int tok = tile * kTile + t;
#pragma unroll
        for (int vg = 0; vg < NG; ++vg) {
          const int64_t midx = b * a.vm_sb + kvh * a.vm_sh + (int64_t)tok * NG + vg;
          const DeqRow r = deq_row(meta_load(a.v_mn, midx, a.meta_dtype), meta_load(a.v_scale, midx, a.meta_dtype),
                                   qmax, true);
          const uint8_t* prow = a.v_packed + b * a.vp_sb + kvh * a.vp_sh + ((int64_t)tok * NG + vg) * QB;
          uint32_t w[QB / 4];
#pragma unroll
          for (int i = 0; i < QB / 4; ++i) w[i] = ((const uint32_t*)prow)[i];
          const uint8_t* bytes = (const uint8_t*)w;
#pragma unroll
          for (int c = 0; c < 64; ++c) {
            if (64 * vg + c < D) {
              const uint32_t q = unpack_code<BITS>(bytes, c);
              kv[(64 * vg + c) * L::V_LD + t] = f2h(M::load(M::cvt(deq_value(r, q, EV))));
            }
          }
        }
      } else if (t < n_valid) {
        const uint16_t* src = (const uint16_t*)a.v_res + b * a.vr_sb + kvh * a.vr_sh + (int64_t)(r0 + t) * a.vr_st;
#pragma unroll
        for (int c = 0; c < D; c += 8) {
          const u32x4 v = *(const u32x4*)(src + c);
          const uint16_t* hv = (const uint16_t*)&v;
#pragma unroll
          for (int e = 0; e < 8; ++e) kv[(c + e) * L::V_LD + t] = IO == MZ_F16 ? hv[e] : f2h(bf2f(hv[e]));
        }
      } else {
#pragma unroll
        for (int c = 0; c < D; ++c) kv[c * L::V_LD + t] = 0;
      }
    }
    wave_lds_sync();

    // ---------------- acc += P V : A = P[m=n][32ks+8g..], B = V[32ks+8g..][16jn+n]
#pragma unroll
    for (int ks = 0; ks < kTile / 32; ++ks) {
      const u32x4 pa = *(const u32x4*)(pb + n * L::P_LD + 32 * ks + 8 * g);
#pragma unroll
      for (int jn = 0; jn < D / 16; ++jn) {
        const u32x4 vb = *(const u32x4*)(kv + (16 * jn + n) * L::V_LD + 32 * ks + 8 * g);
        acc[jn] = Mfma<MZ_F16>::run(pa, vb, acc[jn]);
      }
    }
    wave_lds_sync();
  }

  // ---------------- merge the 4 waves' states, write the split partial
  __syncthreads();
  float* red = (float*)lds;  // per wave: m[16], l[16], acc[16][D]
  constexpr int RED = 32 + 16 * D;
  {
    float* w = red + wave * RED;
    if (n == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) { w[4 * g + i] = m_run[i]; w[16 + 4 * g + i] = l_run[i]; }
    }
#pragma unroll
    for (int jn = 0; jn < D / 16; ++jn) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[32 + (4 * g + i) * D + 16 * jn + n] = acc[jn][i];
    }
  }
  __syncthreads();
  float* ws = (float*)a.workspace;
  const int Hq = a.kv_heads * n_rep;
  for (int e = threadIdx.x; e < n_rep * (D + 2); e += 256) {
    const int h = e / (D + 2);
    const int c = e - h * (D + 2);
    float M_ = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M_ = fmaxf(M_, red[w * RED + h]);
    float val = 0.f;
    if (c == D) {
      val = M_;
    } else if (M_ != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = __expf(red[w * RED + h] - M_);
        val += f * (c == D + 1 ? red[w * RED + 16 + h] : red[w * RED + 32 + h * D + c]);
      }
    }
    const int64_t row = ((int64_t)b * Hq + kvh * n_rep + h) * n_split + split;
    ws[row * (D + 2) + c] = val;
  }
}

// Merge the splits of one (batch, q-head): out = sum_s e^{m_s-M} acc_s / sum_s e^{m_s-M} l_s.
template <int D>
__global__ __launch_bounds__(D) void decode_combine_kernel(const float* __restrict__ ws, int n_split, int Hq,
                                                           void* out, int out_dtype, int64_t out_sb, int64_t out_sh) {
  const int bh = blockIdx.x;
  const int c = threadIdx.x;
  const float* base = ws + (int64_t)bh * n_split * (D + 2);
  float M_ = -INFINITY;
  for (int s = 0; s < n_split; ++s) M_ = fmaxf(M_, base[s * (D + 2) + D]);
  float num = 0.f, den = 0.f;
  if (M_ != -INFINITY) {
    for (int s = 0; s < n_split; ++s) {
      const float f = __expf(base[s * (D + 2) + D] - M_);
      num += f * base[s * (D + 2) + c];
      den += f * base[s * (D + 2) + D + 1];
    }
  }
  const float o = den > 0.f ? num / den : 0.f;
  const int b = bh / Hq, h = bh - b * Hq;
  store_val(out, b * out_sb + (int64_t)h * out_sh + c, o, out_dtype);
}

bool fold_supported(const mz_decode_args* a);
int fold_choose_split(const mz_decode_args* a, int* tiles_per_split);
int fold_launch_partials(const mz_decode_args* a, hipStream_t s, bool direct);

static int choose_split(const mz_decode_args* a, int* tiles_per_split) {
  const int n_tiles = a->n_groups + (a->n_residual + kTile - 1) / kTile;
  if (n_tiles <= 0) { *tiles_per_split = 1; return 1; }
  int ns = a->n_split;
  if (ns <= 0) {
    const int64_t units = (int64_t)a->batch * a->kv_heads;
    const int64_t target = 2048;  // workgroups: several per CU on 256 CUs
    ns = (int)((target + units - 1) / units);
    // at least 4 tiles per split so each wave has work
    ns = max(1, min(ns, (n_tiles + 3) / 4));
  }
  ns = min(ns, n_tiles);
  const int tps = (n_tiles + ns - 1) / ns;
  *tiles_per_split = tps;
  return (n_tiles + tps - 1) / tps;
}

static int check_args(const mz_decode_args* a) {
  if (!a) return MZ_EINVAL;
  if (a->batch < 0 || a->kv_heads <= 0 || a->n_rep <= 0 || a->n_groups < 0 || a->n_residual < 0) return MZ_EINVAL;
  if (a->bits < 1 || a->bits > 8) return MZ_EINVAL;
  if (a->io_dtype != MZ_BF16 && a->io_dtype != MZ_F16) return MZ_EINVAL;
  if (a->meta_dtype != MZ_F16 && a->meta_dtype != MZ_BF16 && a->meta_dtype != MZ_F32) return MZ_EINVAL;
  if (a->out_dtype != a->io_dtype && a->out_dtype != MZ_F32) return MZ_EINVAL;
  if (a->kernel_path < MZ_PATH_AUTO || a->kernel_path > MZ_PATH_FOLD) return MZ_EINVAL;
  if (a->head_dim != 64 && a->head_dim != 128) return MZ_EUNSUPPORTED;
  if (a->n_rep > 16) return MZ_EUNSUPPORTED;
  if (a->batch == 0) return MZ_OK;
  if (!a->query || !a->out) return MZ_EINVAL;
  if (a->n_groups > 0 && (!a->k_packed || !a->k_mn || !a->k_scale || !a->v_packed || !a->v_mn || !a->v_scale ||
                          !a->e_key || !a->e_value))
    return MZ_EINVAL;
  if (a->n_residual > 0 && (!a->k_res || !a->v_res)) return MZ_EINVAL;
  // 16-byte vector loads of query rows and residual rows
  if (((uintptr_t)a->query & 15) || (a->q_sh & 7) || (a->q_sb & 7)) return MZ_EINVAL;
  if (a->n_residual > 0 && (((uintptr_t)a->k_res & 15) || ((uintptr_t)a->v_res & 15) || (a->kr_st & 7) ||
                            (a->kr_sh & 7) || (a->kr_sb & 7) || (a->vr_st & 7) || (a->vr_sh & 7) || (a->vr_sb & 7)))
    return MZ_EINVAL;
  if (a->n_groups > 0 && (((uintptr_t)a->k_packed & 3) || ((uintptr_t)a->v_packed & 3) || (a->kp_sb & 3) ||
                          (a->kp_sh & 3) || (a->vp_sb & 3) || (a->vp_sh & 3)))
    return MZ_EINVAL;
  return MZ_OK;
}

// Which kernel runs and with how many splits (both kernels share the
// workspace layout and the combine kernel).
static bool use_fold(const mz_decode_args* a) {
  if (a->kernel_path == MZ_PATH_EXACT) return false;
  return fold_supported(a);
}

static int plan_split(const mz_decode_args* a, int* tps) {
  return use_fold(a) ? fold_choose_split(a, tps) : choose_split(a, tps);
}

}  // namespace mz

using namespace mz;

extern "C" int64_t muzero_decode_workspace_bytes(const mz_decode_args* a, int* n_split_out) {
  if (check_args(a) != MZ_OK) return -1;
  if (a->kernel_path == MZ_PATH_FOLD && !fold_supported(a)) return -1;
  int tps;
  const int ns = plan_split(a, &tps);
  if (n_split_out) *n_split_out = ns;
  return (int64_t)a->batch * a->kv_heads * a->n_rep * ns * (a->head_dim + 2) * (int64_t)sizeof(float);
}

extern "C" int muzero_decode_uses_fold(const mz_decode_args* a) {
  if (check_args(a) != MZ_OK) return -1;
  return use_fold(a) ? 1 : 0;
}

template <int D, int IO>
static int launch_partials(const mz_decode_args* a, hipStream_t s) {
  int tps;
  const int ns = choose_split(a, &tps);
  static_assert(D == 64 || D == 128, "head_dim");
  const int64_t need = (int64_t)a->batch * a->kv_heads * a->n_rep * ns * (D + 2) * (int64_t)sizeof(float);
  if (!a->workspace || a->workspace_bytes < need) return MZ_EWORKSPACE;
  const dim3 grid(ns, a->kv_heads, a->batch);
  const size_t lds = Lds<D>::BYTES;
  switch (a->bits) {
#define MZ_CASE(BB)                                                                                      \
  case BB: {                                                                                             \
    static const hipError_t attr = hipFuncSetAttribute(                                                  \
        (const void*)decode_split_kernel<D, BB, IO>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds); \
    if (attr != hipSuccess) return (int)attr;                                                            \
    hipLaunchKernelGGL((decode_split_kernel<D, BB, IO>), grid, dim3(256), lds, s, *a, tps, ns);          \
  } break;
    MZ_CASE(1) MZ_CASE(2) MZ_CASE(3) MZ_CASE(4) MZ_CASE(5) MZ_CASE(6) MZ_CASE(7) MZ_CASE(8)
#undef MZ_CASE
    default: return MZ_EINVAL;
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

template <int D, int IO>
static int launch_combine(const mz_decode_args* a, hipStream_t s) {
  int tps;
  const int ns = plan_split(a, &tps);
  const int64_t need = (int64_t)a->batch * a->kv_heads * a->n_rep * ns * (D + 2) * (int64_t)sizeof(float);
  if (!a->workspace || a->workspace_bytes < need) return MZ_EWORKSPACE;
  const int Hq = a->kv_heads * a->n_rep;
  hipLaunchKernelGGL((decode_combine_kernel<D>), dim3(a->batch * Hq), dim3(D), 0, s,
                     (const float*)a->workspace, ns, Hq, a->out, a->out_dtype, a->out_sb, a->out_sh);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

static int decode_check_launchable(const mz_decode_args* a) {
  int st = check_args(a);
  if (st != MZ_OK) return st;
  if (a->batch == 0) return 1;
  if (a->n_groups + a->n_residual == 0) return MZ_EINVAL;  // nothing to attend to
  return MZ_OK;
}

extern "C" int muzero_decode_partials(const mz_decode_args* a, mz_stream_t stream) {
  const int st = decode_check_launchable(a);
  if (st) return st == 1 ? MZ_OK : st;
  hipStream_t s = (hipStream_t)stream;
  if (a->kernel_path == MZ_PATH_FOLD && !fold_supported(a)) return MZ_EUNSUPPORTED;
  if (use_fold(a)) {
    int tps;
    const int ns = fold_choose_split(a, &tps);
    const int64_t need = (int64_t)a->batch * a->kv_heads * a->n_rep * ns * (a->head_dim + 2) * (int64_t)sizeof(float);
    if (!a->workspace || a->workspace_bytes < need) return MZ_EWORKSPACE;
    return fold_launch_partials(a, s, false);
  }
  if (a->head_dim == 128)
    return a->io_dtype == MZ_BF16 ? launch_partials<128, MZ_BF16>(a, s) : launch_partials<128, MZ_F16>(a, s);
  return a->io_dtype == MZ_BF16 ? launch_partials<64, MZ_BF16>(a, s) : launch_partials<64, MZ_F16>(a, s);
}

extern "C" int muzero_decode_combine(const mz_decode_args* a, mz_stream_t stream) {
  const int st = decode_check_launchable(a);
  if (st) return st == 1 ? MZ_OK : st;
  if (!a->out) return MZ_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  if (a->head_dim == 128)
    return a->io_dtype == MZ_BF16 ? launch_combine<128, MZ_BF16>(a, s) : launch_combine<128, MZ_F16>(a, s);
  return a->io_dtype == MZ_BF16 ? launch_combine<64, MZ_BF16>(a, s) : launch_combine<64, MZ_F16>(a, s);
}

extern "C" int muzero_decode_attention(const mz_decode_args* a, mz_stream_t stream) {
  // fold path with one split: the split kernel writes the output (no workspace, no combine)
  if (decode_check_launchable(a) == MZ_OK && a->out && use_fold(a)) {
    int tps;
    if (fold_choose_split(a, &tps) == 1) return fold_launch_partials(a, (hipStream_t)stream, true);
  }
  const int st = muzero_decode_partials(a, stream);
  if (st != MZ_OK) return st;
  return muzero_decode_combine(a, stream);
}
