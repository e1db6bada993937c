// Separate QK and AV launches over a packed prefix (gfx950, wave64).
//
// The reference's default decode path (muzero/cache/attention.py:179-295,
// MUZERO_FUSED_PREFIX_DECODE unset) runs three steps: qk writes the logits of
// the packed key prefix in the query dtype, torch takes the softmax, av writes
// the weighted sum of the packed value prefix.  This file implements qk and
// av with the reference's argument meaning (muzero/kernels/loader.py:46-53);
// the fused decode kernels (decode.hip, decode_fold.hip) do all three steps in
// one pass and are what the cache's decode hook runs.
//
// Both launches are one computation on 64-code rows: a wave takes a chunk of
// up to 64 rows, lane i dequantizes code i of every row and adds
// coefficient(row, head) * value to one accumulator per query head of the
// kv-head.
//   qk: rows = the D channels of one key group (64 tokens), lane = token,
//       coefficient = the query's channel; the accumulators are the group's
//       logits.  A wave owns two key groups.
//   av: rows = tokens of one value group (64 channels), lane = channel,
//       coefficient = the token's attention weight.  A workgroup owns a
//       (batch, kv-head, value group); its 4 waves take every 4th 64-token
//       chunk and add their sums through LDS in a fixed order (no atomics:
//       results are deterministic).
// Per chunk, in the wave's LDS area: the rows' packed bytes (one row per lane,
// 8-byte global loads, written at an odd dword pitch so that neither the
// stores nor the per-row code reads meet on a bank), each row's
// dequantization parameters (from the stored metadata), and for codes of up
// to 5 bits a codebook of every code's value per row, lane r writing row r's
// 2^bits entries, so a row costs 2^bits / 64 dequantizations per lane instead
// of one.  Wider codes are dequantized one per lane and row from the row's
// parameters (an LDS broadcast).  Every value is the reference's fp32
// dequantized value exactly (deq_value: muzero/quantizer.py:229-255 op for
// op, the expm1 rows read from the host-built table: copied to LDS once per
// workgroup for codes of up to 6 bits, read from global memory for 7 and 8);
// sums are fp32 multiply-adds, rounded once to the io dtype at the end.
#include <atomic>

#include "decode_common.hpp"

namespace mz {

namespace rowdot {

constexpr int kRows = 64;   // rows per chunk
constexpr int kWaves = 4;   // waves per workgroup
constexpr int kMaxHeadDim = 256;
constexpr int kMaxRep = 16;
constexpr int kGroupsPerWave = 2;  // qk: key groups per wave

// Byte layout of one wave's LDS area.
template <int BITS, int NR>
struct Area {
  static constexpr int QB = 8 * BITS;        // bytes per packed row
  static constexpr int PITCH = QB + 4;       // staged row pitch: an odd number of dwords
  static constexpr bool CB = BITS <= 5;      // codebook per row
  static constexpr int NCB = 1 << BITS;
  // codebook row pitch in floats: rows 8 apart share banks, so the 16-byte
  // stores of a row's entries (8 lanes at a time) do not conflict
  static constexpr int CBP = NCB == 2 ? 2 : NCB + 4;
  static constexpr int STAGE = kRows * PITCH + 16;  // + the dword read past the last row's end
  // wider codes: 48 bytes of parameters per row, read by every lane
  static constexpr int PAR_OFF = STAGE;
  static constexpr int CB_OFF = PAR_OFF + (CB ? 0 : kRows * 48);
  static constexpr int COEF_OFF = CB_OFF + (CB ? kRows * CBP * 4 : 0);
  // `coef`: the area also holds the chunk's coefficients [row][NR] (av)
  static constexpr int bytes(bool coef) { return COEF_OFF + (coef ? kRows * NR * 4 : 0); }
  static_assert(STAGE % 16 == 0 && (CB_OFF % 16) == 0, "16-byte aligned parts");
};

// The reference's fp32 dequantized value of code q (muzero/quantizer.py:250-
// 255): the same operations as deq_value, in the same order, with the branch
// on q >= zl turned into selects (za - ne*e is computed as za + (-ne)*e, which
// rounds identically), so a lane issues its table read without waiting on a
// branch.
__device__ __forceinline__ float deq_select(const DeqRow& r, uint32_t q, const float* E) {
  const float qf = (float)q;
  const bool pos = qf >= r.zl;
  const int dp = min(max((int)(qf - r.zl), 0), (int)r.pb);
  const int dn = min(max((int)(r.zl - qf), 0), (int)r.nb);
  const float e = E[pos ? r.offp + dp : r.offn + dn];
  const float t = (pos ? r.pe : -r.ne) * e;
  const float norm = clamp01(r.za + t);
  const float u = norm * r.s;
  return u + r.mn;
}

// expm1 rows in LDS (codes of up to 6 bits; 7- and 8-bit rows, up to 128 KB,
// stay in global memory): EF floats, rounded up to 16 bytes.
template <int BITS>
constexpr int etab_bytes() {
  return BITS <= 6 ? ((((1 << BITS) - 1) * ((1 << BITS) + 2) / 2) * 4 + 15) & ~15 : 0;
}

// Copy the expm1 rows to the start of LDS (all threads; the caller syncs).
template <int BITS>
__device__ __forceinline__ const float* stage_etab(uint8_t* lds, const float* e) {
  if constexpr (etab_bytes<BITS>() == 0) {
    return e;
  } else {
    constexpr int EF = ((1 << BITS) - 1) * ((1 << BITS) + 2) / 2;
    float* t = (float*)lds;
    for (int i = threadIdx.x; i < EF; i += 256) t[i] = e[i];
    return t;
  }
}

__device__ __forceinline__ void put_row(uint8_t* p, const DeqRow& r) {
  float4* f = (float4*)p;
  f[0] = make_float4(r.mn, r.s, r.za, r.zl);
  f[1] = make_float4(r.pb, r.nb, r.pe, r.ne);
  f[2] = make_float4(__int_as_float(r.offp), __int_as_float(r.offn), 0.f, 0.f);
}

__device__ __forceinline__ DeqRow get_row(const uint8_t* p) {
  const float4* f = (const float4*)p;
  const float4 a = f[0], b = f[1], c = f[2];
  DeqRow r;
  r.mn = a.x; r.s = a.y; r.za = a.z; r.zl = a.w;
  r.pb = b.x; r.nb = b.y; r.pe = b.z; r.ne = b.w;
  r.offp = __float_as_int(c.x); r.offn = __float_as_int(c.y);
  return r;
}

// A chunk's global inputs, held in registers: a wave loads chunk c+1's while
// it computes chunk c.  Lane r holds row r's packed bytes and metadata (and,
// for av, the weights of token r).
template <int BITS, int NR>
struct Fetch {
  uint2 row[BITS];
  float mn, sc;
  float w[NR];
};

// Row r's packed bytes start at rows + r*row_stride, its metadata at index
// meta0 + r*meta_stride of mn / sc (r < nrows).
template <int BITS, int NR>
__device__ __forceinline__ void fetch_rows(Fetch<BITS, NR>& f, const uint8_t* rows, int64_t row_stride,
                                           const void* mn, const void* sc, int64_t meta0, int64_t meta_stride,
                                           int mdt, int nrows) {
  const int lane = threadIdx.x & 63;
  if (lane < nrows) {
    const uint2* src = (const uint2*)(rows + lane * row_stride);
#pragma unroll
    for (int k = 0; k < BITS; ++k) f.row[k] = src[k];
    const int64_t m = meta0 + lane * meta_stride;
    f.mn = load_any(mn, m, mdt);
    f.sc = load_any(sc, m, mdt);
  }
}

// One chunk of `nrows` (<= 64) fetched rows; row r's coefficients are
// coef[r*NR + h] (LDS).  acc[h] += coef[r][h] * value(r, lane) over the rows.
template <int BITS, int NR>
__device__ __forceinline__ void chunk(uint8_t* area, const Fetch<BITS, NR>& f, const float* E, const float* coef,
                                      int nrows, float (&acc)[NR]) {
  using A = Area<BITS, NR>;
  constexpr float qmax = (float)((1 << BITS) - 1);
  const int lane = threadIdx.x & 63;
  if (lane < nrows) {
    uint32_t* dst = (uint32_t*)(area + lane * A::PITCH);
#pragma unroll
    for (int k = 0; k < BITS; ++k) {
      dst[2 * k] = f.row[k].x;
      dst[2 * k + 1] = f.row[k].y;
    }
    const DeqRow r = deq_row(f.mn, f.sc, qmax, true);
    if constexpr (A::CB) {
      // lane r writes row r's codebook
      float* cbr = (float*)(area + A::CB_OFF) + lane * A::CBP;
      if constexpr (A::NCB == 2) {
        *(float2*)cbr = make_float2(deq_select(r, 0, E), deq_select(r, 1, E));
      } else {
#pragma unroll
        for (int q = 0; q < A::NCB; q += 4)
          *(float4*)(cbr + q) = make_float4(deq_select(r, q, E), deq_select(r, q + 1, E), deq_select(r, q + 2, E),
                                            deq_select(r, q + 3, E));
      }
    } else {
      put_row(area + A::PAR_OFF + 48 * lane, r);
    }
  }
  wave_lds_sync();
  const float* cb = (const float*)(area + A::CB_OFF);
  // lane's code: bits [lane*BITS, lane*BITS + BITS) of the row
  const int bit = lane * BITS;
  const uint8_t* lrow = area + (bit >> 5) * 4;
  const uint32_t sh = bit & 31;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  constexpr bool straddle = (32 % BITS) != 0;
  auto row = [&](const int r) __attribute__((always_inline)) {
    const uint8_t* rp = lrow + r * A::PITCH;
    const uint32_t d0 = *(const uint32_t*)rp;
    uint32_t code;
    if constexpr (straddle) code = __builtin_amdgcn_alignbit(*(const uint32_t*)(rp + 4), d0, sh) & mask;
    else code = __builtin_amdgcn_ubfe(d0, sh, BITS);
    float x;
    if constexpr (A::CB) x = cb[r * A::CBP + code];
    else x = deq_select(get_row(area + A::PAR_OFF + 48 * r), code, E);
#pragma unroll
    for (int h = 0; h < NR; ++h) acc[h] = __builtin_fmaf(coef[r * NR + h], x, acc[h]);
  };
  if (nrows == kRows) {
    // a full chunk: every row's offsets are compile-time constants (immediate
    // offsets of the LDS reads), so a row costs its extract and multiply-adds
#pragma unroll
    for (int r = 0; r < kRows; ++r) row(r);
  } else {
#pragma unroll 4
    for (int r = 0; r < nrows; ++r) row(r);
  }
}

__host__ __device__ constexpr int qc_bytes(int D, int NR) { return (D * NR * 4 + 15) & ~15; }

template <int BITS, int NR>
constexpr int qk_lds_bytes(int D) {
  return etab_bytes<BITS>() + qc_bytes(D, NR) + kWaves * Area<BITS, NR>::bytes(false);
}
template <int BITS, int NR>
constexpr int av_lds_bytes() {
  constexpr int areas = kWaves * Area<BITS, NR>::bytes(true);
  constexpr int red = kWaves * NR * kRows * 4;
  return etab_bytes<BITS>() + (areas > red ? areas : red);
}

// grid (ceil(n_groups / 8), kv_heads, batch); wave w of workgroup x takes key
// groups 2(4x + w) and 2(4x + w) + 1.
template <int BITS, int NR>
__global__ __launch_bounds__(256) void qk_kernel(const mz_qk_args a) {
  using A = Area<BITS, NR>;
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int D = a.head_dim;
  const float* E = stage_etab<BITS>(lds, a.e_key);
  // the kv-head's query rows as fp32 coefficients [D][NR] (heads past n_rep are 0)
  float* qc = (float*)(lds + etab_bytes<BITS>());
  for (int i = threadIdx.x; i < D * NR; i += 256) {
    const int d = i / NR, h = i % NR;
    qc[i] = h < a.n_rep ? load_any(a.query, b * a.q_sb + (int64_t)(kvh * a.n_rep + h) * a.q_sh + d, a.io_dtype) : 0.f;
  }
  __syncthreads();
  const int g0 = (blockIdx.x * kWaves + wave) * kGroupsPerWave;
  const int groups = min(kGroupsPerWave, a.n_groups - g0);
  if (groups <= 0) return;
  uint8_t* area = lds + etab_bytes<BITS>() + qc_bytes(D, NR) + wave * A::bytes(false);
  const uint8_t* gp = a.k_packed + b * a.kp_sb + kvh * a.kp_sh + (int64_t)g0 * D * A::QB;
  const int64_t m0 = b * a.km_sb + kvh * a.km_sh + (int64_t)g0 * D;
  // items = (group, chunk of up to 64 channels); the wave's groups are
  // contiguous rows, channel d of its group i being row i*D + d
  const int cpg = (D + kRows - 1) / kRows;
  const int items = groups * cpg;
  auto rows_of = [&](int it) { return min(kRows, D - (it % cpg) * kRows); };
  auto row0_of = [&](int it) { return (it / cpg) * D + (it % cpg) * kRows; };
  Fetch<BITS, NR> f;
  fetch_rows(f, gp, A::QB, a.k_mn, a.k_scale, m0, 1, a.meta_dtype, rows_of(0));
  float acc[NR];
  for (int it = 0; it < items; ++it) {
    const Fetch<BITS, NR> cur = f;
    if (it + 1 < items) {
      const int r1 = row0_of(it + 1);
      fetch_rows(f, gp + (int64_t)r1 * A::QB, A::QB, a.k_mn, a.k_scale, m0 + r1, 1, a.meta_dtype, rows_of(it + 1));
    }
    const int c = it % cpg;
    if (c == 0) {
#pragma unroll
      for (int h = 0; h < NR; ++h) acc[h] = 0.f;
    }
    wave_lds_sync();  // the previous item's reads of the area are done
    chunk<BITS, NR>(area, cur, E, qc + c * kRows * NR, rows_of(it), acc);
    if (c == cpg - 1) {
      const int64_t o = b * a.o_sb + (int64_t)(g0 + it / cpg) * kRows + lane;
#pragma unroll
      for (int h = 0; h < NR; ++h)
        if (h < a.n_rep)
          store_val(a.logits, o + (int64_t)(kvh * a.n_rep + h) * a.o_sh, acc[h] * a.scaling, a.io_dtype);
    }
  }
}

// grid (value groups, kv_heads, batch).
template <int BITS, int NR>
__global__ __launch_bounds__(256) void av_kernel(const mz_av_args a) {
  using A = Area<BITS, NR>;
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int ng = (a.head_dim + kRows - 1) / kRows;
  // (no table to read when there are no tokens: the call writes zeros)
  const float* E = a.n_tokens > 0 ? stage_etab<BITS>(lds, a.e_value) : nullptr;
  if constexpr (etab_bytes<BITS>() > 0) __syncthreads();
  uint8_t* work = lds + etab_bytes<BITS>();
  uint8_t* area = work + wave * A::bytes(true);
  float* coef = (float*)(area + A::COEF_OFF);
  float acc[NR];
#pragma unroll
  for (int h = 0; h < NR; ++h) acc[h] = 0.f;
  const uint8_t* vp = a.v_packed + b * a.vp_sb + kvh * a.vp_sh + j * A::QB;
  const int64_t m0 = b * a.vm_sb + kvh * a.vm_sh + j;
  const int64_t w0 = b * a.w_sb + (int64_t)kvh * a.n_rep * a.w_sh;
  // chunk t0 = 64*(wave + 4k): its rows (tokens) and its tokens' weights
  auto fetch = [&](Fetch<BITS, NR>& f, int t0) {
    const int nrows = min(kRows, a.n_tokens - t0);
    fetch_rows(f, vp + (int64_t)t0 * ng * A::QB, (int64_t)ng * A::QB, a.v_mn, a.v_scale, m0 + (int64_t)t0 * ng, ng,
               a.meta_dtype, nrows);
    if (lane < nrows) {
#pragma unroll
      for (int h = 0; h < NR; ++h)
        f.w[h] = h < a.n_rep ? load_any(a.weights, w0 + h * a.w_sh + t0 + lane, a.io_dtype) : 0.f;
    }
  };
  Fetch<BITS, NR> f;
  int t0 = wave * kRows;
  if (t0 < a.n_tokens) fetch(f, t0);
  for (; t0 < a.n_tokens; t0 += kWaves * kRows) {
    const Fetch<BITS, NR> cur = f;
    if (t0 + kWaves * kRows < a.n_tokens) fetch(f, t0 + kWaves * kRows);
    const int nrows = min(kRows, a.n_tokens - t0);
    wave_lds_sync();  // the previous chunk's reads of the area are done
    if (lane < nrows) {
#pragma unroll
      for (int h = 0; h < NR; ++h) coef[lane * NR + h] = cur.w[h];
    }
    chunk<BITS, NR>(area, cur, E, coef, nrows, acc);
  }
  // the 4 waves' sums, added in wave order
  __syncthreads();
  float* red = (float*)work;  // [wave][NR][64]
#pragma unroll
  for (int h = 0; h < NR; ++h) red[(wave * NR + h) * kRows + lane] = acc[h];
  __syncthreads();
  const int c = j * kRows + lane;
  for (int h = wave; h < a.n_rep; h += kWaves) {
    float s = red[h * kRows + lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += red[(w * NR + h) * kRows + lane];
    if (c < a.head_dim) store_val(a.out, b * a.o_sb + (int64_t)(kvh * a.n_rep + h) * a.o_sh + c, s, a.io_dtype);
  }
}

// Query heads per kv-head rounded up to the accumulator count of a kernel.
inline int nr_for(int n_rep) { return n_rep <= 1 ? 1 : n_rep <= 2 ? 2 : n_rep <= 4 ? 4 : n_rep <= 8 ? 8 : 16; }

template <int BITS, int NR>
hipError_t launch_qk(const mz_qk_args& a, hipStream_t s) {
  static std::atomic<uint64_t> raised{0};
  const int bytes = qk_lds_bytes<BITS, NR>(a.head_dim);
  if (bytes > 65536) {
    const hipError_t e = set_dynamic_lds((const void*)qk_kernel<BITS, NR>, bytes, raised);
    if (e != hipSuccess) return e;
  }
  const int per_wg = kWaves * kGroupsPerWave;
  const dim3 grid((a.n_groups + per_wg - 1) / per_wg, a.kv_heads, a.batch);
  qk_kernel<BITS, NR><<<grid, dim3(256), bytes, s>>>(a);
  return hipGetLastError();
}

template <int BITS, int NR>
hipError_t launch_av(const mz_av_args& a, hipStream_t s) {
  static std::atomic<uint64_t> raised{0};
  constexpr int bytes = av_lds_bytes<BITS, NR>();
  if constexpr (bytes > 65536) {
    const hipError_t e = set_dynamic_lds((const void*)av_kernel<BITS, NR>, bytes, raised);
    if (e != hipSuccess) return e;
  }
  const dim3 grid((a.head_dim + kRows - 1) / kRows, a.kv_heads, a.batch);
  av_kernel<BITS, NR><<<grid, dim3(256), bytes, s>>>(a);
  return hipGetLastError();
}

template <int BITS>
hipError_t qk_nr(const mz_qk_args& a, hipStream_t s) {
  switch (nr_for(a.n_rep)) {
    case 1: return launch_qk<BITS, 1>(a, s);
    case 2: return launch_qk<BITS, 2>(a, s);
    case 4: return launch_qk<BITS, 4>(a, s);
    case 8: return launch_qk<BITS, 8>(a, s);
    default: return launch_qk<BITS, 16>(a, s);
  }
}

template <int BITS>
hipError_t av_nr(const mz_av_args& a, hipStream_t s) {
  switch (nr_for(a.n_rep)) {
    case 1: return launch_av<BITS, 1>(a, s);
    case 2: return launch_av<BITS, 2>(a, s);
    case 4: return launch_av<BITS, 4>(a, s);
    case 8: return launch_av<BITS, 8>(a, s);
    default: return launch_av<BITS, 16>(a, s);
  }
}

inline bool dtype_ok(int dt) { return dt == MZ_F32 || dt == MZ_BF16 || dt == MZ_F16; }
inline bool aligned8(const void* p) { return ((uintptr_t)p & 7u) == 0; }

int status(hipError_t e) { return e == hipSuccess ? MZ_OK : (int)e; }

}  // namespace rowdot
}  // namespace mz

using namespace mz;
using namespace mz::rowdot;

extern "C" int muzero_qk(const mz_qk_args* a, mz_stream_t stream) {
  if (a == nullptr) return MZ_EINVAL;
  if (a->batch < 0 || a->kv_heads < 1 || a->n_rep < 1 || a->head_dim < 1 || a->n_groups < 0) return MZ_EINVAL;
  if (a->bits < 1 || a->bits > 8 || !dtype_ok(a->io_dtype) || !dtype_ok(a->meta_dtype)) return MZ_EINVAL;
  if (a->n_rep > kMaxRep || a->head_dim > kMaxHeadDim) return MZ_EUNSUPPORTED;
  if (a->batch > 65535 || a->kv_heads > 65535) return MZ_EUNSUPPORTED;
  if (a->batch == 0 || a->n_groups == 0) return MZ_OK;
  if (!a->query || !a->k_packed || !a->k_mn || !a->k_scale || !a->e_key || !a->logits) return MZ_EINVAL;
  if (!aligned8(a->k_packed) || (a->kp_sb & 7) || (a->kp_sh & 7)) return MZ_EINVAL;
  const hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (a->bits) {
    case 1: e = qk_nr<1>(*a, s); break;
    case 2: e = qk_nr<2>(*a, s); break;
    case 3: e = qk_nr<3>(*a, s); break;
    case 4: e = qk_nr<4>(*a, s); break;
    case 5: e = qk_nr<5>(*a, s); break;
    case 6: e = qk_nr<6>(*a, s); break;
    case 7: e = qk_nr<7>(*a, s); break;
    default: e = qk_nr<8>(*a, s); break;
  }
  return status(e);
}

extern "C" int muzero_av(const mz_av_args* a, mz_stream_t stream) {
  if (a == nullptr) return MZ_EINVAL;
  if (a->batch < 0 || a->kv_heads < 1 || a->n_rep < 1 || a->head_dim < 1 || a->n_tokens < 0) return MZ_EINVAL;
  if (a->bits < 1 || a->bits > 8 || !dtype_ok(a->io_dtype) || !dtype_ok(a->meta_dtype)) return MZ_EINVAL;
  if (a->n_rep > kMaxRep || a->head_dim > kMaxHeadDim) return MZ_EUNSUPPORTED;
  if (a->batch > 65535 || a->kv_heads > 65535) return MZ_EUNSUPPORTED;
  if (a->batch == 0) return MZ_OK;
  if (!a->out || (a->n_tokens > 0 && (!a->weights || !a->v_packed || !a->v_mn || !a->v_scale || !a->e_value)))
    return MZ_EINVAL;
  if (a->n_tokens > 0 && (!aligned8(a->v_packed) || (a->vp_sb & 7) || (a->vp_sh & 7))) return MZ_EINVAL;
  const hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (a->bits) {
    case 1: e = av_nr<1>(*a, s); break;
    case 2: e = av_nr<2>(*a, s); break;
    case 3: e = av_nr<3>(*a, s); break;
    case 4: e = av_nr<4>(*a, s); break;
    case 5: e = av_nr<5>(*a, s); break;
    case 6: e = av_nr<6>(*a, s); break;
    case 7: e = av_nr<7>(*a, s); break;
    default: e = av_nr<8>(*a, s); break;
  }
  return status(e);
}
