// Quantize + bit-pack and dequantize kernels (gfx950, wave64).
//
// Quantize: 2 lanes per 64-value group, 32 consecutive values per lane, so a
// wave quantizes 32 groups.  The group min/max is an in-lane reduction plus
// one DPP step; the group's compander parameters are computed once per lane; every
// per-element op of the reference quantizer (muzero/quantizer.py:161-186) is
// evaluated in its own dtype with IEEE rounding and no contraction, and the
// one transcendental step (round(log1p(alpha*p)/lb*bins)) comes from a
// host-built constant table staged in LDS, so codes and metadata are
// bit-identical to the reference torch path.  8 codes of BITS bits are exactly
// BITS bytes of the LSB-first bitstream (quantizer.py:189-202), so each lane
// packs and stores its own bytes and a wave's stores are contiguous.  The grid
// is persistent (a few workgroups per CU loop over the groups), so each
// workgroup stages the table once.
#include "common.hpp"

#include <algorithm>
#include <type_traits>

namespace mz {

constexpr int QWG = 256;  // threads per quantize workgroup
// Values per lane: each lane quantizes 32 values of a 64-value group (two
// lanes per group), so a wave quantizes 32 groups and a group's parameters
// are formed once per 32 values.  Key groups read their column from an LDS
// tile.
constexpr int QN_ROWS = 32;
constexpr int QN_KEYS = 32;

// Compander parameters of one group (quantizer.py:169-181), every op rounded
// to the input dtype DT.
struct QParams {
  float mn, sc, za, zl, pb, nb, pe, ne, eps;
  float rsc, rpe, rne;  // v_rcp_f32 of sc, pe, ne (16-bit inputs only)
  float ea, ec;         // fp32 inputs: the table's alpha estimate and 1 / log2(1 + ea) (see code_offset_f32)
};

// rnd<DT>(a / b) for a, b values of the 16-bit input dtype, given r = rcp(b).
// bf16: a and b have 8-bit significands, so a / b is never a bf16 rounding
// midpoint and lies at least 2^7 fp32 ulps from one (a = b * odd 9-bit
// significand is impossible; the distance is >= 1/B bf16 half-ulps with the
// odd part B < 2^8); a * rcp(b) is within 3 ulps, so rounding it to bf16 gives
// the reference's round(fp32 division).  fp16 (11-bit significands, distance
// >= 2 ulps) takes one residual correction (< 1 ulp) except where b is 0 or
// inf, where a * rcp(b) is already the IEEE quotient (inf, NaN or 0).  rcp of
// a b above 2^126 would be denormal: such groups use the IEEE division.
template <int DT, bool FAST>
__device__ __forceinline__ float qdiv(float a, float b, float r) {
  if constexpr (DT == MZ_F32 || !FAST) {
    return rnd<DT>(a / b);
  } else if constexpr (DT == MZ_BF16) {
    return rnd<DT>(a * r);
  } else {
    const float q0 = a * r;
    const float q1 = fmaf(fmaf(-b, q0, a), r, q0);
    return rnd<DT>((b != 0.f && b != __builtin_inff()) ? q1 : q0);
  }
}

// Whether the reciprocal form applies to every division of the group.
template <int DT>
__device__ __forceinline__ bool qfast(const struct QParams& g) {
  if constexpr (DT == MZ_F16) return true;  // an fp16 scale is <= 65504 or inf
  return DT != MZ_F32 && !(g.sc > 0x1p126f && g.sc < __builtin_inff());
}

template <int DT, int BITS>
__device__ __forceinline__ QParams qparams(float mn, float mx, float eps_in) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  QParams g;
  g.eps = rnd<DT>(eps_in);
  g.mn = mn;
  g.sc = clamp_min(rnd<DT>(mx - mn), g.eps);
  if constexpr (DT == MZ_BF16) {
    // the reciprocal form of the division (exact for bf16 operands, see
    // qdiv) unless the scale's reciprocal would be denormal; the IEEE
    // division runs only in a wave that holds such a group
    g.rsc = __builtin_amdgcn_rcpf(g.sc);
    const float a = rnd<DT>(0.f - mn);
    float zq = rnd<DT>(a * g.rsc);
    const bool slow = g.sc > 0x1p126f && g.sc < __builtin_inff();
    if (__ballot(slow) != 0) {
      if (slow) zq = rnd<DT>(a / g.sc);
    }
    g.za = clamp01(zq);
  } else {
    g.za = clamp01(rnd<DT>(rnd<DT>(0.f - mn) / g.sc));
  }
  g.zl = rintf(rnd<DT>(g.za * qmax));
  g.pb = clamp_min(rnd<DT>(qmax - g.zl), 1.f);
  g.nb = clamp_min(g.zl, 1.f);
  g.pe = clamp_min(rnd<DT>(1.f - g.za), g.eps);
  g.ne = clamp_min(g.za, g.eps);
  if constexpr (DT != MZ_F32) {
    if constexpr (DT != MZ_BF16) g.rsc = __builtin_amdgcn_rcpf(g.sc);
    g.rpe = __builtin_amdgcn_rcpf(g.pe);
    g.rne = __builtin_amdgcn_rcpf(g.ne);
  }
  return g;
}

// Compander table in LDS: fp32 inputs use the threshold rows of bins 1..qmax
// (#{k : p >= T[bins][k]}, binary search); bf16/fp16 inputs the 16-bit ratio
// table indexed by the pattern of p.  Table bytes staged per workgroup:
template <int DT, int BITS>
struct QTable {
  static constexpr int QMAX = (1 << BITS) - 1;
  static constexpr int BYTES = DT == MZ_F32 ? QMAX * (QMAX + 1) / 2 * 4
                                            : ((DT == MZ_BF16 ? 0x3F80 : 0x3C00) + 1) * 2;
  static constexpr bool IN_LDS = BYTES <= 40 * 1024;  // 8-bit fp32 thresholds (128 KB) stay in global memory
  static constexpr int LDS_BYTES = IN_LDS ? (BYTES + 15) / 16 * 16 : 16;
};

template <int DT, int BITS>
__device__ __forceinline__ void stage_table(uint8_t* lds, const void* table) {
  using TB = QTable<DT, BITS>;
  if constexpr (TB::IN_LDS) {
    const uint16_t* src = (const uint16_t*)table;
    for (int i = threadIdx.x; i < TB::BYTES / 2; i += QWG) ((uint16_t*)lds)[i] = src[i];
    __syncthreads();
  }
}

// fp32 inputs: the code offset #{k in 1..bins : row[k-1] <= p} of a
// normalised distance p over the threshold row of `bins` (monotone: the
// offset is the reference's round(log1p(alpha*p) / lb * bins), tables.py).
// An estimate from the hardware log2 (bins * log2(1 + ea*p) * ec, ea the
// alpha the row of bins 1 implies) is within one of it; four independent
// reads of the thresholds around it give the count, and two of them check
// that the estimate's window [k0, k0 + 2] holds it (every threshold up to
// k0 at or below p, the one after k0 + 2 above).  Where the check fails the
// binary search runs, so the result is exact whatever the estimate.  Used
// from 5 bits (rows of up to 31 .. 255 thresholds: 5 to 8 dependent reads
// of the binary search); 8-bit keys / values 1.65x / 2.3x faster.
__device__ __forceinline__ int code_offset_f32(const float* row, int bins, float p, const QParams& g) {
  const float e = (float)bins * __builtin_amdgcn_logf(fmaf(g.ea, p, 1.f)) * g.ec;
  const float r = rintf(e) - 1.f;
  const int k0 = (int)__builtin_amdgcn_fmed3f(r == r ? r : 0.f, 0.f, (float)max(bins - 2, 0));
  // row[k0 - 1 .. k0 + 2], each index kept inside the row (an entry outside
  // it is not used: its test is decided by the bounds instead)
  const float t0 = row[max(k0 - 1, 0)], t1 = row[min(k0, bins - 1)], t2 = row[min(k0 + 1, bins - 1)],
              t3 = row[min(k0 + 2, bins - 1)];
  const bool below = k0 == 0 || t0 <= p;         // thresholds 1..k0 at or below p
  const bool above = k0 + 3 > bins || t3 > p;    // thresholds k0 + 3.. above p
  const int cnt = k0 + (k0 + 1 <= bins && t1 <= p ? 1 : 0) + (k0 + 2 <= bins && t2 <= p ? 1 : 0);
  if (below && above) return cnt;
  int lo = 0, hi = bins;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (row[mid] <= p) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Code of one value given its group's parameters (quantizer.py:172-184).
// FINITE: the group's mn and scale are finite and every divisor (scale, pe,
// ne) is positive, so no intermediate is NaN or infinite and every clamped
// quantity is >= 0 (v >= mn; the side's offset from za is >= 0): the NaN
// cases and the lower clamps drop out and give the same results.
template <int DT, int BITS, bool FAST, bool FINITE>
__device__ __forceinline__ uint32_t value_code(float v, const QParams& g, const uint8_t* lds, const void* table) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  const float n0 = qdiv<DT, FAST>(rnd<DT>(v - g.mn), g.sc, g.rsc);
  const float norm = FINITE ? fminf(n0, 1.f) : clamp01(n0);
  const bool up = norm >= g.za;  // torch.where(norm >= za, q_pos, q_neg); false on NaN
  // Only the selected side is evaluated: operands are chosen before the one
  // division, which computes exactly what the unselected-branch form would.
  const float p0 = qdiv<DT, FAST>(rnd<DT>(up ? norm - g.za : g.za - norm), up ? g.pe : g.ne, up ? g.rpe : g.rne);
  const float p = FINITE ? fminf(p0, 1.f) : clamp01(p0);
  const float bins = up ? g.pb : g.nb;
  float off;
  if constexpr (DT == MZ_F32) {
    const float* T = QTable<DT, BITS>::IN_LDS ? (const float*)lds : (const float*)table;
    const int ib = (FINITE || bins == bins) ? (int)bins : 1;
    const float* row = T + ib * (ib - 1) / 2;
    int lo;
    if constexpr (BITS >= 5) {
      lo = code_offset_f32(row, ib, p, g);
    } else {
      // up to 15 thresholds a row: the binary search's 4 steps measured as fast as the estimate
      lo = 0;
      int hi = ib;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (row[mid] <= p) lo = mid + 1; else hi = mid;
      }
    }
    off = (FINITE || p == p) ? (float)lo : __builtin_nanf("");
  } else {
    const uint16_t* Y = (const uint16_t*)lds;
    float y;
    if (FINITE || p == p) {
      const uint32_t pat = (DT == MZ_BF16 ? (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)p)  // p is not NaN
                                          : (uint32_t)f2h(p)) & 0x7FFFu;                          // -0 -> 0
      y = DT == MZ_BF16 ? bf2f(Y[pat]) : h2f(Y[pat]);
    } else {
      y = p;
    }
    off = rintf(rnd<DT>(y * bins));
  }
  // zl +- off is an integer in [-1, qmax + 1] <= 256 there: exact in every
  // input dtype, so its rounding is the identity
  const float q = FINITE ? (up ? g.zl + off : g.zl - off) : rnd<DT>(up ? g.zl + off : g.zl - off);
  // clamp(0, qmax).to(uint8); a NaN code converts to 0 (as on the reference CPU)
  if (!FINITE && !(q == q)) return 0u;
  return (uint32_t)fminf(fmaxf(q, 0.f), qmax);
}

// value_code<MZ_BF16, BITS, true, true> of two values at once (the two
// chains interleave; each rounding to bf16 is one v_cvt_pk_bf16_f32).
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void rnd_bf16_pair(float& a, float& b) {
  a = rnd<MZ_BF16>(a);
  b = rnd<MZ_BF16>(b);
}

//
// The same values as the op-by-op chain, in fewer ops (every rewrite below is
// exact for a finite group: mn and the scale finite, the divisors positive):
//  - min(rnd(x), 1) = rnd(min(x, 1)) (1 is a bf16 value and rounding is
//    monotone), and x >= 0, so the clamp rides on the multiply (med3 = the
//    VOP3 clamp bit);
//  - the selected side's difference, za - n below za and n - za above, is
//    |n - za| (fp32 negation is exact, and bf16 rounding is symmetric);
//  - the down side's offset is subtracted: zl - rint(rnd(y * nb)) =
//    zl + rint(rnd(y * -nb)) (both roundings are symmetric);
//  - p is a bf16 value >= +0 with a zero low half, so its ratio-table byte
//    address, pattern * 2, is its bit pattern >> 15.
template <int BITS>
__device__ __forceinline__ void value_code_bf16_pair(float v0, float v1, const QParams& g, const uint8_t* lds,
                                                     uint32_t& c0, uint32_t& c1) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  float a0 = v0 - g.mn, a1 = v1 - g.mn;
  rnd_bf16_pair(a0, a1);
  float n0 = __builtin_amdgcn_fmed3f(a0 * g.rsc, 0.f, 1.f), n1 = __builtin_amdgcn_fmed3f(a1 * g.rsc, 0.f, 1.f);
  rnd_bf16_pair(n0, n1);
  const bool up0 = n0 >= g.za, up1 = n1 >= g.za;
  float d0 = n0 - g.za, d1 = n1 - g.za;
  rnd_bf16_pair(d0, d1);  // |rnd(x)| = rnd(|x|): the absolute value rides on the multiply's operand
  float p0 = __builtin_amdgcn_fmed3f(__builtin_fabsf(d0) * (up0 ? g.rpe : g.rne), 0.f, 1.f);
  float p1 = __builtin_amdgcn_fmed3f(__builtin_fabsf(d1) * (up1 ? g.rpe : g.rne), 0.f, 1.f);
  rnd_bf16_pair(p0, p1);
  const float y0 = bf2f(*(const uint16_t*)(lds + (__float_as_uint(p0) >> 15)));
  const float y1 = bf2f(*(const uint16_t*)(lds + (__float_as_uint(p1) >> 15)));
  float o0 = y0 * (up0 ? g.pb : -g.nb), o1 = y1 * (up1 ? g.pb : -g.nb);
  rnd_bf16_pair(o0, o1);
  // zl + off: an integer in [-1, qmax + 1], exact in bf16 (its rounding is the identity)
  const float q0 = g.zl + rintf(o0), q1 = g.zl + rintf(o1);
  c0 = (uint32_t)__builtin_amdgcn_fmed3f(q0, 0.f, qmax);
  c1 = (uint32_t)__builtin_amdgcn_fmed3f(q1, 0.f, qmax);
}

// value_code<MZ_F16, BITS, true, true> with the rewrites of the bf16 pair
// form, which hold for fp16 as well (they use only that 1 is an fp16 value,
// that rounding is monotone and symmetric, and that in a finite group every
// quotient is >= +0).  Each division is a * rcp(b) plus one residual
// correction (qdiv; b is positive and finite here), the clamp riding on the
// correction's FMA; p's fp16 pattern addresses the ratio table directly.
template <int BITS>
__device__ __forceinline__ uint32_t value_code_f16(float v, const QParams& g, const uint8_t* lds) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  const float a = rnd<MZ_F16>(v - g.mn);
  const float n0 = a * g.rsc;
  const float n = rnd<MZ_F16>(__builtin_amdgcn_fmed3f(__builtin_fmaf(__builtin_fmaf(-g.sc, n0, a), g.rsc, n0), 0.f, 1.f));
  const bool up = n >= g.za;
  const float d = __builtin_fabsf(rnd<MZ_F16>(n - g.za));
  const float b = up ? g.pe : g.ne, r = up ? g.rpe : g.rne;
  const float p0 = d * r;
  const uint32_t pat = f2h(__builtin_amdgcn_fmed3f(__builtin_fmaf(__builtin_fmaf(-b, p0, d), r, p0), 0.f, 1.f));
  const float y = h2f(*(const uint16_t*)(lds + 2 * (pat & 0x7FFFu)));
  const float o = rnd<MZ_F16>(y * (up ? g.pb : -g.nb));
  // zl + off: an integer in [-1, qmax + 1], exact in fp16
  return (uint32_t)__builtin_amdgcn_fmed3f(g.zl + rintf(o), 0.f, qmax);
}

// Min / max over the 8 lanes of a group (lanes 8k..8k+7), NaN-propagating:
// IEEE 754-2019 minimum / maximum (v_minimum3_f32 / v_maximum3_f32), which
// return NaN when either operand is NaN, as torch's amin / amax do.  (Between
// -0 and +0 they pick -0 / +0; torch's choice there depends on its
// vectorisation.  The codes are the same either way: only the sign of a zero
// minimum or maximum in the metadata can differ.)
__device__ __forceinline__ float fmin_nan(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float fmax_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// Over the L lanes of a group (aligned runs of L = 2, 4 or 8 lanes).
template <int L>
__device__ __forceinline__ float group_min(float v) {
  if constexpr (L >= 2) v = fmin_nan(v, dpp_sel<DPP_QUAD_XOR1>(v));
  if constexpr (L >= 4) v = fmin_nan(v, dpp_sel<DPP_QUAD_XOR2>(v));
  if constexpr (L >= 8) v = fmin_nan(v, dpp_sel<DPP_ROW_HALF_MIRROR>(v));
  return v;
}
template <int L>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (L >= 2) v = fmax_nan(v, dpp_sel<DPP_QUAD_XOR1>(v));
  if constexpr (L >= 4) v = fmax_nan(v, dpp_sel<DPP_QUAD_XOR2>(v));
  if constexpr (L >= 8) v = fmax_nan(v, dpp_sel<DPP_ROW_HALF_MIRROR>(v));
  return v;
}

// NaN-propagating min / max of x[0..N) (a balanced tree).
template <int N, int S = 0>
__device__ __forceinline__ float tree_min(const float* x) {
  if constexpr (N == 1) return x[S];
  else return fmin_nan(tree_min<N / 2, S>(x), tree_min<N / 2, S + N / 2>(x));
}
template <int N, int S = 0>
__device__ __forceinline__ float tree_max(const float* x) {
  if constexpr (N == 1) return x[S];
  else return fmax_nan(tree_max<N / 2, S>(x), tree_max<N / 2, S + N / 2>(x));
}

// Quantize the 8 values x[0..7] of a chunk with the group's parameters and
// store their BITS packed bytes at dst.
template <int DT, int BITS>
__device__ __forceinline__ void quantize_chunk8(const float* x, const QParams& g, bool finite, uint8_t* dst,
                                                const uint8_t* lds, const void* table) {
  uint64_t w = 0;
  if (qfast<DT>(g) && finite) {
    if constexpr (DT == MZ_BF16) {
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        uint32_t c0, c1;
        value_code_bf16_pair<BITS>(x[i], x[i + 1], g, lds, c0, c1);
        w |= ((uint64_t)c0 << (i * BITS)) | ((uint64_t)c1 << ((i + 1) * BITS));
      }
    } else if constexpr (DT == MZ_F16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) w |= (uint64_t)value_code_f16<BITS>(x[i], g, lds) << (i * BITS);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) w |= (uint64_t)value_code<DT, BITS, true, true>(x[i], g, lds, table) << (i * BITS);
    }
  } else if (finite) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (uint64_t)value_code<DT, BITS, false, true>(x[i], g, lds, table) << (i * BITS);
  } else if (qfast<DT>(g)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (uint64_t)value_code<DT, BITS, true, false>(x[i], g, lds, table) << (i * BITS);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (uint64_t)value_code<DT, BITS, false, false>(x[i], g, lds, table) << (i * BITS);
  }
  if constexpr (BITS == 8) *(uint64_t*)dst = w;
  else if constexpr (BITS == 4) *(uint32_t*)dst = (uint32_t)w;
  else if constexpr (BITS == 2) *(uint16_t*)dst = (uint16_t)w;
  else if constexpr (BITS == 1) *dst = (uint8_t)w;
  else {
#pragma unroll
    for (int k = 0; k < BITS; ++k) dst[k] = (uint8_t)(w >> (8 * k));
  }
}

// The offset estimate's constants (code_offset_f32) from the threshold t of
// bins 1 (index 0 of the table), where log1p(alpha*t) / lb crosses 1/2:
// (1 + alpha*t)^2 = 1 + alpha, so alpha = (1 - 2t) / t^2.
template <int BITS>
__device__ __forceinline__ void set_estimate(QParams& g, const uint8_t* lds, const void* table) {
  const float t = (QTable<MZ_F32, BITS>::IN_LDS ? (const float*)lds : (const float*)table)[0];
  g.ea = (1.f - 2.f * t) / (t * t);
  g.ec = 1.f / __builtin_amdgcn_logf(1.f + g.ea);
}

// Quantize this lane's N values x[0..N) (positions N*part .. N*part+N-1 of
// its group, which 64 / N lanes share) and store its N*BITS/8 packed bytes
// at prow + part*N*BITS/8; lane part 0 stores the group's metadata at index
// midx.  The group's parameters are formed once per lane, so a larger N
// spreads them over more values.
template <int DT, int BITS, int N>
__device__ __forceinline__ void quantize_lane(const float (&x)[N], int part, uint8_t* prow, void* mn_out,
                                              void* sc_out, int64_t midx, int meta_dtype, float eps,
                                              const uint8_t* lds, const void* table) {
  constexpr int L = 64 / N;
  const float mn = group_min<L>(tree_min<N>(x));
  const float mx = group_max<L>(tree_max<N>(x));
  QParams g = qparams<DT, BITS>(mn, mx, eps);
  if constexpr (DT == MZ_F32 && BITS >= 5) set_estimate<BITS>(g, lds, table);
  // (fp16 rounds eps to 0: a constant group, or za at 0 or 1, then divides by 0).
  // The fp32 8-bit thresholds stay in global memory, where the plain form's
  // binary search measured faster.
  const bool finite = QTable<DT, BITS>::IN_LDS && __builtin_isfinite(g.mn) && __builtin_isfinite(g.sc) &&
                      g.sc > 0.f && g.pe > 0.f && g.ne > 0.f;
  uint8_t* dst = prow + part * (N / 8) * BITS;
#pragma unroll
  for (int c = 0; c < N / 8; ++c) quantize_chunk8<DT, BITS>(x + 8 * c, g, finite, dst + c * BITS, lds, table);
  if (part == 0) {
    store_val(mn_out, midx, mn, meta_dtype);
    store_val(sc_out, midx, g.sc, meta_dtype);
  }
}

// 8 consecutive values at p[i..i+7] (VEC: one or two 16-byte loads).
template <int DT, bool VEC>
__device__ __forceinline__ void load8(float (&x)[8], const void* p, int64_t i) {
  if constexpr (VEC && DT == MZ_F32) {
    const float4 a = *(const float4*)((const float*)p + i);
    const float4 b = *(const float4*)((const float*)p + i + 4);
    x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
  } else if constexpr (VEC) {
    const uint4 a = *(const uint4*)((const uint16_t*)p + i);
    const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = DT == MZ_BF16 ? bf2f((uint16_t)u[k]) : h2f((uint16_t)u[k]);
      x[2 * k + 1] = DT == MZ_BF16 ? bf2f((uint16_t)(u[k] >> 16)) : h2f((uint16_t)(u[k] >> 16));
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = load_val<DT>(p, i + k);
  }
}

// ------------------------------------------------------------- rows
template <int DT, int BITS, bool VEC>
__global__ __launch_bounds__(QWG) void quantize_rows_kernel(const void* __restrict__ x, int64_t nrows,
                                                            int64_t xs, uint8_t* __restrict__ packed, int64_t ps,
                                                            void* mn, void* sc, int meta_dtype, int64_t ms,
                                                            float eps, const void* __restrict__ table) {
  __shared__ __align__(16) uint8_t lds[QTable<DT, BITS>::LDS_BYTES];
  stage_table<DT, BITS>(lds, table);
  constexpr int N = QN_ROWS, L = 64 / N;
  const int lane = threadIdx.x & 63;
  const int part = lane % L;
  const int64_t stride = (int64_t)gridDim.x * (QWG / 64) * N;
  for (int64_t row = ((int64_t)blockIdx.x * (QWG / 64) + (threadIdx.x >> 6)) * N + lane / L;
       row - lane / L < nrows; row += stride) {
    if (row < nrows) {  // lanes of a group share `row`: the whole group takes this branch
      float v[N];
#pragma unroll
      for (int c = 0; c < N / 8; ++c) load8<DT, VEC>(*(float(*)[8])(v + 8 * c), x, row * xs + N * part + 8 * c);
      quantize_lane<DT, BITS, N>(v, part, packed + row * ps, mn, sc, row * ms, meta_dtype, eps, lds, table);
    }
  }
}

// ------------------------------------------------------------- index math
// n / d for 0 <= n < 2^31 by multiply-high (Granlund-Montgomery): l =
// ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(n, m) + n) >> l.
struct FastDiv {
  uint32_t d, m, l;
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return (__umulhi(n, m) + n) >> l; }
};

static FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint64_t m = (((1ull << 32) * ((1ull << l) - d)) / d) + 1;
  return FastDiv{d, (uint32_t)m, l};
}

// ------------------------------------------------------------- values
// Row (b, h, t, j): channels 64j..64j+63 of token t, zero beyond D.  Rows
// are numbered b-major with j fastest; nrows < 2^31 per launch (the host
// splits the batch).
template <int DT, int BITS, bool VEC, bool NARROW>
__global__ __launch_bounds__(QWG) void quantize_values_kernel(const void* __restrict__ x, int nrows, FastDiv fng,
                                                              FastDiv fT, FastDiv fH, int D, int64_t sb, int64_t sh,
                                                              int64_t st, uint8_t* __restrict__ packed, int64_t psb,
                                                              int64_t psh, void* mn, void* sc, int meta_dtype,
                                                              int64_t msb, int64_t msh, float eps,
                                                              const void* __restrict__ table) {
  __shared__ __align__(16) uint8_t lds[QTable<DT, BITS>::LDS_BYTES];
  stage_table<DT, BITS>(lds, table);
  constexpr int QB = 8 * BITS;
  constexpr int N = QN_ROWS, L = 64 / N;  // values per lane, lanes per group
  const int ng = (int)fng.d, T = (int)fT.d, H = (int)fH.d;
  const int TN = T * ng;  // rows per (b, h)
  const int lane = threadIdx.x & 63;
  const int part = lane % L;
  const int k = lane / L;  // the lane's row within its wave's N
  // wave-uniform (the compiler cannot see that threadIdx.x >> 6 is): the
  // (b, h) decomposition of a wave's first row then runs on the scalar unit
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int stride = gridDim.x * (QWG / 64) * N;
  for (int w0 = (blockIdx.x * (QWG / 64) + wave) * N; w0 < nrows; w0 += stride) {
    const int row = w0 + k;
    if (row >= nrows) continue;  // lanes of a group share `row`: the whole group takes this branch
    int64_t xo, po, mo;
    int i;
    if (TN >= N) {
      // the wave's N rows lie in (b, h) slices o0 and o0 + 1 at most (rows
      // are b-major, (t, j) fastest): their offsets are scalar
      const int o0 = (int)fT.div((uint32_t)fng.div((uint32_t)w0));  // w0 / (T*ng)
      const int b0 = (int)fH.div((uint32_t)o0), h0 = o0 - b0 * H;
      const int b1 = h0 + 1 == H ? b0 + 1 : b0, h1 = h0 + 1 == H ? 0 : h0 + 1;
      i = w0 - o0 * TN + k;
      const bool next = i >= TN;
      if (next) i -= TN;
      xo = next ? b1 * sb + h1 * sh : b0 * sb + h0 * sh;
      po = next ? b1 * psb + h1 * psh : b0 * psb + h0 * psh;
      mo = next ? b1 * msb + h1 * msh : b0 * msb + h0 * msh;
    } else {
      // short slices (few tokens): each row decomposed on its own
      const int o = (int)fT.div((uint32_t)fng.div((uint32_t)row));
      const int b = (int)fH.div((uint32_t)o), h = o - b * H;
      i = row - o * TN;
      xo = b * sb + h * sh;
      po = b * psb + h * psh;
      mo = b * msb + h * msh;
    }
    const int t = (int)fng.div((uint32_t)i);
    const int j = i - t * ng;
    const int c = 64 * j + N * part;
    // NARROW: every offset within a slice fits 31 bits (checked on the host)
    const int64_t src = xo + (NARROW ? (int64_t)(t * (int)st + c) : (int64_t)t * st + c);
    float v[N];
#pragma unroll
    for (int e8 = 0; e8 < N / 8; ++e8) {
      float (&v8)[8] = *(float(*)[8])(v + 8 * e8);
      const int c8 = c + 8 * e8;
      if (c8 + 8 <= D) {  // VEC only picks the load width; lanes past D (D % 64 != 0) read nothing
        load8<DT, VEC>(v8, x, src + 8 * e8);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v8[e] = c8 + e < D ? load_val<DT>(x, src + 8 * e8 + e) : 0.f;
      }
    }
    uint8_t* prow = packed + po + (NARROW ? (int64_t)(i * QB) : (int64_t)i * QB);
    quantize_lane<DT, BITS, N>(v, part, prow, mn, sc, mo + i, meta_dtype, eps, lds, table);
  }
}

// ------------------------------------------------------------- keys
// A workgroup loops over (b, h, token group) tiles: the [64 x D] tile is
// staged in LDS in the input dtype (16-bit inputs as they arrive, fp32 as
// fp32) and each wave quantizes 8 channels at a time reading the tile's
// columns, so the reference's permute + contiguous copy (layer.py:276-278)
// never touches HBM.  VEC: the tile arrives as 16-byte vectors (D % 8 == 0,
// D <= 256, aligned rows), and the next tile's vectors are loaded into
// registers before the current tile is quantized.  The grid holds as many
// workgroups per CU as the table and the tile leave room for in LDS (at most
// 4).
// 16-byte vectors per thread per tile on the vector path: 64 tokens x D
// channels / (16 / element bytes) / QWG, so at most D = 256 for 16-bit
// inputs and D = 128 for fp32 (the host sends wider fp32 tiles to the scalar
// path)
constexpr int KEY_MAX_VEC = 8;

template <int DT>
struct Vec16 {
  static constexpr int N = DT == MZ_F32 ? 4 : 8;  // elements per 16 bytes
};

template <int DT>
__device__ __forceinline__ void vec16_store_lds(float* dst, const uint4 u) {
  if constexpr (DT == MZ_F32) {
    dst[0] = __uint_as_float(u.x), dst[1] = __uint_as_float(u.y), dst[2] = __uint_as_float(u.z),
    dst[3] = __uint_as_float(u.w);
  } else {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      dst[2 * k] = DT == MZ_BF16 ? bf2f((uint16_t)w[k]) : h2f((uint16_t)w[k]);
      dst[2 * k + 1] = DT == MZ_BF16 ? bf2f((uint16_t)(w[k] >> 16)) : h2f((uint16_t)(w[k] >> 16));
    }
  }
}

// Staging element of the key tile: 16-bit inputs stay 16-bit in LDS (row
// pitch D + 2 halves), fp32 inputs stay fp32 (pitch D + 1).  Either pitch is
// an odd number of dwords, so a column read of a wave's 8 lane groups meets
// at most two distinct dwords per bank.
template <int DT>
struct KeyStage {
  using T = typename std::conditional<DT == MZ_F32, float, uint16_t>::type;
  static constexpr int PAD = DT == MZ_F32 ? 1 : 2;
  static __device__ __forceinline__ float load(const T* p) {
    if constexpr (DT == MZ_F32) return *p;
    else if constexpr (DT == MZ_BF16) return bf2f(*p);
    else return h2f(*p);
  }
  static __device__ __forceinline__ float load16(uint16_t u) { return DT == MZ_BF16 ? bf2f(u) : h2f(u); }
};

// 16-bit inputs arriving as vectors are staged transposed instead: one row
// of KT_PITCH dwords per channel, dword m = tokens 2m (low half) and 2m + 1
// (high half), so a lane reads its 32 tokens of a column as four 16-byte
// LDS reads.  A staging thread loads the same 8 channels of two adjacent
// tokens and pairs them with v_perm; threads of a wave take consecutive
// token pairs, so their stores fill consecutive dwords of a row.  The pitch
// (36 dwords, a multiple of 4) keeps the 16-byte reads aligned, and the 8
// lanes served in one cycle (4 columns x 2 halves) cover distinct banks.
constexpr int KT_PITCH = 36;
template <int DT, bool VEC>
struct KeyTrans {
  static constexpr bool ON = VEC && DT != MZ_F32;
  static constexpr size_t bytes(int D) { return (size_t)D * KT_PITCH * 4; }
};

template <int DT, int BITS, bool VEC>
__global__ __launch_bounds__(QWG) void quantize_keys_kernel(const void* __restrict__ x, int B, int H, int T, int D,
                                                            int64_t sb, int64_t sh, int64_t st,
                                                            uint8_t* __restrict__ packed, int64_t psb, int64_t psh,
                                                            void* mn, void* sc, int meta_dtype, int64_t msb,
                                                            int64_t msh, float eps, const void* __restrict__ table) {
  using KS = KeyStage<DT>;
  using ET = typename KS::T;
  extern __shared__ __align__(16) uint8_t dyn[];
  uint8_t* lds = dyn;                                                 // compander table
  ET* tile = (ET*)(dyn + QTable<DT, BITS>::LDS_BYTES);                // [64][D + PAD]
  stage_table<DT, BITS>(lds, table);
  const int nsg = T / 64;
  const int ntiles = B * H * nsg;  // < 2^31 (host check)
  const int ld = D + KS::PAD;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int part = lane % (64 / QN_KEYS);
  constexpr int QB = 8 * BITS;
  constexpr int NE = Vec16<DT>::N;
  const int vpr = D / NE;             // vectors per token row (VEC)
  const int nvec = 64 * vpr;          // vectors per tile (VEC)
  auto tile_base = [&](int ti) -> int64_t {
    const int s = ti % nsg, h = (ti / nsg) % H, b = ti / (nsg * H);
    return b * sb + h * sh + (int64_t)(64 * s) * st;
  };
  constexpr bool TRANS = KeyTrans<DT, VEC>::ON;
  uint32_t* tileT = (uint32_t*)tile;  // TRANS: [D][KT_PITCH] token-pair dwords
  const int npair = 32 * vpr;         // TRANS: (token pair, 8-channel block) items per tile
  uint4 nxt[KEY_MAX_VEC];
  auto fetch = [&](int ti) {
    if constexpr (TRANS) {
      const int64_t base = tile_base(ti);
      const uint16_t* xb = (const uint16_t*)x;
#pragma unroll
      for (int k = 0; k < KEY_MAX_VEC / 2; ++k) {
        const int e = threadIdx.x + k * QWG;
        if (e < npair) {
          const int tp = e & 31, cb = e >> 5;
          const int64_t a = base + (int64_t)(2 * tp) * st + NE * cb;
          nxt[2 * k] = *(const uint4*)(xb + a);
          nxt[2 * k + 1] = *(const uint4*)(xb + a + st);
        }
      }
    } else if constexpr (VEC) {
      const int64_t base = tile_base(ti);
      const char* xb = (const char*)x;
#pragma unroll
      for (int k = 0; k < KEY_MAX_VEC; ++k) {
        const int e = threadIdx.x + k * QWG;
        if (e < nvec) {
          const int t = e / vpr, c = (e - t * vpr) * NE;
          nxt[k] = *(const uint4*)(xb + (base + (int64_t)t * st + c) * (DT == MZ_F32 ? 4 : 2));
        }
      }
    }
  };
  if (blockIdx.x < ntiles) fetch(blockIdx.x);
  for (int ti = blockIdx.x; ti < ntiles; ti += gridDim.x) {
    const int s = ti % nsg, h = (ti / nsg) % H, b = ti / (nsg * H);
    __syncthreads();  // the previous tile's columns are consumed
    if constexpr (TRANS) {
#pragma unroll
      for (int k = 0; k < KEY_MAX_VEC / 2; ++k) {
        const int e = threadIdx.x + k * QWG;
        if (e < npair) {
          const int tp = e & 31, cb = e >> 5;
          const uint32_t a4[4] = {nxt[2 * k].x, nxt[2 * k].y, nxt[2 * k].z, nxt[2 * k].w};
          const uint32_t b4[4] = {nxt[2 * k + 1].x, nxt[2 * k + 1].y, nxt[2 * k + 1].z, nxt[2 * k + 1].w};
          uint32_t* col = tileT + (NE * cb) * KT_PITCH + tp;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            col[(2 * q) * KT_PITCH] = __builtin_amdgcn_perm(b4[q], a4[q], 0x05040100u);      // channel 2q
            col[(2 * q + 1) * KT_PITCH] = __builtin_amdgcn_perm(b4[q], a4[q], 0x07060302u);  // channel 2q+1
          }
        }
      }
      if (ti + (int)gridDim.x < ntiles) fetch(ti + gridDim.x);  // lands while this tile is quantized
    } else if constexpr (VEC) {
#pragma unroll
      for (int k = 0; k < KEY_MAX_VEC; ++k) {
        const int e = threadIdx.x + k * QWG;
        if (e < nvec) {
          const int t = e / vpr, c = (e - t * vpr) * NE;
          if constexpr (DT == MZ_F32) {
            vec16_store_lds<DT>(tile + t * ld + c, nxt[k]);
          } else {
            uint32_t* d32 = (uint32_t*)(tile + t * ld + c);  // 4-byte aligned: ld and c are even
            d32[0] = nxt[k].x, d32[1] = nxt[k].y, d32[2] = nxt[k].z, d32[3] = nxt[k].w;
          }
        }
      }
      if (ti + (int)gridDim.x < ntiles) fetch(ti + gridDim.x);  // lands while this tile is quantized
    } else {
      const int64_t base = tile_base(ti);
      for (int e = threadIdx.x; e < 64 * D; e += QWG) {
        const int t = e / D, c = e - t * D;
        if constexpr (DT == MZ_F32) tile[t * ld + c] = load_val<DT>(x, base + t * st + c);
        else tile[t * ld + c] = ((const uint16_t*)x)[base + t * st + c];
      }
    }
    __syncthreads();
    uint8_t* gbase = packed + b * psb + h * psh + (int64_t)s * D * QB;
    const int64_t mbase = b * msb + h * msh + (int64_t)s * D;
    constexpr int N = QN_KEYS, L = 64 / N;  // values per lane, lanes per group (one column)
    for (int c0 = (64 / L) * wave; c0 < D; c0 += (64 / L) * (QWG / 64)) {
      const int c = c0 + lane / L;
      if (c < D) {  // a group's lanes share c
        float v[N];
        if constexpr (TRANS) {
          static_assert(N == 32, "a lane reads 16 token-pair dwords");
          const uint4* src = (const uint4*)(tileT + c * KT_PITCH + 16 * part);
#pragma unroll
          for (int m4 = 0; m4 < 4; ++m4) {
            const uint4 u = src[m4];
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              v[8 * m4 + 2 * q] = KS::load16((uint16_t)w[q]);
              v[8 * m4 + 2 * q + 1] = KS::load16((uint16_t)(w[q] >> 16));
            }
          }
        } else {
#pragma unroll
          for (int k = 0; k < N; ++k) v[k] = KS::load(tile + (N * part + k) * ld + c);
        }
        quantize_lane<DT, BITS, N>(v, part, gbase + (int64_t)c * QB, mn, sc, mbase + c, meta_dtype, eps, lds, table);
      }
    }
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


// Persistent grid: enough workgroups to fill the GPU a few times over, each
// looping over its share of the 64-value groups (table staged once).
static int quantize_grid(int64_t work_groups, int groups_per_wave) {
  const int64_t per_wg = (int64_t)(QWG / 64) * groups_per_wave;
  const int64_t need = (work_groups + per_wg - 1) / per_wg;
  return (int)std::max<int64_t>(1, std::min<int64_t>(need, (int64_t)device_cu_count() * 8));
}

// Alignment the packed rows need: a lane stores its `bits` bytes as one
// 2/4/8-byte word when bits is 2/4/8, byte by byte otherwise.
static int packed_align(int bits) { return (bits == 2 || bits == 4 || bits == 8) ? bits : 1; }

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
static int64_t dtype_size(int dt) { return dt == MZ_F32 ? 4 : 2; }

extern "C" int muzero_quantize_rows(const void* x, int x_dtype, int64_t nrows, int64_t x_row_stride,
                                    uint8_t* packed, int64_t packed_row_stride, void* mn, void* scale,
                                    int meta_dtype, int64_t meta_stride, int bits, float eps, const void* table,
                                    mz_stream_t stream) {
  if (nrows < 0 || !dtype_ok(x_dtype) || !dtype_ok(meta_dtype) || bits < 1 || bits > 8) return MZ_EINVAL;
  if (nrows == 0) return MZ_OK;
  if (!x || !packed || !mn || !scale || !table) return MZ_EINVAL;
  if (x_row_stride < 64 || packed_row_stride < 8 * bits || meta_stride < 1) return MZ_EINVAL;
  // packed bytes are stored 1/2/4/8 at a time at offsets part*bits: rows must keep that alignment
  if (((uintptr_t)packed | (uintptr_t)packed_row_stride) % packed_align(bits) != 0) return MZ_EINVAL;
  const bool vec = aligned16(x) && x_row_stride % 8 == 0;
  const dim3 grid((unsigned)quantize_grid(nrows, QN_ROWS));
  hipStream_t s = (hipStream_t)stream;
  MZ_DT_SWITCH(x_dtype, MZ_BITS_SWITCH(bits,
      if (vec) hipLaunchKernelGGL((quantize_rows_kernel<D_, B_, true>), grid, dim3(QWG), 0, s, x, nrows,
                                  x_row_stride, packed, packed_row_stride, mn, scale, meta_dtype, meta_stride, eps,
                                  table);
      else hipLaunchKernelGGL((quantize_rows_kernel<D_, B_, false>), grid, dim3(QWG), 0, s, x, nrows,
                              x_row_stride, packed, packed_row_stride, mn, scale, meta_dtype, meta_stride, eps,
                              table)));
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
  if (((uintptr_t)packed | (uintptr_t)p_sb | (uintptr_t)p_sh) % packed_align(bits) != 0) return MZ_EINVAL;
  const int64_t ntiles = (int64_t)B * H * (T / 64);
  if (ntiles >= (int64_t)1 << 31) return MZ_EINVAL;
  const size_t es = x_dtype == MZ_F32 ? 4 : 2;
  // the vector path stages a whole tile in KEY_MAX_VEC 16-byte loads per thread
  const bool vec = aligned16(keys) && D % 8 == 0 && (int64_t)64 * D * (int64_t)es <= (int64_t)KEY_MAX_VEC * QWG * 16 &&
                   (x_sb * es) % 16 == 0 && (x_sh * es) % 16 == 0 && (x_st * es) % 16 == 0;
  hipStream_t s = (hipStream_t)stream;
  MZ_DT_SWITCH(x_dtype, MZ_BITS_SWITCH(bits,
      const size_t lds = (size_t)QTable<D_, B_>::LDS_BYTES +
                         (vec && D_ != MZ_F32 ? KeyTrans<D_, true>::bytes(D)
                                              : (size_t)64 * (D + KeyStage<D_>::PAD) * sizeof(typename KeyStage<D_>::T));
      if (lds > 160 * 1024) return MZ_EUNSUPPORTED;
      const void* fn = vec ? (const void*)quantize_keys_kernel<D_, B_, true> : (const void*)quantize_keys_kernel<D_, B_, false>;
      if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return (int)e;
      }
      const int per_cu = std::max<int>(1, std::min<int>(4, (int)((160 * 1024) / lds)));
      const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>(ntiles, per_cu * (int64_t)device_cu_count())));
      if (vec) hipLaunchKernelGGL((quantize_keys_kernel<D_, B_, true>), grid, dim3(QWG), lds, s, keys, B, H, T, D,
                                  x_sb, x_sh, x_st, packed, p_sb, p_sh, mn, scale, meta_dtype, m_sb, m_sh, eps, table);
      else hipLaunchKernelGGL((quantize_keys_kernel<D_, B_, false>), grid, dim3(QWG), lds, s, keys, B, H, T, D,
                              x_sb, x_sh, x_st, packed, p_sb, p_sh, mn, scale, meta_dtype, m_sb, m_sh, eps, table)));
  return launch_status();
}

extern "C" int muzero_quantize_values(const void* values, int x_dtype, int B, int H, int T, int D, int64_t x_sb,
                                      int64_t x_sh, int64_t x_st, uint8_t* packed, int64_t p_sb, int64_t p_sh,
                                      void* mn, void* scale, int meta_dtype, int64_t m_sb, int64_t m_sh, int bits,
                                      float eps, const void* table, mz_stream_t stream) {
  int st = check_block(values, x_dtype, B, H, T, D, packed, mn, scale, meta_dtype, bits, table);
  if (st == 1) return MZ_OK;
  if (st) return st;
  if (((uintptr_t)packed | (uintptr_t)p_sb | (uintptr_t)p_sh) % packed_align(bits) != 0) return MZ_EINVAL;
  const int ng = (D + 63) / 64;
  const int64_t rows_per_b = (int64_t)H * T * ng;
  if (rows_per_b >= (int64_t)1 << 31) return MZ_EINVAL;
  const size_t es = x_dtype == MZ_F32 ? 4 : 2;
  const bool vec = aligned16(values) && D % 8 == 0 && (x_sb * es) % 16 == 0 && (x_sh * es) % 16 == 0 &&
                   (x_st * es) % 16 == 0;
  const FastDiv fng = make_fastdiv((uint32_t)ng), fT = make_fastdiv((uint32_t)T), fH = make_fastdiv((uint32_t)H);
  // offsets within one (b, h) slice in 32-bit arithmetic when they all fit
  const bool narrow = x_st >= 0 && (int64_t)(T - 1) * x_st + D < ((int64_t)1 << 31) &&
                      (int64_t)T * ng * 8 * bits < ((int64_t)1 << 31);
  hipStream_t s = (hipStream_t)stream;
  // row numbers stay below 2^31 per launch: batches go in slices of bstep
  const int bstep = (int)std::min<int64_t>(B, (((int64_t)1 << 31) - 1) / rows_per_b);
  for (int b0 = 0; b0 < B; b0 += bstep) {
    const int nb = std::min(bstep, B - b0);
    const int nrows = (int)(nb * rows_per_b);
    const void* xs = (const char*)values + b0 * x_sb * (int64_t)es;
    uint8_t* ps = packed + b0 * p_sb;
    void* mns = (char*)mn + b0 * m_sb * (int64_t)dtype_size(meta_dtype);
    void* scs = (char*)scale + b0 * m_sb * (int64_t)dtype_size(meta_dtype);
    const dim3 grid((unsigned)quantize_grid(nrows, QN_ROWS));
#define MZ_QV(VECV, NARV)                                                                                     \
  hipLaunchKernelGGL((quantize_values_kernel<D_, B_, VECV, NARV>), grid, dim3(QWG), 0, s, xs, nrows, fng, fT, fH, D, \
                     x_sb, x_sh, x_st, ps, p_sb, p_sh, mns, scs, meta_dtype, m_sb, m_sh, eps, table)
    MZ_DT_SWITCH(x_dtype, MZ_BITS_SWITCH(bits,
        if (vec && narrow) MZ_QV(true, true);
        else if (vec) MZ_QV(true, false);
        else if (narrow) MZ_QV(false, true);
        else MZ_QV(false, false)));
#undef MZ_QV
    const int st2 = launch_status();
    if (st2 != MZ_OK) return st2;
  }
  return MZ_OK;
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
    case MZ_ESCRATCH: return "the call needs more than the static decode scratch (MZ_DECODE_SCRATCH_BYTES = 8 MiB)";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown error";
  }
}
