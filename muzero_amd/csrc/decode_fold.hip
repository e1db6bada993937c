// Packed-KV decode attention, fast path for 4-bit codes (gfx950, wave64).
//
// Dequantization folded into the MFMA operands.  For a group with stored
// (mn, s) the reference dequantizes code q as (muzero/quantizer.py:241-255)
//   x = mn + s * (za + pe * E[pb][q - zl])   (q >= zl)
//   x = mn + s * (za - ne * E[nb][zl - q])   (q <  zl)
// which is x = a + bp * P(zl, q) + bn * N(zl, q) with per-group scalars
// a = mn + s*za, bp = s*pe, bn = -s*ne and a 16 x 16 table of pairs
// (P, N) = (E[pb][q-zl], 0) or (0, E[nb][zl-q]).  So
//   q.k = sum_c (Q_c*a_c) + sum_c [(Q_c*bp_c) P + (Q_c*bn_c) N]
// is an MFMA whose A operand carries the group scalars times the query (for
// P.V: the softmax weight times the token's scalars) and whose B operand is
// one table lookup (an fp16 pair) per code, contracting over (channel, side)
// pairs.  The constant part sum_c Q_c*a_c is one more MFMA against a ones
// operand.  No element is ever dequantized to memory.  The dequantized
// values are those of the reference's fused CUDA kernels: full precision
// (their fp32 codebooks, loader.py:197-263), not rounded to the layer dtype.
//
// Work of one wave: a 64-token tile = one key group (or 64 residual tokens).
//   QK: MFMA M rows = query heads of the kv-head (GQA grouping), columns =
//   token positions 4n+{0,2,1,3} of N-tiles 0..3; lane (n, g) of k-tile kt
//   holds channels 16kt+4g+{0..3}, and reads for each one 16 bits of the
//   channel's packed row (4 codes) straight from HBM.
//   PV: columns = channels 64vg+4n+{0,2,1,3}, k = (token, side); lane (n, g)
//   reads 16 bits of a token's packed row per value group (4 channels).
// The 16 lanes of a lane group always look up one zero-level row of the
// table, and each lane group has its own copy of the table in a disjoint
// bank range, so the per-code lookups are bank-conflict free.  The softmax of
// a tile is redistributed through LDS so every lane computes exps.  fp16
// operands are kept in range by a power-of-two scale per key group and per
// value tile, folded into the logits and into the online-softmax rescale.
//
// Launch: one workgroup of 4 waves per (batch, kv-head, split); a split is a
// run of tiles, waves take every 4th tile; the split's (m, l, acc) goes to the
// workspace and the shared combine kernel merges splits.
#include "decode_common.hpp"

namespace mz {

namespace fold {

constexpr int D = 128;
constexpr int QB = 32;       // bytes per packed 64-code group (4-bit)
constexpr int NG = 2;        // value groups per token
constexpr int TILE = 64;     // tokens per tile
constexpr int WAVES = 4;
constexpr uint32_t ONES_F16X2 = 0x3C003C00u;
// N-tile jt of a 16-bit code word holds code PERM_POS[jt] of its 4 codes
// (byte order produced by expand(): q0, q2, q1, q3).
__device__ constexpr int PERM_POS[4] = {0, 2, 1, 3};

// Static LDS layout (bytes).  Per workgroup: the two (P, N) tables (16 zero
// levels x 4 lane-group copies x 16 codes, uint32 each) and the query in three
// forms; per wave: group scalars, logits, weights, rescale factors.
template <int NREP>
struct Smem {
  static constexpr int TBL = 16 * 4 * 16 * 4;  // 4 KB per table
  static constexpr int TBL_K = 0;
  static constexpr int TBL_V = TBL;
  static constexpr int Q16 = 2 * TBL;              // fp16 [NREP][D]
  static constexpr int Q_IO = Q16 + NREP * D * 2;   // io dtype [NREP][D]
  static constexpr int WAVE0 = Q_IO + NREP * D * 2;
  // per-wave region
  static constexpr int KZL = 0;                        // uint32 [D]      zl << 8
  static constexpr int KBP = KZL + D * 4;              // float2 [D]      (bp, bn), scaled
  static constexpr int KA = KBP + D * 8;               // fp16 [D]        a, scaled
  static constexpr int VZL = KA + D * 2;               // uint32 [NG][TILE]
  static constexpr int VBP = VZL + NG * TILE * 4;      // uint32 [NG][TILE]
  static constexpr int VA = VBP + NG * TILE * 4;       // fp16 [NG][TILE]
  static constexpr int LOGIT = VA + NG * TILE * 2;     // f32 [NREP][TILE]
  static constexpr int P2 = LOGIT + NREP * TILE * 4;   // uint32 [NREP][TILE]  (p, p)
  static constexpr int P1 = P2 + NREP * TILE * 4;      // fp16 [NREP][TILE]
  static constexpr int CORR = P1 + NREP * TILE * 2;    // f32 [NREP]
  static constexpr int PER_WAVE = (CORR + NREP * 4 + 15) / 16 * 16;
  static constexpr int MERGE = (2 * NREP + NREP * D) * 4;  // per wave at the end (aliases the wave area)
  static constexpr int WAVE_AREA = WAVES * (PER_WAVE > MERGE ? PER_WAVE : MERGE);
  static constexpr int TOTAL = WAVE0 + WAVE_AREA;
};

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_mul(uint32_t x, uint32_t y) {
  const h2 r = __builtin_bit_cast(h2, x) * __builtin_bit_cast(h2, y);
  return __builtin_bit_cast(uint32_t, r);
}

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// q*b0 and q*b1 as fp16 pairs hi + lo with hi + lo = q*b to about 2^-22
// relative: one fp16 rounding of the product would cost 2^-12 per channel,
// which the logits of long contexts amplify past the attention tolerance.
// (Compiles to v_fma_mix{lo,hi}_f16: the fp16 q feeds the fp32 FMA directly.)
__device__ __forceinline__ uint2 split_product(_Float16 q, float b0, float b1) {
  const float fq = (float)q;
  const _Float16 h0 = (_Float16)__builtin_fmaf(fq, b0, 0.f);
  const _Float16 h1 = (_Float16)__builtin_fmaf(fq, b1, 0.f);
  const _Float16 l0 = (_Float16)__builtin_fmaf(fq, b0, -(float)h0);
  const _Float16 l1 = (_Float16)__builtin_fmaf(fq, b1, -(float)h1);
  return uint2{__builtin_bit_cast(uint32_t, h2{h0, h1}), __builtin_bit_cast(uint32_t, h2{l0, l1})};
}

// Exponent k with |v| * 2^k < 2^15 (fp16 operands and products stay finite).
__device__ __forceinline__ int range_exp(float mx) {
  if (!(mx > 0.f) || !(mx < INFINITY)) return 0;
  int e;
  frexpf(mx, &e);  // mx = f * 2^e, f in [0.5, 1)
  return min(max(15 - e, -60), 60);
}

struct GroupScalars {
  float a, bp, bn;
  uint32_t zlb;  // zl << 8
};

// (a, bp, bn, zl) of one stored group (mn, s); the scale is guarded like the
// reference CUDA extension (loader.py:201), so an all-zero group gives x = mn.
__device__ __forceinline__ GroupScalars group_scalars(float mn, float s) {
  constexpr float qmax = 15.f;
  const float eps = 1e-8f;
  if (!(s >= eps)) s = eps;
  const float za = clamp01((0.f - mn) / s);  // IEEE division: zl must match the reference
  const float zl = rintf(za * qmax);
  const float pe = clamp_min(1.f - za, eps);
  const float ne = clamp_min(za, eps);
  GroupScalars r;
  r.a = mn + s * za;
  r.bp = s * pe;
  r.bn = -(s * ne);
  r.zlb = (uint32_t)(zl == zl ? (int)zl : 0) << 8;
  return r;
}

// 16-bit word of 4 codes -> bytes (4*q0, 4*q2, 4*q1, 4*q3) | lane-group copy.
__device__ __forceinline__ uint32_t expand(uint32_t h, uint32_t grep) {
  return (((h << 2) | (h << 14)) & 0x3C3C3C3Cu) | grep;
}

template <int IO, int NREP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void fold_kernel(
    const mz_decode_args a, int tiles_per_split, int n_split,
                                                   const uint32_t* __restrict__ ftab_k,
                                                   const uint32_t* __restrict__ ftab_v) {
  using M = Mfma<IO>;
  using S = Smem<NREP>;
  constexpr int LPH = 64 / NREP;   // softmax layout: lanes per head
  constexpr int TPL = TILE / LPH;  // tokens per lane
  __shared__ __align__(16) uint8_t smem[S::TOTAL];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;

  // ---------------- workgroup setup: tables and query in LDS
  // entry (zl, q) is replicated for the 4 lane groups at byte zl*256 + 64*group + 4*q
  for (int i = threadIdx.x; i < 1024; i += 256) {
    const int zl = i >> 6, q = i & 15;
    ((uint32_t*)(smem + S::TBL_K))[i] = ftab_k[zl * 16 + q];
    ((uint32_t*)(smem + S::TBL_V))[i] = ftab_v[zl * 16 + q];
  }
  float qabs = 0.f;
  for (int i = threadIdx.x; i < NREP * D; i += 256) {
    const int h = i / D, c = i - h * D;
    const uint16_t raw = ((const uint16_t*)a.query)[b * a.q_sb + (int64_t)(kvh * NREP + h) * a.q_sh + c];
    const float qf = M::load(raw);
    const uint16_t qh = f2h(qf);
    ((uint16_t*)(smem + S::Q16))[i] = qh;
    ((uint16_t*)(smem + S::Q_IO))[i] = raw;
    qabs = fmaxf(qabs, fabsf(qf));
  }
  qabs = wave_max(qabs);
  float* wq = (float*)(smem + S::WAVE0);
  if (lane == 0) wq[wave] = qabs;
  __syncthreads();
  qabs = fmaxf(fmaxf(wq[0], wq[1]), fmaxf(wq[2], wq[3]));
  __syncthreads();

  uint8_t* W = smem + S::WAVE0 + wave * S::PER_WAVE;
  float* logit = (float*)(W + S::LOGIT);
  uint32_t* p2 = (uint32_t*)(W + S::P2);
  uint16_t* p1 = (uint16_t*)(W + S::P1);
  float* corrs = (float*)(W + S::CORR);

  // A-operand row of this lane: a query head; rows >= NREP (MFMA padding)
  // repeat head 0 and their outputs are never read
  const int hA = n < NREP ? n : 0;
  const uint32_t grep = 0x40404040u * (uint32_t)g;
  const int sh = lane / LPH;           // softmax layout: head
  const int st0 = (lane % LPH) * TPL;  // and first token

  float m_run = -INFINITY, l_run = 0.f;  // head sh
  f32x4 acc[NG][4], acc_a[NG];
#pragma unroll
  for (int vg = 0; vg < NG; ++vg) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[vg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc_a[vg] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  int kacc = 0;  // acc holds sum p * x * 2^kacc
  bool kacc_init = false;

  const int n_tiles_d = (a.n_residual + TILE - 1) / TILE;
  const int n_tiles = a.n_groups + n_tiles_d;
  const int t_begin = split * tiles_per_split;
  const int t_end = min(n_tiles, t_begin + tiles_per_split);
  const uint8_t* kp_bh = a.k_packed + b * a.kp_sb + kvh * a.kp_sh;
  const uint8_t* vp_bh = a.v_packed + b * a.vp_sb + kvh * a.vp_sh;
  const int64_t km_bh = b * a.km_sb + kvh * a.km_sh;
  const int64_t vm_bh = b * a.vm_sb + kvh * a.vm_sh;

  for (int tile = t_begin + wave; tile < t_end; tile += WAVES) {
    const bool quant = tile < a.n_groups;
    int n_valid, pos0, r0 = 0;
    if (quant) {
      n_valid = TILE;
      pos0 = TILE * tile;
    } else {
      r0 = (tile - a.n_groups) * TILE;
      n_valid = min(TILE, a.n_residual - r0);
      pos0 = TILE * a.n_groups + r0;
    }

    f32x4 s[4];
    int kv_exp = 0;
    float unscale = a.scaling;
    uint32_t vc[4][4][NG];  // value code words (16 bits each) of a quantized tile
    if (quant) {
      // ---------- loads: metadata first, then code words
      float kmn[2], ksc[2], vmn[NG], vsc[NG];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int64_t mi = km_bh + (int64_t)tile * D + lane + 64 * cc;
        kmn[cc] = meta_load(a.k_mn, mi, a.meta_dtype);
        ksc[cc] = meta_load(a.k_scale, mi, a.meta_dtype);
      }
#pragma unroll
      for (int vg = 0; vg < NG; ++vg) {
        const int64_t mi = vm_bh + (int64_t)(pos0 + lane) * NG + vg;
        vmn[vg] = meta_load(a.v_mn, mi, a.meta_dtype);
        vsc[vg] = meta_load(a.v_scale, mi, a.meta_dtype);
      }
      // K: k-tile kt, slot ii -> channel 16kt+4g+ii, 16 bits at byte 2n of its row
      uint32_t kc[8][4];
      const uint16_t* kgrp = (const uint16_t*)(kp_bh + (int64_t)tile * D * QB + 4 * g * QB + 2 * n);
#pragma unroll
      for (int kt = 0; kt < 8; ++kt)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) kc[kt][ii] = kgrp[(16 * kt + ii) * (QB / 2)];

      // ---------- key group scalars (lane: channels lane, lane+64)
      GroupScalars ks[2];
      float kmx = 0.f;
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        ks[cc] = group_scalars(kmn[cc], ksc[cc]);
        kmx = fmaxf(kmx, fmaxf(fabsf(ks[cc].a), fmaxf(ks[cc].bp, -ks[cc].bn)));
      }
      kmx = wave_max(kmx);
      const int kexp = min(range_exp(kmx * fmaxf(qabs, 1.f)), range_exp(kmx));
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int c = lane + 64 * cc;
        ((uint32_t*)(W + S::KZL))[c] = ks[cc].zlb;
        ((float2*)(W + S::KBP))[c] = float2{ldexpf(ks[cc].bp, kexp), ldexpf(ks[cc].bn, kexp)};
        ((uint16_t*)(W + S::KA))[c] = f2h(ldexpf(ks[cc].a, kexp));
      }
      unscale = ldexpf(a.scaling, -kexp);
      // ---------- value scalars (lane: token lane, both value groups)
      GroupScalars vs[NG];
      float vmx = 0.f;
#pragma unroll
      for (int vg = 0; vg < NG; ++vg) {
        vs[vg] = group_scalars(vmn[vg], vsc[vg]);
        vmx = fmaxf(vmx, fmaxf(fabsf(vs[vg].a), fmaxf(vs[vg].bp, -vs[vg].bn)));
      }
      // keep the accumulators' exponent unless this tile needs a smaller one
      kv_exp = min(kacc_init ? kacc : 60, range_exp(wave_max(vmx)));
#pragma unroll
      for (int vg = 0; vg < NG; ++vg) {
        ((uint32_t*)(W + S::VZL))[vg * TILE + lane] = vs[vg].zlb;
        ((uint32_t*)(W + S::VBP))[vg * TILE + lane] = pack_h2(ldexpf(vs[vg].bp, kv_exp), ldexpf(vs[vg].bn, kv_exp));
        ((uint16_t*)(W + S::VA))[vg * TILE + lane] = f2h(ldexpf(vs[vg].a, kv_exp));
      }
      wave_lds_sync();

      // ---------- S = Q K^T: constant part (ones operand), then the folded codes
      f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        const u32x4 qv = *(const u32x4*)(smem + S::Q16 + (hA * D + 32 * kq + 8 * g) * 2);
        const u32x4 av = *(const u32x4*)(W + S::KA + (32 * kq + 8 * g) * 2);
        u32x4 A;
#pragma unroll
        for (int p = 0; p < 4; ++p) A[p] = pk_mul(qv[p], av[p]);
        s0 = Mfma<MZ_F16>::run(A, u32x4{ONES_F16X2, ONES_F16X2, ONES_F16X2, ONES_F16X2}, s0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] = s0;
#pragma unroll
      for (int kt = 0; kt < 8; ++kt) {
        const h4 q4 = *(const h4*)(smem + S::Q16 + (hA * D + 16 * kt + 4 * g) * 2);
        const f32x4 b01 = *(const f32x4*)(W + S::KBP + (16 * kt + 4 * g) * 8);
        const f32x4 b23 = *(const f32x4*)(W + S::KBP + (16 * kt + 4 * g) * 8 + 16);
        const u32x4 zl4 = *(const u32x4*)(W + S::KZL + (16 * kt + 4 * g) * 4);
        const uint2 p0 = split_product(q4[0], b01[0], b01[1]);
        const uint2 p1_ = split_product(q4[1], b01[2], b01[3]);
        const uint2 p2_ = split_product(q4[2], b23[0], b23[1]);
        const uint2 p3 = split_product(q4[3], b23[2], b23[3]);
        const u32x4 Ahi = u32x4{p0.x, p1_.x, p2_.x, p3.x};
        const u32x4 Alo = u32x4{p0.y, p1_.y, p2_.y, p3.y};
        uint32_t e[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) e[ii] = expand(kc[kt][ii], grep);
        u32x4 B[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii)
            B[jt][ii] = *(const uint32_t*)(smem + S::TBL_K +
                                           __builtin_amdgcn_perm(zl4[ii], e[ii], 0x0C0C0500u | (uint32_t)jt));
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) s[jt] = Mfma<MZ_F16>::run(Ahi, B[jt], s[jt]);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) s[jt] = Mfma<MZ_F16>::run(Alo, B[jt], s[jt]);
      }
      // V code words, issued after the key words are consumed (their latency
      // is covered by the softmax): k-tile kt, slot ii -> token 16kt+4g+ii,
      // 16 bits at byte 32vg+2n of its row
      const uint16_t* vtok = (const uint16_t*)(vp_bh + (int64_t)(pos0 + 4 * g) * (NG * QB) + 2 * n);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
#pragma unroll
          for (int vg = 0; vg < NG; ++vg)
            vc[kt][ii][vg] = vtok[((16 * kt + ii) * (NG * QB) + QB * vg) / 2];
    } else {
      // ---------- residual tile: S = Q K^T with dense operands
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint16_t* kres = (const uint16_t*)a.k_res + b * a.kr_sb + kvh * a.kr_sh;
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        const u32x4 qv = *(const u32x4*)(smem + S::Q_IO + (hA * D + 32 * kq + 8 * g) * 2);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          const int t = 4 * n + PERM_POS[jt];
          const u32x4 kb = t < n_valid ? *(const u32x4*)(kres + (int64_t)(r0 + t) * a.kr_st + 32 * kq + 8 * g)
                                       : u32x4{0, 0, 0, 0};
          s[jt] = M::run(qv, kb, s[jt]);
        }
      }
    }

    // ---------- softmax over the tile (redistributed: lane -> head sh, tokens st0..)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * g + i;
      if (h < NREP)
        *(f32x4*)(logit + h * TILE + 4 * n) = f32x4{s[0][i], s[2][i], s[1][i], s[3][i]} * unscale;
    }
    wave_lds_sync();
    float x[TPL];
    float tmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
      const int tt = st0 + t;
      float v = logit[sh * TILE + tt];
      if (tt >= n_valid) v = -INFINITY;
      else if (a.mask) v += a.mask[b * a.mask_sb + pos0 + tt];
      x[t] = v;
      tmax = fmaxf(tmax, v);
    }
#pragma unroll
    for (int o = LPH / 2; o > 0; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float corr = (m_new == -INFINITY) ? 1.f : __expf(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < TPL; ++t) {
      const float p = (x[t] == -INFINITY) ? 0.f : __expf(x[t] - m_new);
      const uint16_t ph = f2h(p);
      psum += h2f(ph);
      p2[sh * TILE + st0 + t] = (uint32_t)ph | ((uint32_t)ph << 16);
      p1[sh * TILE + st0 + t] = ph;
    }
#pragma unroll
    for (int o = LPH / 2; o > 0; o >>= 1) psum += __shfl_xor(psum, o, 64);
    l_run = l_run * corr + psum;
    if ((lane % LPH) == 0) corrs[sh] = corr;
    wave_lds_sync();

    // ---------- rescale the accumulators (softmax correction and value-tile exponent),
    // skipped when no head's maximum moved and the exponent is unchanged
    // (residual tiles add p*v unscaled, so they need exponent 0)
    if (__ballot(corr != 1.f) != 0 || kv_exp != kacc || !kacc_init) {
      const float fexp = ldexpf(1.f, kv_exp - kacc);
      kacc = kv_exp;
      kacc_init = true;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * g + i;
        const float f = (h < NREP ? corrs[h] : 1.f) * fexp;
#pragma unroll
        for (int vg = 0; vg < NG; ++vg) {
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[vg][j][i] *= f;
          acc_a[vg][i] *= f;
        }
      }
    }

    // ---------- acc += P V
    if (quant) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const u32x4 pd = *(const u32x4*)(p2 + hA * TILE + 16 * kt + 4 * g);
#pragma unroll
        for (int vg = 0; vg < NG; ++vg) {
          const u32x4 bq = *(const u32x4*)(W + S::VBP + (vg * TILE + 16 * kt + 4 * g) * 4);
          const u32x4 zl4 = *(const u32x4*)(W + S::VZL + (vg * TILE + 16 * kt + 4 * g) * 4);
          u32x4 A;
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) A[ii] = pk_mul(pd[ii], bq[ii]);
          uint32_t e[4];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) e[ii] = expand(vc[kt][ii][vg], grep);
          u32x4 B[4];
#pragma unroll
          for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
              B[jt][ii] = *(const uint32_t*)(smem + S::TBL_V +
                                             __builtin_amdgcn_perm(zl4[ii], e[ii], 0x0C0C0500u | (uint32_t)jt));
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) acc[vg][jt] = Mfma<MZ_F16>::run(A, B[jt], acc[vg][jt]);
        }
      }
      // constant part: sum_t p_t * a_t against a ones operand
#pragma unroll
      for (int kq = 0; kq < 2; ++kq) {
        const u32x4 pv = *(const u32x4*)(p1 + hA * TILE + 32 * kq + 8 * g);
#pragma unroll
        for (int vg = 0; vg < NG; ++vg) {
          const u32x4 av = *(const u32x4*)(W + S::VA + (vg * TILE + 32 * kq + 8 * g) * 2);
          u32x4 A;
#pragma unroll
          for (int p = 0; p < 4; ++p) A[p] = pk_mul(pv[p], av[p]);
          acc_a[vg] = Mfma<MZ_F16>::run(A, u32x4{ONES_F16X2, ONES_F16X2, ONES_F16X2, ONES_F16X2}, acc_a[vg]);
        }
      }
    } else {
      // residual values: B pairs (v, 0) against A pairs (p, p)
      const uint16_t* vres = (const uint16_t*)a.v_res + b * a.vr_sb + kvh * a.vr_sh;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const u32x4 pd = *(const u32x4*)(p2 + hA * TILE + 16 * kt + 4 * g);
#pragma unroll
        for (int vg = 0; vg < NG; ++vg) {
          uint32_t v4[4][2];
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const int t = 16 * kt + 4 * g + ii;
            if (t < n_valid) {
              const uint2 raw = *(const uint2*)(vres + (int64_t)(r0 + t) * a.vr_st + 64 * vg + 4 * n);
              v4[ii][0] = raw.x;
              v4[ii][1] = raw.y;
            } else {
              v4[ii][0] = 0u;
              v4[ii][1] = 0u;
            }
          }
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) {
            const int ch = PERM_POS[jt];  // channel 4n + ch
            u32x4 B;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const uint32_t w = v4[ii][ch >> 1];
              const uint16_t h = (ch & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFFu);
              B[ii] = IO == MZ_F16 ? (uint32_t)h : (uint32_t)f2h(bf2f(h));
            }
            acc[vg][jt] = Mfma<MZ_F16>::run(pd, B, acc[vg][jt]);
          }
        }
      }
    }
    wave_lds_sync();
  }

  // ---------------- merge the 4 waves and write this split's partial records
  __syncthreads();
  float* red = (float*)(smem + S::WAVE0);
  constexpr int RED = 2 * NREP + NREP * D;  // per wave: m[NREP], l[NREP], acc[NREP][D]
  {
    float* w = red + wave * RED;
    if ((lane % LPH) == 0) { w[sh] = m_run; w[NREP + sh] = l_run; }
    const float unit = ldexpf(1.f, -kacc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * g + i;
      if (h < NREP) {
#pragma unroll
        for (int vg = 0; vg < NG; ++vg)
#pragma unroll
          for (int jt = 0; jt < 4; ++jt)
            w[2 * NREP + h * D + 64 * vg + 4 * n + PERM_POS[jt]] = (acc[vg][jt][i] + acc_a[vg][i]) * unit;
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < NREP * (D + 2); e += 256) {
    const int h = e / (D + 2);
    const int c = e - h * (D + 2);
    float M_ = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M_ = fmaxf(M_, red[w * RED + h]);
    float val = 0.f;
    if (c == D) {
      val = M_;
    } else if (M_ != -INFINITY) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float f = __expf(red[w * RED + h] - M_);
        val += f * (c == D + 1 ? red[w * RED + NREP + h] : red[w * RED + 2 * NREP + h * D + c]);
      }
    }
    ws_record<D>(a, b, kvh * NREP + h, split, n_split)[c] = val;
  }
}

}  // namespace fold

// ------------------------------------------------------------------ host side

bool fold_supported(const mz_decode_args* a) {
  return a->bits == 4 && a->head_dim == 128 && a->n_groups > 0 &&
         (a->n_rep == 1 || a->n_rep == 2 || a->n_rep == 4 || a->n_rep == 8) && a->fold_k && a->fold_v;
}

int fold_choose_split(const mz_decode_args* a, int* tiles_per_split) {
  const int n_tiles = a->n_groups + (a->n_residual + fold::TILE - 1) / fold::TILE;
  int ns = a->n_split;
  if (ns <= 0) {
    const int64_t units = (int64_t)a->batch * a->kv_heads;
    const int64_t target = 2048;  // workgroups: several per CU on 256 CUs
    ns = (int)((target + units - 1) / units);
    ns = max(1, min(ns, (n_tiles + 7) / 8));  // at least 2 tiles per wave
  }
  ns = min(ns, n_tiles);
  const int tps = (n_tiles + ns - 1) / ns;
  *tiles_per_split = tps;
  return (n_tiles + tps - 1) / tps;
}

int fold_launch_partials(const mz_decode_args* a, hipStream_t s) {
  int tps;
  const int ns = fold_choose_split(a, &tps);
  const dim3 grid(ns, a->kv_heads, a->batch);
  const uint32_t* fk = (const uint32_t*)a->fold_k;
  const uint32_t* fv = (const uint32_t*)a->fold_v;
#define MZ_FOLD(IOV, NR) hipLaunchKernelGGL((fold::fold_kernel<IOV, NR>), grid, dim3(256), 0, s, *a, tps, ns, fk, fv)
#define MZ_FOLD_NREP(IOV)             \
  switch (a->n_rep) {                 \
    case 1: MZ_FOLD(IOV, 1); break;   \
    case 2: MZ_FOLD(IOV, 2); break;   \
    case 4: MZ_FOLD(IOV, 4); break;   \
    case 8: MZ_FOLD(IOV, 8); break;   \
    default: return MZ_EUNSUPPORTED;  \
  }
  if (a->io_dtype == MZ_BF16) { MZ_FOLD_NREP(MZ_BF16) } else { MZ_FOLD_NREP(MZ_F16) }
#undef MZ_FOLD_NREP
#undef MZ_FOLD
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

}  // namespace mz
