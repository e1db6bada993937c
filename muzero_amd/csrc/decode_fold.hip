// Packed-KV decode attention, fast path for 1- to 7-bit codes (gfx950, wave64).
//
// Dequantization folded into the MFMA operands.  For a group with stored
// (mn, s) the reference dequantizes code q as (muzero/quantizer.py:241-255)
//   x = mn + s * (za + pe * E[pb][q - zl])   (q >= zl)
//   x = mn + s * (za - ne * E[nb][zl - q])   (q <  zl)
// which is x = a + bp * P(zl, q) + bn * N(zl, q) with per-group scalars
// a = mn + s*za + (bp + bn)/2, bp = s*pe, bn = -s*ne and a (qmax+1)^2 table of
// pairs (P, N) = (E[pb][q-zl], 0) or (0, E[nb][zl-q]), stored shifted by 1/2
// (entries in [-1/2, 1/2] halve their worst fp16 rounding error; the shift's
// share, (bp + bn)/2, rides in a).  So
//   q.k = sum_c (Q_c*a_c) + sum_c [(Q_c*bp_c) P + (Q_c*bn_c) N]
// is an MFMA whose A operand carries the group scalars times the query (for
// P.V: the softmax weight times the token's scalars) and whose B operand is
// a table lookup (an fp16 pair) per code, contracting over (channel, side)
// pairs.  The constant part sum_c Q_c*a_c is two more MFMAs per 32 channels:
// A = the fp16 query (exact), B = a's high fp16 part, then its low part (a
// is the group's value nearest zero, large for one-signed groups, so one fp16
// rounding of it would not do); the values' constant part sum_t p_t*a_t is
// an fp32 row reduction.  No element is ever dequantized to memory.  The dequantized
// values are those of the reference's fused CUDA kernels: full precision
// (their fp32 codebooks, loader.py:197-263), not rounded to the layer dtype.
//
// Work of one wave: a 64-token tile = one key group (or 64 residual tokens).
//   QK: MFMA columns = tokens 4n+jt of N-tiles jt = 0..3; lane (n, g) of
//   k-tile kt holds channels 16kt+4g+{0..3} and needs, for each, the 4 codes
//   of its tokens 4n..4n+3 (4*BITS bits of the channel's row).
//   PV: columns = channels 64vg+4n+jt, k = (token, side); lane (n, g) needs
//   the codes of channels 4n..4n+3 of tokens 16kt+4g+{0..3}.
//   Lane pairs load the rows' shared words straight from HBM (buffer loads,
//   the tile offset in a scalar register) and swap them with one DPP move.
//   MFMA rows = query heads of the kv-head, spread to rows h*16/NREP: every
//   lane group of the MFMA output then holds real logits, so the softmax
//   runs in registers (row reductions on DPP) with no LDS round trip.
// Each 3- or 4-bit code is one conflict-free ds_read_b32 from a per-lane-
// group copy of the (P, N) table in LDS, addressed by one v_perm (plus about
// 0.75 VALU ops of code extraction), read straight into the MFMA B register;
// 2-bit codes go two to a ds_read_b64 and 1-bit codes four to a ds_read_b128
// (a B operand's rows at one token), the address one v_dot4_u32_u8 of the
// codes; 5- to 7-bit codes are bit-field extracts onto one table copy.  The
// lookups of the next k-tile are issued before the MFMAs of the current one.
// The
// key-side products q*bp, q*bn are formed per (head, channel) per tile as
// fp16 hi + lo pairs, on two rows of the same MFMA (fp32 accuracy at no extra
// MFMA); the PV operands p*bp, p*bn, p*a are formed per (head, token) by the
// softmax.  A tile's group scalars are computed during the previous tile's
// P.V, in chunks between its MFMA steps.  fp16 operands are kept in range by
// a power-of-two scale per key group and an accumulator exponent for the
// values, folded into the logits and into the online-softmax rescale.
//
// head_dim 64 runs the same layout with the k-tiles of channels 64..127 and
// the second value group absent.
//
// Launch: one workgroup of 4 waves (7 bits with up to 4 heads: 8) per (batch, kv-head, split); a split is a
// run of tiles (residual tiles first), waves take every 4th; the split's
// (m, l, acc) goes to the workspace and the shared combine kernel merges
// splits.  With a single split (the grid already fills the GPU) the kernel
// writes the output itself.
#include <type_traits>

#include "decode_tile.hpp"

namespace mz {

namespace fold {

constexpr int D = 128;
constexpr int NG = 2;     // value groups per token
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kLn2 = 0.693147180559945309f;
constexpr int TILE = 64;  // tokens per tile
// Waves per workgroup (one per SIMD; two workgroups share a CU).  Six-wave
// workgroups (three waves per SIMD; they fit the registers and LDS for up to
// 4 query heads) measured 13 % slower at config 1: more waves per CU contend
// for its LDS rather than hide more latency.
// 7-bit codes: one workgroup of 8 waves per CU (its 64 KB table then serves
// the CU's two waves per SIMD); with 8 query heads one workgroup of 4 (the
// per-wave operand staging of 16 MFMA rows brings it to 89 KB of LDS, so a CU
// holds one).
template <int NREP, int BITS>
constexpr int waves_for() { return BITS >= 7 && NREP <= 4 ? 8 : 4; }
template <int NREP>
constexpr int waves_per_simd() { return 2; }
// (P, N) table in LDS.  Up to 4 bits: entry (zl, q) replicated for the 4
// lane groups at byte zl*256 + 64*group + 4*q; the 16 lanes of a group always
// read one zero level (one channel / one token-group) and each group owns a
// disjoint bank range, so the per-code lookups are free of bank conflicts.
// 5 and 6 bits ("wide"): one copy, entry (zl, q) at byte zl*256 + 4*q (a
// group's 32 or 64 codes span every bank anyway, so copies would not help;
// two lane groups of a half-wave can meet on a bank).  7 bits: zl*512 + 4*q,
// one 64 KB table for keys and values (the launcher requires one alpha).
// 2 bits ("pair"): entry (z, e) = the (P, N) pairs of two codes q0 = e & 3,
// q1 = e >> 2 of two rows with zero levels z & 3, z >> 2, as two words at
// byte z*128 + 8*e: one ds_read_b64 fills two B registers.  A 64-bit read
// serves 16 lanes (one lane group, one row pair, so one 128-byte block) per
// cycle: no conflicts and no copies.
// 1 bit ("quad"): entry (z, e) = the (P, N) pairs of the 4 rows' codes
// (e >> ii) & 1 at zero levels (z >> ii) & 1, as four words at byte
// z*256 + 16*e: one ds_read_b128 is a whole B operand.
template <int BITS>
struct Fmt {
  static constexpr int QMAX = (1 << BITS) - 1;
  static constexpr int QB = 8 * BITS;  // bytes per packed 64-code row
  static constexpr bool WIDE = BITS >= 5;
  // 2 bits: one lookup serves two codes (rows 2p, 2p+1 of a k-slice at one
  // token); 1 bit: four (the k-slice's 4 rows), a whole B operand
  static constexpr bool PAIR = BITS == 2;
  static constexpr bool QUAD = BITS == 1;
  static constexpr int WPK = WIDE ? 4 : 2;  // code words per lane and k-tile
  // wide: bytes per zero level of the table, and the byte that stands for a
  // zero level in the zero-level words (the table row is that byte * 256)
  static constexpr int ZROW = (4 << BITS) > 256 ? (4 << BITS) : 256;
  static constexpr int ZS = ZROW / 256;
  static constexpr int TBL = WIDE ? (1 << BITS) * ZROW : (PAIR ? 16 * 16 * 8 : 16 * 4 * 16 * 4);  // bytes per table
  static constexpr bool SHARED = TBL > 16384;  // one table for keys and values
};

// Wide codes: each lane loads, per row of its k-tile, the dword holding its 4
// codes (4*BITS bits at bit 4*BITS*n, read unaligned; the last lane's dword
// is moved back inside the row), then extracts them with bit-field ops.
template <int BITS>
__device__ __forceinline__ int wide_byte(int n) {
  return min((4 * BITS * n) >> 3, Fmt<BITS>::QB - 4);
}

// Lanes 2m and 2m+1 of a lane group need the codes of tokens 8m..8m+7 of a
// row: 8*BITS bits starting at byte BITS*m.  The pair's word (1-bit: a byte,
// 2-bit: 16 bits, 4-bit: 32 bits, 3-bit: a dword read unaligned, the last
// pair's moved back inside the row) starts at pair_byte(m); pair_shift(n) is
// the bit offset of lane n's own 4 codes in it.
template <int BITS>
__device__ __forceinline__ int pair_byte(int m) {
  return BITS == 3 ? min(3 * m, 3 * 8 - 4) : BITS * m;
}
template <int BITS>
__device__ __forceinline__ uint32_t pair_shift(int n) {
  if constexpr (Fmt<BITS>::WIDE) return (uint32_t)(4 * BITS * n - 8 * wide_byte<BITS>(n));
  const int m = n >> 1;
  return (uint32_t)(8 * (BITS * m - pair_byte<BITS>(m)) + 4 * BITS * (n & 1));
}

// Padded row lengths (in 4-byte words) of the [head][...] arrays so that the
// rows read together by lanes of different heads start in different banks.
constexpr int AROW = D + 4;         // uint32 per head row of the key A operand
constexpr int HROW = D / 2 + 4;     // uint32 per head row of fp16 [D] arrays
constexpr int LROW = TILE + 4;      // uint32 per head row of per-token arrays

// Static LDS layout (bytes).  Per workgroup: the two (P, N) tables and the
// query in two forms; per wave: the current tile's operands and weights.
template <int NREP, int WAVES, int TBLB, bool SHARED>
struct Smem {
  static constexpr int TBL_K = 0;
  static constexpr int TBL_V = SHARED ? 0 : TBLB;
  static constexpr int Q16 = (SHARED ? 1 : 2) * TBLB;  // fp16 [NREP][HROW*2]
  static constexpr int Q_IO = Q16 + NREP * HROW * 4;  // io dtype [NREP][HROW*2]
  static constexpr int ZERO = Q_IO + NREP * HROW * 4;  // AROW zero words: A rows that must be 0
  static constexpr int WAVE0 = ZERO + AROW * 4;
  // per-wave region
  static constexpr int KZP = 0;                      // uint32 [4 g][8 kt]    zl of channels 16kt+4g+{0..3}
  static constexpr int AHI = KZP + 4 * 8 * 4;        // uint32 [NREP][AROW]   (q*bp, q*bn) fp16, high part
  static constexpr int ALO = AHI + NREP * AROW * 4;  // uint32 [NREP][AROW]   low part
  static constexpr int KA = ALO + NREP * AROW * 4;   // fp16 [2][D]           a per channel: high part, low part
  static constexpr int VZP = KA + 2 * D * 2;         // uint32 [NG][4 g][4 kt] zl of tokens 16kt+4g+{0..3}
  static constexpr int VBP = VZP + NG * 4 * 4 * 4;   // fp32 [NG][TILE]       bp
  static constexpr int VBN = VBP + NG * TILE * 4;    // fp32 [NG][TILE]       bn
  static constexpr int VA = VBN + NG * TILE * 4;     // fp32 [NG][TILE]       a
  static constexpr int PA = VA + NG * TILE * 4;      // uint32 [NG][NREP][LROW]   (p*bp, p*bn) fp16, high part
  static constexpr int PALO = PA + NG * NREP * LROW * 4;  // uint32 [NG][NREP][LROW]   low part
  static constexpr int PER_WAVE = (PALO + NG * NREP * LROW * 4 + 15) / 16 * 16;
  static constexpr int MERGE = (2 * NREP + NREP * D) * 4;  // per wave at the end (aliases the wave area)
  static constexpr int WAVE_AREA = WAVES * (PER_WAVE > MERGE ? PER_WAVE : MERGE);
  static constexpr int TOTAL = WAVE0 + WAVE_AREA;
};

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
}

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

// x0, x1 as fp16 pairs hi = (hi0, hi1), lo = (lo0, lo1) with hi + lo = x to
// about 2^-22 relative.
__device__ __forceinline__ uint2 split_values(float x0, float x1) {
  const _Float16 h0 = (_Float16)x0, h1 = (_Float16)x1;
  const _Float16 l0 = (_Float16)(x0 - (float)h0), l1 = (_Float16)(x1 - (float)h1);
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
  uint32_t zl;    // zero level: the group's row of the (P, N) table
};

// (a, bp, bn, zl) of one stored group (mn, s); the scale is guarded like the
// reference CUDA extension (loader.py:201), so an all-zero group gives x = mn.
// The clamps are single max / med3 ops: for any finite metadata they are
// torch's clamp / clamp_min; a NaN in the metadata cannot carry the zero level
// outside 0..QMAX (med3 returns one of its bounds), so the table reads stay in
// range.
template <int QMAX>
__device__ __forceinline__ GroupScalars group_scalars(float mn, float s) {
  constexpr float qmax = (float)QMAX;
  const float eps = 1e-8f;
  s = fmaxf(s, eps);
  const float za = __builtin_amdgcn_fmed3f((0.f - mn) / s, 0.f, 1.f);  // IEEE division: zl must match the reference
  const float zl = rintf(za * qmax);
  const float pe = fmaxf(1.f - za, eps);
  const float ne = fmaxf(za, eps);
  GroupScalars r;
  r.bp = s * pe;
  r.bn = -(s * ne);
  // the table holds (P - 1/2, N - 1/2): the constant part carries (bp + bn) / 2
  r.a = (mn + s * za) + 0.5f * (r.bp + r.bn);
  r.zl = (uint32_t)zl;
  return r;
}

// Code words of a quantized tile: lanes 2m and 2m+1 of a
// lane group read the same 2*LB bytes of two rows of a pair (key: channels,
// value: tokens); addr_ktile() later swaps halves between them so each lane
// ends with the bytes of both rows that hold ITS codes.
//   4-bit: kw[kt*2+p] = 32 bits of row 16kt+4g+2p+(n&1)
//   2-bit: kw[kt*2+h] = 16 bits of row 16kt+4g+2h+(n&1)
// (values: vw[(kt*NG+vg)*2 + p|h], rows = tokens, bytes of value group vg).
// `imm` (a compile-time offset within the tile) rides in the scalar offset
// with the tile's own; the tile index is always a quantized tile, so the
// address stays inside the buffer whatever the range check counts.
template <int BITS>
__device__ __forceinline__ uint32_t load_code_word(const __amdgpu_buffer_rsrc_t& r, int voff, int soff, int imm) {
  if constexpr (BITS >= 3) return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff + imm, 0);
  else if constexpr (BITS == 2) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff + imm, 0);
  else return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, voff, soff + imm, 0);
}

// Key code words of a tile (issued once the previous tile's key words are
// consumed: they land while the previous tile's P.V runs).
template <int BITS, int HD>
__device__ __forceinline__ void load_kw(uint32_t (&kw)[8 * Fmt<BITS>::WPK], const Bufs& bf, int tile, int lane) {
  using F = Fmt<BITS>;
  const int n = lane & 15, g = lane >> 4;
  const int soff = tile * HD * F::QB;
  if constexpr (F::WIDE) {
    // kw[kt*4+ii] = the lane's dword of row 16kt+4g+ii
    const int voff = 4 * g * F::QB + wide_byte<BITS>(n);
#pragma unroll
    for (int kt = 0; kt < HD / 16; ++kt)
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        kw[kt * 4 + ii] = __builtin_amdgcn_raw_buffer_load_b32(bf.kp, voff, soff + (16 * kt + ii) * F::QB, 0);
    return;
  }
  const int voff = (4 * g + (n & 1)) * F::QB + pair_byte<BITS>(n >> 1);
#pragma unroll
  for (int kt = 0; kt < HD / 16; ++kt)
#pragma unroll
    for (int p = 0; p < 2; ++p) kw[kt * 2 + p] = load_code_word<BITS>(bf.kp, voff, soff, (16 * kt + 2 * p) * F::QB);
}

// Value code words of a tile (issued at the start of the tile: they land
// while its Q.K runs).
template <int BITS, int HD>
__device__ __forceinline__ void load_vw(uint32_t (&vw)[8 * Fmt<BITS>::WPK], const Bufs& bf, int tile, int lane) {
  using F = Fmt<BITS>;
  constexpr int NGH = HD / 64;
  const int n = lane & 15, g = lane >> 4;
  const int soff = tile * TILE * NGH * F::QB;
  if constexpr (F::WIDE) {
    // vw[(kt*NGH+vg)*4+ii] = the lane's dword of token row 16kt+4g+ii, value group vg
    const int voff = 4 * g * (NGH * F::QB) + wide_byte<BITS>(n);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
          vw[(kt * NGH + vg) * 4 + ii] = __builtin_amdgcn_raw_buffer_load_b32(
              bf.vp, voff, soff + (16 * kt + ii) * (NGH * F::QB) + F::QB * vg, 0);
    return;
  }
  const int voff = (4 * g + (n & 1)) * (NGH * F::QB) + pair_byte<BITS>(n >> 1);
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int vg = 0; vg < NGH; ++vg)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        vw[(kt * NGH + vg) * 2 + p] =
            load_code_word<BITS>(bf.vp, voff, soff, (16 * kt + 2 * p) * (NGH * F::QB) + F::QB * vg);
}

// The table addresses of one k-tile's B operands (4 rows ii of this lane's
// k-slice x its 4 codes, jt = code index) from the two raw words w0, w1 of
// the k-tile (1-4 bits; wide codes: one dword per row).  The codes are spread
// to bytes as table offsets 4*q + 64*group (two ops per 4 codes); one v_perm
// per code then joins the offset (low byte) with row ii's zero level (byte ii
// of zp, as the high byte: the table row zl*256).  read_ktile() then fetches each (P, N) pair with one ds_read_b32
// straight into the operand register.  `odd` = lane n is odd.
template <int BITS>
__device__ __forceinline__ void addr_ktile(const uint32_t* w, uint32_t zp, uint32_t grep, bool odd, uint32_t sh,
                                           uint32_t (&ad)[4][4]) {
  const uint32_t w0 = w[0], w1 = w[1];
  if constexpr (Fmt<BITS>::WIDE) {
    // w[ii]: the lane's dword of row ii; code jt at bit sh + BITS*jt; the
    // table row of row ii's zero level starts at byte zl*256 (byte ii of zp
    // moved to byte 1)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const uint32_t row = __builtin_amdgcn_perm(zp, 0u, 0x0C0C000Cu | ((uint32_t)(4 + ii) << 8));
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
        ad[jt][ii] = (__builtin_amdgcn_ubfe(w[ii], sh + BITS * jt, BITS) << 2) + row;
    }
  } else if constexpr (BITS == 3) {
    // w0 / w1: the pair's dword of rows (0 | 1) / (2 | 3); after the swap the
    // lane holds all four rows, its code jt of row ii at bit sh + 3*jt; the
    // row's table copy for this lane group starts at byte zl*256 + 64*group
    // (the zero level, byte ii of zp, moved to byte 1 over grep's byte 0)
    const uint32_t s0 = dpp_swap_pairs(w0), s1 = dpp_swap_pairs(w1);
    const uint32_t r[4] = {odd ? s0 : w0, odd ? w0 : s0, odd ? s1 : w1, odd ? w1 : s1};
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const uint32_t row = __builtin_amdgcn_perm(zp, grep, 0x0C0C0000u | ((uint32_t)(4 + ii) << 8));
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) ad[jt][ii] = (__builtin_amdgcn_ubfe(r[ii], sh + 3 * jt, 3) << 2) + row;
    }
  } else if constexpr (BITS == 1) {
    // w0 / w1: byte m of rows (0 | 1) / (2 | 3) (even / odd lane); gather the
    // byte of rows 0..3 into one word; shifted by sh, bit jt of byte ii is
    // this lane's code jt of row ii.  zp = the row quad's block offset
    // (z*256).  One dot product per token forms 16*e (e = the 4 rows' codes
    // as bits 0..3) plus the block: ad[jt][0] addresses token jt's B operand.
    const uint32_t own = w0 | (w1 << 16);
    const uint32_t w = __builtin_amdgcn_perm(dpp_swap_pairs(own), own, odd ? 0x02060004u : 0x06020400u);
    const uint32_t ws = w >> sh;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
      ad[jt][0] = __builtin_amdgcn_udot4(ws & (0x01010101u << jt), 0x80402010u >> jt, zp, false);
  } else if constexpr (BITS == 4) {
    // w0 / w1: rows (0,1) / (2,3) of the pair, 32 bits = codes of lanes 2m, 2m+1;
    // this lane keeps 16 bits of each row: low half = row 2p, high half = row 2p+1
    const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
    const uint32_t r01 = __builtin_amdgcn_perm(dpp_swap_pairs(w0), w0, sel);
    const uint32_t r23 = __builtin_amdgcn_perm(dpp_swap_pairs(w1), w1, sel);
    // even / odd nibbles of each half: bytes (4*q0 | 4*q2 | ...) of rows ii
    const uint32_t ev[2] = {((r01 << 2) & 0x3C3C3C3Cu) | grep, ((r23 << 2) & 0x3C3C3C3Cu) | grep};
    const uint32_t od[2] = {((r01 >> 2) & 0x3C3C3C3Cu) | grep, ((r23 >> 2) & 0x3C3C3C3Cu) | grep};
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const uint32_t e = (jt & 1) ? od[ii >> 1] : ev[ii >> 1];
        const uint32_t s = 0x0C0C0000u | ((uint32_t)(4 + ii) << 8) | (uint32_t)((ii & 1) * 2 + (jt >> 1));
        ad[jt][ii] = __builtin_amdgcn_perm(zp, e, s);
      }
  } else if constexpr (Fmt<BITS>::PAIR) {
    // w0 / w1 as below; byte ii of w = this lane's codes of row ii (token jt
    // at bits 2jt).  zp = the two row pairs' block offsets (z*128, 16 bits
    // each).  One dot product per pair and token forms the entry offset
    // 8*q0 + 32*q1 from the two rows' codes (masked in place) plus the block:
    // ad[jt][p] is the byte address of rows (2p, 2p+1) at token jt.
    const uint32_t own = w0 | (w1 << 16);
    const uint32_t sel = odd ? 0x03070105u : 0x06020400u;
    const uint32_t w = __builtin_amdgcn_perm(dpp_swap_pairs(own), own, sel);
    const uint32_t w2 = w >> 4;  // tokens 2, 3 at bits 0 / 2 of each byte
    const uint32_t c0 = zp & 0xFFFFu, c1 = zp >> 16;
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const int s2 = 2 * (jt & 1);
      const uint32_t t = (jt < 2 ? w : w2) & (0x03030303u << s2);
      ad[jt][0] = __builtin_amdgcn_udot4(t, s2 ? 0x00000802u : 0x00002008u, c0, false);
      ad[jt][1] = __builtin_amdgcn_udot4(t, s2 ? 0x08020000u : 0x20080000u, c1, false);
    }
  } else {
    // w0 / w1: 16 bits of rows (0 | 1) / (2 | 3) (even / odd lane), one byte per
    // lane of the pair; gather this lane's byte of rows 0..3 into one word
    const uint32_t own = w0 | (w1 << 16);
    const uint32_t sel = odd ? 0x03070105u : 0x06020400u;
    const uint32_t w = __builtin_amdgcn_perm(dpp_swap_pairs(own), own, sel);  // byte ii = row ii
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const uint32_t e = (jt == 0 ? (w << 2) : (w >> (2 * jt - 2))) & 0x0C0C0C0Cu;
      const uint32_t ej = e | grep;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
        ad[jt][ii] = __builtin_amdgcn_perm(zp, ej, 0x0C0C0000u | ((uint32_t)(4 + ii) << 8) | ii);
    }
  }
}

template <int TBASE, bool PAIR = false, bool QUAD = false>
__device__ __forceinline__ void read_ktile(const uint8_t* smem, const uint32_t (&ad)[4][4], u32x4 B[4]) {
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    if constexpr (QUAD) {
      B[jt] = *(const u32x4*)(smem + TBASE + ad[jt][0]);
    } else if constexpr (PAIR) {
      const uint2 r0 = *(const uint2*)(smem + TBASE + ad[jt][0]);
      const uint2 r1 = *(const uint2*)(smem + TBASE + ad[jt][1]);
      B[jt] = u32x4{r0.x, r0.y, r1.x, r1.y};
    } else {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) B[jt][ii] = *(const uint32_t*)(smem + TBASE + ad[jt][ii]);
    }
  }
}

// HD: head_dim, 64 or 128.  The LDS layout is the 128-channel one either way;
// with 64 channels the k-tiles of channels 64..127 and the second value group
// are simply absent (lanes 32..63 compute no key scalar of the tile).
template <int IO, int NREP, int BITS, int MW, int HD>
__global__ __launch_bounds__((64 * waves_for<NREP, BITS>()))
__attribute__((amdgpu_waves_per_eu(waves_per_simd<NREP>(), waves_per_simd<NREP>()))) void fold_kernel(
    const mz_decode_args a, int tiles_per_split, int n_split, const uint32_t* __restrict__ ftab_k,
    const uint32_t* __restrict__ ftab_v, int direct, int cus) {
  constexpr int WAVES = waves_for<NREP, BITS>();
  constexpr int NT = 64 * WAVES;  // threads per workgroup
  using M = Mfma<IO>;
  using F = Fmt<BITS>;
  using S = Smem<NREP, WAVES, F::TBL, F::SHARED>;
  static_assert(S::TOTAL <= 160 * 1024, "LDS of one workgroup");
  constexpr int TBL = F::TBL;
  constexpr int RS = 16 / NREP;                 // MFMA row stride between query heads
  static_assert(RS >= 2, "QK needs a second row per head for the low part of the key product");
  constexpr int HS = NREP > 4 ? NREP / 4 : 1;   // head slots per lane of the MFMA output
  static_assert(HD == 64 || HD == 128, "head_dim");
  constexpr int NGH = HD / 64;                  // value groups per token
  __shared__ __align__(16) uint8_t smem[S::TOTAL];

  const int lane = threadIdx.x & 63;
  // wave-uniform (the compiler cannot see that threadIdx.x >> 6 is): tile
  // bookkeeping and load offsets then live in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const bool odd = (n & 1) != 0;
  const uint32_t lsh = pair_shift<BITS>(n);  // bit offset of this lane's codes in its pair's word
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;

  const int n_tiles_d = (a.n_residual + TILE - 1) / TILE;
  const int n_tiles = a.n_groups + n_tiles_d;
  const int t_begin = split * tiles_per_split;
  const int t_end = min(n_tiles, t_begin + tiles_per_split);
  constexpr int meta_es = 2 * MW;
  Bufs bf;
  {
    const int64_t ng = a.n_groups;
    bf.kp = make_buf(a.k_packed + b * a.kp_sb + kvh * a.kp_sh, ng * HD * F::QB);
    bf.vp = make_buf(a.v_packed + b * a.vp_sb + kvh * a.vp_sh, ng * TILE * NGH * F::QB);
    const int64_t km = b * a.km_sb + kvh * a.km_sh, vm = b * a.vm_sb + kvh * a.vm_sh;
    bf.kmn = make_buf((const uint8_t*)a.k_mn + km * meta_es, ng * HD * meta_es);
    bf.ksc = make_buf((const uint8_t*)a.k_scale + km * meta_es, ng * HD * meta_es);
    bf.vmn = make_buf((const uint8_t*)a.v_mn + vm * meta_es, ng * TILE * NGH * meta_es);
    bf.vsc = make_buf((const uint8_t*)a.v_scale + vm * meta_es, ng * TILE * NGH * meta_es);
    bf.kr = (const uint16_t*)a.k_res + b * a.kr_sb + kvh * a.kr_sh;
    bf.vr = (const uint16_t*)a.v_res + b * a.vr_sb + kvh * a.vr_sh;
  }

  // The split's tiles in virtual order: residual tiles first (their loads
  // then overlap the setup), quantized tiles after; wave w takes virtual
  // tiles w, w + WAVES, ...
  const int n_quant = max(0, min(t_end, a.n_groups) - t_begin);  // quantized tiles of the split
  const int n_res = (t_end - t_begin) - n_quant;                  // residual tiles of the split
  const int n_virt = t_end - t_begin;
  auto tile_of = [&](int v) { return v < n_res ? max(t_begin, a.n_groups) + v : t_begin + (v - n_res); };
  // Tile loads are issued unconditionally (the compiler's wait counts then
  // stay exact and a prefetch is never waited for early); a tile index that
  // is not a quantized tile is replaced by one this split reads anyway, so
  // the spare load hits the cache.
  const int q_last = max(0, min(t_end, a.n_groups) - 1);
  const int v0 = wave;  // first virtual tile of this wave

  // ---------------- workgroup setup: tables and query in LDS.  Their loads
  // are issued before the first tile's, so the setup waits for them only.
  constexpr int TW = (TBL / 4 + NT - 1) / NT;     // table words per thread (each table)
  constexpr int QW = (NREP * D + NT - 1) / NT;    // query elements per thread
  uint32_t tk[TW], tv[TW];
  uint16_t qraw[QW];
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    const int i = min(threadIdx.x + j * NT, TBL / 4 - 1);
    // narrow: word i = (zl, group, q) of the 16 x 16 host table; wide: the
    // host table's [zl][64] words as they are; pair / quad: two / four of its words
    // pair: word i = half (i & 1) of entry ((i >> 1) & 15) of block z = i >> 5
    // quad: word i = row (i & 3) of entry ((i >> 2) & 15) of block z = i >> 6
    const int e = (i >> 1) & 15, z = i >> 5;
    const int e4 = (i >> 2) & 15, z4 = i >> 6, r4 = i & 3;
    const int src = F::WIDE ? i
                    : F::PAIR ? ((i & 1) ? (z >> 2) * 16 + (e >> 2) : (z & 3) * 16 + (e & 3))
                    : F::QUAD ? ((z4 >> r4) & 1) * 16 + ((e4 >> r4) & 1)
                              : (i >> 6) * 16 + (i & 15);
    tk[j] = ftab_k[src];
    if constexpr (!F::SHARED) tv[j] = ftab_v[src];
  }
#pragma unroll
  for (int j = 0; j < QW; ++j) {
    const int i = threadIdx.x + j * NT, h = i / D, c = i - h * D;
    // heads past n_rep (a kernel built for more heads) get a zero query; their
    // outputs are not written.  Channels past HD (head_dim 64 in the
    // 128-channel layout) are zero too.
    qraw[j] = h < a.n_rep && c < HD
                  ? ((const uint16_t*)a.query)[b * a.q_sb + (int64_t)(kvh * a.n_rep + h) * a.q_sh + c]
                  : 0;
  }
  MetaWords<MW> MT;              // metadata of the current tile
  uint32_t KW[8 * F::WPK], VW[8 * F::WPK];  // key / value code words of the current tile
  load_meta_tile<MW, HD>(MT, bf, min(tile_of(v0), q_last), lane);
  load_kw<BITS, HD>(KW, bf, min(tile_of(v0), q_last), lane);
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    if (threadIdx.x + j * NT < TBL / 4) {
      ((uint32_t*)(smem + S::TBL_K))[threadIdx.x + j * NT] = tk[j];
      if constexpr (!F::SHARED) ((uint32_t*)(smem + S::TBL_V))[threadIdx.x + j * NT] = tv[j];
    }
  }
  for (int i = threadIdx.x; i < AROW; i += NT) ((uint32_t*)(smem + S::ZERO))[i] = 0u;
  float qabs = 0.f;
#pragma unroll
  for (int j = 0; j < QW; ++j) {
    const int i = threadIdx.x + j * NT, h = i / D, c = i - h * D;
    if (i >= NREP * D) break;
    const uint16_t raw = qraw[j];
    const float qf = M::load(raw);
    ((uint16_t*)(smem + S::Q16))[h * HROW * 2 + c] = f2h(qf);
    ((uint16_t*)(smem + S::Q_IO))[h * HROW * 2 + c] = raw;
    qabs = fmaxf(qabs, fabsf(qf));
  }
  qabs = wave_max_fast(qabs);
  float* wq = (float*)(smem + S::WAVE0);
  if (lane == 0) wq[wave] = qabs;
  __syncthreads();
  {
    float m4 = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) m4 = fmaxf(m4, wq[w]);
    qabs = m4;
  }
  __syncthreads();

  uint8_t* W = smem + S::WAVE0 + wave * S::PER_WAVE;
  // fp16 query of channels 2*lane, 2*lane+1 per head (the key-side products'
  // left factor), kept in registers: an LDS read in the scalar chunks would
  // make their wait take the table reads in flight with it
  uint32_t q16_pair[NREP];
#pragma unroll
  for (int h = 0; h < NREP; ++h) q16_pair[h] = *(const uint32_t*)(smem + S::Q16 + (h * HROW + lane) * 4);
  uint32_t* pa = (uint32_t*)(W + S::PA);
  uint32_t* pa_lo = (uint32_t*)(W + S::PALO);

  // A-operand row n of this lane belongs to query head hA = n / RS.  For
  // QK, row 0 of a head's rows carries the high fp16 part of the key-side
  // products (q*bp, q*bn against the codes) and row 1 their low part (summed
  // per logit), the head's remaining rows are zero; the constant part uses
  // row 0 only (the query against a's high, then low parts).  For PV row 0
  // carries the high fp16 part of p*bp, p*bn and row 1 the low part (summed
  // at the end); the other rows repeat row 1 and are not read.
  const int hA = n / RS;
  const int rA = n % RS;
  const uint8_t* a_hi_row = rA == 0 ? W + S::AHI + hA * AROW * 4
                                    : (rA == 1 ? W + S::ALO + hA * AROW * 4 : smem + S::ZERO);
  const uint8_t* q16_row = rA == 0 ? smem + S::Q16 + hA * HROW * 4 : smem + S::ZERO;
  // the constant part's A operand (the fp16 query on row 0 of each head's
  // rows, zero elsewhere) is the same for every tile: kept in registers
  // (wide codes, whose code words take twice the registers, re-read it)
  u32x4 q16_op[4];
#pragma unroll
  for (int kq = 0; kq < HD / 32; ++kq)
    q16_op[kq] = F::WIDE ? u32x4{0u, 0u, 0u, 0u} : *(const u32x4*)(q16_row + (32 * kq + 8 * g) * 2);
  const uint32_t* pv_row = (rA == 0 ? pa : pa_lo) + hA * LROW;  // PV A operand: this row's head
  const uint8_t* qio_row = rA == 0 ? smem + S::Q_IO + hA * HROW * 4 : smem + S::ZERO;
  const uint32_t grep = 0x40404040u * (uint32_t)g;  // this lane group's table copy
  // MFMA output element (g, i) = row 4g+i: head slot s is element i = s*RS
  // when 4g % RS == 0 (the lane group holds query heads), head 4g/RS + s
  const bool owner = ((4 * g) % RS) == 0;
  const int h0 = (4 * g) / RS;

  float m_run[HS], l_run[HS];
#pragma unroll
  for (int s = 0; s < HS; ++s) m_run[s] = -INFINITY, l_run[s] = 0.f;
  f32x4 acc[NGH][4];
  // the values' constant part sum_t p_t * a_t per head slot and value group
  // (fp32; the same in the 16 lanes of a head's row)
  float acc_a[HS][NGH];
#pragma unroll
  for (int vg = 0; vg < NGH; ++vg) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[vg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) acc_a[sl][vg] = 0.f;
  }
  int kacc = 0;  // acc and acc_a hold sum p * x * 2^kacc
  bool kacc_init = false;

  // ---------------- per-tile scalars, computed for the NEXT tile in 8 chunks
  // that ride along the current tile's 8 P.V steps (their division, DPP and
  // LDS latencies then hide behind the lookups and MFMAs).  They write the
  // next tile's Q.K operands (AHI, ALO, QA), zero levels (KZP, VZP) and value
  // scalars (VBP, VA): the current tile read its own before its P.V began.
  struct ScalState {
    GroupScalars k0, k1, v0, v1;
    float kmx, vmx;
  } sc;
  // logits are kept in base-2 units (times log2(e)): the softmax exponentials
  // are then single v_exp_f32 ops
  const float scaling2 = a.scaling * kLog2e;
  float unscale_n = scaling2;  // next tile's logit factor: scaling * log2(e) * 2^-kexp
  int kvexp_n = 0;              // next tile's value exponent
  auto scal_chunk = [&](const MetaWords<MW>& Mw, const int chunk) __attribute__((always_inline)) {
    constexpr int HPC = (NREP + 3) / 4;  // heads per chunk 4..7
    if (chunk == 0) {
      // key group scalars (lane: channels 2*lane, 2*lane+1)
      const float2 kmn = meta_cvt<MW>(Mw.kmn, a.meta_dtype), ksc = meta_cvt<MW>(Mw.ksc, a.meta_dtype);
      sc.k0 = group_scalars<F::QMAX>(kmn.x, ksc.x);
      sc.k1 = group_scalars<F::QMAX>(kmn.y, ksc.y);
      sc.kmx = fmaxf(fmaxf(fabsf(sc.k0.a), fmaxf(sc.k0.bp, -sc.k0.bn)),
                     fmaxf(fabsf(sc.k1.a), fmaxf(sc.k1.bp, -sc.k1.bn)));
      // head_dim 64: lanes 32..63 hold no channel of the tile (their stores
      // below land in layout slots the tile does not read)
      if constexpr (HD < D) sc.kmx = 2 * lane < HD ? sc.kmx : 0.f;
      // zero levels of channels 2*lane, 2*lane+1 = (kt, g, ii) = (lane/8, lane/2 % 4, 2*(lane%2) + {0,1})
      // (pair codes: the row pair's block offset in the table; quad codes: the
      // row quad's, from this lane's rows and its partner's)
      if constexpr (F::QUAD) {
        const uint32_t zpair = sc.k0.zl + 2 * sc.k1.zl;
        const uint32_t other = dpp_swap_pairs(zpair);
        if (!(lane & 1))
          *(uint32_t*)(W + S::KZP + (((lane >> 1) & 3) * 8 + (lane >> 3)) * 4) = (zpair + 4 * other) * 256;
      } else {
        *(uint16_t*)(W + S::KZP + (((lane >> 1) & 3) * 8 + (lane >> 3)) * 4 + (lane & 1) * 2) =
            F::PAIR ? (uint16_t)((sc.k0.zl + 4 * sc.k1.zl) * 128)
                    : (uint16_t)(sc.k0.zl * F::ZS | (sc.k1.zl * F::ZS << 8));
      }
    } else if (chunk == 1) {
      // value group scalars (lane: token lane, both value groups)
      const float2 vmn = meta_cvt<MW>(Mw.vmn, a.meta_dtype), vsc = meta_cvt<MW>(Mw.vsc, a.meta_dtype);
      sc.v0 = group_scalars<F::QMAX>(vmn.x, vsc.x);
      sc.v1 = group_scalars<F::QMAX>(vmn.y, vsc.y);
      sc.vmx = fmaxf(fabsf(sc.v0.a), fmaxf(sc.v0.bp, -sc.v0.bn));
      // one value group (head_dim 64): the second entry is the next token's
      if constexpr (NGH > 1) sc.vmx = fmaxf(sc.vmx, fmaxf(fabsf(sc.v1.a), fmaxf(sc.v1.bp, -sc.v1.bn)));
      // zero levels of token lane = (kt, g, ii) = (lane/16, lane/4 % 4, lane % 4), both value groups
      const int vzo = (((lane >> 2) & 3) * 4 + (lane >> 4)) * 4 + (lane & 3);
      if constexpr (F::QUAD) {
        // tokens 0..3 of a k-slice are lanes 4m..4m+3: their zero levels as
        // bits of the quad index, summed over the quad; its first lane writes
        // the block offset
        uint32_t q0 = sc.v0.zl << (lane & 3), q1 = sc.v1.zl << (lane & 3);
        q0 += dpp_sel_u<DPP_QUAD_XOR1>(q0);
        q1 += dpp_sel_u<DPP_QUAD_XOR1>(q1);
        q0 += dpp_sel_u<DPP_QUAD_XOR2>(q0);
        q1 += dpp_sel_u<DPP_QUAD_XOR2>(q1);
        if (!(lane & 3)) {
          *(uint32_t*)(W + S::VZP + vzo) = q0 * 256;
          *(uint32_t*)(W + S::VZP + 64 + vzo) = q1 * 256;
        }
      } else if constexpr (F::PAIR) {
        // tokens (2p, 2p+1) are lanes (2m, 2m+1): the even lane writes the pair's block offset
        const uint32_t z0n = dpp_swap_pairs(sc.v0.zl), z1n = dpp_swap_pairs(sc.v1.zl);
        if (!(lane & 1)) {
          *(uint16_t*)(W + S::VZP + vzo) = (uint16_t)((sc.v0.zl + 4 * z0n) * 128);
          *(uint16_t*)(W + S::VZP + 64 + vzo) = (uint16_t)((sc.v1.zl + 4 * z1n) * 128);
        }
      } else {
        W[S::VZP + vzo] = (uint8_t)(sc.v0.zl * F::ZS);
        W[S::VZP + 64 + vzo] = (uint8_t)(sc.v1.zl * F::ZS);
      }
    } else if (chunk == 2) {
      // power-of-two scales keeping the fp16 operands in range (one reduction for both)
      wave_max2_bound(sc.kmx, sc.vmx);
      const int kexp = min(range_exp(sc.kmx * fmaxf(qabs, 1.f)), range_exp(sc.kmx));
      unscale_n = ldexpf(scaling2, -kexp);
      sc.k0.bp = ldexpf(sc.k0.bp, kexp), sc.k0.bn = ldexpf(sc.k0.bn, kexp);
      sc.k1.bp = ldexpf(sc.k1.bp, kexp), sc.k1.bn = ldexpf(sc.k1.bn, kexp);
      // a of channels 2*lane, 2*lane+1 in high and low parts: the constant part's B operands
      const uint2 ka = split_values(ldexpf(sc.k0.a, kexp), ldexpf(sc.k1.a, kexp));
      ((uint32_t*)(W + S::KA))[lane] = ka.x;
      ((uint32_t*)(W + S::KA))[D / 2 + lane] = ka.y;
      kvexp_n = range_exp(sc.vmx);
    } else if (chunk == 3) {
      // keep the accumulators' exponent unless the tile needs a smaller one
      kvexp_n = min(kacc_init ? kacc : 60, kvexp_n);
      ((float*)(W + S::VBP))[lane] = ldexpf(sc.v0.bp, kvexp_n);
      ((float*)(W + S::VBN))[lane] = ldexpf(sc.v0.bn, kvexp_n);
      ((float*)(W + S::VBP))[TILE + lane] = ldexpf(sc.v1.bp, kvexp_n);
      ((float*)(W + S::VBN))[TILE + lane] = ldexpf(sc.v1.bn, kvexp_n);
      ((float*)(W + S::VA))[lane] = ldexpf(sc.v0.a, kvexp_n);
      ((float*)(W + S::VA))[TILE + lane] = ldexpf(sc.v1.a, kvexp_n);
    } else {
      // key-side products of heads HPC*(chunk-4) ...: q*bp, q*bn as fp16 hi + lo
#pragma unroll
      for (int hh = 0; hh < HPC; ++hh) {
        const int h = HPC * (chunk - 4) + hh;
        if (h < NREP) {
          const h2 qh = __builtin_bit_cast(h2, q16_pair[h]);
          const uint2 p0 = split_product(qh.x, sc.k0.bp, sc.k0.bn);
          const uint2 p1_ = split_product(qh.y, sc.k1.bp, sc.k1.bn);
          *(uint2*)(W + S::AHI + (h * AROW + 2 * lane) * 4) = uint2{p0.x, p1_.x};
          *(uint2*)(W + S::ALO + (h * AROW + 2 * lane) * 4) = uint2{p0.y, p1_.y};
        }
      }
    }
  };

  // one tile.  Loads in flight: this tile's value words (issued here, used by
  // its P.V), the next tile tn's metadata (issued here, used by the scalars
  // computed during this tile's P.V) and the next tile's key words (issued
  // after this tile's Q.K).
  // `quant` (a compile-time tag): a quantized tile, or a residual tile; the two
  // kinds run in separate loops, so neither carries the other's branches
  auto process = [&](auto quant_tag, const int tile, const int tn) {
    constexpr bool quant = decltype(quant_tag)::value;
    const int tl = min(tn, q_last);
    load_vw<BITS, HD>(VW, bf, min(tile, q_last), lane);
    MetaWords<MW> MN;
    load_meta_tile<MW, HD>(MN, bf, tl, lane);
    int n_valid, pos0, r0 = 0;
    if constexpr (quant) {
      n_valid = TILE;
      pos0 = TILE * tile;
    } else {
      r0 = (tile - a.n_groups) * TILE;
      n_valid = min(TILE, a.n_residual - r0);
      pos0 = TILE * a.n_groups + r0;
    }

    f32x4 s[4];
    // this lane's value scalars (a, bp, bn of tokens 4n..4n+3, per value
    // group), read once the tile's scalars are in LDS: at the start of a
    // quantized tile, so the reads complete behind its Q.K
    f32x4 va_r[NGH], vbp_r[NGH], vbn_r[NGH];
    auto read_value_scalars = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg) {
        va_r[vg] = *(const f32x4*)(W + S::VA + (vg * TILE + 4 * n) * 4);
        vbp_r[vg] = *(const f32x4*)(W + S::VBP + (vg * TILE + 4 * n) * 4);
        vbn_r[vg] = *(const f32x4*)(W + S::VBN + (vg * TILE + 4 * n) * 4);
      }
    };
    int kv_exp = kvexp_n;
    float unscale = unscale_n;
    if constexpr (quant) {
      wave_lds_sync();  // this tile's scalars were written by other lanes
      read_value_scalars();
      // ---------- S = Q K^T: constant part (the same for every token: the
      // query against a's high part, then its low part), then the folded codes
      f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kq = 0; kq < HD / 32; ++kq) {
        const u32x4 A = F::WIDE ? *(const u32x4*)(q16_row + (32 * kq + 8 * g) * 2) : q16_op[kq];
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const u32x4 Bq = *(const u32x4*)(W + S::KA + (part * D + 32 * kq + 8 * g) * 2);
          s0 = Mfma<MZ_F16>::run(A, Bq, s0);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] = s0;
      // k-tiles software-pipelined in three stages: the table reads of
      // k-tile kt+1 are issued, then the addresses of k-tile kt+2 computed,
      // then the MFMAs of k-tile kt run.  The address work sits between the
      // reads and the wait for them: a k-tile has 16 reads and the LDS
      // counter can leave at most 15 outstanding, so the wait before the
      // MFMAs also takes the oldest reads of the next k-tile.
      const u32x4 kz0 = *(const u32x4*)(W + S::KZP + g * 32);
      const u32x4 kz1 = *(const u32x4*)(W + S::KZP + g * 32 + 16);
      auto kzp = [&](int kt) { return kt < 4 ? kz0[kt] : kz1[kt - 4]; };
      u32x4 Ac = *(const u32x4*)(a_hi_row + (4 * g) * 4);
      u32x4 Bc[4], Bn[4];
      uint32_t adc[4][4], adn[4][4];
      addr_ktile<BITS>(KW, kzp(0), grep, odd, lsh, adc);
      read_ktile<S::TBL_K, F::PAIR, F::QUAD>(smem, adc, Bc);
      addr_ktile<BITS>(KW + F::WPK, kzp(1), grep, odd, lsh, adn);
      constexpr int KT = HD / 16;  // k-tiles of 16 channels
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        u32x4 An;
        if (kt < KT - 1) {
          An = *(const u32x4*)(a_hi_row + (16 * (kt + 1) + 4 * g) * 4);
          read_ktile<S::TBL_K, F::PAIR, F::QUAD>(smem, adn, Bn);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kt < KT - 2) addr_ktile<BITS>(KW + F::WPK * (kt + 2), kzp(kt + 2), grep, odd, lsh, adn);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) s[jt] = Mfma<MZ_F16>::run(Ac, Bc[jt], s[jt]);
        __builtin_amdgcn_sched_barrier(0);
        if (kt < KT - 1) {
          Ac = An;
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) Bc[jt] = Bn[jt];
        }
      }
    } else {
      // ---------- residual tile: S = Q K^T with dense operands; the weight
      // products below then use (bp, bn) = (2^kv_exp, 0) and a = 0: A =
      // (p * 2^kv_exp, 0), exact in fp16 (low parts 0), so the accumulators
      // keep their exponent (at most 15: p * 2^15 stays finite in fp16)
      // whatever the tile order
      kv_exp = min(kacc_init ? kacc : 15, 15);
      unscale = scaling2;
      const float unit = ldexpf(1.f, kv_exp);
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg) {
        ((float*)(W + S::VBP))[vg * TILE + lane] = unit;
        ((float*)(W + S::VBN))[vg * TILE + lane] = 0.f;
        ((float*)(W + S::VA))[vg * TILE + lane] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      // key vectors in two batches of 8 per lane, each batch in flight at once.
      // The buffer starts at the tile's first row and ends after its last
      // filled row, so the per-lane offset (row, lane group's column) carries
      // every bound: rows past the residual read 0 (their logits are masked);
      // the 32-column step rides in the scalar offset and never leaves a row.
      const int kst = a.kr_st * 2;
      const __amdgpu_buffer_rsrc_t krb = make_buf(bf.kr + (int64_t)r0 * a.kr_st, (n_valid - 1) * kst + HD * 2);
#pragma unroll
      for (int kh = 0; kh < HD / 64; ++kh) {
        u32x4 kb[2][4];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
          for (int jt = 0; jt < 4; ++jt)
            kb[k2][jt] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           krb, (4 * n + jt) * kst + 16 * g, 64 * (2 * kh + k2), 0));
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const u32x4 qv = *(const u32x4*)(qio_row + (32 * (2 * kh + k2) + 8 * g) * 2);
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) s[jt] = M::run(qv, kb[k2][jt], s[jt]);
        }
      }
      wave_lds_sync();  // the (1, 0) / 0 scalars above are read by other lanes below
      read_value_scalars();
    }
    load_kw<BITS, HD>(KW, bf, tl, lane);

    // ---------- online softmax in registers: head slot s of this lane group
    // owns tokens 4n+jt (jt = 0..3) of the 16 lanes of its row
    float corr[HS];
    // factor taking the accumulators from exponent kacc to this tile's kv_exp
    const float fexp = ldexpf(1.f, kv_exp - kacc);
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const int i = sl * RS;  // MFMA output element of this head slot
      float x[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int tt = 4 * n + jt;
        float v = (s[jt][i] + s[jt][i + 1]) * unscale;
        if (tt >= n_valid) v = -INFINITY;
        else if (a.mask) v = add_mask_log2(v, a.mask[b * a.mask_sb + pos0 + tt]);
        x[jt] = v;
        tmax = fmaxf(tmax, v);
      }
      tmax = group_reduce<16>(tmax, OpMax());
      const float m_new = fmaxf(m_run[sl], tmax);
      // while a row is fully masked its maximum stays -inf; 0 stands in for
      // it, so exp2(-inf - 0) gives the zero weights, and a zero correction
      // of the still all-zero sums, with no per-element test
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      corr[sl] = __builtin_amdgcn_exp2f(m_run[sl] - m_use);
      m_run[sl] = m_new;
      // weights rounded to fp16 (the P.V operand precision); the row sum uses
      // the same rounded weights
      const h2 p01 = h2{(_Float16)__builtin_amdgcn_exp2f(x[0] - m_use), (_Float16)__builtin_amdgcn_exp2f(x[1] - m_use)};
      const h2 p23 = h2{(_Float16)__builtin_amdgcn_exp2f(x[2] - m_use), (_Float16)__builtin_amdgcn_exp2f(x[3] - m_use)};
      const h2 one2 = h2{(_Float16)1.f, (_Float16)1.f};
      // l_run and acc_a are per-lane partial sums (this lane's 4 tokens of
      // every tile; the rescale factors are the same in the 16 lanes of the
      // row): they are summed over the row once, at the end
      const float psum = __builtin_amdgcn_fdot2(p23, one2, __builtin_amdgcn_fdot2(p01, one2, 0.f, false), false);
      l_run[sl] = l_run[sl] * corr[sl] + psum;
      // the values' constant part of this head: the running sum rescaled,
      // plus sum_t p_t * a_t over the tile, in fp32 with the same (fp16)
      // weights as the rest of the row
      const float fa = corr[sl] * fexp;
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg) {
        const f32x4 av = va_r[vg];
        float c = (float)p01.x * av[0];
        c = __builtin_fmaf((float)p01.y, av[1], c);
        c = __builtin_fmaf((float)p23.x, av[2], c);
        c = __builtin_fmaf((float)p23.y, av[3], c);
        acc_a[sl][vg] = __builtin_fmaf(acc_a[sl][vg], fa, c);
      }
      if (owner) {
        // PV A operands of this head's 4 tokens: p times the token's (bp, bn),
        // as fp16 hi + lo pairs
        const int h = h0 + sl;
#pragma unroll
        for (int vg = 0; vg < NGH; ++vg) {
          const f32x4 bp = vbp_r[vg];
          const f32x4 bn = vbn_r[vg];
          const uint2 w0 = split_product(p01.x, bp[0], bn[0]);
          const uint2 w1 = split_product(p01.y, bp[1], bn[1]);
          const uint2 w2 = split_product(p23.x, bp[2], bn[2]);
          const uint2 w3 = split_product(p23.y, bp[3], bn[3]);
          *(u32x4*)(pa + (vg * NREP + h) * LROW + 4 * n) = u32x4{w0.x, w1.x, w2.x, w3.x};
          *(u32x4*)(pa_lo + (vg * NREP + h) * LROW + 4 * n) = u32x4{w0.y, w1.y, w2.y, w3.y};
        }
      }
    }
    wave_lds_sync();

    // ---------- rescale the accumulators (softmax correction and value-tile
    // exponent; acc_a was rescaled above).  Unconditional: a branch around it
    // costs the accumulators a register copy on every tile.
    kacc = kv_exp;
    kacc_init = true;
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const int i = sl * RS;
      const float f = corr[sl] * fexp;
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[vg][j][i] *= f, acc[vg][j][i + 1] *= f;
      }
    }

    // ---------- acc += P V
    if constexpr (quant) {
      // steps st = (kt, vg), software-pipelined like Q.K
      u32x4 vz[NGH];
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg) vz[vg] = *(const u32x4*)(W + S::VZP + vg * 64 + g * 16);
      auto vzp = [&](int st) { return vz[st % NGH][st / NGH]; };
      constexpr int NST = 4 * NGH;  // P.V steps (k-tile, value group)
      constexpr int CPS = 8 / NST;  // scalar chunks per step
      u32x4 Ac = *(const u32x4*)(pv_row + 4 * g);
      u32x4 Bc[4], Bn[4];
      uint32_t adc[4][4], adn[4][4];
      addr_ktile<BITS>(VW, vzp(0), grep, odd, lsh, adc);
      read_ktile<S::TBL_V, F::PAIR, F::QUAD>(smem, adc, Bc);
      addr_ktile<BITS>(VW + F::WPK, vzp(1), grep, odd, lsh, adn);
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const int vg = st % NGH;
        u32x4 An;
        if (st + 1 < NST) {
          const int kt1 = (st + 1) / NGH, vg1 = (st + 1) % NGH;
          An = *(const u32x4*)(pv_row + vg1 * NREP * LROW + 16 * kt1 + 4 * g);
          read_ktile<S::TBL_V, F::PAIR, F::QUAD>(smem, adn, Bn);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (st + 2 < NST) addr_ktile<BITS>(VW + F::WPK * (st + 2), vzp(st + 2), grep, odd, lsh, adn);
#pragma unroll
        for (int c = 0; c < CPS; ++c) scal_chunk(MN, CPS * st + c);  // the next tile's scalars
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) acc[vg][jt] = Mfma<MZ_F16>::run(Ac, Bc[jt], acc[vg][jt]);
        __builtin_amdgcn_sched_barrier(0);
        if (st + 1 < NST) {
          Ac = An;
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) Bc[jt] = Bn[jt];
        }
      }
    } else {
      // residual values: B pairs (v, 0) against A pairs (p, 0); each k-tile's
      // 8 value vectors are loaded together through a buffer that starts at
      // the k-tile's first row and ends after its last filled row (padding
      // rows read 0, p = 0 there); the value-group column step rides in the
      // scalar offset and never leaves a row
      const int vst = a.vr_st * 2;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const u32x4 pd = *(const u32x4*)(pv_row + 16 * kt + 4 * g);  // (p, 0) pairs (row 1: zeros)
        const int rows = n_valid - 16 * kt;
        const __amdgpu_buffer_rsrc_t vrb =
            make_buf(bf.vr + (int64_t)(r0 + 16 * kt) * a.vr_st, rows > 0 ? (rows - 1) * vst + HD * 2 : 0);
        uint32_t vv[NGH][4][2];
#pragma unroll
        for (int vg = 0; vg < NGH; ++vg)
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const auto raw =
                __builtin_amdgcn_raw_buffer_load_b64(vrb, (4 * g + ii) * vst + 8 * n, 128 * vg, 0);
            vv[vg][ii][0] = raw[0];
            vv[vg][ii][1] = raw[1];
          }
#pragma unroll
        for (int vg = 0; vg < NGH; ++vg) {
          uint32_t (&v4)[4][2] = vv[vg];
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) {  // channel 64vg + 4n + jt
            u32x4 B;
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
              const uint32_t w = v4[ii][jt >> 1];
              const uint16_t h = (jt & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xFFFFu);
              B[ii] = IO == MZ_F16 ? (uint32_t)h : (uint32_t)f2h(bf2f(h));
            }
            acc[vg][jt] = Mfma<MZ_F16>::run(pd, B, acc[vg][jt]);
          }
        }
      }
    #pragma unroll
      for (int c = 0; c < 8; ++c) scal_chunk(MN, c);  // the next tile's scalars
    }
    wave_lds_sync();
  };

  // tiles of this wave: tile0, tile0 + 4, ...
  // Two waves (of two workgroups) share a SIMD and its issue slots go to the
  // older one first: with equal shares one wave would finish early and leave
  // the other to run alone.  Every wave has the same number of tiles, so a
  // wave's priority falls with its progress (4 levels) and the SIMD favours
  // the wave that is behind.  Workgroups are placed in launch order, one per
  // CU and then a second one, so the younger workgroup of a CU (linear index
  // >= `cus`) starts one level higher.  The tile assignment itself is fixed:
  // results do not depend on timing.
#pragma unroll
  for (int c = 0; c < 8; ++c) scal_chunk(MT, c);  // the first tile's scalars
  const int n_mine = (n_virt - v0 + WAVES - 1) / WAVES;
  const int wg_lin = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  const int older = wg_lin < cus ? 1 : 0;  // the first workgroup of its CU: one level lower
  int done = 0;
  if (older) __builtin_amdgcn_s_setprio(2);
  else __builtin_amdgcn_s_setprio(3);
  auto step = [&](auto quant_tag, const int v) {
    process(quant_tag, tile_of(v), v + WAVES < n_virt ? tile_of(v + WAVES) : q_last);
    ++done;
    switch ((4 * done) / max(n_mine, 1) + older) {  // wave-uniform
      case 0: break;
      case 1: __builtin_amdgcn_s_setprio(2); break;
      case 2: __builtin_amdgcn_s_setprio(1); break;
      default: __builtin_amdgcn_s_setprio(0); break;
    }
  };
  int v = v0;
  for (; v < n_res; v += WAVES) step(std::false_type{}, v);  // residual tiles come first
  for (; v < n_virt; v += WAVES) step(std::true_type{}, v);
  __builtin_amdgcn_s_setprio(0);

  // ---------------- merge the waves and write this split's partial records
  __syncthreads();
  float* red = (float*)(smem + S::WAVE0);
  constexpr int RED = 2 * NREP + NREP * D;  // per wave: m[NREP], l[NREP], acc[NREP][D] (first HD used)
  // lane-derived indices recomputed from the lane id (mbcnt) instead of kept
  // live across the tile loop, where every register is taken
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int tid_e = wave * 64 + lane_e;  // threadIdx.x, recomputed for the same reason
  const int n_e = lane_e & 15, g_e = lane_e >> 4;
  if (((4 * g_e) % RS) == 0) {
    const int h0 = (4 * g_e) / RS, n = n_e;
    float* w = red + wave * RED;
    const float unit = ldexpf(1.f, -kacc);
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const int i = sl * RS, h = h0 + sl;
      // the row's partial sums (the 16 lanes of lane group g_e)
      const float l_row = group_reduce<16>(l_run[sl], OpAdd());
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg) acc_a[sl][vg] = group_reduce<16>(acc_a[sl][vg], OpAdd());
      if (n == 0) {
        w[h] = m_run[sl];
        w[NREP + h] = l_row;
      }
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg)
        *(f32x4*)(w + 2 * NREP + h * D + 64 * vg + 4 * n) =
            f32x4{acc[vg][0][i] + acc[vg][0][i + 1] + acc_a[sl][vg], acc[vg][1][i] + acc[vg][1][i + 1] + acc_a[sl][vg],
                  acc[vg][2][i] + acc[vg][2][i + 1] + acc_a[sl][vg], acc[vg][3][i] + acc[vg][3][i + 1] + acc_a[sl][vg]} *
            unit;
    }
  }
  __syncthreads();
  if (direct) {
    // one split: the final output, exactly as the combine kernel would form it
    for (int e = tid_e; e < a.n_rep * HD; e += NT) {
      const int h = e / HD;
      const int c = e - h * HD;
      float M_ = -INFINITY;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) M_ = fmaxf(M_, red[w * RED + h]);
      float num = 0.f, den = 0.f;
      if (M_ != -INFINITY) {
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          const float f = __builtin_amdgcn_exp2f(red[w * RED + h] - M_);
          num += f * red[w * RED + 2 * NREP + h * D + c];
          den += f * red[w * RED + NREP + h];
        }
      }
      store_val(a.out, b * a.out_sb + (int64_t)(kvh * a.n_rep + h) * a.out_sh + c, den > 0.f ? num / den : 0.f,
                a.out_dtype);
    }
    return;
  }
  for (int e = tid_e; e < a.n_rep * (HD + 2); e += NT) {
    const int h = e / (HD + 2);
    const int c = e - h * (HD + 2);
    float M_ = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M_ = fmaxf(M_, red[w * RED + h]);
    float val = 0.f;
    if (c == HD) {
      val = M_ * kLn2;  // the record's maximum in natural-log units
    } else if (M_ != -INFINITY) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float f = __builtin_amdgcn_exp2f(red[w * RED + h] - M_);
        val += f * (c == HD + 1 ? red[w * RED + NREP + h] : red[w * RED + 2 * NREP + h * D + c]);
      }
    }
    ws_record<HD>(a, b, kvh * a.n_rep + h, split, n_split)[c] = val;
  }
}

}  // namespace fold

// ------------------------------------------------------------------ host side

static bool fold_meta_aligned(const void* p, int64_t sb, int64_t sh, int dt) {
  const int pair = dt == MZ_F32 ? 8 : 4;  // two adjacent entries are read at once
  return ((uintptr_t)p % pair) == 0 && sb % 2 == 0 && sh % 2 == 0;
}

bool fold_supported(const mz_decode_args* a) {
  const int64_t es = a->meta_dtype == MZ_F32 ? 4 : 2;
  const int64_t qb = 8 * (int64_t)a->bits;
  // buffer-resource ranges are 32-bit
  const int64_t ngv = a->head_dim / 64;  // value groups per token
  const bool fits = (int64_t)a->n_groups * fold::TILE * ngv * qb < ((int64_t)1 << 31) &&
                    (int64_t)a->n_groups * a->head_dim * es < ((int64_t)1 << 31);
  const bool aligned = a->v_prefix == 0 || a->v_prefix == a->n_groups * fold::TILE;
  // 8 query heads per kv-head take one workgroup per CU (their per-wave
  // operand staging is twice that of 4 heads; at 7 bits a workgroup of 4
  // waves beside the 64 KB table).  Other head counts run the kernel built
  // for the next larger count (3 -> 4, 5..7 -> 8) with the extra heads'
  // queries zero and their outputs unwritten
  const bool nrep_ok = a->n_rep >= 1 && a->n_rep <= 8;
  const bool one_table = a->bits < 7 || a->fold_k == a->fold_v;
  return a->bits >= 1 && a->bits <= 7 && (a->head_dim == 128 || a->head_dim == 64) && a->n_groups > 0 && fits && aligned && nrep_ok &&
         one_table && a->fold_k && a->fold_v &&
         ((uintptr_t)a->fold_k % 4) == 0 && ((uintptr_t)a->fold_v % 4) == 0 &&
         ((uintptr_t)a->k_packed % 4) == 0 && ((uintptr_t)a->v_packed % 4) == 0 && a->kp_sb % 4 == 0 &&
         a->kp_sh % 4 == 0 && a->vp_sb % 4 == 0 && a->vp_sh % 4 == 0 &&
         fold_meta_aligned(a->k_mn, a->km_sb, a->km_sh, a->meta_dtype) &&
         fold_meta_aligned(a->k_scale, a->km_sb, a->km_sh, a->meta_dtype) &&
         fold_meta_aligned(a->v_mn, a->vm_sb, a->vm_sh, a->meta_dtype) &&
         fold_meta_aligned(a->v_scale, a->vm_sb, a->vm_sh, a->meta_dtype);
}


int fold_choose_split(const mz_decode_args* a, int* tiles_per_split) {
  const int n_tiles = a->n_groups + (a->n_residual + fold::TILE - 1) / fold::TILE;
  int ns = a->n_split;
  if (ns <= 0) {
    // fill the resident workgroup slots once: every workgroup then runs its
    // tiles in one pass with its tables loaded once.  Two workgroups fit a
    // CU up to 4 query heads per kv-head and 6 bits; the 8-head kernels and
    // the 7-bit workgroups take a CU alone.
    const int64_t units = std::max<int64_t>(1, (int64_t)a->batch * a->kv_heads);  // an empty batch splits nothing
    const int per_cu = (a->n_rep > 4 || a->bits >= 7) ? 1 : 2;
    const int64_t slots = per_cu * (int64_t)device_cu_count();
    ns = (int)((slots + units - 1) / units);
    ns = max(1, min(ns, (n_tiles + 7) / 8));  // at least 2 tiles per wave
  }
  ns = min(ns, n_tiles);
  const int tps = (n_tiles + ns - 1) / ns;
  *tiles_per_split = tps;
  return (n_tiles + tps - 1) / tps;
}

int fold_launch_partials(const mz_decode_args* a, hipStream_t s, bool direct) {
  int tps;
  const int ns = fold_choose_split(a, &tps);
  const dim3 grid(ns, a->kv_heads, a->batch);
  const uint32_t* fk = (const uint32_t*)a->fold_k;
  const uint32_t* fv = (const uint32_t*)a->fold_v;
  const int dir = direct ? 1 : 0;
  const int cus = device_cu_count();
  // query heads per kv-head of the kernel that runs: n_rep rounded up to a power of two
  const int nrep_pad = a->n_rep <= 1 ? 1 : a->n_rep <= 2 ? 2 : a->n_rep <= 4 ? 4 : a->n_rep <= 8 ? 8 : 0;
#define MZ_FOLD_HD(IOV, NR, BB, HD)                                                                     \
  if (a->meta_dtype == MZ_F32)                                                                          \
    hipLaunchKernelGGL((fold::fold_kernel<IOV, NR, BB, 2, HD>), grid, dim3(64 * fold::waves_for<NR, BB>()), 0, s, *a, tps, ns, fk, fv, dir, cus); \
  else                                                                                                       \
    hipLaunchKernelGGL((fold::fold_kernel<IOV, NR, BB, 1, HD>), grid, dim3(64 * fold::waves_for<NR, BB>()), 0, s, *a, tps, ns, fk, fv, dir, cus)
#define MZ_FOLD(IOV, NR, BB)                                        \
  if (a->head_dim == 128) { MZ_FOLD_HD(IOV, NR, BB, 128); } \
  else { MZ_FOLD_HD(IOV, NR, BB, 64); }
#define MZ_FOLD_NREP(IOV, BB)            \
  switch (nrep_pad) {                    \
    case 1: MZ_FOLD(IOV, 1, BB); break;  \
    case 2: MZ_FOLD(IOV, 2, BB); break;  \
    case 4: MZ_FOLD(IOV, 4, BB); break;  \
    case 8: MZ_FOLD(IOV, 8, BB); break;  \
    default: return MZ_EUNSUPPORTED;     \
  }
#define MZ_FOLD_BITS(IOV)                              \
  if (a->bits == 4) { MZ_FOLD_NREP(IOV, 4) }           \
  else if (a->bits == 3) { MZ_FOLD_NREP(IOV, 3) }      \
  else if (a->bits == 2) { MZ_FOLD_NREP(IOV, 2) }      \
  else if (a->bits == 1) { MZ_FOLD_NREP(IOV, 1) }      \
  else if (a->bits == 5) { MZ_FOLD_NREP(IOV, 5) }      \
  else if (a->bits == 6) { MZ_FOLD_NREP(IOV, 6) }      \
  else if (a->bits == 7) { MZ_FOLD_NREP(IOV, 7) }      \
  else return MZ_EUNSUPPORTED;
  if (a->io_dtype == MZ_BF16) { MZ_FOLD_BITS(MZ_BF16) } else { MZ_FOLD_BITS(MZ_F16) }
#undef MZ_FOLD_BITS
#undef MZ_FOLD_NREP
#undef MZ_FOLD
#undef MZ_FOLD_HD
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

}  // namespace mz
