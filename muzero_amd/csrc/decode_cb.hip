// Packed-KV decode attention over per-tile codebooks, 1- to 5-bit codes
// (gfx950, wave64, MFMA 16x16x32 in the layer dtype).
//
// Every value this kernel attends with is the reference's dequantize-then-
// attend value bit for bit: a quantized group (one key channel or one value
// token-group of 64 elements) has only 2^bits distinct values, so each wave
// forms, for each group of its tile, those values with the reference's own
// fp32 operation order (muzero/quantizer.py:241-255: t = pe*E or -ne*E,
// unit = za + t, x = unit*s + mn) rounded to the layer dtype
// (muzero/cache/layer.py:263) -- the group's codebook, in LDS -- and then
// reads each code's value straight into an MFMA operand register.  Q.K is
// then an MFMA of the query (in its own dtype) against the keys' values,
// P.V one of the softmax weights against the values' values, both
// accumulated in fp32: no operand products, no constant-part MFMAs, 32 MFMAs
// per tile.
//
// Work of one wave: a 64-token tile = one key group per channel and one
// value group per (token, 64 channels).
//   QK: MFMA rows = query heads (row RS*h, RS = 16 / NREP; the other rows
//   zero); columns = tokens 4n+jt of N-tiles jt = 0..3; lane (n, g) of
//   k-step kt holds channels 32kt+8g+{0..7} and needs, for each, the 4 codes
//   of its tokens 4n..4n+3 (16 bits of the channel's 32-byte row).
//   PV: rows RS*h / RS*h+1 = the high / low parts of the head's weights in
//   the layer dtype (their sum carries each weight to ~2^-17); columns =
//   channels 64vg+4n+jt; lane (n, g) of step (kt, vg) holds tokens
//   32kt+8g+{0..7} and needs, for each, the codes of its channels 4n..4n+3.
//   Lanes 2m, 2m+1 load a word of two different rows and swap halves with
//   one DPP move, so each lane then holds its 16 bits of both rows.
// 4-bit codebook layout (per wave, keys and values alike): group r's 16
// entries (2 bytes each) at byte 288*(r/8) + 32*(r%8) + 2q.  One lookup
// instruction reads one group per lane group (16 lanes, 32 bytes = 8 banks),
// and the 32 bytes of padding per 8 groups put the 4 lane groups of every
// instruction in disjoint bank octets: the lookups are free of bank
// conflicts.  The address is one v_perm per code: byte 0 = 2q (+32g), bytes
// 1-3 = the lane group's block base; the row and step offsets ride in the
// instruction.  Two lookups fill one B register (rows 2i, 2i+1).
// 3-bit codes: group r's 8 entries at byte 144*(r/8) + 16*(r%8) + 2q; the 16
// bytes of padding per 8 groups put the 4 lane groups of a lookup in 4
// different 16-byte bank slots and 8 consecutive lanes' codebook stores (16
// bytes each) in 8.  The address is a bit-field extract of the code and one
// shift-or onto the lane group's base per code (3-bit codes straddle bytes).
// 5-bit codes: group r's 32 entries (64 bytes) at byte 512*(r/8) +
// 64*((r%8) ^ (r/8 % 2)): the groups of lane groups g and g ^ 1 in one lookup
// lie in opposite bank halves (two lane bases per lane, for even and odd
// rows), and each lane stores its 16-byte codebook chunks in a rotated order
// so that 8 lanes' stores hit 8 bank slots.  Each lane reads its own dword
// of every row (4 codes of 5 bits); the address is a bit-field extract and a
// shift-or per code.  The (E+, E-) table is 32 x 32 pairs; one table serves
// keys and values (5-bit calls with two alphas run the fold kernel).
// 2-bit codes: the two rows of a B register (channels or tokens 2i, 2i+1)
// share a joint codebook of their 4 x 4 code pairs, each entry the two
// values as one dword: one 32-bit read per code pair fills a B register,
// its address one v_dot4_u32_u8 of the two codes (masked in place) plus the
// lane group's base.  A pair's 16 entries take 64 bytes = 16 banks; pair
// (step s, i, lane group g) lies at byte 272*(4s + i) + 64g: the pairs of
// lane groups g and g ^ 1 (one half-wave) lie in opposite bank halves, and
// the 16 bytes of padding per 4 pairs put the pairs that 8 consecutive lanes
// write (i = 0..3, two lane groups) in 8 different 16-byte bank slots, so the
// 128-bit codebook stores are free of conflicts too.
// 1-bit codes: the four rows of two B registers (4h .. 4h + 3) share a quad
// codebook of their 16 code combinations, each entry the four values as two
// dwords: one 64-bit read per four codes, its address one v_dot4_u32_u8 of
// the four code bits.  A quad's 128 bytes lie in a 256-byte slot, offset
// within it so that the 8 lanes of one 128-bit store (4 quads, two halves
// each) hit 8 different 16-byte bank slots; a 64-bit read serves one lane
// group (one quad) per cycle, free of conflicts.
// The (E+, E-) pairs the codebooks are formed from (E+ = E[pb][q-zl] above
// the zero level, E- = E[nb][zl-q] below it, the other 0) are a 16 x 16
// table per alpha in LDS, built at setup from the expm1 rows; a pair turns
// the side's product into t = fma(pe, E+, -ne*E-) with no per-code select.
//
// Launch, splits, wave priorities and the final merge are those of the fold
// kernel (decode_fold.hip): one workgroup of 4 waves per (batch, kv-head,
// split), residual tiles first, waves take every 4th tile; one split writes
// the output itself, more go through the workspace and the combine kernel.
#include <type_traits>

#include "decode_tile.hpp"

namespace mz {

namespace cb {

constexpr int D = 128;
constexpr int TILE = 64;
constexpr int WAVES = 4;
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kLn2 = 0.693147180559945309f;

// 4 bits: per group 16 entries of 2 bytes, 32 bytes of padding per 8 groups
constexpr int CB_GROUP = 32;
constexpr int CB_BLOCK = 8 * CB_GROUP + 32;
// 1 bit: per row quad 16 entries of 8 bytes, in a 256-byte slot
constexpr int CB_QUAD = 256;
// 5 bits: per group 32 entries of 2 bytes, 8 groups per 512-byte block
constexpr int CB_BLOCK5 = 8 * 64;
// 3 bits: per group 8 entries of 2 bytes, 16 bytes of padding per 8 groups
constexpr int CB_BLOCK3 = 8 * 16 + 16;
// 2 bits: per row pair 16 entries of 4 bytes; the 4 lane groups' pairs of one
// (step, i) in a block of 4 pairs + 16 bytes
constexpr int CB_PAIR = 64;
constexpr int CB_PAIRS = 4 * CB_PAIR + 16;

template <int BITS>
struct Fmt {
  static constexpr int QMAX = (1 << BITS) - 1;
  static constexpr int QB = 8 * BITS;       // bytes per packed 64-code row
  static constexpr bool PAIR = BITS == 2;   // joint codebooks of row pairs
  static constexpr bool QUAD = BITS == 1;   // joint codebooks of row quads
  static constexpr bool WIDE = BITS == 5;   // one dword per lane and row
  // (E+, E-) table: rows of zero levels, 8 bytes per code, 8 bytes of padding;
  // 5 bits: one table for keys and values
  static constexpr int ET_ROW = (QMAX + 1 > 16 ? QMAX + 1 : 16) * 8 + 8;
  static constexpr int ET_BYTES = (QMAX + 1 > 16 ? QMAX + 1 : 16) * ET_ROW;
  static constexpr int ET_TABLES = WIDE ? 1 : 2;
  static constexpr int CODE_WORDS = WIDE ? 32 : 16;  // code words per lane and tile, each of keys and values
  // codebook bytes per side and wave (128 groups; 2 bits: 64 row pairs), a multiple of 256
  static constexpr int CB_BYTES =
      WIDE ? 16 * CB_BLOCK5 : QUAD ? 32 * CB_QUAD : PAIR ? 16 * CB_PAIRS : BITS == 3 ? 16 * CB_BLOCK3 : 16 * CB_BLOCK;
};
constexpr int QROW = D * 2 + 16;       // bytes per head row of the query copy
constexpr int PROW = TILE * 2 + 16;    // bytes per head row of the weight staging

template <int NREP, int BITS>
struct Smem {
  static constexpr int CB_BYTES = Fmt<BITS>::CB_BYTES;
  // (E+, E-) tables: rows padded by 8 bytes so that lanes reading different
  // zero levels at one code use different banks
  static constexpr int ETK = 0;
  static constexpr int ETV = Fmt<BITS>::ET_TABLES == 2 ? Fmt<BITS>::ET_BYTES : 0;
  static constexpr int QIO = Fmt<BITS>::ET_TABLES * Fmt<BITS>::ET_BYTES;  // query, io dtype [NREP][QROW]
  static constexpr int ZERO = QIO + NREP * QROW;      // 256 zero bytes: A rows that must be 0
  static constexpr int WAVE0 = (ZERO + 256 + 255) / 256 * 256;
  // per wave (256-aligned: a lane group's codebook base has byte 0 = 32g)
  static constexpr int KCB = 0;
  static constexpr int VCB = CB_BYTES;
  static constexpr int PST = 2 * CB_BYTES;            // io dtype [2 parts][NREP][PROW]: weights hi / lo
  static constexpr int PER_WAVE = (PST + 2 * NREP * PROW + 255) / 256 * 256;
  static constexpr int MERGE = (2 * NREP + NREP * D) * 4;  // per wave at the end (aliases the wave area)
  static constexpr int TOTAL = WAVE0 + WAVES * (PER_WAVE > MERGE ? PER_WAVE : MERGE);
};

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t lds_u16(const uint8_t* smem, uint32_t addr) {
  return *(const uint16_t*)(smem + addr);
}

// Two fp32 values rounded to the io dtype (round to nearest even), packed
// low / high.
template <int IO>
__device__ __forceinline__ uint32_t pack_io2(float x0, float x1) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  if constexpr (IO == MZ_BF16) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{x0, x1}), b2));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{x0, x1}), h2));
  }
}

template <int IO>
__device__ __forceinline__ float io_to_f32(uint16_t h) {
  return IO == MZ_BF16 ? bf2f(h) : h2f(h);
}

// Dequantization quantities of one stored group (mn, s), as the reference
// forms them from the stored metadata (quantizer.py:241-249), the scale
// guarded like the reference CUDA extension (loader.py:201) so that an
// all-zero group (stored scale 0) gives x = mn.
struct Group {
  float mn, s, za, pe, mne;  // mne = -ne
  uint32_t row;              // byte offset of the zero level's (E+, E-) row
};

template <int QMAX, int ET_ROW>
__device__ __forceinline__ Group group_of(float mn, float s) {
  const float eps = 1e-8f;
  Group r;
  r.mn = mn;
  r.s = s >= eps ? s : eps;                        // NaN -> eps, as deq_row
  r.za = clamp01((0.f - mn) / r.s);                // IEEE division: the zero level must match
  const float zl = rintf(r.za * (float)QMAX);
  r.pe = clamp_min(1.f - r.za, eps);
  r.mne = -clamp_min(r.za, eps);
  // a NaN zero level (NaN metadata) reads row 0: the values are NaN anyway
  r.row = (uint32_t)__builtin_amdgcn_fmed3f(zl == zl ? zl : 0.f, 0.f, (float)QMAX) * ET_ROW;
  return r;
}

// The value of the code whose (E+, E-) pair is `v`: the reference's fp32
// operation order (quantizer.py:250-255).  unit = za + t needs no clamp: for
// finite metadata it lies in [0, 1] already (t = pe*E with pe = fl(1 - za)
// gives za + t <= 1 after rounding; t = -za*E gives za + t >= 0), and NaN
// metadata propagates.
__device__ __forceinline__ float code_value(const Group& gr, float2 v) {
  const float t = __builtin_fmaf(gr.pe, v.x, gr.mne * v.y);
  const float unit = gr.za + t;
  const float u = unit * gr.s;
  return u + gr.mn;
}

// A group's 4 values (2-bit codes) in the io dtype: (x0, x1), (x2, x3).
template <int IO>
__device__ __forceinline__ uint2 values4(const uint8_t* smem, int et, const Group& gr) {
  float2 pn[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) pn[q] = *(const float2*)(smem + et + gr.row + 8 * q);
  return uint2{pack_io2<IO>(code_value(gr, pn[0]), code_value(gr, pn[1])),
               pack_io2<IO>(code_value(gr, pn[2]), code_value(gr, pn[3]))};
}

// A group's 2 values (1-bit codes) in the io dtype, packed (x0, x1).
template <int IO>
__device__ __forceinline__ uint32_t values2(const uint8_t* smem, int et, const Group& gr) {
  const float2 p0 = *(const float2*)(smem + et + gr.row), p1 = *(const float2*)(smem + et + gr.row + 8);
  return pack_io2<IO>(code_value(gr, p0), code_value(gr, p1));
}

// Half B3 of a quad codebook (entries 8*B3 .. 8*B3 + 7, 64 bytes at `dst`)
// from the four rows' packed values R[r] = (x_r(0), x_r(1)): entry e =
// (x_0(b0), x_1(b1)), (x_2(b2), x_3(b3)) for the bits b of e.  `hsel` = the
// selector half taking x_3(B3): 0x07060000 for B3 = 1, else 0x05040000.
__device__ __forceinline__ void build_quad_half(const uint32_t (&R)[4], uint32_t hsel, uint8_t* dst) {
  uint32_t d0[4], d1[2];
#pragma unroll
  for (int b = 0; b < 4; ++b)
    d0[b] = __builtin_amdgcn_perm(R[1], R[0], (b & 1 ? 0x0302u : 0x0100u) | (b & 2 ? 0x07060000u : 0x05040000u));
#pragma unroll
  for (int b2 = 0; b2 < 2; ++b2) d1[b2] = __builtin_amdgcn_perm(R[3], R[2], (b2 ? 0x0302u : 0x0100u) | hsel);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    *(u32x4*)(dst + 16 * k) = u32x4{d0[2 * (k & 1)], d1[k >> 1], d0[2 * (k & 1) + 1], d1[k >> 1]};
}

// 1-bit codes: the B operands of one step from its 4 code words: w[p] = the
// byte of the step's row 2p + (n & 1) holding the codes of the lane pair
// (tokens / channels 8m .. 8m + 7, m = n / 2); this lane's codes from bit
// sh1 = 4 (n & 1).  lb[h]: the lane group's base of its quad h codebook;
// IMM[h]: the step's offset of quad h.
template <int IMM0, int IMM1>
__device__ __forceinline__ void lookup1(const uint8_t* smem, const uint32_t* w, const uint32_t (&lb)[2], bool odd,
                                        uint32_t sh1, u32x4 (&B)[4]) {
  const uint32_t sel = odd ? 0x02060004u : 0x06020400u;
  uint32_t W[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t own = w[2 * h] | (w[2 * h + 1] << 16);
    W[h] = __builtin_amdgcn_perm(dpp_swap_pairs(own), own, sel) >> sh1;  // byte r: codes of row 4h + r, bit jt
  }
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t ad = __builtin_amdgcn_udot4(W[h] & (0x01010101u << jt), 0x40201008u >> jt, lb[h], false);
      const uint2 v = *(const uint2*)(smem + ad + (h ? IMM1 : IMM0));
      B[jt][2 * h] = v.x;
      B[jt][2 * h + 1] = v.y;
    }
}

// Values 8c .. 8c + 7 of a 5-bit group's codebook, written to its 16 bytes at
// `cbg` + 16c (cbg: the group's 64 bytes).
template <int IO>
__device__ __forceinline__ void build_chunk5(const uint8_t* smem, int et, const Group& gr, uint8_t* cbg, int c) {
  float2 pn[8];
  const uint8_t* src = smem + et + gr.row + 64 * c;
#pragma unroll
  for (int e = 0; e < 8; ++e) pn[e] = *(const float2*)(src + 8 * e);
  uint32_t w[4];
#pragma unroll
  for (int q2 = 0; q2 < 4; ++q2) w[q2] = pack_io2<IO>(code_value(gr, pn[2 * q2]), code_value(gr, pn[2 * q2 + 1]));
  *(u32x4*)(cbg + 16 * c) = u32x4{w[0], w[1], w[2], w[3]};
}

__device__ __forceinline__ uint32_t cb5_offset(int r) {
  return (uint32_t)((r >> 3) * CB_BLOCK5 + 64 * ((r & 7) ^ ((r >> 3) & 1)));
}

// 5-bit codes: the B operands of one step from its 8 code words: w[j] = this
// lane's dword of the step's row j, its code jt at bit sh + 5jt.  lb[j % 2]:
// the lane group's base for even / odd rows (bits 0-5 zero); IMM: the step's
// first block.
template <int IMM>
__device__ __forceinline__ void lookup5(const uint8_t* smem, const uint32_t* w, const uint32_t (&lb)[2], uint32_t sh,
                                        u32x4 (&B)[4]) {
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a0 = (__builtin_amdgcn_ubfe(w[2 * i], sh + 5 * jt, 5) << 1) | lb[0];
      const uint32_t a1 = (__builtin_amdgcn_ubfe(w[2 * i + 1], sh + 5 * jt, 5) << 1) | lb[1];
      const uint16_t lo = lds_u16(smem, a0 + (IMM + 2 * i * 64));
      const uint16_t hi = lds_u16(smem, a1 + (IMM + (2 * i + 1) * 64));
      B[jt][i] = __builtin_bit_cast(uint32_t, u16x2{lo, hi});
    }
}

// A group's 8 values (3-bit codes) in the io dtype, written as its codebook (16 bytes at `dst`).
template <int IO>
__device__ __forceinline__ void build_group8(const uint8_t* smem, int et, const Group& gr, uint8_t* dst) {
  float2 pn[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) pn[q] = *(const float2*)(smem + et + gr.row + 8 * q);
  uint32_t w[4];
#pragma unroll
  for (int q2 = 0; q2 < 4; ++q2) w[q2] = pack_io2<IO>(code_value(gr, pn[2 * q2]), code_value(gr, pn[2 * q2 + 1]));
  *(u32x4*)dst = u32x4{w[0], w[1], w[2], w[3]};
}

__device__ __forceinline__ uint32_t cb3_offset(int r) { return (uint32_t)((r >> 3) * CB_BLOCK3 + (r & 7) * 16); }

// The joint codebook of a row pair from the rows' values lo (first row) and
// hi (second): entry q0 + 4*q1 = (lo[q0], hi[q1]) as one dword, 64 bytes at `dst`.
__device__ __forceinline__ void build_pair(const uint2 lo, const uint2 hi, uint8_t* dst) {
  uint32_t w[16];
#pragma unroll
  for (int q1 = 0; q1 < 4; ++q1)
#pragma unroll
    for (int q0 = 0; q0 < 4; ++q0) {
      const uint32_t l = q0 < 2 ? lo.x : lo.y, h = q1 < 2 ? hi.x : hi.y;
      const uint32_t sel = (q0 & 1 ? 0x0302u : 0x0100u) | (q1 & 1 ? 0x07060000u : 0x05040000u);
      w[q0 + 4 * q1] = __builtin_amdgcn_perm(h, l, sel);
    }
#pragma unroll
  for (int k = 0; k < 4; ++k) *(u32x4*)(dst + 16 * k) = u32x4{w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
}

// Values 8*half .. 8*half + 7 of the group's codebook in the io dtype,
// written to its 16 bytes at `cbg` + 16*half (cbg: the group's 32 bytes).
template <int IO>
__device__ __forceinline__ void build_half(const uint8_t* smem, int et, const Group& gr, uint8_t* cbg, int half) {
  float2 pn[8];
  const uint8_t* src = smem + et + gr.row + 64 * half;
#pragma unroll
  for (int e = 0; e < 8; ++e) pn[e] = *(const float2*)(src + 8 * e);
  uint32_t w[4];
#pragma unroll
  for (int q2 = 0; q2 < 4; ++q2) {
    float x[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) x[e] = code_value(gr, pn[2 * q2 + e]);
    w[q2] = pack_io2<IO>(x[0], x[1]);
  }
  *(u32x4*)(cbg + 16 * half) = u32x4{w[0], w[1], w[2], w[3]};
}

__device__ __forceinline__ uint32_t cb_offset(int r) { return (uint32_t)((r >> 3) * CB_BLOCK + (r & 7) * CB_GROUP); }

// 4-bit codes: the B operands (columns jt = 0..3) of one step from its 4
// code words: w[p] = this lane's word of the step's row 2p + (n & 1).  `lb`:
// the lane group's codebook base (byte 0 = 32g); IMM: the step's block offset.
template <int IMM>
__device__ __forceinline__ void lookup4(const uint8_t* smem, const uint32_t* w, uint32_t lb, uint32_t gb,
                                            bool odd, u32x4 (&B)[4]) {
  // after the swap: low half = the lane's 4 codes of row 2p, high half =
  // those of row 2p + 1 (code jt at bits 4jt)
  const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
  uint32_t ev[4], od[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t r = __builtin_amdgcn_perm(dpp_swap_pairs(w[p]), w[p], sel);
    ev[p] = ((r << 1) & 0x1E1E1E1Eu) | gb;  // 2q of codes 0, 2 of each row, one per byte
    od[p] = ((r >> 3) & 0x1E1E1E1Eu) | gb;  // codes 1, 3
  }
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t e = (jt & 1) ? od[i] : ev[i];
      const uint32_t a0 = __builtin_amdgcn_perm(lb, e, 0x07060500u | (uint32_t)(jt >> 1));
      const uint32_t a1 = __builtin_amdgcn_perm(lb, e, 0x07060500u | (uint32_t)(2 + (jt >> 1)));
      const uint16_t lo = lds_u16(smem, a0 + (IMM + 2 * i * CB_GROUP));
      const uint16_t hi = lds_u16(smem, a1 + (IMM + (2 * i + 1) * CB_GROUP));
      B[jt][i] = __builtin_bit_cast(uint32_t, u16x2{lo, hi});
    }
}

// 3-bit codes: the B operands of one step from its 4 code words: w[p] = the
// dword of the step's row 2p + (n & 1) holding the codes of the lane pair
// (read at byte min(3m, 20) of the 24-byte row, m = n / 2); this lane's code
// jt of a row is at bit sh + 3jt of it.  `lb`: the lane group's block base
// (its low 4 bits 0); IMM: the step's first block.
template <int IMM>
__device__ __forceinline__ void lookup3(const uint8_t* smem, const uint32_t* w, uint32_t lb, bool odd, uint32_t sh,
                                        u32x4 (&B)[4]) {
  uint32_t R[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t o = dpp_swap_pairs(w[p]);
    R[2 * p] = odd ? o : w[p];
    R[2 * p + 1] = odd ? w[p] : o;
  }
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t a0 = (__builtin_amdgcn_ubfe(R[2 * i], sh + 3 * jt, 3) << 1) | lb;
      const uint32_t a1 = (__builtin_amdgcn_ubfe(R[2 * i + 1], sh + 3 * jt, 3) << 1) | lb;
      const uint16_t lo = lds_u16(smem, a0 + (IMM + 2 * i * 16));
      const uint16_t hi = lds_u16(smem, a1 + (IMM + (2 * i + 1) * 16));
      B[jt][i] = __builtin_bit_cast(uint32_t, u16x2{lo, hi});
    }
}

// 2-bit codes: the B operands of one step from its 4 code words: w[p] = 16
// bits of the step's row 2p + (n & 1) (the codes of tokens / channels 8m ..
// 8m + 7, m = n / 2).  After the swap, byte r of W[h] = this lane's 4 codes
// of row 4h + r (code jt at bits 2jt).  `lb`: the lane group's base (pair
// g of the step); IMM: the step's first pair block; pair i's lies CB_PAIRS further.
template <int IMM>
__device__ __forceinline__ void lookup2(const uint8_t* smem, const uint32_t* w, uint32_t lb, bool odd,
                                        u32x4 (&B)[4]) {
  const uint32_t sel = odd ? 0x03070105u : 0x06020400u;
  uint32_t W[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t own = w[2 * h] | (w[2 * h + 1] << 16);
    W[h] = __builtin_amdgcn_perm(dpp_swap_pairs(own), own, sel);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t W2 = W[h] >> 4;  // codes 2, 3 at bits 0 and 2 of each byte
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      // the two rows' codes of column jt in place (times 1 or 4), then the
      // entry offset 4*q0 + 16*q1 of each of the word's two pairs
      const uint32_t t = (jt < 2 ? W[h] : W2) & ((jt & 1) ? 0x0C0C0C0Cu : 0x03030303u);
      const uint32_t w0 = (jt & 1) ? 0x00000401u : 0x00001004u;
#pragma unroll
      for (int pp = 0; pp < 2; ++pp) {
        const int i = 2 * h + pp;
        const uint32_t ad = __builtin_amdgcn_udot4(t, w0 << (16 * pp), lb, false);
        B[jt][i] = *(const uint32_t*)(smem + ad + (IMM + CB_PAIRS * i));
      }
    }
  }
}

template <int IO, int NREP, int MW, int BITS>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2))) void cb_kernel(
    const mz_decode_args a, int tiles_per_split, int n_split, int direct, int cus) {
  constexpr int NT = 64 * WAVES;
  using M = Mfma<IO>;
  using F = Fmt<BITS>;
  using S = Smem<NREP, BITS>;
  constexpr int QMAX = F::QMAX;
  constexpr int QB = F::QB;
  static_assert(S::TOTAL <= 80 * 1024, "two workgroups per CU");
  constexpr int RS = 16 / NREP;               // MFMA row stride between query heads
  static_assert(RS >= 2, "P.V needs a second row per head for the weights' low part");
  constexpr int HS = NREP > 4 ? NREP / 4 : 1;  // head slots per lane of the MFMA output
  constexpr int NGH = 2;                        // value groups per token
  __shared__ __align__(256) uint8_t smem[S::TOTAL];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const bool odd = (n & 1) != 0;
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
    bf.kp = make_buf(a.k_packed + b * a.kp_sb + kvh * a.kp_sh, ng * D * QB);
    bf.vp = make_buf(a.v_packed + b * a.vp_sb + kvh * a.vp_sh, ng * TILE * NGH * QB);
    const int64_t km = b * a.km_sb + kvh * a.km_sh, vm = b * a.vm_sb + kvh * a.vm_sh;
    bf.kmn = make_buf((const uint8_t*)a.k_mn + km * meta_es, ng * D * meta_es);
    bf.ksc = make_buf((const uint8_t*)a.k_scale + km * meta_es, ng * D * meta_es);
    bf.vmn = make_buf((const uint8_t*)a.v_mn + vm * meta_es, ng * TILE * NGH * meta_es);
    bf.vsc = make_buf((const uint8_t*)a.v_scale + vm * meta_es, ng * TILE * NGH * meta_es);
    bf.kr = (const uint16_t*)a.k_res + b * a.kr_sb + kvh * a.kr_sh;
    bf.vr = (const uint16_t*)a.v_res + b * a.vr_sb + kvh * a.vr_sh;
  }

  // the split's tiles in virtual order: residual tiles first, quantized
  // after; wave w takes virtual tiles w, w + WAVES, ...
  const int n_quant = max(0, min(t_end, a.n_groups) - t_begin);
  const int n_res = (t_end - t_begin) - n_quant;
  const int n_virt = t_end - t_begin;
  auto tile_of = [&](int v) { return v < n_res ? max(t_begin, a.n_groups) + v : t_begin + (v - n_res); };
  // loads are issued unconditionally; an index that is not a quantized tile
  // is replaced by one this split reads anyway
  const int q_last = max(0, min(t_end, a.n_groups) - 1);
  const int v0 = wave;

  // ---------------- workgroup setup: (E+, E-) tables and the query in LDS
  constexpr int EZ = F::ET_BYTES / F::ET_ROW;   // zero-level rows per table (16, or 32 at 5 bits)
  constexpr int EN = F::ET_TABLES * EZ * EZ;    // table entries
  constexpr int EW = (EN + NT - 1) / NT;        // table entries per thread
  constexpr int QW = (NREP * D + NT - 1) / NT;  // query elements per thread
  float2 et[EW];
  uint16_t qraw[QW];
#pragma unroll
  for (int j = 0; j < EW; ++j) {
    const int i = min(threadIdx.x + j * NT, EN - 1);
    const int t = i / (EZ * EZ), zl = (i / EZ) % EZ, q = i % EZ;
    const float* E = t ? a.e_value : a.e_key;
    float ep = 0.f, en = 0.f;
    if (zl > QMAX || q > QMAX) {
      // not a code of this width: never read
    } else if (q >= zl) {
      const int pb = max(QMAX - zl, 1);
      ep = E[expm1_row(pb) + q - zl];
    } else {
      const int nb = max(zl, 1);
      en = E[expm1_row(nb) + zl - q];
    }
    et[j] = float2{ep, en};
  }
#pragma unroll
  for (int j = 0; j < QW; ++j) {
    const int i = threadIdx.x + j * NT, h = i / D, c = i - h * D;
    qraw[j] = h < a.n_rep ? ((const uint16_t*)a.query)[b * a.q_sb + (int64_t)(kvh * a.n_rep + h) * a.q_sh + c] : 0;
  }
  MetaWords<MW> MT;  // metadata of the current tile
  uint32_t KW[F::CODE_WORDS], VW[F::CODE_WORDS];
  // the lane pair's word of a row: the codes of tokens (keys) / channels
  // (values) 8m .. 8m + 7, m = n / 2: 32 bits at 4 bits, 16 at 2, 8 at 1; at 3
  // bits the dword at byte min(3m, 20) (read unaligned; the last pair's moved
  // back inside the row), this lane's codes from bit sh3
  const int pbyte = BITS == 3 ? min(3 * (n >> 1), QB - 4) : BITS * (n >> 1);
  // 5 bits: this lane's own dword of each row (its 4 codes at bit 20n; the
  // last lane's dword moved back inside the 40-byte row)
  const int wbyte = min((20 * n) >> 3, QB - 4);
  const uint32_t sh5 = (uint32_t)(20 * n - 8 * wbyte);
  const uint32_t sh3 = (uint32_t)(8 * (3 * (n >> 1) - pbyte) + 12 * (n & 1));
  auto load_word = [&](const __amdgpu_buffer_rsrc_t& r, int voff, int soff) __attribute__((always_inline)) {
    if constexpr (BITS >= 3) return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    else if constexpr (BITS == 2) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
    else return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
  };
  // key words: KW[4kt + p] = this lane's word of channel row 32kt + 8g + 2p + (n & 1)
  const int kvoff = (8 * g + (n & 1)) * QB + pbyte;
  auto load_kw = [&](int tile) __attribute__((always_inline)) {
    const int soff = tile * D * QB;
    if constexpr (F::WIDE) {
      // KW[8kt + j] = this lane's dword of channel row 32kt + 8g + j
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          KW[8 * kt + j] = __builtin_amdgcn_raw_buffer_load_b32(bf.kp, 8 * g * QB + wbyte, soff + (32 * kt + j) * QB, 0);
      return;
    }
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int p = 0; p < 4; ++p) KW[4 * kt + p] = load_word(bf.kp, kvoff, soff + (32 * kt + 2 * p) * QB);
  };
  // value words: VW[4(2kt + vg) + p] = this lane's word of token row 32kt + 8g + 2p + (n & 1), group vg
  const int vvoff = (8 * g + (n & 1)) * (NGH * QB) + pbyte;
  auto load_vw = [&](int tile) __attribute__((always_inline)) {
    const int soff = tile * TILE * NGH * QB;
    if constexpr (F::WIDE) {
      // VW[8(2kt + vg) + j] = this lane's dword of token row 32kt + 8g + j, group vg
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int vg = 0; vg < NGH; ++vg)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            VW[8 * (2 * kt + vg) + j] = __builtin_amdgcn_raw_buffer_load_b32(
                bf.vp, 8 * g * (NGH * QB) + wbyte, soff + (32 * kt + j) * (NGH * QB) + QB * vg, 0);
      return;
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg)
#pragma unroll
        for (int p = 0; p < 4; ++p)
          VW[4 * (2 * kt + vg) + p] = load_word(bf.vp, vvoff, soff + (32 * kt + 2 * p) * (NGH * QB) + QB * vg);
  };
  load_meta_tile<MW, D>(MT, bf, min(tile_of(v0), q_last), lane);
  load_kw(min(tile_of(v0), q_last));
#pragma unroll
  for (int j = 0; j < EW; ++j) {
    const int i = threadIdx.x + j * NT;
    const int t = i / (EZ * EZ), zl = (i / EZ) % EZ, q = i % EZ;
    if (i < EN) *(float2*)(smem + (t ? S::ETV : S::ETK) + zl * F::ET_ROW + 8 * q) = et[j];
  }
  for (int i = threadIdx.x; i < 64; i += NT) ((uint32_t*)(smem + S::ZERO))[i] = 0u;
#pragma unroll
  for (int j = 0; j < QW; ++j) {
    const int i = threadIdx.x + j * NT, h = i / D, c = i - h * D;
    if (i < NREP * D) *(uint16_t*)(smem + S::QIO + h * QROW + 2 * c) = qraw[j];
  }
  __syncthreads();

  uint8_t* W = smem + S::WAVE0 + wave * S::PER_WAVE;
  const uint32_t wbase = (uint32_t)(S::WAVE0 + wave * S::PER_WAVE);  // LDS byte address of W (smem is at 0)
  // this lane group's codebook bases: 4 bits, its block (byte 0 = 32g); 2 bits, its pair of each step
  constexpr int LGSTRIDE = F::WIDE ? CB_BLOCK5 : F::QUAD ? CB_QUAD : F::PAIR ? CB_PAIR : BITS == 3 ? CB_BLOCK3 : CB_BLOCK;
  const uint32_t lbk = wbase + S::KCB + LGSTRIDE * g;
  const uint32_t lbv = wbase + S::VCB + LGSTRIDE * g;
  // 1 bit: quad (step, h, lane group g) at slot (4*(2*step + h) + g) * 256,
  // offset 16 * ((h + 2 z) % 4) within it (z = g for keys, the value group
  // for values): the lane bases of a step's quads h = 0, 1
  const uint32_t lbk1[2] = {lbk + 16u * (uint32_t)((2 * g) & 3), lbk + 16u * (uint32_t)((1 + 2 * g) & 3)};
  const uint32_t lbv1[2] = {lbv, lbv};
  const uint32_t sh1 = 4u * (uint32_t)(n & 1);
  // 5 bits: the lane group's bases of even and odd rows (group j of its block at 64 * (j ^ (g & 1)))
  const uint32_t lbk5[2] = {lbk + 64u * (uint32_t)(g & 1), lbk - 64u * (uint32_t)(g & 1)};
  const uint32_t lbv5[2] = {lbv + 64u * (uint32_t)(g & 1), lbv - 64u * (uint32_t)(g & 1)};
  const uint32_t gb = 0x20202020u * (uint32_t)g;

  // MFMA A rows: row n of this lane belongs to head hA = n / RS; for Q.K row
  // 0 of a head's rows is its query, the others zero; for P.V row 0 is the
  // weights' high part, row 1 their low part, the others zero
  const int hA = n / RS;
  const int rA = n % RS;
  u32x4 qa[4];
#pragma unroll
  for (int kq = 0; kq < 4; ++kq)
    qa[kq] = rA == 0 ? *(const u32x4*)(smem + S::QIO + hA * QROW + (32 * kq + 8 * g) * 2) : u32x4{0u, 0u, 0u, 0u};
  const uint8_t* pv_row = rA < 2 ? W + S::PST + (rA * NREP + hA) * PROW : smem + S::ZERO;
  // MFMA output element (g, i) = row 4g + i: head slot s is element i = s*RS
  // when 4g % RS == 0 (the lane group holds query heads), head 4g/RS + s
  const bool owner = ((4 * g) % RS) == 0;
  const int h0 = (4 * g) / RS;

  float m_run[HS], l_run[HS];
#pragma unroll
  for (int s = 0; s < HS; ++s) m_run[s] = -INFINITY, l_run[s] = 0.f;
  f32x4 acc[NGH][4];
#pragma unroll
  for (int vg = 0; vg < NGH; ++vg)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[vg][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // logits in base-2 units (times log2(e)): the exponentials are single v_exp_f32 ops
  const float scaling2 = a.scaling * kLog2e;

  // Codebooks.  The key groups of a tile are channels 2*lane, 2*lane + 1,
  // its value groups token lane's two.  The value codebooks of a tile are
  // built during its Q.K, the key codebooks of the next tile during its P.V:
  // each is written after the last read of the one it replaces and read
  // after the wave fence that follows.  4 bits: a quarter per step (quarter
  // c: group c/2, half c%2 xor a lane bit: 8 consecutive lanes then store to
  // 8 different 16-byte bank slots).  2 bits: all in the first step; the lane's two
  // channels are one key row pair (pair lane of the tile: step lane/16, lane
  // group lane/4 % 4, pair lane % 4); the value row pair of tokens 2m, 2m+1
  // of group vg is built by lane 2m + vg from its own and its partner's values.
  uint8_t* const kcb0 = W + S::KCB + (F::PAIR ? 0 : cb_offset(2 * lane));
  uint8_t* const kcb1 = W + S::KCB + (F::PAIR ? 0 : cb_offset(2 * lane + 1));
  uint8_t* const vcb0 = W + S::VCB + (F::PAIR ? 0 : cb_offset(lane));
  uint8_t* const vcb1 = W + S::VCB + (F::PAIR ? 0 : cb_offset(TILE + lane));
  const int kpair = ((lane >> 4) * 4 + (lane & 3)) * CB_PAIRS + ((lane >> 2) & 3) * CB_PAIR;
  // 1 bit: the key quad of this lane's channels (Q = lane / 2: step Q / 8, lane group Q / 2 % 4,
  // h = Q % 2) and the value quad this lane builds (tokens of Q' = lane / 4, value group
  // (lane >> 1) & 1), each at its half (lane & 1)
  const int kq = lane >> 1, kqg = (kq >> 1) & 3, kqh = kq & 1;
  const int kquad = ((2 * (kq >> 3) + kqh) * 4 + kqg) * CB_QUAD + 16 * ((kqh + 2 * kqg) & 3) + 64 * (lane & 1);
  const int vq = lane >> 2, vqg = (vq >> 1) & 3, vqh = vq & 1, vqv = (lane >> 1) & 1;
  const int vquad = ((2 * (2 * (vq >> 3) + vqv) + vqh) * 4 + vqg) * CB_QUAD + 16 * ((vqh + 2 * vqv) & 3) + 64 * (lane & 1);
  const int vm = lane >> 1;
  const int vpair = (((vm >> 4) * 2 + (lane & 1)) * 4 + (vm & 3)) * CB_PAIRS + ((vm >> 2) & 3) * CB_PAIR;
  auto key_groups = [&](const MetaWords<MW>& Mw, Group& g0, Group& g1) __attribute__((always_inline)) {
    const float2 mn = meta_cvt<MW>(Mw.kmn, a.meta_dtype), sc = meta_cvt<MW>(Mw.ksc, a.meta_dtype);
    g0 = group_of<QMAX, F::ET_ROW>(mn.x, sc.x);
    g1 = group_of<QMAX, F::ET_ROW>(mn.y, sc.y);
  };
  auto value_groups = [&](const MetaWords<MW>& Mw, Group& g0, Group& g1) __attribute__((always_inline)) {
    const float2 mn = meta_cvt<MW>(Mw.vmn, a.meta_dtype), sc = meta_cvt<MW>(Mw.vsc, a.meta_dtype);
    g0 = group_of<QMAX, F::ET_ROW>(mn.x, sc.x);
    g1 = group_of<QMAX, F::ET_ROW>(mn.y, sc.y);
  };
  // 4 bits: the half a lane builds in parts 0 and 2 (see above)
  const int krot = (lane >> 1) & 1, vrot = (lane >> 2) & 1;
  // part c (0..3) of the key (VALUES false) or value codebooks of groups g0, g1
  auto build_part = [&](auto values_tag, const Group& g0, const Group& g1, auto part) __attribute__((always_inline)) {
    constexpr bool values = decltype(values_tag)::value;
    constexpr int c = decltype(part)::value;
    constexpr int et = values ? S::ETV : S::ETK;
    if constexpr (F::WIDE) {
      // part c: group c / 2 of the two, its chunks 2(c % 2) and 2(c % 2) + 1 in the lane's
      // rotated order (keys: channels 2*lane + c/2; values: token lane, group c/2)
      const int rot = values ? (lane >> 1) & 3 : lane & 3;
      uint8_t* cbg = W + (values ? S::VCB + cb5_offset(TILE * (c >> 1) + lane) : S::KCB + cb5_offset(2 * lane + (c >> 1)));
      build_chunk5<IO>(smem, et, c < 2 ? g0 : g1, cbg, (2 * (c & 1) + rot) & 3);
      build_chunk5<IO>(smem, et, c < 2 ? g0 : g1, cbg, (2 * (c & 1) + 1 + rot) & 3);
    } else if constexpr (F::QUAD) {
      if constexpr (c == 0) {
        const uint32_t x0 = values2<IO>(smem, et, g0), x1 = values2<IO>(smem, et, g1);
        // this lane builds half b3 = lane & 1 of one quad
        const uint32_t hsel = (lane & 1) ? 0x07060000u : 0x05040000u;
        uint32_t R[4];
        if constexpr (values) {
          // the quad of tokens 4Q'..4Q'+3 (lanes 4Q'+r) and value group (lane >> 1) & 1: every
          // lane of the lane quad reads both groups' values of the four, then keeps its group's
          const bool vg1 = (lane & 2) != 0;
          const uint32_t a0 = dpp_sel_u<0x00>(x0), a1 = dpp_sel_u<0x55>(x0), a2 = dpp_sel_u<0xAA>(x0), a3 = dpp_sel_u<0xFF>(x0);
          const uint32_t b0 = dpp_sel_u<0x00>(x1), b1 = dpp_sel_u<0x55>(x1), b2 = dpp_sel_u<0xAA>(x1), b3 = dpp_sel_u<0xFF>(x1);
          R[0] = vg1 ? b0 : a0;
          R[1] = vg1 ? b1 : a1;
          R[2] = vg1 ? b2 : a2;
          R[3] = vg1 ? b3 : a3;
          build_quad_half(R, hsel, W + S::VCB + vquad);
        } else {
          // the quad of channels 4Q..4Q+3 (lanes 2Q, 2Q+1: two channels each)
          const uint32_t o0 = dpp_swap_pairs(x0), o1 = dpp_swap_pairs(x1);
          R[0] = odd ? o0 : x0;
          R[1] = odd ? o1 : x1;
          R[2] = odd ? x0 : o0;
          R[3] = odd ? x1 : o1;
          build_quad_half(R, hsel, W + S::KCB + kquad);
        }
      }
    } else if constexpr (BITS == 3) {
      // group c of the two (keys: channels 2*lane + c; values: token lane, group c)
      if constexpr (c < 2)
        build_group8<IO>(smem, et, c == 0 ? g0 : g1,
                         W + (values ? S::VCB + cb3_offset(TILE * c + lane) : S::KCB + cb3_offset(2 * lane + c)));
    } else if constexpr (F::PAIR) {
      if constexpr (c == 0) {
        const uint2 x0 = values4<IO>(smem, et, g0), x1 = values4<IO>(smem, et, g1);
        if constexpr (values) {
          // lane 2m builds group 0's pair of tokens 2m, 2m+1, lane 2m+1 group 1's
          const uint2 give = odd ? x0 : x1;
          const uint2 got = uint2{dpp_swap_pairs(give.x), dpp_swap_pairs(give.y)};
          build_pair(odd ? got : x0, odd ? x1 : got, W + S::VCB + vpair);
        } else {
          build_pair(x0, x1, W + S::KCB + kpair);
        }
      }
    } else {
      build_half<IO>(smem, et, c < 2 ? g0 : g1, values ? (c < 2 ? vcb0 : vcb1) : (c < 2 ? kcb0 : kcb1),
                     (c & 1) ^ (values ? vrot : krot));
    }
  };
  using KEYS = std::false_type;
  using VALUES = std::true_type;
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;
  using Q2 = std::integral_constant<int, 2>;
  using Q3 = std::integral_constant<int, 3>;
  // The B operands of key step kt (Q.K, channels 32kt ..) and of value step
  // st = 2kt + vg (P.V, tokens 32kt .., channels 64vg ..) from their code words.
  // PIPE (1 and 2 bits, where the kernel waits on LDS more than it computes):
  // a step's lookups are issued one step ahead, before the previous step's
  // MFMAs; at 3-5 bits, which are bound by their VALU work, that measured
  // slower and the lookups stay in step order.
  constexpr bool PIPE = BITS <= 2;
  auto k_lookup = [&](auto kt_tag, u32x4(&B)[4]) __attribute__((always_inline)) {
    constexpr int kt = decltype(kt_tag)::value;
    if constexpr (F::WIDE) lookup5<kt * 4 * CB_BLOCK5>(smem, KW + 8 * kt, lbk5, sh5, B);
    else if constexpr (F::QUAD)
      lookup1<(2 * kt) * 4 * CB_QUAD, (2 * kt + 1) * 4 * CB_QUAD>(smem, KW + 4 * kt, lbk1, odd, sh1, B);
    else if constexpr (F::PAIR) lookup2<kt * 4 * CB_PAIRS>(smem, KW + 4 * kt, lbk, odd, B);
    else if constexpr (BITS == 3) lookup3<kt * 4 * CB_BLOCK3>(smem, KW + 4 * kt, lbk, odd, sh3, B);
    else lookup4<kt * 4 * CB_BLOCK>(smem, KW + 4 * kt, lbk, gb, odd, B);
  };
  auto v_lookup = [&](auto st_tag, u32x4(&B)[4]) __attribute__((always_inline)) {
    constexpr int st = decltype(st_tag)::value, kt = st >> 1, vg = st & 1;
    if constexpr (F::WIDE) lookup5<vg * 8 * CB_BLOCK5 + kt * 4 * CB_BLOCK5>(smem, VW + 8 * st, lbv5, sh5, B);
    else if constexpr (F::QUAD)
      lookup1<(2 * st) * 4 * CB_QUAD + 16 * ((2 * vg) & 3), (2 * st + 1) * 4 * CB_QUAD + 16 * ((1 + 2 * vg) & 3)>(
          smem, VW + 4 * st, lbv1, odd, sh1, B);
    else if constexpr (F::PAIR) lookup2<st * 4 * CB_PAIRS>(smem, VW + 4 * st, lbv, odd, B);
    else if constexpr (BITS == 3) lookup3<vg * 8 * CB_BLOCK3 + kt * 4 * CB_BLOCK3>(smem, VW + 4 * st, lbv, odd, sh3, B);
    else lookup4<vg * 8 * CB_BLOCK + kt * 4 * CB_BLOCK>(smem, VW + 4 * st, lbv, gb, odd, B);
  };
  // the first tile's key codebooks
  {
    Group g0, g1;
    key_groups(MT, g0, g1);
    build_part(KEYS{}, g0, g1, Q0{});
    build_part(KEYS{}, g0, g1, Q1{});
    build_part(KEYS{}, g0, g1, Q2{});
    build_part(KEYS{}, g0, g1, Q3{});
  }
  wave_lds_sync();

  // one tile.  Loads in flight: this tile's value words and the next tile's
  // metadata (issued here), the next tile's key words (after this tile's Q.K)
  auto process = [&](auto quant_tag, const int tile, const int tn) {
    constexpr bool quant = decltype(quant_tag)::value;
    const int tl = min(tn, q_last);
    load_vw(min(tile, q_last));
    MetaWords<MW> MN;
    load_meta_tile<MW, D>(MN, bf, tl, lane);
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
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (quant) {
      // ---------- S = Q K^T over the keys' values; this tile's value
      // codebooks are built alongside
      Group gv0, gv1;
      value_groups(MT, gv0, gv1);
      // PIPE: the next step's lookups are issued before this step's MFMAs
      u32x4 Bc[4], Bn[4];
      if constexpr (PIPE) k_lookup(Q0{}, Bc);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        switch (kt) {
          case 0: PIPE ? k_lookup(Q1{}, Bn) : k_lookup(Q0{}, Bc); build_part(VALUES{}, gv0, gv1, Q0{}); break;
          case 1: PIPE ? k_lookup(Q2{}, Bn) : k_lookup(Q1{}, Bc); build_part(VALUES{}, gv0, gv1, Q1{}); break;
          case 2: PIPE ? k_lookup(Q3{}, Bn) : k_lookup(Q2{}, Bc); build_part(VALUES{}, gv0, gv1, Q2{}); break;
          default:
            if constexpr (!PIPE) k_lookup(Q3{}, Bc);
            build_part(VALUES{}, gv0, gv1, Q3{});
            break;
        }
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) s[jt] = M::run(qa[kt], Bc[jt], s[jt]);
        if constexpr (PIPE) {
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) Bc[jt] = Bn[jt];
        }
      }
    } else {
      // ---------- residual tile: dense keys; rows past the filled ones read 0
      // (their logits are masked below)
      const int kst = a.kr_st * 2;
      const __amdgpu_buffer_rsrc_t krb = make_buf(bf.kr + (int64_t)r0 * a.kr_st, (n_valid - 1) * kst + D * 2);
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        u32x4 kb[2][4];
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
          for (int jt = 0; jt < 4; ++jt)
            kb[k2][jt] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(krb, (4 * n + jt) * kst + 16 * g, 64 * (2 * kh + k2), 0));
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) s[jt] = M::run(qa[2 * kh + k2], kb[k2][jt], s[jt]);
      }
    }
    load_kw(tl);

    // ---------- online softmax in registers: head slot sl of this lane group
    // owns tokens 4n + jt (jt = 0..3) of the 16 lanes of its row
    float corr[HS];
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const int i = sl * RS;  // MFMA output element of this head slot
      float x[4];
      float tmax = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int tt = 4 * n + jt;
        float v = s[jt][i] * scaling2;
        if (tt >= n_valid) v = -INFINITY;
        else if (a.mask) v = add_mask_log2(v, a.mask[b * a.mask_sb + pos0 + tt]);
        x[jt] = v;
        tmax = fmaxf(tmax, v);
      }
      tmax = group_reduce<16>(tmax, OpMax());
      const float m_new = fmaxf(m_run[sl], tmax);
      // while a row is fully masked its maximum stays -inf; 0 stands in for
      // it, so exp2(-inf - 0) gives zero weights and a zero correction
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      corr[sl] = __builtin_amdgcn_exp2f(m_run[sl] - m_use);
      m_run[sl] = m_new;
      float p[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) p[jt] = __builtin_amdgcn_exp2f(x[jt] - m_use);
      // l_run is a per-lane partial sum (this lane's 4 tokens of every tile;
      // the correction is the same in the 16 lanes of the row): summed over
      // the row once, at the end
      l_run[sl] = l_run[sl] * corr[sl] + ((p[0] + p[1]) + (p[2] + p[3]));
      if (owner) {
        // the weights as high + low parts in the io dtype
        const uint32_t h01 = pack_io2<IO>(p[0], p[1]), h23 = pack_io2<IO>(p[2], p[3]);
        const uint32_t l01 = pack_io2<IO>(p[0] - io_to_f32<IO>((uint16_t)h01), p[1] - io_to_f32<IO>((uint16_t)(h01 >> 16)));
        const uint32_t l23 = pack_io2<IO>(p[2] - io_to_f32<IO>((uint16_t)h23), p[3] - io_to_f32<IO>((uint16_t)(h23 >> 16)));
        const int h = h0 + sl;
        *(uint2*)(W + S::PST + h * PROW + 8 * n) = uint2{h01, h23};
        *(uint2*)(W + S::PST + (NREP + h) * PROW + 8 * n) = uint2{l01, l23};
      }
    }
    // ---------- rescale the accumulators (rows i, i + 1 of each head slot)
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const int i = sl * RS;
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[vg][j][i] *= corr[sl], acc[vg][j][i + 1] *= corr[sl];
    }
    wave_lds_sync();  // the weights and value codebooks were written by other lanes

    // ---------- acc += P V; the next tile's key codebooks are built alongside
    Group gk0, gk1;
    key_groups(MN, gk0, gk1);
    if constexpr (quant) {
      u32x4 Bc[4], Bn[4];
      if constexpr (PIPE) v_lookup(Q0{}, Bc);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int kt = st >> 1, vg = st & 1;
        const u32x4 A = *(const u32x4*)(pv_row + (32 * kt + 8 * g) * 2);
        switch (st) {
          case 0: PIPE ? v_lookup(Q1{}, Bn) : v_lookup(Q0{}, Bc); build_part(KEYS{}, gk0, gk1, Q0{}); break;
          case 1: PIPE ? v_lookup(Q2{}, Bn) : v_lookup(Q1{}, Bc); build_part(KEYS{}, gk0, gk1, Q1{}); break;
          case 2: PIPE ? v_lookup(Q3{}, Bn) : v_lookup(Q2{}, Bc); build_part(KEYS{}, gk0, gk1, Q2{}); break;
          default:
            if constexpr (!PIPE) v_lookup(Q3{}, Bc);
            build_part(KEYS{}, gk0, gk1, Q3{});
            break;
        }
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) acc[vg][jt] = M::run(A, Bc[jt], acc[vg][jt]);
        if constexpr (PIPE) {
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) Bc[jt] = Bn[jt];
        }
      }
    } else {
      // residual values: lane (n, g) of step (kt, vg) needs tokens
      // 32kt + 8g + j (j = 0..7) of channels 64vg + 4n + jt: one 8-byte load
      // per token (its 4 channels), then the halves paired per token pair.
      // The buffer starts at the step's first row and ends after its last
      // filled row (padding rows read 0; their weights are 0)
      const int vst = a.vr_st * 2;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const u32x4 A = *(const u32x4*)(pv_row + (32 * kt + 8 * g) * 2);
        const int rows = n_valid - 32 * kt;
        const __amdgpu_buffer_rsrc_t vrb =
            make_buf(bf.vr + (int64_t)(r0 + 32 * kt) * a.vr_st, rows > 0 ? (rows - 1) * vst + D * 2 : 0);
#pragma unroll
        for (int vg = 0; vg < NGH; ++vg) {
          uint32_t vv[8][2];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const auto raw = __builtin_amdgcn_raw_buffer_load_b64(vrb, (8 * g + j) * vst + 8 * n, 128 * vg, 0);
            vv[j][0] = raw[0];
            vv[j][1] = raw[1];
          }
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) {
            u32x4 B;
            const uint32_t sel = (jt & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
            for (int i = 0; i < 4; ++i) B[i] = __builtin_amdgcn_perm(vv[2 * i + 1][jt >> 1], vv[2 * i][jt >> 1], sel);
            acc[vg][jt] = M::run(A, B, acc[vg][jt]);
          }
        }
      }
      build_part(KEYS{}, gk0, gk1, Q0{});
      build_part(KEYS{}, gk0, gk1, Q1{});
      build_part(KEYS{}, gk0, gk1, Q2{});
      build_part(KEYS{}, gk0, gk1, Q3{});
    }
    MT = MN;
    wave_lds_sync();  // the next tile's key codebooks were written by other lanes; this tile's weights
                      // and value codebooks are read before the next tile overwrites them
  };

  // tiles of this wave; the wave priority falls with its progress (as in the
  // fold kernel: the SIMD then favours the wave that is behind)
  const int n_mine = (n_virt - v0 + WAVES - 1) / WAVES;
  const int wg_lin = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
  const int older = wg_lin < cus ? 1 : 0;
  int done = 0;
  if (older) __builtin_amdgcn_s_setprio(2);
  else __builtin_amdgcn_s_setprio(3);
  auto step = [&](auto quant_tag, const int v) {
    process(quant_tag, tile_of(v), v + WAVES < n_virt ? tile_of(v + WAVES) : q_last);
    ++done;
    switch ((4 * done) / max(n_mine, 1) + older) {
      case 0: break;
      case 1: __builtin_amdgcn_s_setprio(2); break;
      case 2: __builtin_amdgcn_s_setprio(1); break;
      default: __builtin_amdgcn_s_setprio(0); break;
    }
  };
  int v = v0;
  for (; v < n_res; v += WAVES) step(std::false_type{}, v);
  for (; v < n_virt; v += WAVES) step(std::true_type{}, v);
  __builtin_amdgcn_s_setprio(0);

  // ---------------- merge the waves and write this split's partial records
  __syncthreads();
  float* red = (float*)(smem + S::WAVE0);
  constexpr int RED = 2 * NREP + NREP * D;  // per wave: m[NREP], l[NREP], acc[NREP][D]
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int tid_e = wave * 64 + lane_e;
  const int n_e = lane_e & 15, g_e = lane_e >> 4;
  if (((4 * g_e) % RS) == 0) {
    const int h0e = (4 * g_e) / RS;
    float* w = red + wave * RED;
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const int i = sl * RS, h = h0e + sl;
      const float l_row = group_reduce<16>(l_run[sl], OpAdd());
      if (n_e == 0) {
        w[h] = m_run[sl];
        w[NREP + h] = l_row;
      }
#pragma unroll
      for (int vg = 0; vg < NGH; ++vg)
        *(f32x4*)(w + 2 * NREP + h * D + 64 * vg + 4 * n_e) =
            f32x4{acc[vg][0][i] + acc[vg][0][i + 1], acc[vg][1][i] + acc[vg][1][i + 1],
                  acc[vg][2][i] + acc[vg][2][i + 1], acc[vg][3][i] + acc[vg][3][i + 1]};
    }
  }
  __syncthreads();
  if (direct) {
    for (int e = tid_e; e < a.n_rep * D; e += NT) {
      const int h = e / D;
      const int c = e - h * D;
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
  for (int e = tid_e; e < a.n_rep * (D + 2); e += NT) {
    const int h = e / (D + 2);
    const int c = e - h * (D + 2);
    float M_ = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M_ = fmaxf(M_, red[w * RED + h]);
    float val = 0.f;
    if (c == D) {
      val = M_ * kLn2;  // the record's maximum in natural-log units
    } else if (M_ != -INFINITY) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float f = __builtin_amdgcn_exp2f(red[w * RED + h] - M_);
        val += f * (c == D + 1 ? red[w * RED + NREP + h] : red[w * RED + 2 * NREP + h * D + c]);
      }
    }
    ws_record<D>(a, b, kvh * a.n_rep + h, split, n_split)[c] = val;
  }
}

}  // namespace cb

// ------------------------------------------------------------------ host side

static bool cb_meta_aligned(const void* p, int64_t sb, int64_t sh, int dt) {
  const int pair = dt == MZ_F32 ? 8 : 4;  // two adjacent entries are read at once
  return ((uintptr_t)p % pair) == 0 && sb % 2 == 0 && sh % 2 == 0;
}

bool cb_supported(const mz_decode_args* a) {
  const int64_t es = a->meta_dtype == MZ_F32 ? 4 : 2;
  const int64_t qb = 8 * (int64_t)a->bits;
  // 5 bits: one (E+, E-) table for keys and values, up to 4 query heads (LDS)
  const bool bits_ok = (a->bits >= 1 && a->bits <= 4) || (a->bits == 5 && a->e_key == a->e_value && a->n_rep <= 4);
  // buffer-resource ranges are 32-bit
  const bool fits = (int64_t)a->n_groups * cb::TILE * 2 * qb < ((int64_t)1 << 31) &&
                    (int64_t)a->n_groups * a->head_dim * es < ((int64_t)1 << 31);
  const bool aligned = a->v_prefix == 0 || a->v_prefix == a->n_groups * cb::TILE;
  return bits_ok && a->head_dim == cb::D && a->n_groups > 0 && fits && aligned && a->n_rep >= 1 &&
         a->n_rep <= 8 && a->e_key && a->e_value && ((uintptr_t)a->k_packed % 4) == 0 &&
         ((uintptr_t)a->v_packed % 4) == 0 && a->kp_sb % 4 == 0 && a->kp_sh % 4 == 0 && a->vp_sb % 4 == 0 &&
         a->vp_sh % 4 == 0 && cb_meta_aligned(a->k_mn, a->km_sb, a->km_sh, a->meta_dtype) &&
         cb_meta_aligned(a->k_scale, a->km_sb, a->km_sh, a->meta_dtype) &&
         cb_meta_aligned(a->v_mn, a->vm_sb, a->vm_sh, a->meta_dtype) &&
         cb_meta_aligned(a->v_scale, a->vm_sb, a->vm_sh, a->meta_dtype);
}

int cb_choose_split(const mz_decode_args* a, int* tiles_per_split) {
  const int n_tiles = a->n_groups + (a->n_residual + cb::TILE - 1) / cb::TILE;
  int ns = a->n_split;
  if (ns <= 0) {
    // fill the resident workgroup slots (two per CU) once
    const int64_t units = std::max<int64_t>(1, (int64_t)a->batch * a->kv_heads);
    const int64_t slots = 2 * (int64_t)device_cu_count();
    ns = (int)((slots + units - 1) / units);
    ns = max(1, min(ns, (n_tiles + 7) / 8));  // at least 2 tiles per wave
  }
  ns = min(ns, n_tiles);
  const int tps = (n_tiles + ns - 1) / ns;
  *tiles_per_split = tps;
  return (n_tiles + tps - 1) / tps;
}

// One width's kernel (meta dtype picked at run time).
template <int IO, int NR, int BB>
static void cb_launch_one(const mz_decode_args* a, hipStream_t s, dim3 grid, int tps, int ns, int dir, int cus) {
  if (a->meta_dtype == MZ_F32)
    hipLaunchKernelGGL((cb::cb_kernel<IO, NR, 2, BB>), grid, dim3(64 * cb::WAVES), 0, s, *a, tps, ns, dir, cus);
  else
    hipLaunchKernelGGL((cb::cb_kernel<IO, NR, 1, BB>), grid, dim3(64 * cb::WAVES), 0, s, *a, tps, ns, dir, cus);
}

template <int IO, int NR>
static int cb_launch_nr(const mz_decode_args* a, hipStream_t s, dim3 grid, int tps, int ns, int dir, int cus) {
  switch (a->bits) {
    case 1: cb_launch_one<IO, NR, 1>(a, s, grid, tps, ns, dir, cus); break;
    case 2: cb_launch_one<IO, NR, 2>(a, s, grid, tps, ns, dir, cus); break;
    case 3: cb_launch_one<IO, NR, 3>(a, s, grid, tps, ns, dir, cus); break;
    case 4: cb_launch_one<IO, NR, 4>(a, s, grid, tps, ns, dir, cus); break;
    case 5:
      // the 5-bit workgroup's LDS holds up to 4 query heads' staging
      if constexpr (NR <= 4) {
        cb_launch_one<IO, NR, 5>(a, s, grid, tps, ns, dir, cus);
        break;
      } else {
        return MZ_EUNSUPPORTED;
      }
    default: return MZ_EUNSUPPORTED;
  }
  return MZ_OK;
}

template <int IO>
static int cb_launch_io(const mz_decode_args* a, hipStream_t s, dim3 grid, int tps, int ns, int dir, int cus) {
  // query heads per kv-head of the kernel that runs: n_rep rounded up to a power of two
  switch (a->n_rep <= 1 ? 1 : a->n_rep <= 2 ? 2 : a->n_rep <= 4 ? 4 : a->n_rep <= 8 ? 8 : 0) {
    case 1: return cb_launch_nr<IO, 1>(a, s, grid, tps, ns, dir, cus);
    case 2: return cb_launch_nr<IO, 2>(a, s, grid, tps, ns, dir, cus);
    case 4: return cb_launch_nr<IO, 4>(a, s, grid, tps, ns, dir, cus);
    case 8: return cb_launch_nr<IO, 8>(a, s, grid, tps, ns, dir, cus);
    default: return MZ_EUNSUPPORTED;
  }
}

int cb_launch_partials(const mz_decode_args* a, hipStream_t s, bool direct) {
  int tps;
  const int ns = cb_choose_split(a, &tps);
  const dim3 grid(ns, a->kv_heads, a->batch);
  const int st = a->io_dtype == MZ_BF16 ? cb_launch_io<MZ_BF16>(a, s, grid, tps, ns, direct ? 1 : 0, device_cu_count())
                                        : cb_launch_io<MZ_F16>(a, s, grid, tps, ns, direct ? 1 : 0, device_cu_count());
  if (st != MZ_OK) return st;
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

}  // namespace mz
