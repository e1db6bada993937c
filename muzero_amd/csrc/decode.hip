// Packed-KV decode attention, general path (gfx950, wave64, MFMA 16x16x32):
// every bit width 1-8, head_dim 64 or 128, up to 16 query heads per kv-head.
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
// Per tile, through one per-wave LDS staging buffer:
//   K in chunks of 32 tokens (head_dim 64: one chunk of 64) -> [token][D] in
//   the io dtype, dequantized like the reference's _dequantize_rows_torch and
//   rounded to the layer dtype; QK^T with MFMA (A = Q rows, B = the chunk);
//   online softmax on the MFMA accumulator layout, P -> LDS in fp16;
//   V in chunks of 64 channels (one value group) -> [channel][64 tokens] in
//   fp16 (an MFMA B operand is 8 consecutive tokens of one channel), then
//   acc += P V.
// Dequantization runs in registers, two codes per lane per LDS store: a lane
// owns two adjacent channels of a K chunk (two key groups) or two adjacent
// tokens of a V chunk (two value groups), so a group's parameters are formed
// once per tile and each code costs one table read and a few branch-free ops.
// Every width reproduces the reference's dequantized value bit for bit before
// the rounding to the layer dtype (its op order, its fp32 expm1 rows): codes
// of up to 6 bits read the rows from LDS, the 7- and 8-bit rows (32 KB and
// 128 KB per alpha, too large to sit next to the staging buffers) are read
// from the host-built table in global memory (L2-resident).
// A tile's packed words are loaded one tile ahead: the next tile's key words
// are issued as soon as this tile's keys are staged, its value words as soon
// as this tile's values are.
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
  static constexpr int KT = D == 128 ? 32 : 64;  // tokens per K chunk
  static constexpr int KCH = kTile / KT;         // K chunks per tile
  static constexpr int NG = D / 64;              // V chunks (value groups) per tile
  static constexpr int K_LD = D + kPad;          // K chunk row: one token
  static constexpr int V_LD = kTile + kPad;      // V chunk row: one channel
  // V chunk rows 32..63 start 64 halves (32 banks) further on: the two lane
  // halves of a staging store (rows i and 32 + i) then use disjoint banks
  static constexpr int V_HI = 64;
  static constexpr int STAGE = (KT * K_LD > 64 * V_LD + V_HI) ? KT * K_LD : 64 * V_LD + V_HI;
  static constexpr int P_LD = kTile + kPad;
  static constexpr int P_HALVES = 16 * P_LD;
  static constexpr int WAVE_HALVES = STAGE + P_HALVES;
  static constexpr int RED_FLOATS = 32 + 16 * D;  // per wave at the end (aliases the wave areas)
  static constexpr int WAVES_BYTES =
      kWaves * WAVE_HALVES * 2 > kWaves * RED_FLOATS * 4 ? kWaves * WAVE_HALVES * 2 : kWaves * RED_FLOATS * 4;
  // per-wave codebooks (codes of up to 4 bits): the lane's two groups' 2^bits
  // staged values, [group r][code q][64 lane slots] halves, the slots of
  // lanes L and L + 32 side by side in one dword (a half-wave's 32 lanes then
  // read 32 different banks)
  static constexpr int cb_halves(int bits) { return bits <= 4 ? 2 * (1 << bits) * 64 : 0; }
  static constexpr int CB_BYTES4 = kWaves * 2 * 16 * 64 * 2;  // the largest (4 bits), for offsets
  // expm1 rows for bins 1..qmax (codes of up to 6 bits), forward and
  // reversed, one pair of tables per alpha
  static constexpr int e_floats(int bits) { return bits <= 6 ? ((1 << bits) - 1) * ((1 << bits) + 2) / 2 : 0; }
  static constexpr size_t cb_bytes(int bits) { return (size_t)kWaves * cb_halves(bits) * 2; }
  static constexpr size_t bytes(int bits) { return (size_t)WAVES_BYTES + cb_bytes(bits) + 4 * (size_t)e_floats(bits) * 4; }
};

// One group's dequantization parameters (muzero/quantizer.py:241-255, from the
// stored metadata, scale guarded as in loader.py:201).
struct DeqG {
  float za, s, mn, pe, mne;  // mne = -ne
  int zl;                    // zero level, an integer in 0..qmax
  // <= 6 bits: LDS byte address of code q's expm1 entry is (q >= zl ? bp : bn) + 4q;
  // 7/8 bits: its index in the global table is q >= zl ? bp + q : bn - q
  int bp, bn;
  const float* eg;           // 7/8 bits: the global expm1 table
};

// `ebase`: LDS byte address of the forward expm1 rows E[bins][d]; the reversed
// rows R[bins][k] = E[bins][bins - k] follow them (same row offsets), so a
// code below the zero level reads R[nb][q] = E[nb][zl - q] (nb = zl then)
// and both sides index with +q.
template <int BITS>
__device__ __forceinline__ DeqG deq_group(float mn, float s, int ebase, const float* eg) {
  constexpr float qmax = (float)((1 << BITS) - 1);
  constexpr int EF = ((1 << BITS) - 1) * ((1 << BITS) + 2) / 2;
  const DeqRow r = deq_row(mn, s, qmax, true);
  DeqG g;
  g.za = r.za;
  g.s = r.s;
  g.mn = r.mn;
  g.pe = r.pe;
  g.mne = -r.ne;
  g.zl = r.zl == r.zl ? (int)r.zl : 0;  // a NaN zero level reads row 1 (pb = nb = 1), never past the table
  if constexpr (BITS <= 6) {
    g.bp = ebase + 4 * (r.offp - g.zl);
    g.bn = ebase + 4 * (EF + r.offn);
  } else {
    // E[pb][q - zl] and E[nb][zl - q] (row offsets expm1_row(bins)); q and zl
    // lie in 0..qmax, so the index stays inside the table for any metadata
    g.bp = r.offp - g.zl;
    g.bn = r.offn + g.zl;
    g.eg = eg;
  }
  return g;
}

// An LDS load from a byte address (the dynamic LDS array starts at address 0:
// these kernels have no static LDS).
__device__ __forceinline__ float lds_load_f32(int addr) {
  return *(const __attribute__((address_space(3))) float*)(size_t)(uint32_t)addr;
}

// Dequantized fp32 value of code q, the reference's value exactly: norm =
// za + pe*E[pb][q-zl] or za - ne*E[nb][zl-q] (the sign folded into mne is
// exact), clamped, times s, plus mn, with no contraction.  Split in two so a
// block of codes can issue all its table reads before using any: deq_fetch
// returns the table entry, deq_apply finishes the value.
template <int BITS>
__device__ __forceinline__ float deq_fetch(const DeqG& g, int q) {
  const bool pos = q >= g.zl;
  if constexpr (BITS <= 6) return lds_load_f32((pos ? g.bp : g.bn) + 4 * q);
  else return g.eg[pos ? g.bp + q : g.bn - q];
}
template <int BITS>
__device__ __forceinline__ float deq_apply(const DeqG& g, int q, float z) {
  const bool pos = q >= g.zl;
  const float t = (pos ? g.pe : g.mne) * z;
  const float norm = __builtin_amdgcn_fmed3f(g.za + t, 0.f, 1.f);
  return norm * g.s + g.mn;
}
template <int BITS>
__device__ __forceinline__ float deq_code(const DeqG& g, int q) {
  return deq_apply<BITS>(g, q, deq_fetch<BITS>(g, q));
}

// Code `idx` of an LSB-first bitstream held in registers (idx is a constant
// after unrolling, so this is one bit-field extract, or two ops when the code
// straddles two words).
template <int BITS>
__device__ __forceinline__ int code_at(const uint32_t* w, const int idx) {
  const int bit = idx * BITS, i = bit >> 5, o = bit & 31;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if (o + BITS <= 32) return (int)((w[i] >> o) & mask);
  return (int)(__builtin_amdgcn_alignbit(w[i + 1], w[i], o) & mask);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two values rounded to the io dtype, packed (first value in the low half).
template <int IO>
__device__ __forceinline__ uint32_t pack_io(float x0, float x1) {
  if constexpr (IO == MZ_BF16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{x0, x1}), bf16x2_t));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{x0, x1}), f16x2_t));
}
// Two values rounded to the io dtype, then converted to fp16 (exact for
// normal-range bf16 values), packed.
template <int IO>
__device__ __forceinline__ uint32_t pack_io_f16(float x0, float x1) {
  if constexpr (IO == MZ_BF16) {
    const uint32_t b = pack_io<MZ_BF16>(x0, x1);
    const f32x2_t f{__uint_as_float(b << 16), __uint_as_float(b & 0xFFFF0000u)};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2_t));
  } else {
    return pack_io<MZ_F16>(x0, x1);
  }
}
// A pair of io-dtype halves converted to fp16.
template <int IO>
__device__ __forceinline__ uint32_t io_pair_to_f16(uint16_t h0, uint16_t h1) {
  if constexpr (IO == MZ_F16) return (uint32_t)h0 | ((uint32_t)h1 << 16);
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{bf2f(h0), bf2f(h1)}), f16x2_t));
}

template <int D, int BITS, int IO>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_split_kernel(
    const mz_decode_args a, int tiles_per_split, int n_split, int direct) {
  using L = Lds<D>;
  using M = Mfma<IO>;
  constexpr int QB = 8 * BITS;      // bytes per packed 64-code row
  constexpr int NG = L::NG;
  constexpr int KT = L::KT;
  constexpr int KCH = L::KCH;
  constexpr int CPW = D / 2;        // K: channel pairs (one per lane, D = 64: two token halves)
  constexpr int KTPL = D == 128 ? 64 : 32;  // K tokens per lane and tile
  constexpr int KWR = KTPL * BITS / 32;  // K words per row and lane
  constexpr int EF = L::e_floats(BITS);
  constexpr bool kTab = BITS <= 6;

  extern __shared__ __align__(16) uint16_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int n_rep = a.n_rep;

  uint16_t* kv = lds + wave * L::WAVE_HALVES;
  uint16_t* pb = kv + L::STAGE;
  // codes of up to 4 bits are staged through per-group codebooks: the 2^bits
  // exact values of each of the lane's two groups, built once per tile (keys)
  // or value chunk, then one LDS read per code instead of its dequantization
  constexpr bool kCB = BITS <= 4;
  constexpr int NQ = 1 << BITS;
  constexpr int CB_BASE = L::WAVES_BYTES;
  constexpr int EK_BASE = L::WAVES_BYTES + (int)L::cb_bytes(BITS);  // key table
  constexpr int EV_BASE = EK_BASE + 8 * EF;                          // value table
  // this lane's codebook slots (group 0, code 0) and (group 1, code 0); code q is 64 halves further
  uint16_t* cb0 = (uint16_t*)((uint8_t*)lds + CB_BASE) + wave * L::cb_halves(BITS) + 2 * (lane & 31) + (lane >> 5);
  uint16_t* cb1 = cb0 + NQ * 64;
  if constexpr (kTab) {
    // the expm1 tables exist only when there is a quantized prefix
    if (a.n_groups > 0 || a.v_prefix > 0) {
      float* eK = (float*)((uint8_t*)lds + EK_BASE);
      float* eV = (float*)((uint8_t*)lds + EV_BASE);
      for (int i = threadIdx.x; i < EF; i += 256) {
        // row of entry i: the largest bins with (bins - 1)(bins + 2)/2 <= i
        int bins = (int)((__builtin_sqrtf((float)(8 * i + 9)) - 1.f) * 0.5f);
        if ((bins - 1) * (bins + 2) / 2 > i) --bins;
        if (bins * (bins + 3) / 2 <= i) ++bins;
        const int off = (bins - 1) * (bins + 2) / 2, k = i - off;
        eK[i] = a.e_key[i];
        eV[i] = a.e_value[i];
        eK[EF + i] = a.e_key[off + bins - k];
        eV[EF + i] = a.e_value[off + bins - k];
      }
    }
    __syncthreads();
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

  // Lane roles.  K: channels 2cp, 2cp+1, token range ts (D = 64: two halves).
  // V: tokens 2tp, 2tp+1 of the tile, channels 32cs..32cs+31 of each value group.
  const int cp = lane % CPW;
  const int ts = lane / CPW;
  const int tp = lane & 31;
  const int cs = lane >> 5;
  const uint8_t* kbase = a.k_packed + b * a.kp_sb + kvh * a.kp_sh;
  const uint8_t* vbase = a.v_packed + b * a.vp_sb + kvh * a.vp_sh;
  const int64_t kmb = b * a.km_sb + kvh * a.km_sh;
  const int64_t vmb = b * a.vm_sb + kvh * a.vm_sh;
  // quantized value tokens past the key prefix (logq_compatible_layout), 0 when aligned
  const int dv = a.v_prefix > 0 ? a.v_prefix - a.n_groups * kTile : 0;

  // packed words and metadata of the tile being staged next (loaded one tile ahead)
  uint32_t kw[2][KWR];
  uint32_t vw[NG][2][BITS];
  float kmeta[2][2], vmeta[NG][2][2];
  auto load_k = [&](int tile) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t* row = (const uint32_t*)(kbase + ((int64_t)tile * D + 2 * cp + r) * QB) + ts * KWR;
#pragma unroll
      for (int i = 0; i < KWR; ++i) kw[r][i] = row[i];
      const int64_t mi = kmb + (int64_t)tile * D + 2 * cp + r;
      kmeta[r][0] = meta_load(a.k_mn, mi, a.meta_dtype);
      kmeta[r][1] = meta_load(a.k_scale, mi, a.meta_dtype);
    }
  };
  auto load_v = [&](int tile) __attribute__((always_inline)) {
#pragma unroll
    for (int vg = 0; vg < NG; ++vg)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int64_t tok = (int64_t)tile * kTile + 2 * tp + r;
        const uint32_t* row = (const uint32_t*)(vbase + (tok * NG + vg) * QB) + cs * BITS;
#pragma unroll
        for (int i = 0; i < BITS; ++i) vw[vg][r][i] = row[i];
        const int64_t mi = vmb + tok * NG + vg;
        vmeta[vg][r][0] = meta_load(a.v_mn, mi, a.meta_dtype);
        vmeta[vg][r][1] = meta_load(a.v_scale, mi, a.meta_dtype);
      }
  };
  // The 2^bits staged values of the lane's two groups: each the reference's
  // exact dequantized value (deq_code), rounded as `pack` stages it, into the
  // lane's own codebook slots (only this lane reads them back, so program
  // order is the only ordering needed).
  auto build_codebooks = [&](const DeqG (&gg)[2], auto pack) __attribute__((always_inline)) {
    if constexpr (kCB) {
      float z0[NQ], z1[NQ];
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        z0[q] = deq_fetch<BITS>(gg[0], q);
        z1[q] = deq_fetch<BITS>(gg[1], q);
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const uint32_t h = pack(deq_apply<BITS>(gg[0], q, z0[q]), deq_apply<BITS>(gg[1], q, z1[q]));
        cb0[q * 64] = (uint16_t)h;
        cb1[q * 64] = (uint16_t)(h >> 16);
      }
    }
  };
  {
    const int t0 = t_begin + wave;
    if (t0 < t_end && t0 < a.n_groups) {
      load_k(t0);
      load_v(t0);
    }
  }

  for (int tile = t_begin + wave; tile < t_end; tile += kWaves) {
    const bool quant = tile < a.n_groups;
    const int r0 = quant ? 0 : (tile - a.n_groups) * kTile;
    const int n_valid = quant ? kTile : min(kTile, a.n_residual - r0);
    const int pos0 = quant ? tile * kTile : a.n_groups * kTile + r0;
    const int next = tile + kWaves;
    const bool next_quant = next < t_end && next < a.n_groups;

    // ---------------- S = Q K^T, one K chunk at a time: lane (n, g) gets heads 4g+i of token 16j+n
    f32x4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    DeqG gk[2];
    if (quant) {
#pragma unroll
      for (int r = 0; r < 2; ++r) gk[r] = deq_group<BITS>(kmeta[r][0], kmeta[r][1], EK_BASE, a.e_key);
      if constexpr (kCB) build_codebooks(gk, [](float x0, float x1) { return pack_io<IO>(x0, x1); });
    }
#pragma unroll
    for (int kc = 0; kc < KCH; ++kc) {
      if (quant && kCB) {
        // the staged pair of each token: one codebook read per code
#pragma unroll
        for (int u = 0; u < 32; ++u) {
          const int wi = (KCH == 2 ? 32 * kc : 0) + u;  // code index in the lane's words
          const int row = (KCH == 2 ? 0 : 32 * ts) + u;  // token row of the chunk
          const uint32_t h0 = cb0[code_at<BITS>(kw[0], wi) * 64];
          const uint32_t h1 = cb1[code_at<BITS>(kw[1], wi) * 64];
          *(uint32_t*)(kv + row * L::K_LD + 2 * cp) = h0 | (h1 << 16);
        }
      } else if (quant) {
        // blocks of 8 tokens: all 16 table reads issued, then used
#pragma unroll
        for (int i0 = 0; i0 < 32; i0 += 8) {
          int q0[8], q1[8];
          float z0[8], z1[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int wi = (KCH == 2 ? 32 * kc : 0) + i0 + u;  // code index in the lane's words
            q0[u] = code_at<BITS>(kw[0], wi);
            q1[u] = code_at<BITS>(kw[1], wi);
            z0[u] = deq_fetch<BITS>(gk[0], q0[u]);
            z1[u] = deq_fetch<BITS>(gk[1], q1[u]);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int row = (KCH == 2 ? 0 : 32 * ts) + i0 + u;  // token row of the chunk
            *(uint32_t*)(kv + row * L::K_LD + 2 * cp) =
                pack_io<IO>(deq_apply<BITS>(gk[0], q0[u], z0[u]), deq_apply<BITS>(gk[1], q1[u], z1[u]));
          }
        }
      } else {
        // residual rows: LPT lanes per token, each copying D / LPT halves (rows past the window are 0)
        constexpr int LPT = 64 / KT;
        const int t = lane / LPT, part = lane % LPT;
        const int tok = KT * kc + t;
        u32x4* dst = (u32x4*)(kv + t * L::K_LD + part * (D / LPT));
        if (tok < n_valid) {
          const uint16_t* src = (const uint16_t*)a.k_res + b * a.kr_sb + kvh * a.kr_sh + (int64_t)(r0 + tok) * a.kr_st +
                                part * (D / LPT);
#pragma unroll
          for (int c = 0; c < D / LPT / 8; ++c) dst[c] = ((const u32x4*)src)[c];
        } else {
#pragma unroll
          for (int c = 0; c < D / LPT / 8; ++c) dst[c] = u32x4{0, 0, 0, 0};
        }
      }
      wave_lds_sync();
#pragma unroll
      for (int jj = 0; jj < KT / 16; ++jj) {
        const int j = kc * (KT / 16) + jj;
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
          const u32x4 kb = *(const u32x4*)(kv + (16 * jj + n) * L::K_LD + 32 * ks + 8 * g);
          s[j] = M::run(qa[ks], kb, s[j]);
        }
      }
      wave_lds_sync();
    }
    if (next_quant) load_k(next);

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
    for (int i = 0; i < 4; ++i) tmax[i] = group_reduce<16>(tmax[i], OpMax());
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
      psum[i] = group_reduce<16>(psum[i], OpAdd());
      l_run[i] = l_run[i] * corr[i] + psum[i];
    }
#pragma unroll
    for (int jn = 0; jn < D / 16; ++jn) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[jn][i] *= corr[i];
    }

    // ---------------- acc += P V, one value group (64 channels) at a time
#pragma unroll
    for (int vc = 0; vc < NG; ++vc) {
      // V^T chunk -> kv[c * V_LD + t]: lane = tokens 2tp, 2tp+1, channels 32cs..32cs+31
      if (quant && kCB) {
        DeqG gv[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) gv[r] = deq_group<BITS>(vmeta[vc][r][0], vmeta[vc][r][1], EV_BASE, a.e_value);
        build_codebooks(gv, [](float x0, float x1) { return pack_io_f16<IO>(x0, x1); });
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const uint32_t h0 = cb0[code_at<BITS>(vw[vc][0], i) * 64];
          const uint32_t h1 = cb1[code_at<BITS>(vw[vc][1], i) * 64];
          *(uint32_t*)(kv + (32 * cs + i) * L::V_LD + cs * L::V_HI + 2 * tp) = h0 | (h1 << 16);
        }
      } else if (quant) {
        DeqG gv[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) gv[r] = deq_group<BITS>(vmeta[vc][r][0], vmeta[vc][r][1], EV_BASE, a.e_value);
#pragma unroll
        for (int i0 = 0; i0 < 32; i0 += 8) {
          int q0[8], q1[8];
          float z0[8], z1[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            q0[u] = code_at<BITS>(vw[vc][0], i0 + u);
            q1[u] = code_at<BITS>(vw[vc][1], i0 + u);
            z0[u] = deq_fetch<BITS>(gv[0], q0[u]);
            z1[u] = deq_fetch<BITS>(gv[1], q1[u]);
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < 8; ++u)
            *(uint32_t*)(kv + (32 * cs + i0 + u) * L::V_LD + cs * L::V_HI + 2 * tp) =
                pack_io_f16<IO>(deq_apply<BITS>(gv[0], q0[u], z0[u]), deq_apply<BITS>(gv[1], q1[u], z1[u]));
        }
      } else if (dv > 0) {
        // misaligned value prefix (logq_compatible_layout): the first dv
        // tokens past the key prefix have quantized values, the rest dense
        // ones starting at v_res row 0; one token at a time
#pragma unroll 1
        for (int r = 0; r < 2; ++r) {
          const int tok = 2 * tp + r;
          const int vt = r0 + tok;  // token index past the key prefix
          uint16_t* col = kv + (32 * cs) * L::V_LD + cs * L::V_HI + tok;
          if (tok < n_valid && vt < dv) {
            const int64_t at = (int64_t)a.n_groups * kTile + vt;
            const uint32_t* row = (const uint32_t*)(vbase + (at * NG + vc) * QB) + cs * BITS;
            uint32_t w[BITS];
#pragma unroll
            for (int i = 0; i < BITS; ++i) w[i] = row[i];
            const int64_t mi = vmb + at * NG + vc;
            const DeqG gq = deq_group<BITS>(meta_load(a.v_mn, mi, a.meta_dtype), meta_load(a.v_scale, mi, a.meta_dtype),
                                            EV_BASE, a.e_value);
#pragma unroll
            for (int i = 0; i < 32; i += 2) {
              const uint32_t h = pack_io_f16<IO>(deq_code<BITS>(gq, code_at<BITS>(w, i)),
                                                 deq_code<BITS>(gq, code_at<BITS>(w, i + 1)));
              col[i * L::V_LD] = (uint16_t)h;
              col[(i + 1) * L::V_LD] = (uint16_t)(h >> 16);
            }
          } else if (tok < n_valid) {
            const uint16_t* src = (const uint16_t*)a.v_res + b * a.vr_sb + kvh * a.vr_sh +
                                  (int64_t)(vt - dv) * a.vr_st + 64 * vc + 32 * cs;
#pragma unroll
            for (int i = 0; i < 32; i += 2)
              {
                const uint32_t h = io_pair_to_f16<IO>(src[i], src[i + 1]);
                col[i * L::V_LD] = (uint16_t)h;
                col[(i + 1) * L::V_LD] = (uint16_t)(h >> 16);
              }
          } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) col[i * L::V_LD] = 0;
          }
        }
      } else {
        u32x4 rv[2][4];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int tok = 2 * tp + r;
          if (tok < n_valid) {
            const uint16_t* src = (const uint16_t*)a.v_res + b * a.vr_sb + kvh * a.vr_sh +
                                  (int64_t)(r0 + tok) * a.vr_st + 64 * vc + 32 * cs;
#pragma unroll
            for (int c = 0; c < 4; ++c) rv[r][c] = ((const u32x4*)src)[c];
          } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) rv[r][c] = u32x4{0, 0, 0, 0};
          }
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const uint32_t w0 = rv[0][i >> 3][(i >> 1) & 3], w1 = rv[1][i >> 3][(i >> 1) & 3];
          const uint16_t h0 = (i & 1) ? (uint16_t)(w0 >> 16) : (uint16_t)w0;
          const uint16_t h1 = (i & 1) ? (uint16_t)(w1 >> 16) : (uint16_t)w1;
          *(uint32_t*)(kv + (32 * cs + i) * L::V_LD + cs * L::V_HI + 2 * tp) = io_pair_to_f16<IO>(h0, h1);
        }
      }
      wave_lds_sync();
      // A = P[m=n][32ks+8g..], B = V[32ks+8g..][16jn+n]
#pragma unroll
      for (int ks = 0; ks < kTile / 32; ++ks) {
        const u32x4 pa = *(const u32x4*)(pb + n * L::P_LD + 32 * ks + 8 * g);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const u32x4 vb = *(const u32x4*)(kv + (16 * jj + n) * L::V_LD + (jj >= 2 ? L::V_HI : 0) + 32 * ks + 8 * g);
          acc[4 * vc + jj] = Mfma<MZ_F16>::run(pa, vb, acc[4 * vc + jj]);
        }
      }
      wave_lds_sync();
    }
    if (next_quant) load_v(next);
  }

  // ---------------- merge the 4 waves' states, write the split partial
  __syncthreads();
  float* red = (float*)lds;  // per wave: m[16], l[16], acc[16][D]
  constexpr int RED = L::RED_FLOATS;
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
  if (direct) {
    // one split: the final output, exactly as the combine kernel would form it
    for (int e = threadIdx.x; e < n_rep * D; e += 256) {
      const int h = e / D;
      const int c = e - h * D;
      float M_ = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M_ = fmaxf(M_, red[w * RED + h]);
      float num = 0.f, den = 0.f;
      if (M_ != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const float f = __expf(red[w * RED + h] - M_);
          num += f * red[w * RED + 32 + h * D + c];
          den += f * red[w * RED + 16 + h];
        }
      }
      store_val(a.out, b * a.out_sb + (int64_t)(kvh * n_rep + h) * a.out_sh + c, den > 0.f ? num / den : 0.f,
                a.out_dtype);
    }
    return;
  }
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

// The online-softmax state of a packed prefix, for one (batch, q-head): the
// split records merged into (acc, m, l) with acc and l relative to the merged
// maximum m (the state the reference's prefix_decode kernels return, and what
// its reduce kernel forms from its chunk records, loader.py:1251-1285), and,
// when requested, the records themselves as the reference's chunk partials
// (chunks past the split count hold the empty state acc = 0, m = -inf, l = 0,
// as an empty reference chunk does).
template <int D>
__global__ __launch_bounds__(D) void prefix_state_kernel(const float* __restrict__ ws, int n_split, int Hq,
                                                         mz_prefix_state_args st) {
  const int bh = blockIdx.x;
  const int c = threadIdx.x;
  const float* base = ws + (int64_t)bh * n_split * (D + 2);
  float M_ = -INFINITY;
  for (int s = 0; s < n_split; ++s)
    if (base[s * (D + 2) + D + 1] > 0.f) M_ = fmaxf(M_, base[s * (D + 2) + D]);
  float acc = 0.f, l = 0.f;
  if (M_ != -INFINITY) {
    for (int s = 0; s < n_split; ++s) {
      const float ls = base[s * (D + 2) + D + 1];
      if (!(ls > 0.f)) continue;  // an empty record (every logit masked) adds nothing
      const float f = __expf(base[s * (D + 2) + D] - M_);
      acc += f * base[s * (D + 2) + c];
      l += f * ls;
    }
  }
  const int b = bh / Hq, h = bh - b * Hq;
  st.acc[b * st.acc_sb + (int64_t)h * st.acc_sh + c] = acc;
  if (c == 0) {
    st.m[b * st.ml_sb + h] = M_;
    st.l[b * st.ml_sb + h] = l;
  }
  if (st.n_chunks > 0) {
    for (int s = 0; s < st.n_chunks; ++s) {
      const bool real = s < n_split;
      const int64_t row = (int64_t)bh * st.n_chunks + s;
      st.part_acc[row * D + c] = real ? base[s * (D + 2) + c] : 0.f;
      if (c == 0) {
        st.part_m[row] = real ? base[s * (D + 2) + D] : -INFINITY;
        st.part_l[row] = real ? base[s * (D + 2) + D + 1] : 0.f;
      }
    }
  }
}

bool fold_supported(const mz_decode_args* a);
int fold_choose_split(const mz_decode_args* a, int* tiles_per_split);
int fold_launch_partials(const mz_decode_args* a, hipStream_t s, bool direct);
bool cb_supported(const mz_decode_args* a);
int cb_choose_split(const mz_decode_args* a, int* tiles_per_split);
int cb_launch_partials(const mz_decode_args* a, hipStream_t s, bool direct);
bool tp_supported(const mz_decode_args* a);
int tp_choose_split(const mz_decode_args* a, int* tiles_per_split);
int64_t tp_workspace_bytes(const mz_decode_args* a, int ns);
int tp_launch_partials(const mz_decode_args* a, hipStream_t s);


static int choose_split(const mz_decode_args* a, int* tiles_per_split) {
  const int n_tiles = a->n_groups + (a->n_residual + kTile - 1) / kTile;
  if (n_tiles <= 0) { *tiles_per_split = 1; return 1; }
  int ns = a->n_split;
  if (ns <= 0) {
    // fill the resident workgroup slots (two per CU) once: each workgroup then
    // loads its tables and query once and runs all its tiles in one pass
    const int64_t units = std::max<int64_t>(1, (int64_t)a->batch * a->kv_heads);  // an empty batch splits nothing
    const int64_t slots = 2 * (int64_t)device_cu_count();
    ns = (int)((slots + units - 1) / units);
    ns = max(1, min(ns, (n_tiles + 7) / 8));  // at least 2 tiles per wave
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
  if (a->kernel_path < MZ_PATH_AUTO || a->kernel_path > MZ_PATH_GENERAL) return MZ_EINVAL;
  if (a->head_dim != 64 && a->head_dim != 128) return MZ_EUNSUPPORTED;
  if (a->n_rep > 16) return MZ_EUNSUPPORTED;
  if (a->batch == 0) return MZ_OK;
  if (!a->query || !a->out) return MZ_EINVAL;
  if (a->n_groups > 0 && (!a->k_packed || !a->k_mn || !a->k_scale || !a->v_packed || !a->v_mn || !a->v_scale ||
                          !a->e_key || !a->e_value))
    return MZ_EINVAL;
  // dense value rows: the residual window minus the quantized value tokens past the key prefix
  const int64_t v_dense = (int64_t)a->n_residual - (a->v_prefix ? a->v_prefix - (int64_t)a->n_groups * 64 : 0);
  if (a->n_residual > 0 && !a->k_res) return MZ_EINVAL;
  if (v_dense > 0 && !a->v_res) return MZ_EINVAL;
  if (a->v_prefix != 0) {
    const int64_t lk = (int64_t)a->n_groups * 64;
    if (a->v_prefix < lk || a->v_prefix > lk + a->n_residual) return MZ_EINVAL;
    if (a->v_prefix > lk && (!a->v_packed || !a->v_mn || !a->v_scale || !a->e_value)) return MZ_EINVAL;
  }
  // 16-byte vector loads of query rows and residual rows
  if (((uintptr_t)a->query & 15) || (a->q_sh & 7) || (a->q_sb & 7)) return MZ_EINVAL;
  if (a->n_residual > 0 && (((uintptr_t)a->k_res & 15) || ((uintptr_t)a->v_res & 15) || (a->kr_st & 7) ||
                            (a->kr_sh & 7) || (a->kr_sb & 7) || (a->vr_st & 7) || (a->vr_sh & 7) || (a->vr_sb & 7)))
    return MZ_EINVAL;
  if ((a->n_groups > 0 || a->v_prefix > 0) &&
      (((uintptr_t)a->k_packed & 3) || ((uintptr_t)a->v_packed & 3) || (a->kp_sb & 3) || (a->kp_sh & 3) ||
       (a->vp_sb & 3) || (a->vp_sh & 3)))
    return MZ_EINVAL;
  return MZ_OK;
}

// Which kernel runs and with how many splits (the kernels share the
// workspace layout and the combine kernel).
enum Kernel { K_GENERAL = 0, K_FOLD = 1, K_CODEBOOK = 2, K_TWOPASS = 3 };

// AUTO: the codebook kernel where it applies (1-5 bits, the layer-dtype
// values: at 1-4 bits at the fold kernel's speed or better, at 5 bits ~13 %
// slower, kept for the values), else the fold kernel (6-7 bits, head_dim
// 64, 5 bits with two alphas or more query heads), else the two-pass kernel
// (8 bits, 7 bits with two alphas: the layer-dtype values), else the general
// one.
// EXACT: the codebook kernel where it applies, else the two-pass kernel
// (5-8 bits), else the general kernel.
static Kernel which_kernel(const mz_decode_args* a) {
  switch (a->kernel_path) {
    case MZ_PATH_GENERAL: return K_GENERAL;
    case MZ_PATH_FOLD: return fold_supported(a) ? K_FOLD : K_GENERAL;
    case MZ_PATH_CODEBOOK: return cb_supported(a) ? K_CODEBOOK : K_GENERAL;
    case MZ_PATH_EXACT: return cb_supported(a) ? K_CODEBOOK : tp_supported(a) ? K_TWOPASS : K_GENERAL;
    default:
      return cb_supported(a) ? K_CODEBOOK : fold_supported(a) ? K_FOLD : tp_supported(a) ? K_TWOPASS : K_GENERAL;
  }
}

// A forced kernel that does not take these arguments.
static bool forced_unsupported(const mz_decode_args* a) {
  return (a->kernel_path == MZ_PATH_FOLD && !fold_supported(a)) ||
         (a->kernel_path == MZ_PATH_CODEBOOK && !cb_supported(a));
}

static int plan_split(const mz_decode_args* a, int* tps) {
  switch (which_kernel(a)) {
    case K_FOLD: return fold_choose_split(a, tps);
    case K_CODEBOOK: return cb_choose_split(a, tps);
    case K_TWOPASS: return tp_choose_split(a, tps);
    default: return choose_split(a, tps);
  }
}

// Workspace bytes of a planned call: the split records, and for the
// two-pass kernel its logits after them.
static int64_t plan_workspace(const mz_decode_args* a, int ns) {
  if (which_kernel(a) == K_TWOPASS) return tp_workspace_bytes(a, ns);
  return (int64_t)a->batch * a->kv_heads * a->n_rep * ns * (a->head_dim + 2) * (int64_t)sizeof(float);
}

// The codebook, fold and two-pass kernels (the two-pass kernel always
// writes records: `direct` is for the other two).
static int launch_fast(const mz_decode_args* a, hipStream_t s, bool direct) {
  switch (which_kernel(a)) {
    case K_FOLD: return fold_launch_partials(a, s, direct);
    case K_TWOPASS: return tp_launch_partials(a, s);
    default: return cb_launch_partials(a, s, direct);
  }
}

}  // namespace mz

using namespace mz;

extern "C" int64_t muzero_decode_workspace_bytes(const mz_decode_args* a, int* n_split_out) {
  if (check_args(a) != MZ_OK) return -1;
  if (forced_unsupported(a)) return -1;
  int tps;
  const int ns = plan_split(a, &tps);
  if (n_split_out) *n_split_out = ns;
  return plan_workspace(a, ns);
}

extern "C" int muzero_decode_uses_fold(const mz_decode_args* a) {
  if (check_args(a) != MZ_OK) return -1;
  return which_kernel(a) == K_FOLD ? 1 : 0;
}

extern "C" int muzero_decode_kernel(const mz_decode_args* a) {
  if (check_args(a) != MZ_OK || forced_unsupported(a)) return -1;
  return (int)which_kernel(a);
}

template <int D, int IO>
static int launch_partials(const mz_decode_args* a, hipStream_t s, bool direct) {
  int tps;
  const int ns = choose_split(a, &tps);
  static_assert(D == 64 || D == 128, "head_dim");
  const int64_t need = (int64_t)a->batch * a->kv_heads * a->n_rep * ns * (D + 2) * (int64_t)sizeof(float);
  if (!direct && (!a->workspace || a->workspace_bytes < need)) return MZ_EWORKSPACE;
  const int dir = direct ? 1 : 0;
  const dim3 grid(ns, a->kv_heads, a->batch);
  switch (a->bits) {
#define MZ_CASE(BB)                                                                                           \
  case BB: {                                                                                                  \
    const size_t lds = Lds<D>::bytes(BB);                                                                     \
    static std::atomic<uint64_t> lds_set{0};                                                                  \
    const hipError_t attr = set_dynamic_lds((const void*)decode_split_kernel<D, BB, IO>, (int)lds, lds_set);  \
    if (attr != hipSuccess) return (int)attr;                                                                 \
    hipLaunchKernelGGL((decode_split_kernel<D, BB, IO>), grid, dim3(256), lds, s, *a, tps, ns, dir);       \
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

static int launch_general(const mz_decode_args* a, hipStream_t s, bool direct) {
  if (a->head_dim == 128)
    return a->io_dtype == MZ_BF16 ? launch_partials<128, MZ_BF16>(a, s, direct)
                                  : launch_partials<128, MZ_F16>(a, s, direct);
  return a->io_dtype == MZ_BF16 ? launch_partials<64, MZ_BF16>(a, s, direct)
                                : launch_partials<64, MZ_F16>(a, s, direct);
}


extern "C" int muzero_decode_partials(const mz_decode_args* a, mz_stream_t stream) {
  const int st = decode_check_launchable(a);
  if (st) return st == 1 ? MZ_OK : st;
  hipStream_t s = (hipStream_t)stream;
  if (forced_unsupported(a)) return MZ_EUNSUPPORTED;
  if (which_kernel(a) != K_GENERAL) {
    int tps;
    const int ns = plan_split(a, &tps);
    const int64_t need = plan_workspace(a, ns);
    if (!a->workspace || a->workspace_bytes < need) return MZ_EWORKSPACE;
    return launch_fast(a, s, false);
  }
  return launch_general(a, s, false);
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

extern "C" int muzero_decode_prefix_state(const mz_decode_args* a, const mz_prefix_state_args* st,
                                          mz_stream_t stream) {
  if (!a || !st) return MZ_EINVAL;
  // the packed prefix alone, keys and values aligned
  if (a->n_residual != 0 || (a->v_prefix != 0 && a->v_prefix != a->n_groups * kTile)) return MZ_EINVAL;
  if (st->n_chunks < 0) return MZ_EINVAL;
  mz_decode_args b = *a;
  b.v_prefix = 0;
  if (st->n_chunks > 0) b.n_split = st->n_chunks;
  int ns = 0;
  const int64_t need = muzero_decode_workspace_bytes(&b, &ns);
  if (need < 0) {
    const int c = check_args(&b);
    return c != MZ_OK ? c : MZ_EUNSUPPORTED;
  }
  if (b.batch == 0) return MZ_OK;
  if (b.n_groups <= 0) return MZ_EINVAL;
  if (!st->acc || !st->m || !st->l) return MZ_EINVAL;
  if (st->n_chunks > 0 && (!st->part_acc || !st->part_m || !st->part_l)) return MZ_EINVAL;
  if (!b.workspace || b.workspace_bytes < need) return MZ_EWORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int r = muzero_decode_partials(&b, stream);
  if (r != MZ_OK) return r;
  const int Hq = b.kv_heads * b.n_rep;
  if (b.head_dim == 128)
    hipLaunchKernelGGL((prefix_state_kernel<128>), dim3(b.batch * Hq), dim3(128), 0, s,
                       (const float*)b.workspace, ns, Hq, *st);
  else
    hipLaunchKernelGGL((prefix_state_kernel<64>), dim3(b.batch * Hq), dim3(64), 0, s,
                       (const float*)b.workspace, ns, Hq, *st);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

extern "C" int muzero_decode_attention(const mz_decode_args* a, mz_stream_t stream) {
  // one split: the split kernel writes the output (no workspace, no combine);
  // the two-pass kernel always goes through the workspace
  if (decode_check_launchable(a) == MZ_OK && a->out && !forced_unsupported(a) && which_kernel(a) != K_TWOPASS) {
    int tps;
    if (plan_split(a, &tps) == 1)
      return which_kernel(a) != K_GENERAL ? launch_fast(a, (hipStream_t)stream, true)
                                          : launch_general(a, (hipStream_t)stream, true);
  }
  const int st = muzero_decode_partials(a, stream);
  if (st != MZ_OK) return st;
  return muzero_decode_combine(a, stream);
}

// ------------------------------------------------------------ allocation-free entry point
// muzero_decode_attention_noalloc keeps a split call's partial records in this
// array instead of a caller workspace: one copy per device, held by each
// device that runs the library until the process ends.  In host code the
// name `scratch` is a stand-in, not a device address: the address comes from
// hipGetSymbolAddress, taken once per device with that device current.
static __device__ __align__(256) float scratch[MZ_DECODE_SCRATCH_BYTES / sizeof(float)];

static hipError_t scratch_address(void** out) {
  static std::atomic<void*> addr[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = addr[dev].load(std::memory_order_acquire);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return hipSuccess;
}

extern "C" int muzero_decode_attention_noalloc(const mz_decode_args* a, mz_stream_t stream) {
  if (!a) return MZ_EINVAL;
  mz_decode_args b = *a;
  int ns = 0;
  int64_t need = muzero_decode_workspace_bytes(&b, &ns);
  if (need < 0) {
    // the status muzero_decode_attention gives for the same arguments
    const int c = check_args(a);
    return c != MZ_OK ? c : MZ_EUNSUPPORTED;  // a forced fold path the fold kernel does not take
  }
  // the two-pass kernel keeps its logits in the workspace as well: a call
  // whose logits do not fit the scratch runs the general kernel instead
  if (need > (int64_t)MZ_DECODE_SCRATCH_BYTES && b.batch > 0 && which_kernel(&b) == K_TWOPASS) {
    b.kernel_path = MZ_PATH_GENERAL;
    need = muzero_decode_workspace_bytes(&b, &ns);
  }
  // a single split of the other kernels writes the output directly and reads no workspace
  const bool reads_ws = ns > 1 || (b.batch > 0 && which_kernel(&b) == K_TWOPASS);
  if (reads_ws && need > (int64_t)MZ_DECODE_SCRATCH_BYTES) return MZ_ESCRATCH;
  const hipError_t e = scratch_address(&b.workspace);
  if (e != hipSuccess) return (int)e;
  b.workspace_bytes = (int64_t)MZ_DECODE_SCRATCH_BYTES;
  return muzero_decode_attention(&b, stream);
}
