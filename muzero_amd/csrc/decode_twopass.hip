// Packed-KV decode attention over 5- to 8-bit codes in two passes, attending
// with the reference's dequantize-then-attend values (gfx950, wave64, MFMA
// 16x16x32 in the layer dtype).
//
// An 8-bit group has 256 possible values for its 64 codes, so per-group
// codebooks cost more than dequantizing each code.  Each code's value is the
// reference's fp32 operation sequence (muzero/quantizer.py:241-255: t = pe*E
// above the zero level or -ne*E below it, unit = za + t, x = unit*s + mn)
// rounded to the layer dtype (muzero/cache/layer.py:263), with E read from the
// expm1 rows of bins 1..2^bits - 1 (the host-built table; 32,895 fp32 entries
// = 128.5 KB at 8 bits) held in LDS.  One such table per alpha: keys and
// values usually have different alphas at 8 bits (quantizer.py:72-77), and
// two 8-bit tables do not fit one CU's 160 KB.  Hence two launches, each with
// its one table in LDS and one workgroup per CU:
//   pass 1 (keys):   12 waves (three per SIMD); S = Q K^T per 64-token tile,
//                    written as fp32 logits in base-2 units (scaled, masked)
//                    to the workspace;
//   pass 2 (values): 8 waves (two per SIMD); the logits back, an online
//                    softmax, P V per tile; each wave owns one contiguous
//                    run of tiles (a split) and
//                    writes its (acc, m, l) record, merged by the combine
//                    kernel of decode.hip.
// The logits' round trip through HBM is 4 bytes per (query head, token),
// written once and read once: at n_rep 4 and 8 bits, 32 bytes per token and
// kv-head against its 256 code bytes.
//
// The same kernels serve 5-7 bits (the exact path where the codebook kernel
// does not apply, and 7 bits with two alphas), with the smaller tables.
//
// Layout of a tile on the MFMA (as the codebook kernel, decode_cb.hip):
//   QK: rows = query heads (row RS*h; the others zero), columns = tokens
//   4n+jt of N-tiles jt = 0..3; lane (n, g) of k-step kt holds channels
//   32kt+8g+{0..7}.  A lane loads, for each of its 8 channel rows of a
//   k-step, the dword holding its tokens 4n..4n+3 (at 8 bits byte jt = the
//   code of token 4n+jt): every code of the tile is loaded once.
//   PV: rows RS*h / RS*h+1 = the high / low parts of the head's weights in
//   the layer dtype; columns = channels 64vg+4n+jt; lane (n, g) of step
//   (kt, vg) holds tokens 32kt+8g+{0..7} and loads, for each, the dword
//   holding its channels 4n..4n+3 of value group vg.
// Group quantities: a lane forms those of two groups of the tile (key
// channels 2*lane, 2*lane+1; value groups 0, 1 of token lane) and stores
// them as 7 words (zl, the byte bases of the up and down rows, pe, za, s, mn)
// in the wave's LDS area, structure of arrays; the lanes of a lane group then
// read the 4 groups of a half step with one 16-byte broadcast read per word.
// Pass 1 keeps the words of 64 key groups at a time (channels 0-63, then
// 64-127: half the area, so that 12 waves' areas fit beside the table).
// A code costs its extract scaled to a byte offset (one SDWA shift at 8
// bits), a compare, a select of the row and one v_sad_u16 for the table
// address, a select of the coefficient, one 32-bit LDS read and the four
// fp32 steps.
#include "decode_tile.hpp"

namespace mz {

namespace tp {

constexpr int D = 128;
constexpr int TILE = 64;
constexpr int WAVES = 8;                            // pass 2
constexpr int NT = 64 * WAVES;
constexpr int WAVES_1 = 12;                         // pass 1
constexpr int NT_1 = 64 * WAVES_1;
constexpr int PW = 7;                               // words per group
constexpr int PS_ROW = 128 * 4;                     // bytes per word row (128 groups), pass 2
constexpr int PS_BYTES = PW * PS_ROW;               // per wave
constexpr int PS_ROW_1 = 64 * 4;                    // pass 1: 64 groups
constexpr int PS_BYTES_1 = PW * PS_ROW_1;

// Code width BITS (5 to 8).
template <int BITS>
struct Fmt {
  static constexpr int QMAX = (1 << BITS) - 1;
  static constexpr int QB = 8 * BITS;                         // bytes per packed 64-code row
  static constexpr int ET_N = QMAX * (QMAX + 3) / 2;           // expm1 entries of bins 1..QMAX: sum of (bins + 1)
  static constexpr int ET_BYTES = (ET_N * 4 + 15) / 16 * 16;
  static constexpr int LDS_BYTES = ET_BYTES + WAVES * PS_BYTES;
  static constexpr int LDS_BYTES_1 = ET_BYTES + WAVES_1 * PS_BYTES_1;
  static_assert(LDS_BYTES <= 160 * 1024 && LDS_BYTES_1 <= 160 * 1024, "one workgroup per CU");
  // a lane's 4 codes of a row (tokens or channels 4n..4n+3) are 4*BITS bits
  // from bit 4*BITS*n: the dword at byte word_byte(n) holds them from bit
  // word_shift(n) (read unaligned; the last lane's dword moved back inside
  // the row)
  static __device__ __forceinline__ int word_byte(int n) { return min((4 * BITS * n) >> 3, QB - 4); }
  static __device__ __forceinline__ uint32_t word_shift(int n) { return (uint32_t)(4 * BITS * n - 8 * word_byte(n)); }
};
constexpr float kLog2e = 1.44269504088896341f;
constexpr float kLn2 = 0.693147180559945309f;
constexpr float kEps = 1e-8f;
enum { P_ZL = 0, P_UP, P_DN, P_PE, P_ZA, P_S, P_MN };

// Two fp32 values rounded to the io dtype (round to nearest even), packed low / high.
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

// The dequantization quantities of one stored group (mn, s), formed as the
// reference forms them from the stored metadata (quantizer.py:241-249), the
// scale guarded like the reference CUDA extension (loader.py:201) so that an
// all-zero group (stored scale 0) gives x = mn.  zl4 = 4 zl; up / down: the
// byte address of expm1 entry 0 of the row for codes above / below the zero
// level, so that code q's entry lies at 4|q - zl| past the side's row start.
template <int QMAX>
__device__ __forceinline__ void group_words(float mn, float s, uint32_t (&w)[PW]) {
  const float sg = s >= kEps ? s : kEps;  // NaN -> eps, as deq_row
  const float za = clamp01((0.f - mn) / sg);  // IEEE division: the zero level must match
  const float zlf = rintf(za * (float)QMAX);
  // a NaN zero level (NaN metadata) reads row 0: the values are NaN anyway
  const int zl = (int)__builtin_amdgcn_fmed3f(zlf == zlf ? zlf : 0.f, 0.f, (float)QMAX);
  const int pb = max(QMAX - zl, 1), nb = max(zl, 1);
  w[P_ZL] = (uint32_t)(4 * zl);
  w[P_UP] = (uint32_t)(4 * expm1_row(pb));
  w[P_DN] = (uint32_t)(4 * expm1_row(nb));
  w[P_PE] = __float_as_uint(clamp_min(1.f - za, kEps));
  w[P_ZA] = __float_as_uint(za);
  w[P_S] = __float_as_uint(sg);
  w[P_MN] = __float_as_uint(mn);
}

// Four groups of a step (rows 4h .. 4h + 3): word k of group j (zl: 4 zl).  mne = -ne.
struct Groups4 {
  uint32_t zl[4], up[4], dn[4];
  float pe[4], mne[4], za[4], s[4], mn[4];
};

// Groups first .. first + 3 of the wave's word arrays, rows of ROW bytes (one
// 16-byte read per word; the lanes of a lane group read the same groups: a
// broadcast).
template <int ROW>
__device__ __forceinline__ void read_groups(const uint8_t* ps, int first, Groups4& G) {
  auto rd = [&](int k) __attribute__((always_inline)) { return *(const u32x4*)(ps + k * ROW + 4 * first); };
  const u32x4 zl = rd(P_ZL), up = rd(P_UP), dn = rd(P_DN), pe = rd(P_PE), za = rd(P_ZA), sc = rd(P_S),
              mn = rd(P_MN);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    G.zl[j] = zl[j];
    G.up[j] = up[j];
    G.dn[j] = dn[j];
    G.pe[j] = __uint_as_float(pe[j]);
    G.za[j] = __uint_as_float(za[j]);
    G.mne[j] = -clamp_min(G.za[j], kEps);
    G.s[j] = __uint_as_float(sc[j]);
    G.mn[j] = __uint_as_float(mn[j]);
  }
}

// The reference's fp32 value of code q of group j (quantizer.py:250-255).
// unit = za + t needs no clamp: every expm1 entry lies in [0, 1], so for
// finite metadata za + pe*E <= 1 and za - ne*E >= 0 after rounding, and NaN
// metadata propagates.  Every address lies inside the table: q - zl <= pb
// above the zero level, zl - q <= nb below it.
__device__ __forceinline__ float code_value(const uint8_t* smem, uint32_t q, const Groups4& G, int j) {
  const uint32_t q4 = 4u * q;
  const bool up = q4 >= G.zl[j];
  // row start + 4|q - zl| (one v_sad_u16: both below 2^16)
  const uint32_t addr = __builtin_amdgcn_sad_u16(q4, G.zl[j], up ? G.up[j] : G.dn[j]);
  const float e = *(const float*)(smem + addr);
  const float t = (up ? G.pe[j] : G.mne[j]) * e;
  const float unit = G.za[j] + t;
  const float u = unit * G.s[j];
  return u + G.mn[j];
}

// Half h of the 4 B operands (N-tiles jt = 0..3) of one step: registers
// 2h, 2h + 1 of each, from the code words w[j] of rows 4h + j (byte jt = the
// code of column jt) and those rows' groups; two rows per B register.
template <int IO, int BITS>
__device__ __forceinline__ void dequant_half(const uint8_t* smem, const uint32_t* w, uint32_t sh, const Groups4& G,
                                             int h, u32x4 (&B)[4]) {
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float x0 = code_value(smem, __builtin_amdgcn_ubfe(w[2 * i], sh + BITS * jt, BITS), G, 2 * i);
      const float x1 = code_value(smem, __builtin_amdgcn_ubfe(w[2 * i + 1], sh + BITS * jt, BITS), G, 2 * i + 1);
      B[jt][2 * h + i] = pack_io2<IO>(x0, x1);
    }
}

// The 4 B operands of one step whose 8 rows' groups start at `first` in the
// word arrays (rows of ROW bytes) and whose code words are w[0..7] (this
// lane's codes from bit sh).
template <int IO, int BITS, int ROW>
__device__ __forceinline__ void dequant_step(const uint8_t* smem, const uint8_t* ps, int first, const uint32_t* w,
                                             uint32_t sh, u32x4 (&B)[4]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    Groups4 G;
    read_groups<ROW>(ps, first + 4 * h, G);
    dequant_half<IO, BITS>(smem, w + 4 * h, sh, G, h, B);
  }
}

// The expm1 rows of bins 1..QMAX of one alpha (the table's first ET_N
// entries) into LDS (bytes 0 .. 4 ET_N of the workgroup's array) by the NTH
// threads of the workgroup: 16 bytes per load, the last ET_N % 4 entries one
// each.
template <int ET_N, int NTH>
__device__ __forceinline__ void load_table(uint8_t* smem, const float* E) {
  constexpr int V = ET_N / 4;
  for (int i = threadIdx.x; i < V; i += NTH) *(u32x4*)(smem + 16 * i) = *(const u32x4*)(E + 4 * i);
  if (threadIdx.x < ET_N - 4 * V) ((float*)smem)[4 * V + threadIdx.x] = E[4 * V + threadIdx.x];
  __syncthreads();
}

// Sum / maximum over the 4 lane groups (lanes n, n + 16, n + 32, n + 48).
__device__ __forceinline__ float across_groups_max(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float across_groups_sum(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---------------------------------------------------------------- pass 1
// Logits of every tile of every (batch, kv-head): the grid is persistent
// (one workgroup of 12 waves per CU); wave u of the grid takes flat tiles
// u, u + 12*grid, ...
// logits[(b*Hq + q-head)*lt + token] = (q . k) * scaling * log2(e), plus the
// additive mask times log2(e); -inf past the filled residual rows.
// Three waves per SIMD hide the table reads' latency with no prefetch of the
// next tile's words: each wave loads a tile's codes and metadata and uses
// them at once (163 VGPRs at 8 bits, none spilled).
template <int IO, int NREP, int MW, int BITS>
__global__ __launch_bounds__(NT_1) void logits_kernel(const mz_decode_args a, float* __restrict__ logits, int n_tiles,
                                                      int64_t lt) {
  using M = Mfma<IO>;
  constexpr int RS = 16 / NREP;
  constexpr int HS = NREP > 4 ? NREP / 4 : 1;
  constexpr int ES = 2 * MW;  // metadata bytes per entry
  using F = Fmt<BITS>;
  constexpr int QB = F::QB;
  __shared__ __align__(16) uint8_t smem[F::LDS_BYTES_1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  load_table<F::ET_N, NT_1>(smem, a.e_key);
  uint8_t* const ps = smem + F::ET_BYTES + wave * PS_BYTES_1;
  const int wbyte = F::word_byte(n);      // this lane's code dword of a row, and its codes' first bit
  const uint32_t wsh = F::word_shift(n);
  const int Hq = a.kv_heads * a.n_rep;
  const int hA = n / RS, rA = n % RS;
  const bool owner = ((4 * g) % RS) == 0;
  const int h0 = (4 * g) / RS;
  const float scaling2 = a.scaling * kLog2e;
  const int64_t ng = a.n_groups;
  // flat tile u = (b*Hkv + kvh)*n_tiles + tile (the host keeps the count below 2^31)
  const uint32_t total = (uint32_t)a.batch * (uint32_t)a.kv_heads * (uint32_t)n_tiles;
  const uint32_t stride = gridDim.x * WAVES_1;
  for (uint32_t u = blockIdx.x * WAVES_1 + wave; u < total; u += stride) {
    const uint32_t tile = u % (uint32_t)n_tiles, bk = u / (uint32_t)n_tiles;
    const int kvh = (int)(bk % (uint32_t)a.kv_heads), b = (int)(bk / (uint32_t)a.kv_heads);
    // the query operand: row n = head hA's query when rA == 0, else zero
    u32x4 qa[4];
    {
      const bool qrow = rA == 0 && hA < a.n_rep;
      const uint16_t* qp =
          (const uint16_t*)a.query + b * a.q_sb + (int64_t)(kvh * a.n_rep + min(hA, a.n_rep - 1)) * a.q_sh;
#pragma unroll
      for (int kq = 0; kq < 4; ++kq) {
        const u32x4 v = *(const u32x4*)(qp + 32 * kq + 8 * g);
        qa[kq] = qrow ? v : u32x4{0u, 0u, 0u, 0u};
      }
    }
    f32x4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    int n_valid, pos0;
    if ((int)tile < a.n_groups) {
      n_valid = TILE;
      pos0 = TILE * (int)tile;
      const __amdgpu_buffer_rsrc_t kp = make_buf(a.k_packed + b * a.kp_sb + kvh * a.kp_sh, ng * D * QB);
      const int64_t km = b * a.km_sb + kvh * a.km_sh;
      const __amdgpu_buffer_rsrc_t kmn = make_buf((const uint8_t*)a.k_mn + km * ES, ng * D * ES);
      const __amdgpu_buffer_rsrc_t ksc = make_buf((const uint8_t*)a.k_scale + km * ES, ng * D * ES);
      // this lane's code words (KW[8kt + i] = the dword of tokens 4n..4n+3
      // of channel row 32kt + 8g + i) and its two key groups' metadata
      // (channels 2*lane, 2*lane + 1)
      uint32_t KW[32], MN[MW], SC[MW];
      load_meta<MW>(MN, kmn, 2 * lane * ES, (int)tile * D * ES);
      load_meta<MW>(SC, ksc, 2 * lane * ES, (int)tile * D * ES);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          KW[8 * kt + i] = __builtin_amdgcn_raw_buffer_load_b32(kp, 8 * g * QB + wbyte,
                                                                (int)tile * D * QB + (32 * kt + i) * QB, 0);
      const float2 mn = meta_cvt<MW>(MN, a.meta_dtype), sc = meta_cvt<MW>(SC, a.meta_dtype);
      uint32_t w0[PW], w1[PW];
      group_words<F::QMAX>(mn.x, sc.x, w0);
      group_words<F::QMAX>(mn.y, sc.y, w1);
      // channel half hh (k-steps 2hh, 2hh + 1): the words of its 64 groups,
      // stored by lanes 32hh .. 32hh + 31, at group index channel - 64hh
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        if ((lane >> 5) == hh) {
#pragma unroll
          for (int k = 0; k < PW; ++k) *(uint2*)(ps + k * PS_ROW_1 + 8 * (lane - 32 * hh)) = uint2{w0[k], w1[k]};
        }
        wave_lds_sync();
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const int kt = 2 * hh + k2;
          u32x4 B[4];
          dequant_step<IO, BITS, PS_ROW_1>(smem, ps, 32 * k2 + 8 * g, KW + 8 * kt, wsh, B);
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) s[jt] = M::run(qa[kt], B[jt], s[jt]);
        }
        wave_lds_sync();  // the group words are read before the next ones are written
      }
    } else {
      // residual tile: dense keys; rows past the filled ones read 0 (masked below)
      const int r0 = ((int)tile - a.n_groups) * TILE;
      n_valid = min(TILE, a.n_residual - r0);
      pos0 = TILE * a.n_groups + r0;
      const int kst = (int)a.kr_st * 2;
      const uint16_t* kr = (const uint16_t*)a.k_res + b * a.kr_sb + kvh * a.kr_sh;
      const __amdgpu_buffer_rsrc_t krb = make_buf(kr + (int64_t)r0 * a.kr_st, (int64_t)(n_valid - 1) * kst + D * 2);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        u32x4 kb[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
          kb[jt] = __builtin_bit_cast(u32x4,
                                      __builtin_amdgcn_raw_buffer_load_b128(krb, (4 * n + jt) * kst + 16 * g, 64 * kt, 0));
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) s[jt] = M::run(qa[kt], kb[jt], s[jt]);
      }
    }
    // this lane's logits: head slot sl = MFMA output element sl*RS, tokens 4n + jt
    if (owner) {
#pragma unroll
      for (int sl = 0; sl < HS; ++sl) {
        const int h = h0 + sl;
        if (h >= a.n_rep) continue;
        float v[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          const int tt = 4 * n + jt;
          float x = s[jt][sl * RS] * scaling2;
          if (tt >= n_valid) x = -INFINITY;
          else if (a.mask) x = add_mask_log2(x, a.mask[b * a.mask_sb + pos0 + tt]);
          v[jt] = x;
        }
        *(f32x4*)(logits + ((int64_t)b * Hq + kvh * a.n_rep + h) * lt + (int64_t)tile * TILE + 4 * n) =
            f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
}

// ---------------------------------------------------------------- pass 2
// One wave per split (a run of tps tiles of one (batch, kv-head)): unit u =
// (b*Hkv + kvh)*ns + split is wave u % 8 of workgroup u / 8.
template <int IO, int NREP, int MW, int BITS>
__global__ __launch_bounds__(NT) void attend_kernel(const mz_decode_args a, const float* __restrict__ logits,
                                                    int n_tiles, int64_t lt, int tps, int ns) {
  using M = Mfma<IO>;
  constexpr int RS = 16 / NREP;
  static_assert(RS >= 2, "P.V needs a second row per head for the weights' low part");
  constexpr int HS = NREP > 4 ? NREP / 4 : 1;
  constexpr int ES = 2 * MW;
  using F = Fmt<BITS>;
  constexpr int QB = F::QB;
  __shared__ __align__(16) uint8_t smem[F::LDS_BYTES];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;
  const int g = lane >> 4;
  load_table<F::ET_N, NT>(smem, a.e_value);
  uint8_t* const ps = smem + F::ET_BYTES + wave * PS_BYTES;
  const int wbyte = F::word_byte(n);      // this lane's code dword of a row, and its codes' first bit
  const uint32_t wsh = F::word_shift(n);

  const int64_t unit = (int64_t)blockIdx.x * WAVES + wave;
  if (unit >= (int64_t)a.batch * a.kv_heads * ns) return;
  const int split = (int)(unit % ns);
  const int64_t bk = unit / ns;
  const int kvh = (int)(bk % a.kv_heads);
  const int b = (int)(bk / a.kv_heads);
  const int t_begin = split * tps;
  const int t_end = min(n_tiles, t_begin + tps);
  const int Hq = a.kv_heads * a.n_rep;
  const int64_t ng = a.n_groups;
  const __amdgpu_buffer_rsrc_t vp = make_buf(a.v_packed + b * a.vp_sb + kvh * a.vp_sh, ng * TILE * 2 * QB);
  const int64_t vm = b * a.vm_sb + kvh * a.vm_sh;
  const __amdgpu_buffer_rsrc_t vmn = make_buf((const uint8_t*)a.v_mn + vm * ES, ng * TILE * 2 * ES);
  const __amdgpu_buffer_rsrc_t vsc = make_buf((const uint8_t*)a.v_scale + vm * ES, ng * TILE * 2 * ES);
  const uint16_t* vr = (const uint16_t*)a.v_res + b * a.vr_sb + kvh * a.vr_sh;

  // A rows: row n is the high (rA == 0) or low (rA == 1) part of head hA's
  // weights, or zero; its lane reads head hA's logits of tokens 32kt+8g+{0..7}
  const int hA = n / RS, rA = n % RS;
  const bool arow = rA < 2 && hA < a.n_rep;
  const float* lrow = logits + ((int64_t)b * Hq + kvh * a.n_rep + min(hA, a.n_rep - 1)) * lt;
  // MFMA output element (g, i) = row 4g + i: head slot sl is element sl*RS of
  // the lane groups whose rows start a head, head h0 + sl
  const bool owner = ((4 * g) % RS) == 0;
  const int h0 = owner ? (4 * g) / RS : 0;

  float m_run[NREP];  // per head, the same in every lane
#pragma unroll
  for (int h = 0; h < NREP; ++h) m_run[h] = -INFINITY;
  float l_part = 0.f;  // head hA: this lane's tokens' share of the sum
  f32x4 acc[2][4];
#pragma unroll
  for (int vg = 0; vg < 2; ++vg)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[vg][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The words of a tile (loaded one tile ahead, into the other of two
  // register sets), for a quantized tile: its code words (VW[8(2kt + vg) +
  // j] = the dword of channels 4n..4n+3 of token row 32kt + 8g + j, group
  // vg) and this lane's two value groups' metadata (groups 0, 1 of token
  // lane).  This lane's logits of a tile (xn[8kt + j] = token 32kt + 8g + j)
  // are loaded halfway through the tile before it, once the first k-step's
  // registers are free (the split's first tile's before the loop).
  struct Words {
    uint32_t VW[32], MN[MW], SC[MW];
  };
  auto issue = [&](Words& W, int t) __attribute__((always_inline)) {
    if (t < a.n_groups) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int vg = 0; vg < 2; ++vg)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            W.VW[8 * (2 * kt + vg) + j] = __builtin_amdgcn_raw_buffer_load_b32(
                vp, 8 * g * (2 * QB) + wbyte, t * TILE * 2 * QB + (32 * kt + j) * (2 * QB) + QB * vg, 0);
      load_meta<MW>(W.MN, vmn, 2 * lane * ES, t * TILE * 2 * ES);
      load_meta<MW>(W.SC, vsc, 2 * lane * ES, t * TILE * 2 * ES);
    }
  };
  float xn[16];
  auto load_x = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int h4 = 0; h4 < 2; ++h4) {
        const f32x4 v = *(const f32x4*)(lrow + (int64_t)t * TILE + 32 * kt + 8 * g + 4 * h4);
#pragma unroll
        for (int j = 0; j < 4; ++j) xn[8 * kt + 4 * h4 + j] = v[j];
      }
  };
  // one tile from the words in C; the next tile's loads go into N first
  auto step = [&](const int tile, Words& C, Words& N) __attribute__((always_inline)) {
    const bool quant = tile < a.n_groups;
    float x[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = xn[j];
    const uint32_t* const VC = C.VW;
    if (quant) {
      const float2 mn = meta_cvt<MW>(C.MN, a.meta_dtype), sc = meta_cvt<MW>(C.SC, a.meta_dtype);
      uint32_t w0[PW], w1[PW];
      group_words<F::QMAX>(mn.x, sc.x, w0);
      group_words<F::QMAX>(mn.y, sc.y, w1);
      // group (token t, vg) at index 64*vg + t
#pragma unroll
      for (int k = 0; k < PW; ++k) {
        *(uint32_t*)(ps + k * PS_ROW + 4 * lane) = w0[k];
        *(uint32_t*)(ps + k * PS_ROW + 4 * (TILE + lane)) = w1[k];
      }
    }
    // the next tile's loads go out before this tile's work
    if (tile + 1 < t_end) issue(N, tile + 1);
    if (quant) wave_lds_sync();

    // ---------- online softmax: the tile's maximum of each head
    float tmax = x[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) tmax = fmaxf(tmax, x[j]);
    tmax = across_groups_max(tmax);
    // mu / cu: the shift and correction of this lane's head hA; cs[sl]: the
    // correction of head slot sl's rows
    float mu = 0.f, cu = 1.f, cs[HS];
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) cs[sl] = 1.f;
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
      const float th = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tmax), RS * h));
      const float m_new = fmaxf(m_run[h], th);
      // while a row is fully masked its maximum stays -inf; 0 stands in for
      // it, so exp2(-inf - 0) gives zero weights and a zero correction
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float corr = __builtin_amdgcn_exp2f(m_run[h] - m_use);
      m_run[h] = m_new;
      if (hA == h) mu = m_use, cu = corr;
#pragma unroll
      for (int sl = 0; sl < HS; ++sl)
        if (h0 + sl == h) cs[sl] = corr;
    }
    float p[16];
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) p[j] = __builtin_amdgcn_exp2f(x[j] - mu), psum += p[j];
    l_part = l_part * cu + psum;
    // the weights as high + low parts in the io dtype (A operand of k-step kt)
    u32x4 pa[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = p[8 * kt + 2 * i], p1 = p[8 * kt + 2 * i + 1];
        const uint32_t hi = pack_io2<IO>(p0, p1);
        const uint32_t lo =
            pack_io2<IO>(p0 - io_to_f32<IO>((uint16_t)hi), p1 - io_to_f32<IO>((uint16_t)(hi >> 16)));
        pa[kt][i] = arow ? (rA == 0 ? hi : lo) : 0u;
      }
    // rescale the accumulators (rows sl*RS, sl*RS + 1 of each head slot)
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const float c = cs[sl];
      const int i = sl * RS;
#pragma unroll
      for (int vg = 0; vg < 2; ++vg)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[vg][j][i] *= c, acc[vg][j][i + 1] *= c;
    }

    if (quant) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int vg = 0; vg < 2; ++vg) {
          u32x4 B[4];
          dequant_step<IO, BITS, PS_ROW>(smem, ps, 64 * vg + 32 * kt + 8 * g, VC + 8 * (2 * kt + vg), wsh, B);
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) acc[vg][jt] = M::run(pa[kt], B[jt], acc[vg][jt]);
          if (kt == 0 && vg == 1 && tile + 1 < t_end) load_x(tile + 1);
        }
      wave_lds_sync();  // the group words are read before the next tile's are written
    } else {
      // residual values: lane (n, g) of step (kt, vg) needs channels
      // 64vg+4n..64vg+4n+3 of tokens 32kt+8g+{0..7}; rows past the filled
      // ones read 0 (their weights are 0)
      const int r0 = (tile - a.n_groups) * TILE;
      const int n_valid = min(TILE, a.n_residual - r0);
      const int vst = (int)a.vr_st * 2;
      const __amdgpu_buffer_rsrc_t vrb = make_buf(vr + (int64_t)r0 * a.vr_st, (int64_t)(n_valid - 1) * vst + D * 2);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int vg = 0; vg < 2; ++vg) {
          // the lane's row offset is formed here, opaque to the compiler: hoisted
          // out of the tile loop, the 16 offsets of a residual tile would hold
          // (or spill) 16 VGPRs through every quantized tile
          int rb = 8 * g * vst + 8 * n;
          asm volatile("" : "+v"(rb));
          uint2 w[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            w[j] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                 vrb, rb + (32 * kt + j) * vst + 128 * vg, 0, 0));
          u32x4 B[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint2 e = w[2 * i], o = w[2 * i + 1];
            B[0][i] = __builtin_amdgcn_perm(o.x, e.x, 0x05040100u);
            B[1][i] = __builtin_amdgcn_perm(o.x, e.x, 0x07060302u);
            B[2][i] = __builtin_amdgcn_perm(o.y, e.y, 0x05040100u);
            B[3][i] = __builtin_amdgcn_perm(o.y, e.y, 0x07060302u);
          }
#pragma unroll
          for (int jt = 0; jt < 4; ++jt) acc[vg][jt] = M::run(pa[kt], B[jt], acc[vg][jt]);
          if (kt == 0 && vg == 1 && tile + 1 < t_end) load_x(tile + 1);
        }
    }
    };
  Words W0, W1;
  if (t_begin < t_end) issue(W0, t_begin), load_x(t_begin);
  for (int tile = t_begin; tile < t_end; tile += 2) {
    step(tile, W0, W1);
    if (tile + 1 >= t_end) break;
    step(tile + 1, W1, W0);
  }

  // ---------------- this split's records: (acc[D], m in natural-log units, l)
  const float l_head = across_groups_sum(l_part);
  float lh[NREP];
#pragma unroll
  for (int h = 0; h < NREP; ++h)
    lh[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_head), RS * h));
  if (owner) {
#pragma unroll
    for (int sl = 0; sl < HS; ++sl) {
      const int h = h0 + sl;
      if (h >= a.n_rep) continue;
      const int i = sl * RS;
      float* rec = ws_record<D>(a, b, kvh * a.n_rep + h, split, ns);
#pragma unroll
      for (int vg = 0; vg < 2; ++vg)
        *(f32x4*)(rec + 64 * vg + 4 * n) =
            f32x4{acc[vg][0][i] + acc[vg][0][i + 1], acc[vg][1][i] + acc[vg][1][i + 1],
                  acc[vg][2][i] + acc[vg][2][i + 1], acc[vg][3][i] + acc[vg][3][i + 1]};
      if (n == 0) {
        float mh = m_run[0], lv = lh[0];
#pragma unroll
        for (int hh = 1; hh < NREP; ++hh)
          if (h == hh) mh = m_run[hh], lv = lh[hh];
        rec[D] = mh * kLn2;
        rec[D + 1] = lv;
      }
    }
  }
}

}  // namespace tp

// ------------------------------------------------------------------ host side

static bool tp_meta_aligned(const void* p, int64_t sb, int64_t sh, int dt) {
  const int pair = dt == MZ_F32 ? 8 : 4;  // two adjacent entries are read at once
  return ((uintptr_t)p % pair) == 0 && sb % 2 == 0 && sh % 2 == 0;
}

bool tp_supported(const mz_decode_args* a) {
  const int64_t es = a->meta_dtype == MZ_F32 ? 4 : 2;
  // buffer-resource ranges are 32-bit
  const bool fits = (int64_t)a->n_groups * tp::TILE * 2 * (8 * a->bits) < ((int64_t)1 << 31) &&
                    (int64_t)a->n_groups * tp::TILE * 2 * es < ((int64_t)1 << 31);
  const bool aligned = a->v_prefix == 0 || a->v_prefix == a->n_groups * tp::TILE;
  // pass 1 counts the flat tiles of all (batch, kv-head) in 32 bits
  const bool count = (int64_t)a->batch * a->kv_heads * (a->n_groups + (a->n_residual + tp::TILE - 1) / tp::TILE) <
                     ((int64_t)1 << 31);
  return a->bits >= 5 && a->bits <= 8 && a->head_dim == tp::D && a->n_groups > 0 && fits && count && aligned &&
         a->n_rep >= 1 &&
         a->n_rep <= 8 && a->e_key && a->e_value && ((uintptr_t)a->e_key % 16) == 0 &&
         ((uintptr_t)a->e_value % 16) == 0 && ((uintptr_t)a->k_packed % 4) == 0 &&
         ((uintptr_t)a->v_packed % 4) == 0 && a->kp_sb % 4 == 0 && a->kp_sh % 4 == 0 && a->vp_sb % 4 == 0 &&
         a->vp_sh % 4 == 0 && tp_meta_aligned(a->k_mn, a->km_sb, a->km_sh, a->meta_dtype) &&
         tp_meta_aligned(a->k_scale, a->km_sb, a->km_sh, a->meta_dtype) &&
         tp_meta_aligned(a->v_mn, a->vm_sb, a->vm_sh, a->meta_dtype) &&
         tp_meta_aligned(a->v_scale, a->vm_sb, a->vm_sh, a->meta_dtype);
}

static int tp_tiles(const mz_decode_args* a) { return a->n_groups + (a->n_residual + tp::TILE - 1) / tp::TILE; }

int tp_choose_split(const mz_decode_args* a, int* tiles_per_split) {
  const int n_tiles = tp_tiles(a);
  int ns = a->n_split;
  if (ns <= 0) {
    // one wave per split: fill the CUs' 8 resident waves once
    const int64_t units = std::max<int64_t>(1, (int64_t)a->batch * a->kv_heads);
    const int64_t slots = (int64_t)tp::WAVES * device_cu_count();
    ns = (int)((slots + units - 1) / units);
    ns = max(1, min(ns, (n_tiles + 1) / 2));  // at least 2 tiles per split
  }
  ns = max(1, min(ns, n_tiles));
  const int tps = (n_tiles + ns - 1) / ns;
  *tiles_per_split = tps;
  return (n_tiles + tps - 1) / tps;
}

// Bytes of the split records, then the logits (256-byte aligned).
static int64_t tp_records_bytes(const mz_decode_args* a, int ns) {
  const int64_t r = (int64_t)a->batch * a->kv_heads * a->n_rep * ns * (tp::D + 2) * (int64_t)sizeof(float);
  return (r + 255) / 256 * 256;
}

int64_t tp_workspace_bytes(const mz_decode_args* a, int ns) {
  return tp_records_bytes(a, ns) +
         (int64_t)a->batch * a->kv_heads * a->n_rep * tp_tiles(a) * tp::TILE * (int64_t)sizeof(float);
}

template <int IO, int NR, int MW, int BB>
static void tp_launch_one(const mz_decode_args* a, hipStream_t s, float* logits, int n_tiles, int tps, int ns) {
  const int64_t lt = (int64_t)n_tiles * tp::TILE;
  const int64_t total = (int64_t)a->batch * a->kv_heads * n_tiles;
  const int64_t g1 = std::min<int64_t>(device_cu_count(), (total + tp::WAVES_1 - 1) / tp::WAVES_1);
  hipLaunchKernelGGL((tp::logits_kernel<IO, NR, MW, BB>), dim3((unsigned)g1), dim3(tp::NT_1), 0, s, *a, logits,
                     n_tiles, lt);
  const int64_t units = (int64_t)a->batch * a->kv_heads * ns;
  hipLaunchKernelGGL((tp::attend_kernel<IO, NR, MW, BB>), dim3((unsigned)((units + tp::WAVES - 1) / tp::WAVES)),
                     dim3(tp::NT), 0, s, *a, (const float*)logits, n_tiles, lt, tps, ns);
}

template <int IO, int NR, int MW>
static int tp_launch_bits(const mz_decode_args* a, hipStream_t s, float* logits, int n_tiles, int tps, int ns) {
  switch (a->bits) {
    case 5: tp_launch_one<IO, NR, MW, 5>(a, s, logits, n_tiles, tps, ns); break;
    case 6: tp_launch_one<IO, NR, MW, 6>(a, s, logits, n_tiles, tps, ns); break;
    case 7: tp_launch_one<IO, NR, MW, 7>(a, s, logits, n_tiles, tps, ns); break;
    case 8: tp_launch_one<IO, NR, MW, 8>(a, s, logits, n_tiles, tps, ns); break;
    default: return MZ_EUNSUPPORTED;
  }
  return MZ_OK;
}

template <int IO, int NR>
static int tp_launch_nr(const mz_decode_args* a, hipStream_t s, float* logits, int n_tiles, int tps, int ns) {
  return a->meta_dtype == MZ_F32 ? tp_launch_bits<IO, NR, 2>(a, s, logits, n_tiles, tps, ns)
                                 : tp_launch_bits<IO, NR, 1>(a, s, logits, n_tiles, tps, ns);
}

template <int IO>
static int tp_launch_io(const mz_decode_args* a, hipStream_t s, float* logits, int n_tiles, int tps, int ns) {
  // query heads per kv-head of the kernel that runs: n_rep rounded up to a power of two
  switch (a->n_rep <= 1 ? 1 : a->n_rep <= 2 ? 2 : a->n_rep <= 4 ? 4 : a->n_rep <= 8 ? 8 : 0) {
    case 1: return tp_launch_nr<IO, 1>(a, s, logits, n_tiles, tps, ns);
    case 2: return tp_launch_nr<IO, 2>(a, s, logits, n_tiles, tps, ns);
    case 4: return tp_launch_nr<IO, 4>(a, s, logits, n_tiles, tps, ns);
    case 8: return tp_launch_nr<IO, 8>(a, s, logits, n_tiles, tps, ns);
    default: return MZ_EUNSUPPORTED;
  }
}

// Both passes; the records go to the start of the workspace (the combine
// kernel's layout), the logits after them.
int tp_launch_partials(const mz_decode_args* a, hipStream_t s) {
  int tps;
  const int ns = tp_choose_split(a, &tps);
  if (!a->workspace || a->workspace_bytes < tp_workspace_bytes(a, ns)) return MZ_EWORKSPACE;
  float* logits = (float*)((uint8_t*)a->workspace + tp_records_bytes(a, ns));
  const int n_tiles = tp_tiles(a);
  const int st = a->io_dtype == MZ_BF16 ? tp_launch_io<MZ_BF16>(a, s, logits, n_tiles, tps, ns)
                                        : tp_launch_io<MZ_F16>(a, s, logits, n_tiles, tps, ns);
  if (st != MZ_OK) return st;
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MZ_OK : (int)e;
}

}  // namespace mz
