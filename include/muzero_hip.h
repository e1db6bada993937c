/*
 * muzero_hip.h — C ABI of the MI355X (gfx950) muZero KV-cache hot path.
 *
 * One shared library, libmuzero_hip.so, built by hipcc for gfx950.  Every
 * entry point takes plain device pointers, explicit sizes and strides, dtype
 * enums and a hipStream_t (0 = the default stream), launches asynchronously
 * and returns an int status (0 = success, negative = argument error, or the
 * positive hipError_t of a failed launch).  Nothing here allocates device
 * memory; callers own every buffer.  Calls are thread-safe, except
 * muzero_decode_attention_noalloc: its calls on one device share that
 * device's static scratch array, so calls that overlap there (from two
 * threads, or on two streams) race.  The library's
 * only mutable state is per device and process: each device's compute-unit
 * count and whether a kernel's dynamic-LDS limit has been raised on it (the
 * general decode kernels, the qk / av kernels with more than 64 KB of LDS),
 * filled on the first call on that device (idempotent, so concurrent first
 * calls are harmless), and the static decode scratch array that
 * muzero_decode_attention_noalloc uses instead of a workspace (each device
 * holds its own copy while the library is loaded).
 *
 * Reference boundary being replaced: the pybind11 module returned by
 * load_mu_zero_cuda_extension() (muzero/kernels/loader.py:37-94, 1862-1880),
 * whose functions take torch tensors and launch on the current stream.
 */
#ifndef MUZERO_HIP_H
#define MUZERO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is an opaque pointer; declared here so C/FFI callers need no HIP headers. */
typedef struct ihipStream_t* mz_stream_t;

/* dtype enums */
enum { MZ_F32 = 0, MZ_BF16 = 1, MZ_F16 = 2 };

/* status codes (besides 0 and positive hipError_t values) */
enum {
  MZ_OK = 0,
  MZ_EINVAL = -1,        /* bad pointer, size, stride or dtype */
  MZ_EUNSUPPORTED = -2,  /* valid for the reference but not built here (e.g. head_dim) */
  MZ_EWORKSPACE = -3,    /* workspace too small */
  MZ_ESCRATCH = -4       /* the call needs more than the static decode scratch (muzero_decode_attention_noalloc) */
};

const char* muzero_version(void);
const char* muzero_strerror(int status);

/*
 * Quantize + bit-pack rows of 64 values (one group per row).
 * Replaces: quantize(grouped, packed_q, mn, scale, bits, alpha, eps)
 *   (muzero/kernels/loader.py:40-42, host :1290-1322; algorithm
 *    muzero/quantizer.py:161-202).
 * x[r*x_row_stride + i] (x_dtype) -> packed[r*packed_row_stride + 0..8*bits-1],
 * mn[r*meta_stride], scale[r*meta_stride] (meta_dtype).
 * `table`: compander table for (alpha, x_dtype) built by the host (see
 * muzero_amd/tables.py): fp32 thresholds for MZ_F32 input, the 16-bit ratio
 * table for MZ_BF16 / MZ_F16 input.  Codes and metadata are bit-identical to
 * the reference torch quantizer on the same input.
 */
int muzero_quantize_rows(const void* x, int x_dtype, int64_t nrows, int64_t x_row_stride,
                         uint8_t* packed, int64_t packed_row_stride,
                         void* mn, void* scale, int meta_dtype, int64_t meta_stride,
                         int bits, float eps, const void* table, mz_stream_t stream);

/*
 * Quantize a key block [B, H, T, D] (T a multiple of 64, last dim contiguous,
 * strides in elements) into the reference key layout: one group per channel
 * over 64 consecutive tokens.
 * Replaces: MuZeroCacheLayer._quantize_key_block (muzero/cache/layer.py:271-285),
 * including its permute+contiguous copy (done here in LDS).
 * Output group (b, h, s, d) goes to packed[b*p_sb + h*p_sh + s*D*qb + d*qb]
 * and mn/scale[b*m_sb + h*m_sh + s*D + d], qb = 8*bits.
 */
int muzero_quantize_keys(const void* keys, int x_dtype, int B, int H, int T, int D,
                         int64_t x_sb, int64_t x_sh, int64_t x_st,
                         uint8_t* packed, int64_t p_sb, int64_t p_sh,
                         void* mn, void* scale, int meta_dtype, int64_t m_sb, int64_t m_sh,
                         int bits, float eps, const void* table, mz_stream_t stream);

/*
 * Quantize a value block [B, H, T, D] into the reference value layout: one
 * group per token over 64 consecutive channels, D zero-padded to a multiple
 * of 64 (ng = ceil(D/64) groups per token).
 * Replaces: MuZeroCacheLayer._quantize_value_block (muzero/cache/layer.py:287-301).
 * Output group (b, h, t, j) goes to packed[b*p_sb + h*p_sh + t*ng*qb + j*qb]
 * and mn/scale[b*m_sb + h*m_sh + t*ng + j].
 */
int muzero_quantize_values(const void* values, int x_dtype, int B, int H, int T, int D,
                           int64_t x_sb, int64_t x_sh, int64_t x_st,
                           uint8_t* packed, int64_t p_sb, int64_t p_sh,
                           void* mn, void* scale, int meta_dtype, int64_t m_sb, int64_t m_sh,
                           int bits, float eps, const void* table, mz_stream_t stream);

/*
 * Dequantize packed rows back to 64 values each (fp32 math, no FMA
 * contraction, expm1 from the host-built table `e_table`).
 * Replaces: dequantize(packed_q, mn, scale, output, bits, alpha)
 *   (muzero/kernels/loader.py:43-45, host :1324-1358; algorithm
 *    muzero/quantizer.py:229-255).
 * Bit-identical to the reference torch dequantizer except for groups stored
 * with scale 0 (all-zero input): like the reference CUDA kernel
 * (loader.py:201) the scale is clamped to 1e-8 instead of producing NaN.
 */
int muzero_dequantize_rows(const uint8_t* packed, int64_t nrows, int64_t packed_row_stride,
                           const void* mn, const void* scale, int meta_dtype, int64_t meta_stride,
                           void* out, int out_dtype, int64_t out_row_stride,
                           int bits, const float* e_table, mz_stream_t stream);

/*
 * Logits of one query token per (batch, q-head) against a packed key prefix.
 * Replaces: qk(query, packed_q, mn, scale, output, bits, alpha,
 *   num_key_value_groups, scaling) (muzero/kernels/loader.py:46-49, host
 *   :1360-1503, kernel :389-450), the first step of the reference's default
 *   decode path (muzero/cache/attention.py:186-211).
 * query [B, Hq, 1, D] (q_sb, q_sh; Hq = kv_heads * n_rep), packed_K
 * [B, Hkv, >=n_groups, D, qb] (kp_sb, kp_sh in bytes, multiples of 8; the
 * pointer 8-byte aligned), K_mn / K_scale [B, Hkv, >=n_groups, D] (km_sb,
 * km_sh) -> logits [B, Hq, 64*n_groups] (o_sb, o_sh; last dim contiguous):
 * logit = (sum_d q[d] * x[d]) * scaling, x the fp32 dequantized key (the
 * reference's value exactly, muzero/quantizer.py:229-255, from the host-built
 * expm1 table e_key), summed in fp32, rounded once to io_dtype.
 * head_dim <= 256, n_rep <= 16 (else MZ_EUNSUPPORTED).
 */
typedef struct mz_qk_args {
  int batch, kv_heads, n_rep, head_dim, bits, n_groups;
  int meta_dtype, io_dtype;
  float scaling;
  const void* query; int64_t q_sb, q_sh;
  const uint8_t* k_packed; int64_t kp_sb, kp_sh;
  const void* k_mn; const void* k_scale; int64_t km_sb, km_sh;
  const float* e_key;
  void* logits; int64_t o_sb, o_sh;
} mz_qk_args;
int muzero_qk(const mz_qk_args* args, mz_stream_t stream);

/*
 * Attention-weighted sum of a packed value prefix.
 * Replaces: av(attn_weights, packed_q, mn, scale, output, bits, alpha,
 *   num_key_value_groups, group_size) (muzero/kernels/loader.py:50-53, host
 *   :1505-1687, kernel :677-751), the third step of the reference's default
 *   decode path (muzero/cache/attention.py:248-272).
 * weights [B, Hq, n_tokens] (w_sb, w_sh; last dim contiguous; io_dtype),
 * packed_V [B, Hkv, >=n_tokens, ng, qb] (vp_sb, vp_sh in bytes, multiples of
 * 8; the pointer 8-byte aligned; ng = ceil(head_dim / 64)), V_mn / V_scale
 * [B, Hkv, >=n_tokens, ng] (vm_sb, vm_sh) -> out [B, Hq, head_dim] (o_sb,
 * o_sh): out = sum_t w[t] * x[t], x the fp32 dequantized value, summed in
 * fp32 (deterministically: no atomics), rounded once to io_dtype.
 * head_dim <= 256, n_rep <= 16 (else MZ_EUNSUPPORTED).
 */
typedef struct mz_av_args {
  int batch, kv_heads, n_rep, head_dim, bits, n_tokens;
  int meta_dtype, io_dtype;
  const void* weights; int64_t w_sb, w_sh;
  const uint8_t* v_packed; int64_t vp_sb, vp_sh;
  const void* v_mn; const void* v_scale; int64_t vm_sb, vm_sh;
  const float* e_value;
  void* out; int64_t o_sb, o_sh;
} mz_av_args;
int muzero_av(const mz_av_args* args, mz_stream_t stream);

/*
 * Decode attention of one query token per (batch, q-head) over a packed
 * key/value prefix of 64*n_groups tokens followed by n_residual dense tokens.
 * Replaces the decode hook's quantized path: qk + softmax + av + dense
 * residual merge (muzero/cache/attention.py:48-295 with the kernels
 * qk/av/prefix_decode_chunked of muzero/kernels/loader.py:46-84), as one
 * split-over-tokens kernel plus a cross-split log-sum-exp combine.
 * Key/value prefix layouts are the reference cache layouts
 * (muzero/cache/layer.py:271-301): packed_K [B,Hkv,>=n_groups,D,qb],
 * K_mn/K_scale [B,Hkv,>=n_groups,D]; packed_V [B,Hkv,>=64*n_groups,ng,qb],
 * V_mn/V_scale [B,Hkv,>=64*n_groups,ng].  Residual K/V: [B,Hkv,R,D] strided
 * views (last dim contiguous).  Strides are in elements, except packed
 * tensors (bytes).  mask: optional additive fp32 [B, L] (L = 64*n_groups+R),
 * row stride mask_sb.  Output [B, Hq, D] (out_sb, out_sh) in out_dtype
 * (io_dtype, i.e. the reference's output dtype, or fp32).
 */
typedef struct mz_decode_args {
  int batch, kv_heads, n_rep, head_dim, bits;
  int n_groups, n_residual;
  int meta_dtype, io_dtype;
  int out_dtype;  /* io_dtype, or MZ_F32 for an unrounded fp32 output */
  float scaling;
  const void* query; int64_t q_sb, q_sh;
  const uint8_t* k_packed; int64_t kp_sb, kp_sh;
  const void* k_mn; const void* k_scale; int64_t km_sb, km_sh;
  const uint8_t* v_packed; int64_t vp_sb, vp_sh;
  const void* v_mn; const void* v_scale; int64_t vm_sb, vm_sh;
  const void* k_res; int64_t kr_sb, kr_sh, kr_st;
  const void* v_res; int64_t vr_sb, vr_sh, vr_st;
  const float* mask; int64_t mask_sb;
  const float* e_key; const float* e_value;
  /* (P, N) fold tables for alpha_key / alpha_value (bits 1 to 7): pairs of
   * fp16 (P - 1/2, N - 1/2) packed in uint32 (P in the low half), row = zero
   * level, column = code; 16 x 16 for bits 1 to 4 (the pair (0, 0) beyond 2^bits - 1),
   * 2^bits x 64 for 5 and 6 bits, 128 x 128 for 7 bits; see
   * muzero_amd/tables.py ("fold1" .. "fold7").  Needed by the fold fast path;
   * may be null (the generic path is used then).  7 bits: the fold path
   * needs fold_k == fold_v (one alpha for keys and values). */
  const void* fold_k; const void* fold_v;
  void* out; int64_t out_sb, out_sh;
  void* workspace; int64_t workspace_bytes;
  int n_split;      /* 0 = let the library choose */
  int kernel_path;  /* MZ_PATH_AUTO, or MZ_PATH_EXACT / _FOLD / _CODEBOOK / _GENERAL (below) */
  /* The compander alphas the expm1 and fold tables were built for.  Recorded
   * for the caller; the kernels read every table value from e_key / e_value /
   * fold_k / fold_v and do not read these. */
  float alpha_key, alpha_value;
  /* Quantized value tokens when they differ from the 64*n_groups quantized
   * key tokens (logq_compatible_layout flushes values per token,
   * muzero/cache/layer.py:389-396): 64*n_groups <= v_prefix <= 64*n_groups
   * + n_residual; v_packed / v_mn / v_scale then hold v_prefix tokens and
   * v_res holds the 64*n_groups + n_residual - v_prefix tokens after them.
   * 0 = aligned prefixes (v_prefix = 64*n_groups).  The fold kernel needs
   * aligned prefixes; a misaligned call runs the general kernel. */
  int v_prefix;
} mz_decode_args;

/* Kernel paths of muzero_decode_attention.  Three kernels:
 *  - codebook: attends with the reference's dequantize-then-attend values
 *    (every dequantized value rounded to the layer dtype, bit for bit);
 *    1- to 4-bit codes, head_dim 128, aligned prefixes, n_rep 1 to 8 (other
 *    counts than 1, 2, 4, 8 run the kernel built for the next larger one),
 *    and 5-bit codes with one expm1 table for keys and values (e_key ==
 *    e_value) and n_rep 1 to 4;
 *  - fold: the reference's fused-kernel values (fp32 dequantized values,
 *    up to the fp16 rounding of its shifted (P, N) table entries); bits 1 to
 *    7, head_dim 64 or 128, aligned prefixes, n_rep 1 to 8, fold tables
 *    given, at 7 bits one table for keys and values;
 *  - two-pass: the dequantize-then-attend values for 5- to 8-bit codes
 *    (keys' logits with the key table in LDS, then softmax and values with
 *    the value table); head_dim 128, aligned prefixes, n_rep 1 to 8; its
 *    logits (4 bytes per query head and token) live in the workspace after
 *    the split records, so it always runs split kernels + combine;
 *  - general: the dequantize-then-attend values, every width and layout.
 * AUTO and EXACT run the codebook kernel where it applies; else AUTO runs
 * the fold kernel where it applies; else both run the two-pass kernel where
 * it applies, else the general one; FOLD, CODEBOOK and GENERAL force that
 * kernel (a forced fold or codebook kernel that does not take the
 * arguments is MZ_EUNSUPPORTED). */
enum { MZ_PATH_AUTO = 0, MZ_PATH_EXACT = 1, MZ_PATH_FOLD = 2, MZ_PATH_CODEBOOK = 3, MZ_PATH_GENERAL = 4 };

/* Bytes of workspace muzero_decode_attention needs for these arguments
 * (and the split count it will use, written to *n_split_out if non-null). */
int64_t muzero_decode_workspace_bytes(const mz_decode_args* args, int* n_split_out);

/* 1 if muzero_decode_attention runs the fold kernel for these arguments, 0 if
 * the exact-dequantize kernel, -1 if the arguments are rejected.  An
 * introspection helper with no counterpart in the reference (its dispatcher,
 * loader.py:1360-1687, picks kernels internally); used by tests and the
 * benchmark to report which kernel they measured. */
int muzero_decode_uses_fold(const mz_decode_args* args);
/* The kernel muzero_decode_attention runs for these arguments: 0 the general
 * exact-dequantize kernel, 1 the fold kernel, 2 the codebook kernel, 3 the
 * two-pass kernel; -1 if the arguments are rejected (or a forced kernel does
 * not take them).  An introspection helper like muzero_decode_uses_fold. */
int muzero_decode_kernel(const mz_decode_args* args);
int muzero_decode_attention(const mz_decode_args* args, mz_stream_t stream);

/* The two launches of muzero_decode_attention, for callers that time or merge
 * them separately.  (When the fold kernel runs with a single split,
 * muzero_decode_attention launches only that kernel, which then writes `out`
 * itself; these two entry points always go through the workspace.)  muzero_decode_partials writes one (acc[D], m, l) fp32
 * record per (batch, q-head, split) into the workspace, laid out
 * [B][Hq][n_split][D + 2]; muzero_decode_combine merges the splits of each
 * (batch, q-head) with a log-sum-exp reduction and writes `out`.
 * Replaces: prefix_decode_chunked + its reduce kernel
 *   (muzero/kernels/loader.py:66-84, kernels :1146-1285), extended to the
 *   residual window and every bit width. */
int muzero_decode_partials(const mz_decode_args* args, mz_stream_t stream);
int muzero_decode_combine(const mz_decode_args* args, mz_stream_t stream);

/*
 * Online-softmax state of a packed prefix: the fused prefix decode that
 * returns (acc, m, l) instead of the normalized output, for the caller to
 * merge with its own dense tail.
 * Replaces: prefix_decode(query, K..., V..., output_accum, output_m,
 *   output_l, alpha_key, alpha_value, num_key_value_groups, scaling) and
 *   prefix_decode_chunked(..., partial_accum, partial_m, partial_l,
 *   output_accum, output_m, output_l, ...) (muzero/kernels/loader.py:54-84,
 *   host :1689-1858, kernels :1046-1285), whose caller merges the residual
 *   window in torch (muzero/cache/attention.py:91-177).  The reference builds
 *   them for 4 bits only; here every width 1-8 (the kernel muzero_decode_attention
 *   would run for these arguments).
 * args: a decode call over the packed prefix alone (n_residual = 0, aligned
 * value prefix), with its workspace (muzero_decode_workspace_bytes of args
 * with n_split set to n_chunks when n_chunks > 0).  Writes, per (b, h):
 * m = the maximum of the scaled (and masked) logits, l = sum_t exp(s_t - m),
 * acc[0..D) = sum_t exp(s_t - m) * v_t (fp32, v_t the dequantized value), to
 * acc[b*acc_sb + h*acc_sh + c], m / l[b*ml_sb + h].  With n_chunks > 0 the
 * prefix is cut into n_chunks runs of ceil(n_groups / n_chunks) groups (the
 * reference's chunks) and each run's own (acc, m, l) also goes to part_acc
 * [B*Hq][n_chunks][D], part_m / part_l [B*Hq][n_chunks] (contiguous); runs
 * past the end of the prefix hold acc = 0, m = -inf, l = 0.
 */
typedef struct mz_prefix_state_args {
  float* acc; int64_t acc_sb, acc_sh;
  float* m; float* l; int64_t ml_sb;
  float* part_acc; float* part_m; float* part_l;
  int n_chunks;  /* 0: the library's split choice, no partials written */
} mz_prefix_state_args;
int muzero_decode_prefix_state(const mz_decode_args* args, const mz_prefix_state_args* state, mz_stream_t stream);

/*
 * muzero_decode_attention without a caller workspace: a split call keeps its
 * partial records in a static device array of MZ_DECODE_SCRATCH_BYTES inside
 * the library (one per device, held until the process ends); args->workspace
 * and args->workspace_bytes are ignored.  Allocates nothing, so it serves
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  Returns MZ_ESCRATCH,
 * launching nothing, when a split call's muzero_decode_workspace_bytes(args)
 * exceeds the array (a single-split call of the other kernels uses no
 * workspace); a two-pass call whose logits and records exceed it runs the
 * general kernel instead (the same dequantize-then-attend values, summed in
 * another order).  Every call on a device shares that device's array (the last call's
 * records stay in it; each call writes every record it reads), so calls that
 * overlap on one device, on different streams or threads, race.  Same
 * results as muzero_decode_attention with a workspace, bit for bit (except
 * for the two-pass calls above that fall back to the general kernel).
 * The first call on a device does one-time runtime set-up there (the
 * scratch array's address, a kernel's LDS limit): a caller that captures
 * the call in a HIP graph makes one call on that device before the capture
 * begins.
 * No counterpart in the reference; it is for callers that cannot allocate.
 */
#define MZ_DECODE_SCRATCH_BYTES (8u << 20)
int muzero_decode_attention_noalloc(const mz_decode_args* args, mz_stream_t stream);

/*
 * Decode-step prologue of one attention layer for a single new token: per
 * head RMSNorm of q and k (Qwen3's q_norm / k_norm; omitted when both weights
 * are null), rotary embedding q*cos + rotate_half(q)*sin (transformers'
 * apply_rotary_pos_emb), the new key and value rows written into the cache
 * layer's residual window, and the query written as the decode-attention
 * query.  Replaces the per-op torch work of the patched attention forward
 * (muzero/integrations/transformers_patch.py:402-431 keeps the model's own
 * norm, rope and cache.update there) with one launch.  q [B, Hq, D], k / v
 * [B, Hkv, D] (the projections with the token dimension dropped), cos / sin
 * [B, D] (cs_sb = 0 broadcasts one row), norm weights [D]; outputs q_out
 * [B, Hq, D] and the residual rows k_dst / v_dst [B, Hkv, D].  Strides in
 * elements, last dimension contiguous; head_dim 64 or 128; bf16 or fp16.
 * The norm's mean of squares is an fp32 wave reduction: normalized values can
 * differ from torch's in the last bit of the io dtype.  No counterpart in the
 * reference's extension: the reference leaves these ops to the model.
 */
typedef struct mz_prologue_args {
  int batch, q_heads, kv_heads, head_dim, io_dtype;
  const void* q; int64_t q_sb, q_sh;
  const void* k; int64_t k_sb, k_sh;
  const void* v; int64_t v_sb, v_sh;
  const void* cos; const void* sin; int64_t cs_sb;
  const void* q_norm_w; const void* k_norm_w; float eps;
  void* q_out; int64_t qo_sb, qo_sh;
  void* k_dst; int64_t kd_sb, kd_sh;
  void* v_dst; int64_t vd_sb, vd_sh;
} mz_prologue_args;
int muzero_decode_prologue(const mz_prologue_args* args, mz_stream_t stream);

/*
 * Streaming-read probe: reads bytes [0, bytes) of src once (16-byte aligned,
 * bytes a multiple of 16; src may be null when bytes is 0) and XOR-folds them, 32-bit word by word, into
 * out[0 .. n_out) (one word per workgroup, n_out workgroups, 1..65535; the
 * XOR of all n_out words is the XOR of every 32-bit word of the buffer).
 * Measures the read bandwidth a streaming kernel attains on the device, the
 * figure the decode kernels' rates are reported against beside the published
 * peak.  No counterpart in the reference: a measurement utility.
 */
int muzero_stream_read(const void* src, int64_t bytes, uint32_t* out, int n_out, mz_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MUZERO_HIP_H */
