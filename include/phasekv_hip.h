/*
 * phasekv_hip.h — C ABI of the MI355X (gfx950) PhaseKV Stage-B decode path.
 *
 * Plain pointers, sizes and a HIP stream handle (hipStream_t passed as void*);
 * no PyTorch types.  Every entry point returns an int status (PK_OK on success),
 * never throws or aborts across the ABI, and launches asynchronously on the
 * given stream.  pk_last_error() returns a thread-local message for the most
 * recent failure of the calling thread.
 *
 * Tensor conventions:
 *   - fp16 / bf16 values are passed as uint16_t bit patterns.
 *   - "packed" buffers are uint8 with the quantized axis moved last and
 *     ceil(len / (8 / bits)) bytes per row, code j of byte k at bits
 *     [j*bits, (j+1)*bits) (LSB first), zero codes in the tail byte.
 *   - "scale"/"mins" buffers are fp16 [rows, ceil(len / group_size)].
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   see the comment above each entry point.
 */
#ifndef PHASEKV_HIP_H
#define PHASEKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
#define PK_OK 0
#define PK_ERR_INVALID (-1)     /* invalid argument: the Python side raises ValueError */
#define PK_ERR_RUNTIME (-2)     /* HIP runtime / launch failure: RuntimeError */

/* ---- dtypes of quantize_pack inputs ---------------------------------------- */
#define PK_DTYPE_F16 0
#define PK_DTYPE_BF16 1
#define PK_DTYPE_F32 2

/* ---- segment kinds of the decode work list --------------------------------- */
#define PK_SEG_KIVI 0    /* K per-channel: packed [.., Hkv, hd, ceil(S/vpb)], meta [.., Hkv, hd, ceil(S/kgs)];
                            V per-token:   packed [.., Hkv, S, ceil(hd/vpb)], meta [.., Hkv, S, ceil(hd/vgs)] */
#define PK_SEG_TOKEN 1   /* K and V both per-token (legacy layout): like V above */
#define PK_SEG_FP16 2    /* uncompressed fp16 K/V [.., Hkv, S, hd], token stride given, hd contiguous */

#define PK_MAX_SEGMENTS_PER_LAUNCH 8

/* Last error message of the calling thread ("" if none). */
const char* pk_last_error(void);

/* Library version string. */
const char* pk_version(void);

/* Device properties the planner uses.  Replaces _device_sm_count
 * (src/phasekv/kernels/attention_triton.py:599-601). */
int pk_device_info(int device, int* cu_count, int* lds_bytes_per_cu, int* wave_size,
                   int* l2_bytes);

/* ---- packing (src/phasekv/kernels/packing.py) ------------------------------- */

/* pack_low_bits (packing.py:41-64): codes uint8 [rows, length] contiguous ->
 * out uint8 [rows, ceil(length / vpb)].  bits in {2, 4, 8}. */
int pk_pack_low_bits(const uint8_t* codes, int64_t rows, int64_t length, int bits,
                     uint8_t* out, void* stream);

/* unpack_low_bits (packing.py:67-79): packed uint8 [rows, packed_len] contiguous ->
 * out uint8 [rows, length], length <= packed_len * vpb. */
int pk_unpack_low_bits(const uint8_t* packed, int64_t rows, int64_t packed_len, int bits,
                       int64_t length, uint8_t* out, void* stream);

/* quantize_pack (packing.py:115-155).  x is any-strided (element strides) with
 * ndim <= 8 dims of the given dtype; axis in [0, ndim); group_size already
 * resolved by the caller to gs = min(group_size, len) (or len).  Outputs are
 * contiguous in the moved layout: out_packed [rows, ceil(len/vpb)],
 * out_scale/out_mins fp16 [rows, ceil(len/gs)], rows = prod(shape) / len in
 * the original order of the remaining dims.  For axis == ndim - 2 only, the
 * layout flags PK_LAYOUT_META_TRANSPOSED / PK_LAYOUT_CODES_TRANSPOSED store
 * scale / mins resp. the codes with those arrays' last two dims transposed
 * ([rows / D, ceil(len/gs), D] and [rows / D, ceil(len/vpb), D], D =
 * shape[ndim - 1]).  Bit-exact with the reference. */
int pk_quantize_pack(const void* x, int dtype, int ndim, const int64_t* shape,
                     const int64_t* strides, int axis, int bits, int group_size,
                     uint8_t* out_packed, uint16_t* out_scale, uint16_t* out_mins,
                     int layout, void* stream);

/* The cache's K/V block pack in one launch (_pack_kv, src/phasekv/phasekv_cache.py:101-107:
 * quantize_pack(K, bits, axis=-2) and quantize_pack(V, bits, axis=-1), groups of
 * 32).  k, v: fp16 [batch, num_kv_heads, seq_len, head_dim] contiguous, 16-byte
 * aligned; seq_len and head_dim multiples of 32.  Outputs as pk_quantize_pack
 * writes them with both layout flags for K: k_packed [B, H, seq_len/vpb,
 * head_dim], k_scale / k_mins [B, H, seq_len/32, head_dim]; v_packed [B, H,
 * seq_len, head_dim/vpb], v_scale / v_mins [B, H, seq_len, head_dim/32]; code
 * buffers 4-byte aligned.  Bit-identical to the two pk_quantize_pack calls. */
int pk_quantize_pack_kv(const uint16_t* k, const uint16_t* v, int batch, int num_kv_heads,
                        int64_t seq_len, int head_dim, int bits, uint8_t* k_packed,
                        uint16_t* k_scale, uint16_t* k_mins, uint8_t* v_packed,
                        uint16_t* v_scale, uint16_t* v_mins, void* stream);

/* unpack_dequantize (packing.py:158-175): inverse of pk_quantize_pack.  Writes
 * fp16 out contiguous in the ORIGINAL layout orig_shape (ndim <= 8), with
 * n_groups = number of groups per row stored in scale/mins. */
int pk_unpack_dequantize(const uint8_t* packed, const uint16_t* scale, const uint16_t* mins,
                         int ndim, const int64_t* orig_shape, int axis, int bits,
                         int group_size, int64_t n_groups, uint16_t* out, void* stream);

/* ---- decode attention (src/phasekv/kernels/attention_triton.py) ------------- */

/* One segment of the decode work list.  All element strides; the two innermost
 * dims of packed / meta buffers are contiguous.  For PK_SEG_FP16 the K/V data
 * pointers are fp16 and k_meta / v_meta strides are unused; tok_stride is the
 * element stride between tokens (hd is contiguous). */
/* Storage of a KIVI K segment (packed along tokens; logical shapes codes
 * [..., head_dim, bytes] and scale / min [..., head_dim, groups]).  Channel major
 * is the reference's contiguous layout.  The transposed storage keeps every
 * channel of one token byte (codes) or one group (scale / min) together,
 * [..., bytes, head_dim] and [..., groups, head_dim] contiguous, so that a few
 * consecutive tokens of all channels are one contiguous run.  pk_quantize_pack
 * writes either (for the second-to-last axis); the decode kernels read either. */
#define PK_META_CHANNEL_MAJOR 0
#define PK_META_GROUP_MAJOR 1
#define PK_CODES_CHANNEL_MAJOR 0
#define PK_CODES_TOKEN_MAJOR 1
/* pk_quantize_pack layout flags */
#define PK_LAYOUT_META_TRANSPOSED 1
#define PK_LAYOUT_CODES_TRANSPOSED 2

typedef struct pk_segment {
  int32_t kind;            /* PK_SEG_* */
  int32_t length;          /* tokens in the segment (max over the batch) */
  int32_t k_bits, v_bits;  /* 2/4/8 (ignored for FP16) */
  int32_t k_group, v_group;/* group sizes as stored in PackedTensor.group_size */
  int32_t splits;          /* requested splits (work items along the tokens), 0 = planner */
  int32_t split_len;       /* tokens per split; with splits > 0 exactly `splits` splits of
                              split_len tokens are launched (trailing ones may be empty, like
                              attention_triton.py:227-240); 0 = split_len = ceil(len / splits) */
  int32_t k_meta_layout;   /* KIVI K scale/min storage: PK_META_CHANNEL_MAJOR or PK_META_GROUP_MAJOR */
  int32_t k_data_layout;   /* KIVI K code storage: PK_CODES_CHANNEL_MAJOR or PK_CODES_TOKEN_MAJOR */
  const int32_t* seq_lens; /* device [batch] valid tokens per row, or NULL (= length) */
  const void* k_data; const uint16_t* k_scale; const uint16_t* k_mins;
  const void* v_data; const uint16_t* v_scale; const uint16_t* v_mins;
  int64_t k_data_bstride, k_data_hstride;
  int64_t k_meta_bstride, k_meta_hstride;
  int64_t v_data_bstride, v_data_hstride;
  int64_t v_meta_bstride, v_meta_hstride;
  int64_t tok_stride;      /* FP16 only */
} pk_segment;

/* One decode problem: q [batch, Hq, hd] fp16 (hd contiguous) against a list of
 * segments of the same kv heads.  Query head h reads kv head h / (Hq / Hkv)
 * (reference.py:61-69).  Scores use 1/sqrt(hd) (attention_triton.py:631). */
typedef struct pk_decode_problem {
  int32_t batch, num_q_heads, num_kv_heads, head_dim;
  const uint16_t* q;
  int64_t q_bstride, q_hstride;
  const pk_segment* segments;  /* host array */
  int32_t num_segments;
  int32_t flags;               /* PK_FLAG_* */
  /* Segments kept in device memory (pk_segment_table_write): entries [0, table_count) of
   * `table` are attended besides `segments`, all in the same partials launch.  The
   * entries must describe segments of this problem's batch, kv heads and head_dim.
   * table_bits: the widest K or V code among them (2 or 4); 0 when table_count is 0. */
  const void* table;
  int32_t table_count;
  int32_t table_bits;
} pk_decode_problem;

#define PK_FLAG_GENERIC_KERNEL 1   /* use the general-shape kernel even where the MFMA one applies */
#define PK_FLAG_REQUIRE_MFMA 2     /* fail (PK_ERR_INVALID) where the MFMA kernel does not apply */

/* ---- device-resident segment table ------------------------------------------
 * The cache's packed segments as descriptors in device memory, so that a decode
 * step over any number of them is one partials launch with a fixed-size argument
 * block.  The reference keeps a Python list of cold segments, one appended per
 * cooling event (src/phasekv/phasekv_cache.py:322-340), and launches once per
 * segment (src/phasekv/kernels/attention_triton.py:662-665).  A table is caller
 * memory of pk_segment_table_entry_bytes() bytes per entry; entries are written
 * on the stream (a small kernel: no host memory is read by the GPU, so the write
 * can be captured in a graph) and read by decode launches ordered after it. */

/* Bytes of one table entry. */
size_t pk_segment_table_entry_bytes(void);

/* Write entries [first, first + count) of `table` from segments[0 .. count).  Each
 * must be a KIVI segment in the storage quantize_pack writes (token-major K codes,
 * group-major K scale / min, 16-byte aligned code rows, V scale / min rows aligned to
 * head_dim / 32 halves), K and V widths of 2 or 4 bits, V groups of 32 and K groups
 * of 32 or a single group; otherwise PK_ERR_INVALID and nothing is written.
 * head_dim: 64 or 128.  A decode attends each entry with one wave per segment, so
 * the table suits many short segments (the cold segments of lazy cooling). */
int pk_segment_table_write(void* table, int32_t first, int32_t count,
                           const pk_segment* segments, int32_t head_dim, void* stream);

/* Bytes of split-K workspace pk_decode_partials needs for this problem: the
 * partials m, l [batch*Hq][splits] and acc [batch*Hq][splits][hd] fp32, each
 * region 256-byte aligned, in that order.  Replaces the torch.empty
 * partial buffers of _kivi_layer_partial (attention_triton.py:624-626). */
int pk_decode_workspace_size(const pk_decode_problem* p, size_t* bytes, int32_t* total_splits);

/* Split-K partial pass over every segment in one launch per
 * PK_MAX_SEGMENTS_PER_LAUNCH segments.  Replaces the per-segment
 * _decode_attn_kivi_split_kernel launches of fused_phasekv_decode
 * (attention_triton.py:514-596, 662-665), the legacy per-token kernels
 * (attention_triton.py:24-92, 145-213) and the FP16 hot partial
 * (attention_triton.py:285-297). */
int pk_decode_partials(const pk_decode_problem* p, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Log-sum-exp combine of the partials (attention_triton.py:257-266, 300-307).
 * If out is non-NULL writes the normalized fp16 output [batch, Hq, hd]
 * contiguous; if out_m/out_l/out_acc are non-NULL writes the unnormalized
 * (m, l, acc) fp32 [batch*Hq], [batch*Hq], [batch*Hq, hd]. */
int pk_decode_combine(const pk_decode_problem* p, const void* workspace, uint16_t* out,
                      float* out_m, float* out_l, float* out_acc, void* stream);

/* pk_decode_partials followed by pk_decode_combine(out) on the same stream: the
 * whole decode step of every segment in two launches (one partial launch per
 * PK_MAX_SEGMENTS_PER_LAUNCH segments).  Replaces fused_phasekv_decode's
 * per-segment launches, _reduce_splits and _merge_partials
 * (attention_triton.py:643-669).  Calls sharing a workspace must be ordered
 * (same stream). */
int pk_fused_decode(const pk_decode_problem* p, void* workspace, size_t workspace_bytes,
                    uint16_t* out, void* stream);

/* pk_fused_decode without a caller workspace and without any allocation: the
 * split-K partials go to a file-scope device array of PK_NOALLOC_SCRATCH_BYTES
 * (16 MiB) that each GPU the library runs on holds until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Problems whose workspace (pk_decode_workspace_size)
 * exceeds the array fail with PK_ERR_INVALID before any launch.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race; calls ordered on one stream do not. */
#define PK_NOALLOC_SCRATCH_BYTES (16u << 20)
int pk_fused_decode_noalloc(const pk_decode_problem* p, uint16_t* out, void* stream);

/* Merge n partials per row: m, l [rows, n] and acc [rows, n, hd] fp32 contiguous.
 * Writes normalized fp16 out [rows, hd] (_merge_partials, attention_triton.py:300-307)
 * or, when out is NULL, unnormalized (m, l, acc) (_reduce_splits,
 * attention_triton.py:257-266). */
int pk_merge_partials(const float* m, const float* l, const float* acc, int64_t rows,
                      int32_t n, int32_t head_dim, uint16_t* out, float* out_m,
                      float* out_l, float* out_acc, void* stream);

/* One set of split partials for pk_merge_partial_sets: m, l [rows, n] and acc
 * [rows, n, head_dim] fp32 contiguous (what pk_decode_partials writes; acc 16-byte
 * aligned).  Output row (o, i) reads the set's row o * outer_stride + i * inner_stride,
 * which must be < rows. */
#define PK_MAX_PARTIAL_SETS 4
typedef struct pk_partial_set {
  const float* m;
  const float* l;
  const float* acc;
  int64_t rows;
  int32_t n;
  int32_t pad_;
  int64_t outer_stride;
  int64_t inner_stride;
} pk_partial_set;

/* Log-sum-exp merge, per output row (o, i) of an [outer, inner] grid, of every
 * partial of 1..PK_MAX_PARTIAL_SETS sets whose rows are numbered differently: the
 * input-chunk attention merges its packed-tier launch (rows (head, token)) with its
 * causal chunk launch (rows (token, head)) this way, with no transpose in between.
 * Writes normalized fp16 out [outer, inner, head_dim] or, when out is NULL,
 * unnormalized (m, l, acc).  The merge of _merge_partials (attention_triton.py:300-307)
 * applied to what the reference computes with one decode call per chunk token
 * (qwen2_attention.py:100-106); the fused chunk itself has no reference counterpart. */
int pk_merge_partial_sets(const pk_partial_set* sets, int32_t nsets, int64_t outer,
                          int64_t inner, int32_t head_dim, uint16_t* out, float* out_m,
                          float* out_l, float* out_acc, void* stream);

/* ---- FP16 hot window lifecycle (src/phasekv/phasekv_cache.py) -------------- */

/* Largest number of hot tokens one cooling step can take. */
#define PK_COOL_MAX_AGED 4096

/* Write one generated token's K and V (fp16 [batch, num_kv_heads, 1, head_dim],
 * element strides of batch and head given, head_dim contiguous) into row
 * `position` of the hot window (fp16 [batch, num_kv_heads, capacity, head_dim],
 * same strides for K and V, head_dim contiguous).  Fails if position is outside
 * [0, capacity).  Replaces PhaseKVCache.append_hot / _append_token
 * (src/phasekv/phasekv_cache.py:292-301, 405-422). */
int pk_append_hot(const uint16_t* k_src, const uint16_t* v_src, int64_t k_bstride,
                  int64_t k_hstride, int64_t v_bstride, int64_t v_hstride, uint16_t* hot_k,
                  uint16_t* hot_v, int64_t hot_bstride, int64_t hot_hstride,
                  int64_t hot_tstride, int batch, int num_kv_heads, int head_dim,
                  int64_t position, int64_t capacity, void* stream);

/* Write `count` consecutive tokens' K and V (fp16 [batch, num_kv_heads, count,
 * head_dim], element strides of batch, head and token given, head_dim
 * contiguous) into rows position .. position + count - 1 of the hot window
 * (layout as pk_append_hot).  Fails unless 0 <= position and position + count
 * <= capacity.  Replaces the per-token append_hot loop over an input chunk
 * (src/phasekv/qwen2_attention.py:100-106, phasekv_cache.py:344-390). */
int pk_append_hot_rows(const uint16_t* k_src, const uint16_t* v_src, int64_t k_bstride,
                       int64_t k_hstride, int64_t k_tstride, int64_t v_bstride,
                       int64_t v_hstride, int64_t v_tstride, uint16_t* hot_k, uint16_t* hot_v,
                       int64_t hot_bstride, int64_t hot_hstride, int64_t hot_tstride,
                       int batch, int num_kv_heads, int head_dim, int64_t position,
                       int64_t count, int64_t capacity, void* stream);

/* One decode token's rotate_half rotary embedding fused with the window append.
 * Inputs are of `dtype` (PK_DTYPE_F16 or PK_DTYPE_BF16).  q ([batch][num_q_heads
 * * head_dim], batch stride q_bstride) is rotated into q_out (fp16 [batch,
 * num_q_heads, head_dim], contiguous); K (same layout with num_kv_heads, batch
 * stride kv_bstride, shared by V) is rotated into row `position` of the fp16 hot
 * window and V is copied there.  cos / sin: [batch][head_dim], batch stride
 * cs_bstride (0: one row for every batch row).  Each output is
 * x * cos + rotate_half(x) * sin evaluated in `dtype` (each product and the sum
 * rounded to it), then rounded to fp16: bit-identical to that expression on
 * tensors of `dtype` followed by `.to(float16)`.  Replaces apply_rotary_pos_emb,
 * the fp16 casts and append_hot in the adapters' decode branch
 * (src/phasekv/qwen2_attention.py:89-92, 77; examples/llama_phasekv_adapter.py:71-74, 89). */
int pk_rope_append_hot(const uint16_t* q, int64_t q_bstride, const uint16_t* k,
                       const uint16_t* v, int64_t kv_bstride, const uint16_t* cos,
                       const uint16_t* sin, int64_t cs_bstride, int dtype, uint16_t* q_out,
                       uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride,
                       int64_t hot_hstride, int64_t hot_tstride, int batch, int num_q_heads,
                       int num_kv_heads, int head_dim, int64_t position, int64_t capacity,
                       void* stream);

/* One lazy cooling step of every (batch, kv head) row of the hot window, in one
 * launch: rank the oldest `aged` tokens by the float32 L2 norm of their V rows,
 * keep the `keep` highest (equal norms: the earlier token; NaN above every
 * number), write the kept K and V rows in token order to out_k / out_v (fp16
 * [batch, num_kv_heads, keep, head_dim] contiguous) and their token indices to
 * out_index (int64 [batch, num_kv_heads, keep], may be NULL), then move rows
 * [aged, hot_len) to [0, hot_len - aged).  keep == aged keeps every token
 * without ranking.  The caller packs out_k / out_v with pk_quantize_pack into
 * the new cold segment.  Replaces PhaseKVCache._cool_aged_tokens and _gather_kv
 * (src/phasekv/phasekv_cache.py:322-340, 110-114). */
int pk_cool_hot(uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride, int64_t hot_hstride,
                int64_t hot_tstride, int batch, int num_kv_heads, int head_dim,
                int64_t hot_len, int64_t aged, int64_t keep, uint16_t* out_k,
                uint16_t* out_v, int64_t* out_index, void* stream);

/* 1 if pk_cool_pack_hot takes this window (the row's hot window and the
 * packing statistics fit one workgroup's LDS and head_dim % 8 == 0), else 0. */
int pk_cool_pack_supported(int64_t hot_len, int head_dim, int64_t aged, int64_t keep,
                           int group_size);

/* pk_cool_hot and the packing of the new cold segment in one launch: the kept
 * rows are quantized with `bits` and `group_size` exactly as pk_quantize_pack
 * would (K along the kept tokens, group min(group_size, keep); V along head_dim,
 * group min(group_size, head_dim)) and written in the storage pk_quantize_pack
 * gives them: K codes [batch, num_kv_heads, ceil(keep / vpb), head_dim] and
 * K scale / mins [batch, num_kv_heads, n_groups, head_dim] (its transposed
 * layout), V codes [batch, num_kv_heads, keep, ceil(head_dim / vpb)] and V scale
 * / mins [batch, num_kv_heads, keep, n_groups], all contiguous.  Hot buffers in
 * 16-byte pieces (16-byte aligned, strides multiples of 8).  Fails without a
 * launch when pk_cool_pack_supported is 0.  Replaces _cool_aged_tokens with its
 * _pack_kv (src/phasekv/phasekv_cache.py:322-340, 101-107). */
int pk_cool_pack_hot(uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride, int64_t hot_hstride,
                     int64_t hot_tstride, int batch, int num_kv_heads, int head_dim,
                     int64_t hot_len, int64_t aged, int64_t keep, int bits, int group_size,
                     uint8_t* k_packed, uint16_t* k_scale, uint16_t* k_mins, uint8_t* v_packed,
                     uint16_t* v_scale, uint16_t* v_mins, int64_t* out_index, void* stream);

/* ---- prefill prompt selection (src/phasekv/prompt_tier.py) ----------------- */

/* Observation-window votes of one layer: votes[b, kv, j] (fp32 [batch,
 * num_kv_heads, kv_len] contiguous) = sum over the kv head's query heads (in
 * order) of the sum over the last min(obs_window, q_len) query rows (in order) of
 * attention[b, h, row, j], in float32.  attention is [batch, num_q_heads, q_len,
 * kv_len] of dtype PK_DTYPE_* with element strides strides[4].  Replaces
 * observation_votes + aggregate_to_kv_heads (src/phasekv/hetero_cache.py:55-77). */
int pk_prompt_votes(const void* attention, int dtype, int64_t batch, int64_t num_q_heads,
                    int64_t q_len, int64_t kv_len, const int64_t* strides, int num_kv_heads,
                    int obs_window, float* votes, void* stream);

/* Kept prompt positions of each of `rows` vote rows (fp32 [rows, kv_len]): the
 * sink positions [0, sink), then the select_k best candidates of [sink,
 * recent_start) after 1-D pooling of their votes (pool_mode 0: max over the
 * window, padding never wins; 1: average with zero padding, divided by
 * pool_kernel; window = pool_kernel positions starting pool_kernel / 2 before the
 * candidate; pool_kernel <= 1: no pooling; equal scores: the earlier position;
 * NaN above every number), then [recent_start, kv_len): int64 keep [rows,
 * sink + select_k + kv_len - recent_start], ascending.  Replaces the selection of
 * select_prompt_indices (src/phasekv/prompt_tier.py:43-75) with pool_scores and
 * topk_per_head (src/phasekv/hetero_cache.py:80-94, 147-157). */
int pk_select_prompt(const float* votes, int64_t rows, int64_t kv_len, int64_t sink,
                     int64_t recent_start, int64_t select_k, int pool_kernel, int pool_mode,
                     int64_t* keep, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PHASEKV_HIP_H */
