/*
 * vfk.h — C ABI of libvfk, the MI355X (gfx950) encoder-attention kernels.
 *
 * Every GPU entry point:
 *   - takes raw device pointers plus element strides (never torch types),
 *   - enqueues its kernels on the caller's `stream` (a hipStream_t; NULL = the
 *     legacy default stream) and never synchronises it,
 *   - allocates nothing: outputs are provided by the caller,
 *   - returns VFK_OK (0) on success, a negative VFK_ERR_* code for a rejected
 *     argument (message in vfk_last_error()), or a positive hipError_t value
 *     when the HIP launch itself failed.
 * The library keeps no mutable global state besides the thread-local error
 * message (and the per-GPU array of vfk_varlen_meta_noalloc, below), so
 * concurrent calls from several host threads are safe, that one excepted.
 *
 * Strides are in elements. A stride of 0 broadcasts that dimension.
 */
#ifndef VFK_H
#define VFK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define VFK_F32 0
#define VFK_BF16 1
#define VFK_F16 2

/* status codes */
#define VFK_OK 0
#define VFK_ERR_INVALID (-1)     /* shape / pointer / stride rejected      */
#define VFK_ERR_UNSUPPORTED (-2) /* valid request this build does not run  */

/* activation codes for vfk_glu_fwd */
#define VFK_ACT_GELU_ERF 0   /* 0.5 x (1 + erf(x / sqrt 2))                     */
#define VFK_ACT_GELU_TANH 1  /* 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) */
#define VFK_ACT_SILU 2       /* x * sigmoid(x)                                  */
#define VFK_ACT_RELU 3       /* max(x, 0)                                       */

/* A strided tensor of up to 4 dimensions. Unused trailing dims: size 1. */
typedef struct vfk_tensor {
  void* data;
  int32_t dtype;       /* VFK_F32 / VFK_BF16 / VFK_F16 */
  int32_t ndim;
  int64_t size[4];
  int64_t stride[4];   /* in elements */
} vfk_tensor;

/* ------------------------------------------------------------------------ */
/* Library information and host-side helpers (no GPU needed)                  */
/* ------------------------------------------------------------------------ */

/* ABI version; bumped on any signature change. */
int vfk_abi_version(void);

/* Message of the last error raised on this host thread ("" if none). */
const char* vfk_last_error(void);

/* T5 relative-position bucket of each relative position rel[i] = key - query,
 * evaluated with the fp32 formula of
 * models/mt5/mt5_encoder.py:124-148 (T5RelativePositionBias._relative_position_bucket)
 * and its Triton twin kernels/flash_attention_rpb.py:12-54. Host only. */
int vfk_t5_bucket(const int64_t* rel, int32_t* out, int64_t n,
                  int32_t bidirectional, int32_t num_buckets,
                  int32_t max_distance);

/* DeBERTa-v2 log bucket of each relative position rel[i] = query - key,
 * following models/deberta_v2/deberta_v2_encoder.py:70-89
 * (make_log_bucket_position). Host only. */
int vfk_deberta_bucket(const int64_t* rel, int32_t* out, int64_t n,
                       int32_t bucket_size, int32_t max_position);

/* 1 when the clamped DeBERTa index c(d) = clamp(bucket(d) + att_span, 0,
 * 2 att_span - 1) changes by at most 1 per unit of d for |d| <= max_len, else
 * 0 (or a negative VFK_ERR code). The bucket formula of
 * models/deberta_v2/deberta_v2_encoder.py:70-89 jumps by 2 or more when
 * max_relative_positions is small against position_buckets (e.g. 256 / 256).
 * The staged vfk_flash_deberta_fwd kernel and vfk_deberta_fused_fwd need unit
 * steps: otherwise the former takes its per-score gather and the latter
 * returns VFK_ERR_UNSUPPORTED. Span and bucket arguments are derived as in
 * kernels/flash_deberta_attention.py:323, :366-368. Host only. */
int vfk_deberta_unit_steps(int32_t position_buckets, int32_t max_relative_distance,
                           int32_t use_log_bucket, int32_t max_len);

/* ------------------------------------------------------------------------ */
/* Attention                                                                 */
/* ------------------------------------------------------------------------ */

/* T5 relative-position-bias flash attention, forward.
 * Replaces kernels/flash_attention_rpb.py:296-412 (flash_attention_rpb_final)
 * and the Triton kernel at :61-230.
 *   q [B,H,Lq,D], k/v [B,H,Lk,D], out [B,H,Lq,D]   (any strides, D == 64)
 *   rpb_table [num_table_buckets, H] or data == NULL (no bias)
 *   mask: additive mask broadcastable to [B,H,Lq,Lk] or data == NULL
 *   is_decoder != 0: causal + unidirectional buckets.
 * out = softmax(q k^T * softmax_scale + table[bucket(k - q), h] + mask) v */
int vfk_flash_rpb_fwd(const vfk_tensor* q, const vfk_tensor* k,
                      const vfk_tensor* v, const vfk_tensor* rpb_table,
                      int32_t num_buckets, int32_t max_distance,
                      int32_t is_decoder, const vfk_tensor* mask,
                      float softmax_scale, vfk_tensor* out, void* stream);

/* vfk_flash_rpb_fwd over packed sequences (no padding, no mask): sequence s
 * is tokens cu_seqlens[s] .. cu_seqlens[s + 1] - 1 of q, k, v, out [T, H, 64]
 * (16-byte aligned rows, any token / head strides; bf16 or fp16) and attends
 * to its own tokens only, with relative positions inside the sequence. This
 * is the reference's padded call (kernels/flash_attention_rpb.py:296-412 with
 * the [B, 1, 1, L] key mask of models/mt5/mt5_encoder.py:571-576) on the
 * valid rows: the flat mT5 callers (plugins/mt5_gliner/model.py:169-201) run
 * on it without re-padding. cu_seqlens: device int32 [num_seqs + 1];
 * max_seqlen >= every sequence length (rows past it are not computed). */
int vfk_flash_rpb_varlen_fwd(const vfk_tensor* q, const vfk_tensor* k,
                             const vfk_tensor* v, const int32_t* cu_seqlens,
                             int32_t num_seqs, int32_t max_seqlen,
                             const vfk_tensor* rpb_table, int32_t num_buckets,
                             int32_t max_distance, int32_t is_decoder,
                             float softmax_scale, vfk_tensor* out, void* stream);

/* DeBERTa-v2/v3 disentangled flash attention, forward, gathering the bias
 * from precomputed position projections (the reference's interface).
 * Replaces kernels/flash_deberta_attention.py:455-499 (flash_deberta_attention)
 * and the Triton kernel at :144-299.
 *   q [B,H,M,D], k/v [B,H,N,D], out [B,H,M,D] (D == 64)
 *   pos_key [B,H,M,2*att_span] or NULL, pos_query [B,H,N,2*att_span] or NULL
 *   seq_lengths: device int32 [B] or NULL (= all N keys valid)
 * Rows >= seq_lengths[b] of out are written as zeros. */
int vfk_flash_deberta_fwd(const vfk_tensor* q, const vfk_tensor* k,
                          const vfk_tensor* v, const int32_t* seq_lengths,
                          const vfk_tensor* pos_key,
                          const vfk_tensor* pos_query, int32_t causal,
                          float sm_scale, int32_t position_buckets,
                          int32_t max_relative_distance,
                          int32_t use_log_bucket, vfk_tensor* out,
                          void* stream);

/* DeBERTa disentangled attention with the position projections computed in
 * the kernel (no counterpart in the reference; it replaces the two
 * [B,H,L,2S] matmuls at models/deberta_v2/deberta_v2_encoder.py:275-286
 * followed by flash_deberta_attention).
 *   key_rel   [H, 2*att_span, D]  = key_proj(rel_emb) per head   (c2p) or NULL
 *   query_rel [H, 2*att_span, D]  = query_proj(rel_emb) per head (p2c) or NULL
 *   either both as given ([H, >= 2 att_span, 64], any strides) or both
 *   chunk-major [H, 8, 2*att_span, 8], contiguous per head (bf16 / fp16 only):
 *   element [h][c][r][i] = table[h][r][8c + i]; the kernel's operand loads
 *   are then contiguous runs, outputs are identical.
 * score(i,j) = (q_i.k_j + q_i.key_rel[c(i-j)] + k_j.query_rel[c(i-j)]) * sm_scale
 * with c(d) = clamp(bucket(d) + att_span, 0, 2*att_span - 1). */
int vfk_deberta_fused_fwd(const vfk_tensor* q, const vfk_tensor* k,
                          const vfk_tensor* v, const int32_t* seq_lengths,
                          const vfk_tensor* key_rel,
                          const vfk_tensor* query_rel, float sm_scale,
                          int32_t position_buckets,
                          int32_t max_relative_distance,
                          int32_t use_log_bucket, vfk_tensor* out,
                          void* stream);

/* vfk_deberta_fused_fwd over packed sequences (no padding): sequence s is
 * tokens cu_seqlens[s] .. cu_seqlens[s + 1] - 1 of q, k, v, out [T, H, 64]
 * (bf16 / fp16, 16-byte aligned rows, any token / head strides) and attends
 * to its own tokens only, relative positions inside the sequence. It is the
 * padded call with seq_lengths on the valid rows: the flat DeBERTa callers
 * (plugins/deberta_gliner/model.py:166-202,
 * plugins/deberta_gliner2/model.py:124-137) run on it without re-padding.
 * cu_seqlens: device int32 [num_seqs + 1]; max_seqlen >= every sequence
 * length (rows past it are not computed); bucket steps must be unit
 * (vfk_deberta_unit_steps). */
int vfk_deberta_fused_varlen_fwd(const vfk_tensor* q, const vfk_tensor* k,
                                 const vfk_tensor* v, const int32_t* cu_seqlens,
                                 int32_t num_seqs, int32_t max_seqlen,
                                 const vfk_tensor* key_rel, const vfk_tensor* query_rel,
                                 float sm_scale, int32_t position_buckets,
                                 int32_t max_relative_distance, int32_t use_log_bucket,
                                 vfk_tensor* out, void* stream);

/* Copies key_rel and / or query_rel ([H, >= 2 att_span, 64], 16-byte aligned
 * rows, bf16 / fp16; either pair may be NULL) into the chunk-major layout the
 * two fused entry points read fastest, out [H, 8, 2 att_span, 8] with
 * out[h][c][r][i] = rel[h][r][8c + i], in one launch. No counterpart in the
 * reference (its pos_key / pos_query matmuls read the projections as
 * stored). */
int vfk_deberta_rel_chunk_major(const vfk_tensor* key_rel, vfk_tensor* key_out,
                                const vfk_tensor* query_rel, vfk_tensor* query_out,
                                int32_t att_span, void* stream);

/* Varlen (packed) bidirectional attention with optional RoPE and sliding
 * window, for ModernBERT (no counterpart kernel in the reference: it replaces
 * the rotary step and F.scaled_dot_product_attention with the dense O(T^2)
 * masks at models/modernbert/modernbert_encoder.py:236-255 and :491-550).
 *   q/k/v [T,H,D] (any strides, D == 64), out [T,H,D]
 *   cu_seqlens: device int32 [num_seqs + 1]; token t of sequence s has
 *     position t - cu_seqlens[s]
 *   max_seqlen: upper bound of the sequence lengths (sizes the grid)
 *   window < 0: global; window >= 0: key j visible iff |i - j| <= window
 *   rope_cos_sin: NULL (no rotation) or the fp32 table written by
 *     vfk_rope_table with rope_positions >= max_seqlen rows; q and k are then
 *     rotated (non-interleaved halves): k by a pre-pass into the workspace, q
 *     in the attention kernel. q, k and v are never written.
 *   key_valid: device uint8 [T] (0 = key masked) or NULL
 *   workspace: device memory of at least vfk_varlen_attn_workspace_bytes()
 *     bytes, 16-byte aligned (NULL when that is 0); its contents on entry do
 *     not matter. Calls that share a workspace must not overlap.
 * Rows that see no key are written as zeros. */
int vfk_varlen_attn_fwd(const vfk_tensor* q, const vfk_tensor* k,
                        const vfk_tensor* v, const int32_t* cu_seqlens,
                        int32_t num_seqs, int32_t max_seqlen, int32_t window,
                        const float* rope_cos_sin, int32_t rope_positions,
                        const uint8_t* key_valid, float softmax_scale,
                        void* workspace, int64_t workspace_bytes,
                        vfk_tensor* out, void* stream);

/* Workspace size of vfk_varlen_attn_fwd for total_tokens rows (q->size[0]),
 * num_heads heads, num_seqs sequences and max_seqlen: for 16-bit dtypes with
 * RoPE, the rotated and scaled K (head-major, total_tokens * num_heads * 64 * 2
 * bytes rounded up to 256) plus four fp32 row-norm maxima per (head,
 * sequence, 64-key tile), one per 16 rows (num_heads * num_seqs *
 * ceil(max_seqlen / 64) * 16 bytes); else 0. */
int64_t vfk_varlen_attn_workspace_bytes(int32_t dtype, int64_t total_tokens,
                                        int32_t num_heads, int32_t rope,
                                        int32_t num_seqs, int32_t max_seqlen);

/* Packed-sequence metadata from vLLM's flat position ids, on the device
 * (no counterpart kernel in the reference: it replaces the boundary detection
 * of models/modernbert/modernbert_encoder.py:491-516
 * (ModernBertModel._build_seq_block_mask, whose [T, T] masks the varlen
 * attention does not need) and the host-side split of
 * plugins/deberta_gliner/model.py:166-170).
 *   positions: device int32 or int64 [total_tokens] (pos_dtype_bytes 4 or 8)
 *   rule: VFK_SEQ_RESET: a sequence starts at token 0 and at every i with
 *     pos[i] <= pos[i-1] (ModernBERT); VFK_SEQ_ZERO: at token 0 and at every
 *     i with pos[i] == 0 (the GLiNER plugins)
 *   cu_seqlens: device int32 [total_tokens + 1]; entries 0..num_seqs are
 *     written (start of each sequence, then total_tokens)
 *   meta: device int32 [4] = {num_seqs, max_seqlen, bad, total_tokens}; bad
 *     counts breaks in the run of positions (a sequence start whose position
 *     is not 0, or a token whose position is not its predecessor's + 1); it
 *     is 0 exactly when every position equals t - cu_seqlens[s], the position
 *     vfk_varlen_attn_fwd gives token t (the reference's RoPE positions)
 *   workspace: device memory of vfk_varlen_meta_workspace_bytes() bytes,
 *     4-byte aligned; calls that share it must not overlap.
 * Four small launches on `stream`; nothing is read back to the host. */
#define VFK_SEQ_RESET 0
#define VFK_SEQ_ZERO 1
int vfk_varlen_meta(const void* positions, int32_t pos_dtype_bytes,
                    int64_t total_tokens, int32_t rule, int32_t* cu_seqlens,
                    int32_t* meta, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* Workspace size of vfk_varlen_meta: 4 bytes per 1024 tokens. */
int64_t vfk_varlen_meta_workspace_bytes(int64_t total_tokens);

/* vfk_varlen_meta with no workspace argument and no allocation of any kind.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid
 * hipMalloc). Same arguments, kernels and results as vfk_varlen_meta; the
 * per-block counts live in a 64 KiB device array built into the library (one
 * per GPU, held until the process ends), so total_tokens is limited to
 * VFK_NOALLOC_MAX_TOKENS (VFK_ERR_UNSUPPORTED above it). Every call on one GPU
 * shares that array: calls that overlap on one GPU (two streams, two host
 * threads) race and must be serialised by the caller. */
#define VFK_NOALLOC_MAX_TOKENS (16384LL * 1024LL)
int vfk_varlen_meta_noalloc(const void* positions, int32_t pos_dtype_bytes,
                            int64_t total_tokens, int32_t rule, int32_t* cu_seqlens,
                            int32_t* meta, void* stream);

/* Flat rows -> padded batch. Replaces the per-row copy loop of
 * plugins/deberta_gliner/model.py:171-191 (batched_ids[row, :length] =
 * input_ids[start:end] with the rest pad_id).
 *   src: device [T, row_bytes] (rows contiguous); dst: device
 *     [num_seqs, max_len, row_bytes]; sequence b = src rows
 *     cu_seqlens[b] .. cu_seqlens[b+1]-1 goes to dst[b, 0 .. len-1] and
 *     dst[b, len .. max_len-1] is filled with the elem_bytes-wide value
 *     fill_bits (little-endian low bytes)
 *   cu_seqlens: device int32 [num_seqs + 1], non-decreasing, last = T
 *   max_len: >= every sequence length (longer sequences are cut at max_len)
 *   seq_lengths: device int32 [num_seqs] receiving the lengths, or NULL
 * num_seqs <= 65535, max_len * row_bytes < 2^31; row_bytes and both
 * addresses multiples of elem_bytes (1, 2, 4 or 8). */
int vfk_pad_rows(const void* src, int64_t row_bytes, const int32_t* cu_seqlens,
                 int32_t num_seqs, int32_t max_len, int32_t elem_bytes,
                 uint64_t fill_bits, void* dst, int32_t* seq_lengths,
                 void* stream);

/* Padded batch -> flat rows, the inverse of vfk_pad_rows. Replaces
 * torch.cat([encoded[row, :length] ...]) at plugins/deberta_gliner/
 * model.py:197-200. src [num_seqs, max_len, row_bytes], dst [T, row_bytes];
 * padded rows are not read. Same limits as vfk_pad_rows. */
int vfk_unpad_rows(const void* src, int64_t row_bytes,
                   const int32_t* cu_seqlens, int32_t num_seqs,
                   int32_t max_len, void* dst, void* stream);

/* GLiNER span pooler front-end over a packed stream: the per-request
 * gathers of _extract_gliner_reps (poolers/gliner.py:313-347), which the
 * reference runs once per request after split_hidden_states
 * (poolers/gliner.py:201, :219-255). Request s owns stream rows
 * cu_seqlens[s] .. cu_seqlens[s + 1] - 1 (int32 [num_seqs + 1]). status
 * (int32, may be NULL) is set to 1 where the reference raises IndexError and
 * is never cleared by these calls.
 *
 * vfk_gliner_class_index: the class-token positions
 * ((iid == ent_token_id).nonzero(), poolers/gliner.py:317) of every request
 * at once. input_ids int64 [total_tokens]. Writes class_idx int32
 * [total_tokens + 1] (stream indices of the class tokens in order, then
 * total_tokens), class_cu int32 [num_seqs + 1] (request s owns
 * class_idx[class_cu[s] .. class_cu[s + 1] - 1]) and meta int32 [4]
 * (meta[0] = number of class tokens). shift is 1 when the model does not
 * embed the class token itself (class_pos + 1, :318-319), else 0; a class
 * token whose row + shift leaves its request sets status. workspace: at least
 * vfk_gliner_class_workspace_bytes(total_tokens) bytes of device memory. */
int64_t vfk_gliner_class_workspace_bytes(int64_t total_tokens);
int vfk_gliner_class_index(const int64_t* input_ids, int64_t total_tokens,
                           int64_t ent_token_id, int32_t shift,
                           const int32_t* cu_seqlens, int32_t num_seqs,
                           int32_t* class_idx, int32_t* class_cu, int32_t* meta,
                           int32_t* status, void* workspace,
                           int64_t workspace_bytes, void* stream);

/* Prompt rows, tok.index_select(0, class_pos) (poolers/gliner.py:321-324):
 * pe[r] = tok[class_idx[r] + shift] for r < meta[0]. tok [total_tokens,
 * row_bytes] and pe [max_rows, row_bytes], rows 16-byte aligned, row_bytes a
 * multiple of 16; max_rows >= meta[0] (read back by the caller). */
int vfk_gliner_prompt_rows(const void* tok, int64_t row_bytes,
                           int64_t total_tokens, const int32_t* class_idx,
                           const int32_t* meta, int32_t shift,
                           int64_t max_rows, void* pe, void* stream);

/* Word index with first-subtoken pooling (poolers/gliner.py:331-341): among
 * the tokens of request s with words_mask > 0, the first token p of each run
 * of equal word ids w gives word_src[word_cu[s] + w - 1] = p + 1.
 * words_mask int64 [total_tokens]; word_cu int32 [num_seqs + 1] (request s
 * owns text_lengths = word_cu[s + 1] - word_cu[s] words); word_src int32
 * [word_cu[num_seqs]], zero-filled by the caller (0 = no token: a zero row,
 * as in the reference's new_zeros). A word id past its request's text length
 * sets status. Word ids that repeat after another word id in between give
 * unordered duplicate writes, as the reference's indexed assignment does. */
int vfk_gliner_word_index(const int64_t* words_mask, int64_t total_tokens,
                          const int32_t* cu_seqlens, int32_t num_seqs,
                          const int32_t* word_cu, int32_t* word_src,
                          int32_t* status, void* stream);

/* Word rows: we[j] = tok[word_src[j] - 1], or a zero row where
 * word_src[j] == 0, for j < num_words. Same row rules as
 * vfk_gliner_prompt_rows. */
int vfk_gliner_word_rows(const void* tok, int64_t row_bytes,
                         int64_t total_tokens, const int32_t* word_src,
                         int64_t num_words, void* we, void* stream);

/* Span pair rows of the GLiNER span marker (SpanMarkerV0.forward with
 * extract_elements, poolers/gliner.py:40-45, :131-145; called at :286-287):
 * for span s of request r (span_cu[r] <= s < span_cu[r + 1]) over r's
 * L = row_cu[r + 1] - row_cu[r] rows of start_rep / end_rep,
 * out[s] = relu(cat(start_rep[row_cu[r] + i], end_rep[row_cu[r] + j])) with
 * i, j = span_idx[s][0 / 1] * span_mask[s] (the reference multiplies the
 * indices by the mask value, :286) clamped to [0, L - 1].
 * L must be the request's fitted row count: the reference first pads (with
 * zero word rows) or truncates its word rows to target_W =
 * span_idx.size(1) // max_width (:285-286, _fit_length :299-311) and
 * projects those, so row_cu describes the projections of the fitted rows.
 * start_rep, end_rep [num_rows = row_cu[num_requests], row_bytes] and out [num_spans,
 * 2 * row_bytes] of dtype VFK_BF16 / VFK_F16 / VFK_F32, rows 16-byte aligned,
 * row_bytes a multiple of 16; span_idx int64 [num_spans, 2], span_mask int64
 * [num_spans], row_cu / span_cu int32 [num_requests + 1]. ReLU maps negative
 * values to +0 and keeps NaN. A request with L == 0 gives zero rows. */
int vfk_gliner_span_rows(const void* start_rep, const void* end_rep,
                         int64_t row_bytes, int64_t num_rows, int32_t dtype,
                         const int32_t* row_cu,
                         int32_t num_requests, const int64_t* span_idx,
                         const int64_t* span_mask, const int32_t* span_cu,
                         int64_t num_spans, void* out, void* stream);

/* The first layer of SpanMarkerV0's out_project (poolers/gliner.py:141-143,
 * create_projection_layer :26-37: Linear(2D, 4D) then ReLU) on every span
 * without the pair rows: since relu(cat(s, e)) = cat(relu(s), relu(e)), the
 * layer's output for the span (i, j) is relu(a[i] + b[j] + bias) with
 * a = relu(start_rep) W1[:, :D]^T and b = relu(end_rep) W1[:, D:]^T computed
 * once per row (the caller's GEMMs) and bias = b1. out[s] = relu(a[row_cu[r]
 * + i] + b[row_cu[r] + j] + bias), summed in fp32 in that order and rounded
 * once to the dtype, with r, i, j as in vfk_gliner_span_rows (a request with
 * L == 0 gives relu(bias)). a, b [num_rows, row_bytes], bias [row_bytes] or
 * NULL (no bias), out [num_spans, row_bytes], same dtypes and layout rules as
 * vfk_gliner_span_rows. */
int vfk_gliner_span_hidden(const void* a, const void* b, const void* bias,
                           int64_t row_bytes, int64_t num_rows, int32_t dtype,
                           const int32_t* row_cu, int32_t num_requests,
                           const int64_t* span_idx, const int64_t* span_mask,
                           const int32_t* span_cu, int64_t num_spans, void* out,
                           void* stream);

/* RoPE cos/sin table of transformers' ModernBertRotaryEmbedding (default rope,
 * head_dim 64; the module the reference calls at
 * models/modernbert/modernbert_encoder.py:236-242): out[p][f] = (cos, sin) of
 * the fp32 product p * inv_freq[f], inv_freq[f] = 1 / theta^(2f/64), for
 * p < max_positions, f < 32. out: device fp32 [max_positions * 64]. */
int vfk_rope_table(float theta, int32_t max_positions, float* out, void* stream);

/* ColBERT output head (no counterpart kernel in the reference: it replaces
 * the encoder's final LayerNorm, models/modernbert/modernbert_encoder.py:
 * 412-415 and :478, followed by the PyLate Dense projection and the L2
 * normalisation of plugins/moderncolbert/model.py:260-267).
 *   x [T, D]: D a multiple of 256 up to 1024, rows contiguous and 8-byte
 *     aligned; residual [T, D] or NULL (the LayerNorm input is x + residual)
 *   ln_weight, ln_bias [D] or NULL; without ln_weight the rows are projected
 *     as given (no LayerNorm)
 *   weight [N, D] (nn.Linear layout; N = 32, 64, 96 or 128; rows 16-byte
 *     aligned) or the same weight packed by vfk_pack_weight_mfma32
 *     ([N / 32, D / 16, 64, 8]: each wave's weight load is then one
 *     contiguous KiB), bias [N] or NULL
 *   hidden_out [T, D] or NULL: receives the LayerNorm output
 *   out [T, N] = y / max(|y|, 1e-8) per row, y = LN(x + residual) W^T + bias
 * x, weight and outputs share one 16-bit dtype; statistics, products and
 * norms are fp32. */
int vfk_colbert_head_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                         const vfk_tensor* ln_weight, const vfk_tensor* ln_bias,
                         float eps, const vfk_tensor* weight,
                         const vfk_tensor* bias, vfk_tensor* hidden_out,
                         vfk_tensor* out, void* stream);

/* The same head in folded form, for callers that do not need the LayerNorm
 * output (no counterpart in the reference; it computes what
 * vfk_colbert_head_fwd does). With u = x + residual rounded to x's dtype (the
 * encoder's residual sum), mu and rstd its LayerNorm statistics:
 *   y_n = rstd (sum_k u_k W'_nk - mu G_n) + C_n,  out = y / max(|y|, 1e-8)
 * so the raw rows go straight into the matrix instructions and each
 * workgroup (128 tokens) streams the weight through LDS once.
 * vfk_colbert_fold_weight makes the three constants once per weight:
 *   weight [N, D] (rows contiguous; N = 32, 64, 96 or 128; D a multiple of
 *     128 up to 4096), ln_weight gamma, ln_bias beta [D] or NULL (beta needs
 *     gamma), bias b [N] or NULL, all of weight's 16-bit dtype
 *   folded [N / 32, D / 16, 64, 8] of weight's dtype: W'_nk = gamma_k W_nk
 *     rounded (W without gamma), in the operand order of
 *     vfk_pack_weight_mfma32
 *   gsum, cvec fp32 [N] (16-byte aligned): G_n = sum_k W'_nk,
 *     C_n = sum_k beta_k W_nk + b_n
 * vfk_colbert_head_folded_fwd:
 *   x [T, D], residual [T, D] or NULL: rows contiguous, 16-byte aligned
 *   folded, cvec as made above; gsum as made above applies the LayerNorm
 *     (eps as given), NULL projects the rows as given (fold without gamma)
 *   out [T, N] (rows 16-byte aligned), x's dtype; the projection is rounded
 *     to that dtype before its norm is taken, as a 16-bit Linear output is. */
int vfk_colbert_fold_weight(const vfk_tensor* weight, const vfk_tensor* ln_weight,
                            const vfk_tensor* ln_bias, const vfk_tensor* bias,
                            vfk_tensor* folded, vfk_tensor* gsum, vfk_tensor* cvec,
                            void* stream);
int vfk_colbert_head_folded_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                                const vfk_tensor* folded, const vfk_tensor* gsum,
                                const vfk_tensor* cvec, float eps, vfk_tensor* out,
                                void* stream);

/* ------------------------------------------------------------------------ */
/* Memory-bound epilogues                                                    */
/* ------------------------------------------------------------------------ */

/* RoPE with a cos/sin table. Replaces kernels/fused_rope_global.py:18-142
 * (_fused_rope_kernel / fused_rope_apply).
 *   x, out [B,S,H,D], any strides, any even D; cos, sin [B,S,D] (stride 0
 *   broadcasts) in x's dtype or fp32 (then used at fp32)
 * out[..d] = x[d] cos[d] - x[d+D/2] sin[d]        (d <  D/2)
 *          = x[d] cos[d] + x[d-D/2] sin[d]        (d >= D/2)
 * The Python mirror uses it where vfk_rope_qk_fwd's D / alignment limits
 * are not met (e.g. D = 36, 40 or 72 in 16 bits).                       */
int vfk_rope_fwd(const vfk_tensor* x, const vfk_tensor* cos,
                 const vfk_tensor* sin, vfk_tensor* out, void* stream);

/* RoPE of q and k in one launch. Replaces kernels/fused_rope_global.py:145-166
 * (fused_rope_global_apply, one _fused_rope_kernel launch per tensor) and
 * kernels/fused_rope_local.py:11-76. Same formula as vfk_rope_fwd.
 *   q, q_out [B,S,Hq,D]; k, k_out [B,S,Hk,D] or both NULL (q only); last dim
 *   contiguous, 16-byte aligned rows, D a multiple of 16 (16-bit) or 8 (fp32)
 *   cos, sin [B|1,S,D] in q's dtype or fp32 (then used at fp32, as the
 *   reference's kernel promotes mixed operands), 16-byte aligned rows.
 * Each cos/sin chunk is loaded once per thread and applied to several heads
 * of q and k; the result is rounded once to q's dtype. */
int vfk_rope_qk_fwd(const vfk_tensor* q, const vfk_tensor* k,
                    const vfk_tensor* cos, const vfk_tensor* sin,
                    vfk_tensor* q_out, vfk_tensor* k_out, void* stream);

/* LayerNorm over the last dim. Replaces kernels/fused_layernorm.py:19-274.
 *   x, out [rows, n] (row stride, unit column stride); weight/bias [n] or
 *   NULL; optional residual [rows, n]: x := x + residual first, and the sum
 *   is written to residual_out when that is not NULL. */
int vfk_layernorm_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                      const vfk_tensor* weight, const vfk_tensor* bias,
                      float eps, vfk_tensor* out, vfk_tensor* residual_out,
                      void* stream);

/* RMSNorm (T5 / vLLM RMSNorm used at models/mt5/mt5_encoder.py:41,461,471,519):
 * out = x * rsqrt(mean(x^2) + eps) * weight, statistics in fp32. Same
 * residual convention as vfk_layernorm_fwd. */
int vfk_rmsnorm_fwd(const vfk_tensor* x, const vfk_tensor* residual,
                    const vfk_tensor* weight, float eps, vfk_tensor* out,
                    vfk_tensor* residual_out, void* stream);

/* Gated activation out = act(a) * b over [rows, n] (row strides).
 * Replaces kernels/fused_glu_mlp.py:23-104 (act on the first operand) and
 * kernels/ff_fused.py:24-125 (act on `gate`). */
int vfk_glu_fwd(int32_t act, const vfk_tensor* a, const vfk_tensor* b,
                vfk_tensor* out, void* stream);

/* GLU projection with the activation and gate product fused into the GEMM:
 * out[t, f] = act(x[t] . w[f]) * (x[t] . w[I + f]), x [M, K], w [2I, K]
 * (activation-input rows, then gate rows), out [M, I]; fp32 accumulation,
 * the [M, 2I] projection is never written. Replaces the Wi projection plus
 * chunk / act / gate product of models/modernbert/modernbert_encoder.py:157-178
 * (ModernBertMLP.forward up to Wo) and the T5 gated FF's wi_0 / wi_1 products
 * (models/mt5/mt5_encoder.py T5DenseGatedActDense); kernels/fused_glu_mlp.py:61-104
 * is the elementwise part. bf16 / fp16; rows contiguous and 16-byte aligned;
 * K a multiple of 64, I a multiple of 8. */
int vfk_glu_linear_fwd(int32_t act, const vfk_tensor* x, const vfk_tensor* w,
                       vfk_tensor* out, void* stream);

/* Dense projection, bias, residual add and LayerNorm in one kernel:
 *   out = LayerNorm(round(x w^T + bias) + residual) * ln_weight + ln_bias,
 * DeBERTa's post-LN output blocks (DebertaV2SelfOutput.forward and
 * DebertaV2Output.forward, models/deberta_v2/deberta_v2_encoder.py:504-508 and
 * :563-567: dense -> dropout (identity) -> LayerNorm(. + input_tensor)). The
 * projection is rounded to the storage type once, after the bias, as the
 * unfused Linear writes it, and the statistics are fp32 over that value plus
 * the residual, as in vfk_layernorm_fwd; the [M, N] projection is never
 * written.
 *   x [M, K], residual and out [M, N]: one dtype, bf16 or fp16, rows
 *     contiguous, base pointers and row strides 16-byte aligned
 *   w_packed [N / 32, K / 16, 64, 8]: the dense weight [N, K] packed by
 *     vfk_pack_weight_mfma32 (same dtype, contiguous)
 *   bias, ln_weight, ln_bias: contiguous 16-byte aligned [N] of that dtype, or
 *     NULL (zeros, ones, zeros)
 *   N in {256, 512, 768, 1024}; K a positive multiple of 64
 *   residual_out [M, N] or NULL: the sum round(x w^T + bias) + residual,
 *     rounded once, as vfk_layernorm_fwd's residual_out: ModernBERT's
 *     pre-LN layers carry it on as the residual stream (Wo at
 *     models/modernbert/modernbert_encoder.py:258 and :177, the residual
 *     adds at :338-342 and :349-353, then mlp_norm :345 or the next
 *     layer's attn_norm)
 *   out and residual_out may each be the residual itself (same rows: updated
 *     in place), must not overlap x or each other. */
int vfk_dense_residual_layernorm_fwd(const vfk_tensor* x, const vfk_tensor* w_packed,
                                     const vfk_tensor* bias, const vfk_tensor* residual,
                                     const vfk_tensor* ln_weight, const vfk_tensor* ln_bias,
                                     float eps, vfk_tensor* out, vfk_tensor* residual_out,
                                     void* stream);

/* The weight layout vfk_dense_residual_layernorm_fwd and
 * vfk_colbert_head_fwd read: w [N, K] (rows contiguous and 16-byte aligned,
 * N a multiple of 32, K a multiple of 16) -> packed [N / 32, K / 16, 64, 8]
 * with packed[f][s][l][i] = w[32 f + l % 32][16 s + 8 (l / 32) + i], the
 * operand order of the 32x32x16 matrix instruction, so that each wave's
 * operand load is one contiguous KiB. Done once per weight (no counterpart
 * in the reference, whose Linear reads w as stored). */
int vfk_pack_weight_mfma32(const vfk_tensor* w, vfk_tensor* packed, void* stream);

/* The q | k | v projection with the K rotation in the GEMM epilogue: the
 * Wqkv linear of models/modernbert/modernbert_encoder.py:236-242
 * (ModernBertAttention: Wqkv, view [T, 3, H, 64], then the rotary step of
 * kernels/fused_rope_global.py / fused_rope_local.py on q and k) without the
 * [T, 3H*64] projection or a separate K pass.
 *   x [M, K], w [3 * num_heads * 64, K] (q rows, k rows, v rows), bf16/fp16,
 *     rows contiguous and 16-byte aligned, K a multiple of 64
 *   positions: device int32 [M], the rotary position of each token (clamped
 *     into the table)
 *   rope_cos_sin: the fp32 table of vfk_rope_table, rope_positions rows
 *   q_out, v_out [M, num_heads, 64]: x . w^T of the q and v heads, rounded
 *     once (q is not rotated: vfk_varlen_attn_krot_fwd rotates it)
 *   workspace (vfk_qkv_rope_workspace_bytes, 16-byte aligned): the k heads,
 *     rotated in fp32, multiplied by softmax_scale * log2(e) and rounded once,
 *     head-major [num_heads][M][64], then per head the largest row norm of
 *     each 32-token block [num_heads][ceil(M / 32)] fp32: the input of
 *     vfk_varlen_attn_krot_fwd with the same M, heads and softmax_scale. */
int vfk_qkv_rope_linear_fwd(const vfk_tensor* x, const vfk_tensor* w,
                            const int32_t* positions, const float* rope_cos_sin,
                            int32_t rope_positions, int32_t num_heads, float softmax_scale,
                            vfk_tensor* q_out, vfk_tensor* v_out, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* Workspace bytes of vfk_qkv_rope_linear_fwd for M tokens and num_heads
 * heads: M * num_heads * 128 rounded up to 256, plus num_heads *
 * ceil(M / 32) * 4. */
int64_t vfk_qkv_rope_workspace_bytes(int64_t tokens, int32_t num_heads);

/* vfk_varlen_attn_fwd with RoPE for K already rotated by
 * vfk_qkv_rope_linear_fwd (krot = its workspace, same tokens, heads and
 * softmax_scale; positions t - cu_seqlens[s]): no K pre-pass. q and v
 * [T, H, 64] bf16/fp16; q is rotated in the kernel with rope_cos_sin. */
int vfk_varlen_attn_krot_fwd(const vfk_tensor* q, const vfk_tensor* v, const void* krot,
                             int64_t krot_bytes, const int32_t* cu_seqlens, int32_t num_seqs,
                             int32_t max_seqlen, int32_t window, const float* rope_cos_sin,
                             int32_t rope_positions, const uint8_t* key_valid,
                             float softmax_scale, vfk_tensor* out, void* stream);

/* Activation out = act(x) over [rows, n] (row strides). Replaces the
 * intermediate activation of models/deberta_v2/deberta_v2_encoder.py:535-550
 * (DebertaV2Intermediate, ACT2FN[hidden_act]) in inference. */
int vfk_act_fwd(int32_t act, const vfk_tensor* x, vfk_tensor* out, void* stream);

/* out = a + b, elementwise over [rows, n] (row strides).
 * Replaces kernels/fused_dropout_residual.py:10-104 in inference mode. */
int vfk_residual_add(const vfk_tensor* a, const vfk_tensor* b,
                     vfk_tensor* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* VFK_H */
