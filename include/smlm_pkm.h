/*
 * smlm_pkm.h -- C ABI of the MI355X (gfx950) product-key-memory lookup.
 *
 * These entry points replace the forward GPU kernels of re133/sparse-memory-lm (smlm/kernels.py, Triton) and
 * the torch einsum that feeds them (smlm/pkm.py).  Every function:
 *   - takes plain device pointers and sizes (no framework types), plus the HIP stream to launch on
 *     (`hipStream_t` passed as `void*`; NULL = the null stream);
 *   - never allocates, frees, synchronises or reads device memory from the host, so a call can be recorded
 *     into a hipGraph by stream capture;
 *   - returns SMLM_OK (0) or a negative smlm_status; the message of the last failure on the calling thread is
 *     returned by smlm_pkm_last_error().
 * Buffers are caller-owned, dense and row-major.  Shapes use the reference's names: N tokens, H heads, NK
 * sub-keys per half (table rows = NK^2), knn lookups per head, K = H*knn lookups per token, D value width.
 */
#ifndef SMLM_PKM_H
#define SMLM_PKM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum smlm_status {
  SMLM_OK = 0,
  SMLM_EINVAL = -1,       /* bad argument: null pointer, shape, dtype or stride */
  SMLM_EUNSUPPORTED = -2, /* valid request outside what the kernels implement */
  SMLM_EHIP = -3          /* the HIP runtime reported an error at launch */
} smlm_status;

typedef enum smlm_dtype {
  SMLM_F32 = 0,
  SMLM_BF16 = 1,
  SMLM_F16 = 2,
  SMLM_I8 = 3,   /* int8 row-quantised table: codes (rows, D) int8 + (rows,) fp16 scales */
  SMLM_Q4 = 4,   /* 4-bit row-quantised table: (rows, D/2) bytes + (rows,) fp16 scales */
  SMLM_I32 = 5,
  SMLM_I64 = 6
} smlm_dtype;

/* Library version string, e.g. "smlm_pkm 0.1.0 gfx950". */
const char *smlm_pkm_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char *smlm_pkm_last_error(void);

/*
 * Device address of a value table (or its scales) kept in pinned host memory (hipHostMalloc).  Replaces the
 * staging path of OffloadTable.bag (smlm/offload.py:57-76: unique rows -> CPU fetch -> pinned staging -> compact
 * device table) for tables held in host RAM (HostTable, smlm/offload.py:79-92): the table-reading entry points
 * (smlm_pkm_bag, smlm_pkm_select_bag) accept the returned address and read the rows over the host link, with no
 * synchronisation, so the call can be captured in a graph.  Host-side only (no device work); fails with
 * SMLM_EINVAL for pageable, device or unknown memory.
 */
int smlm_host_table_pointer(const void *host, void **device);

/*
 * Sub-key scores.  Replaces ProductKeyMemory.subkey_scores (smlm/pkm.py:117-123), the two
 *   s1 = einsum("nhd,hkd->nhk", q[..., :half], keys[:, 0]);  s2 = einsum(..., q[..., half:], keys[:, 1])
 * calls that feed pk_select (smlm/pkm.py:197).
 *   q     (N, H, 2*half) of `dtype`, row n starting at q + n*q_row_stride elements (q_row_stride >= H*2*half)
 *   keys  (H, 2, NK, half) of `dtype`, dense
 *   s1,s2 (N, H, NK) of `dtype` (bf16: fp32 accumulation rounded to nearest even)
 * dtype: SMLM_BF16 (MFMA bf16) or SMLM_F32 (MFMA fp32).  half % 8 == 0 (bf16) / half % 4 == 0 (fp32).
 */
int smlm_pkm_score(const void *q, int64_t q_row_stride, const void *keys, int dtype, int64_t N, int H, int NK,
                   int half, void *s1, void *s2, void *stream);

/*
 * Product-key selection.  Replaces pk_select (smlm/kernels.py:214-226, kernel _pk_select_kernel 146-177) and
 * the torch get_indices + softmax path (smlm/pkm.py:125-136, 205-208):
 *   per (n, h): top-knn of s1[n,h,:] and of s2[n,h,:] (ties -> lower sub-key index), candidates (i, j) with
 *   (i+1)(j+1) <= knn scored as dtype(v1[i] + v2[j]), top-knn of those (ties -> lower table index
 *   i1*NK + i2), softmax in fp32.
 *   s1,s2   (N, H, NK) of `dtype` (SMLM_BF16 or SMLM_F32)
 *   scores  (N, H, knn) of `dtype`, descending
 *   idx     (N, H, knn) int64 table rows in [0, NK^2)
 *   w       (N, H, knn) fp32 softmax weights
 * NK in [knn, 65536]; knn in [1, 128] (the shapes the reference's torch path takes, smlm/pkm.py:48-53).
 */
int smlm_pkm_select(const void *s1, const void *s2, int dtype, int64_t N, int H, int NK, int knn, void *scores,
                    int64_t *idx, float *w, void *stream);

/*
 * Selection fused with the value bag, for any batch (decode steps and prompts): the work of smlm_pkm_select followed by
 * smlm_pkm_bag on its (idx, w) viewed as (N, H*knn), in one launch (one workgroup per token), with identical results.
 * Replaces pk_select + bag_infer of smlm/pkm.py:197-223 (kernels.py:214-226, 364-378).
 *   s1, s2 (N, H, NK) of dtype; table / table_dtype / rows / D / scales / pre / out / out_dtype as smlm_pkm_bag;
 *   scores, idx, w: optional (NULL = not written) copies of the selection, as smlm_pkm_select writes them.
 * H <= 4; NK and knn as smlm_pkm_select; a table row must be whole 16-byte chunks, at most 2*H*64 of them (the
 * bag's additions follow the row-slot layout of smlm_pkm_bag whatever the workgroup's thread count).
 */
int smlm_pkm_select_bag(const void *s1, const void *s2, int dtype, int64_t N, int H, int NK, int knn,
                        const void *table, int table_dtype, int64_t rows, int D, const uint16_t *scales,
                        const uint16_t *pre, void *out, int out_dtype, void *scores, int64_t *idx, float *w,
                        void *stream);

/* Bytes of the static device array that smlm_pkm_lookup_noalloc keeps its sub-key scores in (one per GPU). */
#define SMLM_LOOKUP_SCRATCH_BYTES (8u << 20)

/*
 * No counterpart in the reference.  For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): the decode lookup smlm_pkm_score followed by
 * smlm_pkm_select_bag on the same arguments, with identical results, but with the sub-key score rows s1, s2
 * that those two calls exchange kept in a static device array of SMLM_LOOKUP_SCRATCH_BYTES instead of
 * caller-provided buffers.  The caller passes the inputs (q, keys as smlm_pkm_score; table, scales, pre as
 * smlm_pkm_select_bag) and the output out (N, D) of out_dtype.  Nothing is allocated or freed.
 *   Limit: 2 * N * H * NK * sizeof(dtype) (+ 256 bytes of alignment) <= SMLM_LOOKUP_SCRATCH_BYTES, e.g. N <= 128
 *   for bf16 scores at H = 4, NK = 4096; larger requests fail with SMLM_EUNSUPPORTED before any launch.
 *   The stream must belong to the current device.  The first call on a device looks up the array's address on
 *   that device (hipGetSymbolAddress): make it outside stream capture.  All calls on one GPU share its array:
 *   calls that overlap on one GPU (different streams, or host threads) race on it.
 */
int smlm_pkm_lookup_noalloc(const void *q, int64_t q_row_stride, const void *keys, int dtype, int64_t N, int H,
                            int NK, int half, int knn, const void *table, int table_dtype, int64_t rows, int D,
                            const uint16_t *scales, const uint16_t *pre, void *out, int out_dtype, void *stream);

/*
 * Weighted value bag.  Replaces bag_forward (smlm/kernels.py:229-237) and bag_infer (smlm/kernels.py:364-378):
 *   out[n, :] = sum_{j<K} w[n, j] * row(idx[n, j])        (fp32 accumulation)
 * with row() = table row for SMLM_F32 / SMLM_BF16 tables and scale[r] * code[r, :] for SMLM_I8 / SMLM_Q4 tables
 * (the lookup weight is multiplied by the row scale first, as kernels.py:328-335 does for q4).
 *   idx     (N, K) of idx_dtype (SMLM_I64 or SMLM_I32), rows in [0, rows)
 *   w       (N, K) fp32
 *   table   (rows, D) f32/bf16, (rows, D) int8 codes, or (rows, D/2) q4 bytes (byte i: column i in the low
 *           nibble, column i + D/2 in the high nibble, each stored as code + 8)
 *   scales  (rows,) fp16 bits for SMLM_I8 / SMLM_Q4, else NULL
 *   pre     (N, D) bf16 bits or NULL; if given, out *= bf16(silu(pre)) (smlm/pkm.py:213-224 swilu epilogue)
 *   out     (N, D) of out_dtype (SMLM_F32, or SMLM_BF16 rounded to nearest even)
 * An index outside [0, rows) does not fault: that token's whole output row is written as NaN.
 */
int smlm_pkm_bag(const void *idx, int idx_dtype, const float *w, int64_t N, int K, const void *table,
                 int table_dtype, int64_t rows, int D, const uint16_t *scales, const uint16_t *pre, void *out,
                 int out_dtype, void *stream);

/*
 * Row quantisation of a value table for the inference bag.  Replaces quantize_q4 (smlm/kernels.py:280-300)
 * and gives the int8 scheme of scripts/quantize_table_eval.py:55-61 a device implementation:
 *   m = the row's value of largest magnitude (first on ties); d = fp16(m / lo) (1 if that is 0);
 *   code = clamp(round_half_even(w / d), lo, hi), with (lo, hi) = (-128, 127) for SMLM_I8, (-8, 7) for SMLM_Q4.
 *   src     (rows, D) of src_dtype (SMLM_F32 or SMLM_BF16)
 *   codes   (rows, D) int8 for SMLM_I8; (rows, D/2) bytes for SMLM_Q4 (D even)
 *   scales  (rows,) fp16 bits
 */
int smlm_pkm_quantize(const void *src, int src_dtype, int64_t rows, int D, int kind, void *codes,
                      uint16_t *scales, void *stream);

/*
 * Single-token decode attention over a static KV cache.  Replaces, for T = 1 with a preallocated cache, the
 * attention of smlm/model.py:90-107 after the qkv projection: RoPE on the new q and k (model.py:63-78, the two
 * halves of each head rotated), the cache append (model.py:94-98, here a write at a device-side position) and
 * scaled dot-product attention over positions 0..pos (model.py:100-106), in one launch per layer.
 *   qkv       (B, 3*H*head_dim) bf16, row b at qkv + b*qkv_row_stride: [q | k | v], each (H, head_dim)
 *   rope_cos/rope_sin  (rope_len, head_dim/2) of rope_dtype (SMLM_F32 or SMLM_BF16)
 *   pos       device int64 scalar: the new token's position (also its cache slot)
 *   k_cache, v_cache   (B, H, max_len, head_dim) bf16, written at slot pos
 *   out       (B, H*head_dim) bf16
 * head_dim in {16, 32, 64, 128}.  A pos outside [0, min(max_len, rope_len)) writes no cache slot and NaN output.
 */
int smlm_decode_attention(const void *qkv, int64_t qkv_row_stride, const void *rope_cos, const void *rope_sin,
                          int rope_dtype, int rope_len, const int64_t *pos, void *k_cache, void *v_cache, int64_t B,
                          int H, int head_dim, int max_len, void *out, void *stream);

/*
 * smlm_decode_attention followed by the attention's output projection (smlm/model.py:107, self.wo), per head:
 *   parts[b, h, n] = sum_d bf16(y[b, h, d]) * wo[n, h*head_dim + d]   (fp32, n < n_out)
 * with y the attention output smlm_decode_attention would write.  The sum over h, bf16(sum_h parts[b, h, :]), is
 * the projection (fp32 accumulation, one rounding); the RMSNORM_PARTS prologue of smlm_decode_linear adds it to
 * the residual stream, so the projection needs no launch of its own.
 *   wo     (n_out, >= H*head_dim) bf16 rows at wo + n*wo_row_stride (nn.Linear.weight), 16-byte aligned
 *   parts  (B, H, n_out) fp32, dense
 * Other arguments and the out-of-range position (NaN parts) as smlm_decode_attention.
 */
int smlm_decode_attention_proj(const void *qkv, int64_t qkv_row_stride, const void *rope_cos, const void *rope_sin,
                               int rope_dtype, int rope_len, const int64_t *pos, void *k_cache, void *v_cache,
                               int64_t B, int H, int head_dim, int max_len, const void *wo, int64_t wo_row_stride,
                               int n_out, float *parts, void *stream);

/*
 * SwiGLU activation of the dense FFN.  Replaces `a, b = w13(x).chunk(2, -1); F.silu(a) * b` of
 * smlm/model.py:110-118 (after the w13 projection) in one launch, with the reference's bf16 roundings:
 *   out[m, c] = bf16( bf16(silu(a[m, c])) * b[m, c] ),  a = in[m, :hidden], b = in[m, hidden:2*hidden]
 *   in   (M, 2*hidden) bf16, row m at in + m*in_row_stride;  out (M, hidden) bf16 dense.  hidden % 8 == 0.
 */
int smlm_swiglu(const void *in, int64_t in_row_stride, void *out, int64_t M, int hidden, void *stream);

/*
 * The FFN up-projection of a prompt pass with the SwiGLU activation in its epilogue: replaces self.w13(x) followed
 * by F.silu(a) * b of smlm/model.py:110-118 (SwiGLU.forward) for bf16 activations and weights.
 *   x (M, K) bf16 rows, w13 (2*hidden, K) bf16 (nn.Linear weight: a rows then b rows), out (M, hidden) bf16:
 *   out[m, j] = bf16(bf16(silu(a)) * b), a = bf16(x[m] . w13[j]), b = bf16(x[m] . w13[hidden + j]) with fp32
 *   accumulation (the bf16 projection's roundings followed by smlm_swiglu's).
 * K a multiple of 64, hidden a multiple of 64; 16-byte aligned rows, strides in elements.
 */
int smlm_linear_swiglu(const void *x, int64_t x_row_stride, const void *w13, int64_t w_row_stride, int64_t M, int K,
                       int hidden, void *out, int64_t out_row_stride, void *stream);

/*
 * A projection of a prompt pass, out = bf16(x W^T + bias) with fp32 accumulation (the bias, if any, added in
 * fp32): replaces the nn.Linear calls self.wqkv(x), self.wo(y) and self.w2(h) of smlm/model.py:92, 107, 118 and
 * swilu_proj / value_proj of smlm/pkm.py:213-224 for bf16 activations and weights.  With scale and shift (fp32,
 * N each) every output becomes bf16(bf16(x W^T + bias) * scale + shift): query_proj followed by the eval-mode
 * query BatchNorm of smlm/pkm.py:188-191 (the arithmetic of smlm_affine_bf16) in one launch.
 *   x (M, K) bf16 rows, w (N, K) bf16 (nn.Linear weight), bias (N,) bf16 or NULL, scale / shift both NULL or both
 *   given (16-byte aligned), out (M, N) bf16; K a multiple of 64, N of 128; 16-byte aligned rows, strides in
 *   elements.
 */
int smlm_prompt_linear(const void *x, int64_t x_row_stride, const void *w, int64_t w_row_stride, const void *bias,
                       const float *scale, const float *shift, int64_t M, int K, int N, void *out,
                       int64_t out_row_stride, void *stream);

/*
 * Greedy token choice of the decode loop (smlm/train.py:297-299, `nxt = logits[:, -1:].argmax(-1)`): per row
 * the first index of the largest bf16 logit, written to tok[b]; if hist is given, also to
 * hist[b, *pos + 1] (skipped when that slot is outside [0, hist_len)).
 *   logits (B, V) bf16, row b at logits + b*row_stride;  tok (B,) int64;  pos device int64 scalar.
 */
int smlm_greedy_argmax(const void *logits, int64_t row_stride, int64_t B, int V, const int64_t *pos, int64_t *tok,
                       int64_t *hist, int64_t hist_row_stride, int64_t hist_len, void *stream);

/*
 * Residual add + RMSNorm of the decoder blocks (smlm/model.py:124-126, 156-163: `x = x + sublayer(...)` followed by
 * the next sublayer's `norm(x)`), one launch per pair:
 *   x_out = bf16(x + delta);   h_out = bf16(x_out * rsqrt(mean(x_out^2) + eps) * weight)   (fp32 statistics)
 * With delta == NULL only the norm of x is computed (x_out unused).  x, delta, x_out, h_out (M, C) bf16 dense;
 * weight (C,) bf16.
 */
int smlm_add_rmsnorm(const void *x, const void *delta, const void *weight, float eps, int64_t M, int C, void *x_out,
                     void *h_out, void *stream);

/*
 * Eval-mode BatchNorm of the memory query on bf16 rows in one pass: replaces `q = query_norm(q)` with the running
 * statistics (smlm/pkm.py:188-191; BN in fp32 under autocast, then the bf16 cast of pkm.py:197):
 *   out[m, c] = bf16(x[m, c] * scale[c] + shift[c]),  scale = weight / sqrt(var + eps), shift = bias - mean * scale
 * fp32 arithmetic (one fused multiply-add), round to nearest even.  x, out (M, C) bf16 with row strides (elements,
 * multiples of 8); scale, shift (C,) fp32; C a multiple of 8; pointers 16-byte aligned.
 */
int smlm_affine_bf16(const void *x, int64_t x_row_stride, const float *scale, const float *shift, int64_t M, int C,
                     void *out, int64_t out_row_stride, void *stream);

/*
 * RoPE of a prompt pass in one launch: replaces the chunk / multiply / add / cat ops of smlm/model.py:63-78 applied
 * to q and k of `q, k, v = wqkv(x).view(B, T, 3, H, hd).permute(2, 0, 3, 1, 4)` (smlm/model.py:92-93).  Token t of
 * the (B*T, 3*H*hd) bf16 projection (row b*T + t at qkv + (b*T + t)*qkv_row_stride) is at position pos0 + t:
 *   out[i] = bf16(x[i] c - x[i + hd/2] s),  out[i + hd/2] = bf16(x[i] s + x[i + hd/2] c),  i < hd/2,
 *   c, s = rope_cos / rope_sin[pos0 + t, i] (fp32 or bf16 tables of rope_len rows), fp32 arithmetic;
 * q and k go to q_out / k_out (element (b, h, t, d) at base + b*strides[0] + h*strides[1] + t*strides[2] + d), v is
 * copied to v_out when it is not NULL (e.g. the slots [pos0, pos0 + T) of a static KV cache).  head_dim in
 * {16, 32, 64, 128}; pos0 + T <= rope_len; pointers 16-byte aligned, strides multiples of 8 elements.
 */
int smlm_rope_qkv(const void *qkv, int64_t qkv_row_stride, const void *rope_cos, const void *rope_sin, int rope_dtype,
                  int rope_len, int pos0, void *q_out, const int64_t *q_strides, void *k_out, const int64_t *k_strides,
                  void *v_out, const int64_t *v_strides, int64_t B, int T, int H, int head_dim, void *stream);

/*
 * Causal attention of a prompt / prefill pass (several new tokens at once), flash-style on the matrix cores.
 * Replaces F.scaled_dot_product_attention(q, k, v, is_causal=True) and the masked form for new tokens after a filled
 * cache (mask = ones(T, S).tril(S - T)) of smlm/model.py:97-105:
 *   y[b, t, h, :] = sum_{s <= S-T+t} softmax_s(q[b,h,t] . k[b,h,s] / sqrt(head_dim)) v[b,h,s]
 * bf16 operands, fp32 scores / softmax statistics / accumulation, probabilities rounded to bf16 for the value
 * product, y rounded to bf16.  Element (b, h, t, d) of q is at q + b*q_strides[0] + h*q_strides[1] + t*q_strides[2]
 * + d (d contiguous); likewise k, v (t < S) and y with its own strides.  q, k, v 16-byte aligned with strides that
 * are multiples of 8 elements; y 8-byte aligned, strides multiples of 4.  head_dim in {32, 64, 128}; S >= T;
 * (S + 64) x the larger key / value token stride x 2 bytes below 2^31 (SMLM_EUNSUPPORTED otherwise).
 */
int smlm_prefill_attention(const void *q, const int64_t *q_strides, const void *k, const int64_t *k_strides,
                           const void *v, const int64_t *v_strides, void *y, const int64_t *y_strides, int64_t B,
                           int H, int T, int S, int head_dim, void *stream);

/*
 * Fused linear layer of the single-token decode step (M = decode batch rows):  y = h W^T on the matrix cores with
 * the op in front of it and the op after it in one launch.  Replaces, per decode step, the nn.Linear calls of
 * smlm/model.py:90-118 and 266-293 (wqkv, wo, w13, w2, lm_head) and smlm/pkm.py:188-191, 213-224 (query_proj,
 * swilu_proj, value_proj), together with their neighbours:
 *   prologue SMLM_LIN_PLAIN          h = x
 *            SMLM_LIN_RMSNORM        xs = bf16(x + delta) (delta may be NULL), h = bf16(xs * rsqrt(mean(xs^2) + eps) * g)
 *                                    (the residual add, smlm/model.py:156-163, and the next sublayer's RMSNorm)
 *            SMLM_LIN_EMBED_RMSNORM  xs = emb[tok[m]] (smlm/model.py:268), then as SMLM_LIN_RMSNORM
 *            SMLM_LIN_RMSNORM_PARTS  as SMLM_LIN_RMSNORM with delta = bf16(sum over q < delta_parts of
 *                                    delta[m, q, :]) from fp32 (M, delta_parts, K) parts, summed in q order: the
 *                                    per-head output projections of smlm_decode_attention_proj (1 <= delta_parts
 *                                    <= 8; not with SMLM_LIN_ARGMAX)
 *            SMLM_LIN_EMBED_ARGMAX   as SMLM_LIN_EMBED_RMSNORM with tok[m] = the column of the largest key of
 *                                    tok_partial[m, 0..tok_blocks), the previous step's SMLM_LIN_ARGMAX partials
 *                                    (the greedy choice of smlm/train.py:297-301 made at the start of the next
 *                                    step, so no smlm_argmax_finish launch between steps); the workgroups of
 *                                    column block 0 write it to tok_out[m] (if not NULL) and to hist[m, *pos] (if
 *                                    hist is not NULL and 0 <= *pos < hist_len).  A row without keys (all 0) gets
 *                                    the id 2^32 - 1, outside the embedding: a NaN row, as in SMLM_LIN_EMBED_RMSNORM
 *            with an RMSNorm prologue, xs is also written to x_out (if not NULL): the residual stream
 *   epilogue SMLM_LIN_STORE          v = bf16(acc + bias); on columns < n_affine v = bf16(v * scale + shift) (eval
 *                                    BatchNorm of the memory query); columns < n_split to out, the rest to out2
 *            SMLM_LIN_SWIGLU         out[:, j] = bf16(bf16(silu(a_j)) * b_j), a_j = bf16(acc_j), b_j = bf16(acc_{N/2+j})
 *                                    (w13 followed by the SwiGLU activation, smlm/model.py:110-118)
 *            SMLM_LIN_ARGMAX         no logits are written: partial[m, b] = the largest (order16(bf16 logit) << 32 |
 *                                    ~column) over column block b of smlm_linear_argmax_blocks(N) blocks of 128;
 *                                    smlm_argmax_finish or the next step's SMLM_LIN_EMBED_ARGMAX prologue turns
 *                                    them into tokens (lm_head + greedy argmax); if pos_advance is not NULL, one
 *                                    thread adds 1 to *pos_advance (the decode position; nothing else in the
 *                                    launch reads it)
 * Shapes: W (N, K) bf16 row-major (nn.Linear.weight), K a multiple of 32, N a multiple of 16 (SWIGLU: 32);
 * RMSNorm prologues need K <= 480; x rows at x + m*x_stride; delta, x_out (M, K) dense; bias (N,) bf16;
 * scale/shift (n_affine,) fp32; out/out2 bf16 with row strides in elements.  All inputs 16-byte aligned, outputs
 * 8-byte aligned.  Deterministic (no atomics); the library allocates nothing.
 */
typedef enum smlm_linear_prologue {
  SMLM_LIN_PLAIN = 0,
  SMLM_LIN_RMSNORM = 1,
  SMLM_LIN_EMBED_RMSNORM = 2,
  SMLM_LIN_RMSNORM_PARTS = 3,
  SMLM_LIN_EMBED_ARGMAX = 4
} smlm_linear_prologue;

typedef enum smlm_linear_epilogue {
  SMLM_LIN_STORE = 0,
  SMLM_LIN_SWIGLU = 1,
  SMLM_LIN_ARGMAX = 2
} smlm_linear_epilogue;

typedef struct smlm_linear_args {
  int prologue;             /* smlm_linear_prologue */
  int epilogue;             /* smlm_linear_epilogue */
  int64_t M;                /* rows (tokens) */
  int N;                    /* weight rows (output features; SWIGLU: 2 * hidden) */
  int K;                    /* input features */
  const void *x;            /* (M, K) bf16 rows at x + m*x_stride (PLAIN, RMSNORM) */
  int64_t x_stride;
  const void *delta;        /* (M, K) bf16 or NULL (RMSNORM); (M, delta_parts, K) fp32 (RMSNORM_PARTS) */
  const int64_t *tok;       /* (M,) token ids (EMBED_RMSNORM) */
  const void *emb;          /* (emb_rows, K) bf16 (EMBED_RMSNORM) */
  int64_t emb_rows;
  const void *norm_w;       /* (K,) bf16 RMSNorm weight */
  float eps;
  void *x_out;              /* (M, K) bf16 or NULL: the prologue's xs */
  const void *w;            /* (N, K) bf16 */
  const void *bias;         /* (N,) bf16 or NULL (STORE) */
  const float *scale;       /* (n_affine,) fp32 (STORE) */
  const float *shift;       /* (n_affine,) fp32 (STORE) */
  int n_affine;
  int n_split;              /* STORE: columns [0, n_split) -> out, [n_split, N) -> out2 */
  void *out;                /* STORE: (M, n_split); SWIGLU: (M, N/2) */
  int64_t out_stride;
  void *out2;               /* STORE: (M, N - n_split) */
  int64_t out2_stride;
  uint64_t *partial;        /* ARGMAX: (M, >= smlm_linear_argmax_blocks(N)) */
  int64_t partial_stride;
  int delta_parts;          /* RMSNORM_PARTS: number of fp32 parts of delta */
  const uint64_t *tok_partial;  /* EMBED_ARGMAX: (M, >= tok_blocks) keys, even row stride, 16-byte aligned */
  int64_t tok_partial_stride;
  int tok_blocks;
  int64_t *tok_out;         /* EMBED_ARGMAX: (M,) or NULL */
  int64_t *hist;            /* EMBED_ARGMAX: (M, hist_len) rows at hist + m*hist_stride, or NULL */
  int64_t hist_stride;
  int64_t hist_len;
  const int64_t *pos;       /* EMBED_ARGMAX with hist: the history slot */
  int64_t *pos_advance;     /* ARGMAX: NULL, or the position to advance by one (M >= 1) */
} smlm_linear_args;

/* Number of 128-column blocks of the ARGMAX epilogue for N columns (the width partial needs). */
int smlm_linear_argmax_blocks(int N);

int smlm_decode_linear(const smlm_linear_args *args, void *stream);

/*
 * End of a greedy decode step (smlm/train.py:297-301: nxt = logits.argmax(-1), appended to the sequence), in one
 * workgroup: tok[m] = the column of the largest of partial[m, 0..nblk); if hist is given, hist[m, *pos + 1] = tok[m]
 * (skipped outside [0, hist_len)); then, if advance, *pos += 1 (after every row has read the old value).
 */
int smlm_argmax_finish(const uint64_t *partial, int64_t partial_stride, int nblk, int64_t M, int64_t *pos,
                       int64_t *tok, int64_t *hist, int64_t hist_stride, int64_t hist_len, int advance, void *stream);

/* ---- training side of the lookup ------------------------------------------------------------------------- */

/*
 * Backward of the selection (PKSelect.backward, smlm/kernels.py:253-266):
 *   dl[n,h,k] = w * (g_w - sum_k' w * g_w)  (+ g_scores[n,h,k] if given),  ds = dl rounded to the scores' dtype;
 *   ds1[n,h,:] = dense fp32 sums of ds over the selected pairs per first-half sub-key idx / NK, rounded once to
 *   dtype; ds2 the same per second-half sub-key idx % NK.  Sums run in selection order (deterministic).
 *   idx (N, H, knn) int64 and w (N, H, knn) fp32 from smlm_pkm_select; g_scores (N, H, knn) of dtype or NULL;
 *   g_w (N, H, knn) fp32 or NULL; ds1, ds2 (N, H, NK) of dtype (every element written), 16-byte aligned.
 *   NK a power of two in [8, 65536], knn <= 64.
 */
int smlm_pkm_select_backward(const int64_t *idx, const float *w, const void *g_scores, const float *g_w, int dtype,
                             int64_t N, int H, int NK, int knn, void *ds1, void *ds2, void *stream);

/*
 * Row-sparse value-bag backward (smlm/kernels.py:1-104, smlm/sparse_values.py:94-113):
 *   acc[idx[n,k], :] += w[n,k] * grad_out[n, :]   (fp32 atomic adds: the order of additions is not fixed)
 *   touched[idx[n,k]] = 1
 *   gw[n,k] = sum_d grad_out[n,d] * table[idx[n,k], d]   (the per-sample-weight gradient, fp32)
 *   grad_out (N, D) fp32; idx (N, K) int64; w (N, K) fp32; table (rows, D) SMLM_F32 or SMLM_BF16; acc (rows, D)
 *   fp32; touched (rows,) uint8; gw (N, K) fp32.  D <= 512.  An index outside [0, rows) adds nothing and gives a
 *   NaN gw.
 * gw NULL: the per-sample-weight gradient is not wanted (the reference computes it and its caller discards it when
 *   the weights do not train: the unit weights of the Engram lookups, smlm/engram.py:118); then w may be NULL (unit
 *   weights), table and table_dtype are not read, and the lookups are scattered with one thread per element and no
 *   sort.  With gw given, w and table are required.
 */
int smlm_bag_backward_rows(const float *grad_out, const int64_t *idx, const float *w, int64_t N, int K,
                           const void *table, int table_dtype, int64_t rows, int D, float *acc, uint8_t *touched,
                           float *gw, void *stream);

/*
 * The same row-sparse bag backward in a fixed order (replaces bag_backward_rows, smlm/kernels.py:34-88, with the
 * reference's grouping: the lookups sorted by table row, each row's run added in lookup order):
 *   acc[idx[n,k], :] += w[n,k] * grad_out[n, :], touched[idx[n,k]] = 1, gw[n,k] = grad_out[n, :] . table[idx[n,k], :]
 * Every accumulator row is written by one wavefront (runs that span several 64-lookup chunks add their per-chunk
 * partial sums in chunk order), so the result is the same on every call.  The workspace (caller-owned, 256-byte
 * aligned) holds the sort keys and values, the partial sums and the sort's storage; its size comes from
 * smlm_bag_backward_sorted_workspace.  Shapes as smlm_bag_backward_rows, with rows < 2^32 - 1 and N*K < 2^31 - 1.
 */
int smlm_bag_backward_sorted_workspace(int64_t N, int K, int64_t rows, int D, size_t *bytes);
int smlm_bag_backward_sorted(const float *grad_out, const int64_t *idx, const float *w, int64_t N, int K,
                             const void *table, int table_dtype, int64_t rows, int D, float *acc, uint8_t *touched,
                             float *gw, void *workspace, size_t workspace_bytes, void *stream);

/* Moment storage of smlm_lazy_adam. */
typedef enum smlm_adam_state {
  SMLM_ADAM_F32 = 0,   /* exp_avg, exp_avg_sq (rows, D) fp32 (smlm/kernels.py:380-433) */
  SMLM_ADAM_BF16 = 1,  /* (rows, D) bf16, round to nearest even (smlm/kernels.py:445-492) */
  SMLM_ADAM_INT8 = 2   /* exp_avg (rows, D) int8 codes of sign(m) sqrt(|m| / s_m) * 127, exp_avg_sq (rows, D)
                          uint8 codes of v^(1/4) / s_v * 255 (>= 1 where v > 0), fp32 row scales s_m = max|m|,
                          s_v = max v^(1/4) (smlm/kernels.py:445-492) */
} smlm_adam_state;

/*
 * Lazy Adam step of the value table (LazyRowAdam, smlm/sparse_values.py:148-330, kernels.py:380-515), in place, on
 * the rows with touched[r] != 0 only:
 *   g = acc[r] * (*grad_scale);  m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2;
 *   p[r] -= step_size * m / (sqrt(v) / bc2_sqrt + eps)       (step_size = lr / (1 - b1^step),
 *                                                             bc2_sqrt = sqrt(1 - b2^step), from the host)
 *   then acc[r] = 0 and touched[r] = 0.  SMLM_ADAM_F32 forms 1 - b on the device in fp32 (as the reference's fp32
 *   kernel); the compact states use one_minus_beta1/2 as given (fp32 of the host's 1 - b).  IEEE division and
 *   square root, no fused multiply-add.  param, acc (rows, D) fp32; touched (rows,) uint8; grad_scale a device
 *   fp32 scalar; exp_avg_scale / exp_avg_sq_scale (rows,) fp32 for SMLM_ADAM_INT8 (else NULL).  D <= 512.
 */
int smlm_lazy_adam(float *param, void *exp_avg, void *exp_avg_sq, float *exp_avg_scale, float *exp_avg_sq_scale,
                   int state, float *acc, uint8_t *touched, const float *grad_scale, int64_t rows, int D,
                   float step_size, float bc2_sqrt, float beta1, float beta2, float one_minus_beta1,
                   float one_minus_beta2, float eps, void *stream);

/*
 * Engram n-gram hash.  Replaces NgramHash.forward (smlm/engram.py:60-73): for every position t of B sequences of
 * T tokens, n-gram order o (orders[o] tokens) and hash head h, x = XOR_{i < n} c[t - i] * mult[o, h, i] (64-bit
 * wrap-around), x ^= x >> 17, rows[b, t, o * heads + h] = (x mod rows_per_head) + (o * heads + h) * rows_per_head.
 *   c        (B, c_len) int64 compressed token ids, c_len = T + max(orders) - 1 (the leading columns are the
 *            previous chunk's last tokens, or the pad id)
 *   mult     (n_orders, heads, max_order) int64 odd multipliers
 *   orders   HOST array of n_orders n-gram lengths (1 <= n <= max_order <= 8, n_orders <= 4)
 *   rows_out (B, T, n_orders * heads) int64
 */
int smlm_engram_hash(const int64_t *c, int64_t B, int64_t T, int64_t c_len, const int64_t *mult, const int *orders,
                     int n_orders, int heads, int max_order, int64_t rows_per_head, int64_t *rows_out, void *stream);

/*
 * Row gather out[m] = table[rows[m]] for M int64 row indices (F.embedding), table (table_rows, D) of table_dtype
 * (SMLM_F32 / SMLM_BF16), out (M, D) of the same dtype.  Replaces the Engram row lookup (smlm/engram.py:111-118,
 * F.embedding / row_sparse_embedding_bag with weights 1); a row outside the table gives a NaN output row.
 */
int smlm_row_gather(const int64_t *rows, int64_t M, const void *table, int table_dtype, int64_t table_rows, int D,
                    void *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SMLM_PKM_H */
