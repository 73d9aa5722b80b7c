/*
 * tokquay_amd.h - C ABI of the MI355X (gfx950) paged-attention library.
 *
 * The library replaces the three tensor-level steps of Tokquay's paged
 * attention branch with hand-written HIP kernels:
 *
 *   tq_cache_write    scatter each new token's K/V rows into the block pool
 *                     (tq_paged_gather: the reference view's gathered copy, for its callers)
 *   tq_paged_decode   one-query-per-sequence attention straight off the pool
 *   tq_paged_decode_write  the same, with the new token's cache write folded in
 *                     (tq_paged_decode_write_static: without a workspace argument)
 *   tq_paged_prefill  causal (chunked) prefill attention straight off the pool
 *   tq_paged_mixed    a step's decode rows (with their cache write) and prefill
 *                     rows in one launch
 *
 * plus two kernels of the model step around them:
 *
 *   tq_argmax_rows    index of each logit row's maximum (greedy sampling)
 *   tq_add_layernorm  residual add fused with the LayerNorm that follows it
 *   tq_skinny_linear  linear layer of at most 64 rows, LayerNorm / bias / GELU /
 *                     residual add fused in (small-batch decode steps)
 *   tq_skinny_linear_argmax  the LM head of at most 16 rows with the greedy argmax
 *                     fused in: only ids are written
 *   tq_embed_rows     token + position embeddings of each row
 *
 * KV pool layout (identical to the reference's, bit for bit):
 *
 *   pool[num_blocks][num_layers][2][num_heads][block_size][head_dim]  fp32,
 *   contiguous, dim 2: 0 = K, 1 = V.
 *
 * Logical position p of a sequence lives in block block_table[p / block_size]
 * at offset p % block_size; its flat slot is
 * block_table[p / block_size] * block_size + p % block_size.
 *
 * Conventions
 *   - Every pointer is a device pointer unless its comment says otherwise.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Every entry point only enqueues work on `stream`; none synchronises.
 *   - Row strides are in elements (floats), not bytes; the innermost
 *     (head, dim) block of every q / k / v / out row must be contiguous.
 *   - `d_error` may be NULL. When not NULL it must point to a device int32 the
 *     caller zeroed; kernels OR TQ_DEVERR_* bits into it when they meet an
 *     out-of-range block id, slot or length. Such an entry is skipped (the
 *     kernel never reads or writes outside the pool), so the result for that
 *     row is undefined but the launch is memory safe.
 *   - Only head_dim == 64 is supported (GPT-2 family). block_size may be any
 *     value in [1, 1024].
 *   - Calls are not thread safe with respect to the same pool: the caller
 *     (one engine thread) orders them on one stream.
 */
#ifndef TOKQUAY_AMD_H_
#define TOKQUAY_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum tq_status {
  TQ_OK = 0,
  TQ_ERR_INVALID_ARGUMENT = 1, /* a null pointer, a negative size, a layer out of range ... */
  TQ_ERR_UNSUPPORTED = 2,      /* a shape this build has no kernel for (head_dim != 64 ...) */
  TQ_ERR_WORKSPACE = 3,        /* workspace missing or smaller than the *_workspace_size() asked for */
  TQ_ERR_HIP = 4               /* the HIP runtime refused the launch */
} tq_status;

/* Bits a kernel ORs into *d_error. */
#define TQ_DEVERR_BLOCK_ID 1   /* a block-table entry outside [0, num_blocks) */
#define TQ_DEVERR_SLOT 2       /* a slot_mapping entry >= num_blocks * block_size */
#define TQ_DEVERR_LENGTH 4     /* a context / query length the block table cannot hold */
#define TQ_DEVERR_ORDER 8      /* a seq_order entry outside [0, num_seqs) */

/* Human-readable name of a status code (static storage, never NULL). */
const char* tq_status_string(tq_status status);

/* Version of this ABI; bumped whenever a signature changes (2: seq_order in the decode entry points;
 * 3: seq_order in tq_paged_prefill). */
int32_t tq_abi_version(void);

/* Message of the last TQ_ERR_HIP on the calling thread ("" if none). */
const char* tq_last_hip_error(void);

/*
 * Arms two hipEvent_t handles (passed as void*; either may be NULL) for the
 * calling thread's next decode, prefill or mixed attention call (tq_paged_decode,
 * tq_paged_decode_write, tq_paged_decode_write_static, tq_paged_prefill, tq_paged_mixed): the start
 * event is recorded when that call's first kernel starts and the stop event
 * when its last kernel ends, so hipEventElapsedTime gives the kernels' own
 * duration, without launch gaps. That call disarms them, whatever it returns.
 * No counterpart in the reference (it has no kernels); for benchmarks.
 */
tq_status tq_set_timing_events(void* start_event, void* stop_event);

/*
 * Cache write: for every token n in [0, num_tokens) with slot = slot_mapping[n] >= 0,
 *   pool[slot / block_size][layer][0][h][slot % block_size][:] = k[n * k_row_stride + h * 64 + :]
 *   pool[slot / block_size][layer][1][h][slot % block_size][:] = v[n * v_row_stride + h * 64 + :]
 * for every head h. A negative slot marks a padded token, which writes nothing.
 * The copy is bit exact.
 *
 * Replaces PagedBatch.write (tokquay/kv_cache.py:228-232) together with the
 * scatter targets PagedBatch.__init__ builds for it (tokquay/kv_cache.py:216-226):
 * slot_mapping[n] is block_table[p // block_size] * block_size + p % block_size
 * for the token at position p (tokquay/kv_cache.py:9-10, :223-224).
 */
tq_status tq_cache_write(float* pool, int64_t num_blocks, int32_t num_layers, int32_t num_heads,
                         int32_t block_size, int32_t head_dim, int32_t layer,
                         const float* k, int64_t k_row_stride,
                         const float* v, int64_t v_row_stride,
                         const int64_t* slot_mapping, int64_t num_tokens,
                         int32_t* d_error, void* stream);

/*
 * Paged decode attention: one query per sequence, attending to every cached
 * position of that sequence (the query's own K/V must already be in the pool):
 *
 *   out[b, h, :] = softmax_j(scale * q[b, h, :] . K_b[h, j, :]) @ V_b[h, j, :],  j < context_lens[b]
 *
 * where K_b / V_b are read through block_tables[b * block_table_stride + j / block_size].
 * q row b starts at q + b * q_row_stride (heads contiguous), out row b at
 * out + b * out_row_stride. Rows with context_lens[b] == 0 get zeros.
 * max_context_len must be >= every context_lens[b] (it sizes the grid).
 *
 * seq_order (may be NULL) is the order the sequences' workgroups are dispatched
 * in: a permutation of 0..num_seqs-1 (entries outside that range are reported
 * with TQ_DEVERR_ORDER and skipped). Older waves win arbitration, so listing the
 * longest contexts first shortens the launch's tail (-7 % on 256 sequences of
 * U[256,1024] positions). NULL is the natural order.
 *
 * The kernel splits each sequence into partitions of partition_tokens
 * positions (a multiple of 16, at most 1024; 0 = choose automatically) and merges them with
 * a log-sum-exp pass when a sequence spans several. The merge needs
 * tq_paged_decode_workspace_size(...) bytes of device workspace. With 0, a launch
 * with too few (sequence, head) pairs to fill the GPU runs one workgroup of several
 * waves per pair instead, merged on chip: no workspace (the size function says 0).
 *
 * Replaces PagedBatch.gather (tokquay/kv_cache.py:234-242), the mask it is used
 * with (tokquay/kv_cache.py:208-214) and the attention math of
 * Attention.forward (tokquay/model.py:94-96) for rows that feed one token.
 */
tq_status tq_paged_decode(float* out, int64_t out_row_stride,
                          const float* q, int64_t q_row_stride,
                          const float* pool, int64_t num_blocks, int32_t num_layers,
                          int32_t num_heads, int32_t block_size, int32_t head_dim, int32_t layer,
                          const int32_t* block_tables, int64_t block_table_stride,
                          int32_t max_blocks_per_seq,
                          const int32_t* context_lens, const int32_t* seq_order,
                          int32_t num_seqs, int32_t max_context_len,
                          float scale, int32_t partition_tokens,
                          void* workspace, size_t workspace_bytes,
                          int32_t* d_error, void* stream);

/*
 * Paged decode with the cache write of the new token folded in. For every row b
 * with context_lens[b] = n > 0 the new token sits at position p = n - 1, in slot
 * block_tables[b * block_table_stride + p / block_size] * block_size + p % block_size:
 *
 *   pool[slot / block_size][layer][0][h][slot % block_size][:] = k_new[b * k_new_row_stride + h * 64 + :]
 *   pool[slot / block_size][layer][1][h][slot % block_size][:] = v_new[b * v_new_row_stride + h * 64 + :]
 *
 * for every head h, then out as tq_paged_decode computes it over positions
 * 0..n-1. Output and pool are bit-identical to tq_cache_write (slot_mapping[b]
 * = that slot) followed by tq_paged_decode. Rows with n == 0 write nothing. The
 * same workspace as tq_paged_decode (tq_paged_decode_workspace_size).
 *
 * Replaces PagedBatch.write (tokquay/kv_cache.py:228-232) for rows that feed one
 * token, together with what tq_paged_decode replaces (tokquay/kv_cache.py:208-214,
 * :234-242; tokquay/model.py:94-96).
 */
tq_status tq_paged_decode_write(float* out, int64_t out_row_stride,
                                const float* q, int64_t q_row_stride,
                                const float* k_new, int64_t k_new_row_stride,
                                const float* v_new, int64_t v_new_row_stride,
                                float* pool, int64_t num_blocks, int32_t num_layers,
                                int32_t num_heads, int32_t block_size, int32_t head_dim, int32_t layer,
                                const int32_t* block_tables, int64_t block_table_stride,
                                int32_t max_blocks_per_seq,
                                const int32_t* context_lens, const int32_t* seq_order,
                                int32_t num_seqs, int32_t max_context_len,
                                float scale, int32_t partition_tokens,
                                void* workspace, size_t workspace_bytes,
                                int32_t* d_error, void* stream);

/* Bytes of workspace tq_paged_decode needs for these sizes (0 if none). */
size_t tq_paged_decode_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                      int32_t max_context_len, int32_t partition_tokens);

/* Bytes of the per-GPU device array tq_paged_decode_write_static keeps its partials in. */
#define TQ_STATIC_SCRATCH_BYTES (8u << 20)

/*
 * tq_paged_decode_write without the workspace arguments: it allocates nothing and takes no
 * caller memory beyond its inputs and outputs. Same semantics, kernels and bits as
 * tq_paged_decode_write. When tq_paged_decode_workspace_size(num_seqs, num_heads, head_dim,
 * max_context_len, partition_tokens) is not 0 (explicit partitions that split sequences) the
 * partition partials go to a static device array of TQ_STATIC_SCRATCH_BYTES (8 MiB) per GPU,
 * held until the process ends; a call that would need more returns TQ_ERR_WORKSPACE before any
 * launch. The array's device address is looked up on the first call that needs it on each
 * device (hipGetSymbolAddress, with that device current); `stream` must belong to the current
 * device (else TQ_ERR_INVALID_ARGUMENT). Every call on one GPU shares that GPU's array and it
 * keeps the last call's contents: calls that overlap on one GPU (on different streams) race;
 * order them on one stream.
 *
 * No counterpart in the reference (it has no kernels). For callers that cannot allocate device
 * memory: code under HIP graph capture, serving loops and harnesses that forbid allocation.
 */
tq_status tq_paged_decode_write_static(float* out, int64_t out_row_stride,
                                       const float* q, int64_t q_row_stride,
                                       const float* k_new, int64_t k_new_row_stride,
                                       const float* v_new, int64_t v_new_row_stride,
                                       float* pool, int64_t num_blocks, int32_t num_layers,
                                       int32_t num_heads, int32_t block_size, int32_t head_dim, int32_t layer,
                                       const int32_t* block_tables, int64_t block_table_stride,
                                       int32_t max_blocks_per_seq,
                                       const int32_t* context_lens, const int32_t* seq_order,
                                       int32_t num_seqs, int32_t max_context_len,
                                       float scale, int32_t partition_tokens,
                                       int32_t* d_error, void* stream);

/*
 * Gather: every sequence's K and V as the reference's batch view materialises them,
 *
 *   k_out[b][h][j * block_size + o][:] = pool[block_tables[b][j]][layer][0][h][o][:]
 *   v_out[b][h][j * block_size + o][:] = pool[block_tables[b][j]][layer][1][h][o][:]
 *
 * for j < num_gathered_blocks (tables padded with any valid id, e.g. block 0, as the reference
 * pads them), both outputs contiguous [num_seqs, num_heads, num_gathered_blocks * block_size,
 * head_dim]. A bit-exact copy. An id outside the pool is reported (TQ_DEVERR_BLOCK_ID) and its
 * keys come out as zeros. The attention entry points never need it; it serves callers of the
 * reference's BatchedKV contract.
 *
 * Replaces PagedBatch.gather (tokquay/kv_cache.py:234-242).
 */
tq_status tq_paged_gather(float* k_out, float* v_out, const float* pool, int64_t num_blocks, int32_t num_layers,
                          int32_t num_heads, int32_t block_size, int32_t head_dim, int32_t layer,
                          const int32_t* block_tables, int64_t block_table_stride, int32_t num_gathered_blocks,
                          int32_t num_seqs, int32_t* d_error, void* stream);

/*
 * Paged prefill / chunked-prefill attention. Sequence b feeds
 * n_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] new tokens at positions
 * q_start[b] .. q_start[b] + n_b - 1, whose q rows are
 * q + (cu_seqlens_q[b] + i) * q_row_stride. Its K/V for positions
 * [0, q_start[b] + n_b) must already be in the pool. Causal:
 *
 *   out[row, h, :] = softmax_{j <= q_start[b] + i}(scale * q[row, h, :] . K_b[h, j, :]) @ V_b[h, j, :]
 *
 * cu_seqlens_q has num_seqs + 1 entries, starts at 0 and is non-decreasing;
 * num_q_rows is cu_seqlens_q[num_seqs] (the kernels reject rows beyond it).
 * max_query_len >= every n_b (it sizes the grid).
 *
 * seq_order (may be NULL) is the order the sequences' query tiles are dealt to the
 * GPU in: a permutation of 0..num_seqs-1 (entries outside that range are reported
 * with TQ_DEVERR_ORDER and skipped). Launches with more query tiles than the GPU
 * holds at once use it; listing the sequences by decreasing work
 * (n_b * (q_start[b] + n_b / 2)) first made 32 prompts of U[256,1024] tokens 3-16 %
 * faster. Launches with fewer tiles ignore it. NULL is the natural order; the
 * output does not depend on it.
 *
 * Replaces PagedBatch.gather + mask + Attention.forward's masked softmax
 * (tokquay/kv_cache.py:208-214, :234-242; tokquay/model.py:94-96) for rows that
 * feed several tokens (prefill, recompute after preemption, chunked prefill).
 */
tq_status tq_paged_prefill(float* out, int64_t out_row_stride,
                           const float* q, int64_t q_row_stride,
                           const float* pool, int64_t num_blocks, int32_t num_layers,
                           int32_t num_heads, int32_t block_size, int32_t head_dim, int32_t layer,
                           const int32_t* block_tables, int64_t block_table_stride,
                           int32_t max_blocks_per_seq,
                           const int32_t* cu_seqlens_q, const int32_t* q_start,
                           const int32_t* seq_order,
                           int32_t num_seqs, int32_t num_q_rows, int32_t max_query_len,
                           float scale, int32_t* d_error, void* stream);

/*
 * One step's attention for both kinds of row in one launch: the decode rows as
 * tq_paged_decode_write computes them (their new K/V written into the pool, then one
 * query each over its context; the dec_* arguments, context_lens, seq_order, k_new, v_new
 * and partition_tokens mean what they mean there) and the prefill rows as tq_paged_prefill
 * computes them (the pre_* arguments, cu_seqlens_q, q_start, num_prefill_seqs, num_q_rows,
 * max_query_len as there; their K/V must already be in the pool, e.g. by tq_cache_write).
 * pool, the pool geometry, layer, scale, d_error and stream are shared. The two sets of
 * sequences must not share a pool slot that the decode rows write.
 *
 * The decode rows' waves and the prefill tiles run side by side in one grid, so HBM
 * streaming and MFMA work overlap and the launch cost is paid once. Every output row is
 * bit-identical to the corresponding single-kind call's (for the decode rows: the one with
 * the same partition length; partition_tokens = 0 lets this call choose its own, so compare
 * with an explicit one). With no prefill rows this is tq_paged_decode_write, with no decode
 * rows tq_paged_prefill. Needs tq_paged_mixed_workspace_size(...) bytes of workspace
 * (16-byte aligned; nothing in it needs to start at zero).
 *
 * Replaces one Attention.forward call over a batch that holds both decode and prefill rows:
 * PagedBatch.write + gather + mask + the masked softmax (tokquay/model.py:67-99,
 * tokquay/kv_cache.py:208-214, :228-242).
 */
tq_status tq_paged_mixed(float* dec_out, int64_t dec_out_row_stride,
                         const float* dec_q, int64_t dec_q_row_stride,
                         const float* k_new, int64_t k_new_row_stride,
                         const float* v_new, int64_t v_new_row_stride,
                         const int32_t* dec_block_tables, int64_t dec_block_table_stride,
                         int32_t dec_max_blocks_per_seq,
                         const int32_t* context_lens, const int32_t* seq_order,
                         int32_t num_decode_seqs, int32_t max_context_len, int32_t partition_tokens,
                         float* pre_out, int64_t pre_out_row_stride,
                         const float* pre_q, int64_t pre_q_row_stride,
                         const int32_t* pre_block_tables, int64_t pre_block_table_stride,
                         int32_t pre_max_blocks_per_seq,
                         const int32_t* cu_seqlens_q, const int32_t* q_start,
                         int32_t num_prefill_seqs, int32_t num_q_rows, int32_t max_query_len,
                         float* pool, int64_t num_blocks, int32_t num_layers,
                         int32_t num_heads, int32_t block_size, int32_t head_dim, int32_t layer,
                         float scale, void* workspace, size_t workspace_bytes,
                         int32_t* d_error, void* stream);

/* Bytes of workspace tq_paged_mixed needs for these sizes (0 if none). */
size_t tq_paged_mixed_workspace_size(int32_t num_decode_seqs, int32_t num_heads, int32_t head_dim,
                                     int32_t max_context_len, int32_t partition_tokens,
                                     int32_t num_prefill_seqs, int32_t num_q_rows, int32_t max_query_len);

/*
 * Greedy sampling over a batch of logit rows:
 *
 *   out[r] = the lowest column c with logits[r * row_stride + c] maximal,  c < num_cols
 *
 * with the reference's order: NaN ranks above every number (the first NaN
 * wins) and -0 ties +0. out is int64[num_rows]. num_cols in [1, 2^30];
 * row_stride >= num_cols (elements).
 *
 * Replaces the batched `logits.argmax(-1)` of Engine._sample
 * (tokquay/engine.py:190), so a decode step hands back only [B] token ids.
 */
tq_status tq_argmax_rows(int64_t* out, const float* logits, int64_t num_rows, int64_t num_cols,
                         int64_t row_stride, void* stream);

/*
 * Residual add + LayerNorm over rows of `cols` fp32 values:
 *
 *   s = x[r] + y[r];  x_out[r] = s;  h_out[r] = (s - mean(s)) / sqrt(var(s) + eps) * gamma + beta
 *
 * (biased variance, as torch's LayerNorm). Row r of each matrix starts at
 * ptr + r * stride (elements). cols a multiple of 4, at most 2048; pointers and
 * strides 16-byte aligned. Outputs may alias inputs element for element
 * (x_out == x is the in-place residual update). y may be NULL (y_stride is
 * then ignored): s = x, a plain LayerNorm.
 *
 * Replaces the residual adds of Block.forward (tokquay/model.py:122-123) with
 * the LayerNorm that follows each (ln_2, the next block's ln_1, ln_f at :180).
 */
tq_status tq_add_layernorm(float* x_out, int64_t x_out_stride, float* h_out, int64_t h_out_stride,
                           const float* x, int64_t x_stride, const float* y, int64_t y_stride,
                           const float* gamma, const float* beta, int64_t rows, int32_t cols,
                           float eps, void* stream);

/*
 * Linear layer of a few rows with its neighbours fused in:
 *
 *   h = LN(x) if ln_gamma else x        (LN over K, biased variance, eps = ln_eps)
 *   v = h W^T + bias                    (bias may be NULL)
 *   epilogue 0: y = v;  1: y = gelu_tanh(v);  2: y = y + v (residual add, in place)
 *
 * x [M, K] (row stride x_stride), W [N, K] contiguous (nn.Linear's [out, in]),
 * y [M, N] (row stride y_stride), all fp32. M <= 64; K = 768, or K = 3072 without
 * the LayerNorm (GPT-2's widths; other shapes return TQ_ERR_UNSUPPORTED); x, W,
 * ln_gamma, ln_beta 16-byte aligned, x_stride a multiple of 4. y must not overlap
 * x. Reads W once; the partial products of the K slices are summed in a fixed
 * order (repeated calls give the same bits).
 *
 * Some shapes (K = 3072 with few columns) split K over several workgroups and need a
 * workspace of tq_skinny_linear_workspace_size() bytes (0: none; it grows with M),
 * 256-byte aligned, zeroed once before its first use: each call leaves it ready for
 * the next call with the same N and K (any M). Use one workspace per (N, K); calls
 * that share a workspace must not run concurrently.
 *
 * Replaces, for decode steps of at most 64 sequences, the c_attn / c_proj / c_fc
 * / mlp.c_proj linears (tokquay/model.py:62-63, :103-104) with ln_1 / ln_2 in
 * front (:117-118), the GELU (:107) and the residual adds (:122-123), and the
 * LM head with ln_f (:180-181, W = wte, no bias).
 */
size_t tq_skinny_linear_workspace_size(int32_t M, int32_t N, int32_t K, int32_t has_layernorm);
tq_status tq_skinny_linear(float* y, int64_t y_stride, const float* x, int64_t x_stride, int32_t M,
                           const float* w, const float* bias, int32_t N, int32_t K, const float* ln_gamma,
                           const float* ln_beta, float ln_eps, int32_t epilogue, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * Greedy ids of a linear layer of at most 16 rows, with no logits written:
 *
 *   h = LN(x) if ln_gamma else x;   ids[m] = the lowest n < N with (h[m] W^T + bias)[n] maximal
 *
 * in the order of tq_argmax_rows (NaN above every number, the first NaN wins; -0 ties +0).
 * ids is int64[M]. x [M, 768] (row stride x_stride), W [N, 768] contiguous, bias may be NULL;
 * M <= 16, N < 2^31 - 32; alignment as tq_skinny_linear. Each 32-column slice of the logits is
 * reduced on chip to one candidate per row, kept in the workspace; a second kernel of the same
 * call reduces the candidates of each row. The workspace, of
 * tq_skinny_linear_argmax_workspace_size(N) bytes (16-byte aligned), needs no initialisation;
 * calls sharing a workspace must not run concurrently.
 *
 * Replaces, for decode steps of at most 16 greedy sequences, the tied LM head with ln_f in front
 * (tokquay/model.py:180-181, W = wte, no bias) together with the batched argmax of
 * Engine._sample (tokquay/engine.py:190): only the [M] ids are written.
 */
size_t tq_skinny_linear_argmax_workspace_size(int32_t N);
tq_status tq_skinny_linear_argmax(int64_t* ids, const float* x, int64_t x_stride, int32_t M, const float* w,
                                  const float* bias, int32_t N, int32_t K, const float* ln_gamma,
                                  const float* ln_beta, float ln_eps, void* workspace, size_t workspace_bytes,
                                  void* stream);

/*
 * x[r] = wte[id_r] + wpe[positions[r]] for rows r < rows, C columns (a multiple
 * of 4), x row stride x_stride. id_r = tokens[src[r]] when src is not NULL and
 * src[r] >= 0 (the token a previous step chose for row src[r], left on the
 * device), else ids[r]. Ids outside [0, vocab) or positions outside
 * [0, n_positions) set TQ_DEVERR_LENGTH in d_error and are clamped.
 * Replaces the embedding sum of GPT2.forward (tokquay/model.py:172).
 */
tq_status tq_embed_rows(float* x, int64_t x_stride, const int64_t* ids, const int64_t* src,
                        const int64_t* tokens, const int64_t* positions, const float* wte, const float* wpe,
                        int64_t rows, int32_t C, int64_t vocab, int64_t n_positions, int32_t* d_error,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TOKQUAY_AMD_H_ */
