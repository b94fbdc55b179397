/*
 * C ABI of the MI355X (gfx950) DeepSeek-Sparse-Attention library, libdsa_mi355x.so.
 *
 * The reference (tilelang-ascend) generates, per kernel, a C entry point
 *   extern "C" void call(uint8_t* p0, ..., uint8_t* pN, [int64 shape vars], aclrtStream stream)
 * whose pointer parameters are the PrimFunc's tensors in order (inputs, outputs,
 * workspaces) and which launches on the given stream
 * (src/target/codegen_ascend.cc:1141-1156,1205-1226; a hand-written declaration of
 * one such entry point is examples/torch_tl_ascend/src/_inner.cpp:8-15).
 * The entry points below play that role for the three kernels of the DSA path.
 * They differ from the reference's `call` in two deliberate ways:
 *   - they return an int status (0 = success) and record a message readable
 *     through dsa_last_error(), the convention of the reference's CUDA/HIP
 *     wrappers (tilelang/jit/adapter/wrapper.py:29-41), where `call` is void;
 *   - sizes are explicit int64 arguments rather than baked into the kernel.
 * All pointers are device pointers (except where noted) to contiguous tensors;
 * the library never allocates device memory: outputs and workspaces are the
 * caller's, as with the reference's out_idx / workspace_idx tensors
 * (tilelang/jit/adapter/cython/cython_wrapper.pyx:102-141).  `stream` is a
 * hipStream_t (NULL = the default stream); every call is asynchronous.
 */
#ifndef DSA_MI355X_H_
#define DSA_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define DSA_OK 0
#define DSA_E_INVALID_ARGUMENT 1
#define DSA_E_WORKSPACE_TOO_SMALL 2
#define DSA_E_UNSUPPORTED 3
#define DSA_E_HIP 4

/* Message describing this thread's last failed call ("" if none). */
const char* dsa_last_error(void);
void dsa_clear_error(void);
int dsa_abi_version(void);

/*
 * Row-wise top-k of fp32 scores.
 * Replaces the `call` generated for simple_topk_selector's PrimFunc
 * main(x[B,N] fp32, indices[B,top_k] int32)
 * (examples/topk_selector/example_topk_selector.py:19-54), and the sort/merge
 * top-k stage inside the lightning indexer kernel
 * (examples/deepseek_v4/lightning_indexer.py:945-1036,1116-1196).
 *
 * scores  [rows, ld] fp32, row r uses columns [0, min(row_len[r], cols)) (row_len
 *         may be NULL = all cols).
 * out_idx [rows, k] int32: argsort(-row, stable=True)[:k]; entries <= -1e30 become
 *         -1 when pad_invalid != 0; positions past the row length are -1.
 * out_val [rows, k] fp32 or NULL: the selected values (-inf past the row length).
 * Limits: k <= 8192, cols < 2^31.
 */
int dsa_topk_f32(const float* scores, int64_t rows, int64_t cols, int64_t ld,
                 const int32_t* row_len, int32_t k, int32_t pad_invalid, int32_t* out_idx,
                 float* out_val, void* stream);

/*
 * The same top-k given, for each row, an upper bound of the maximum of every
 * group of 16 consecutive scores: group_max [rows, ld_g] fp32, ld_g >=
 * ceil(cols / 16), group_max[r, g] >= max(scores[r, 16g : 16g + 16] within the
 * row length) (NaN ignored; -inf for an empty group).  The K-th largest group
 * maximum bounds the K-th largest score from below, so only the groups reaching
 * it are read.  The lightning indexer emits exact group maxima with its logits
 * and selects through this path (the fused indexer -> top-k of
 * examples/deepseek_v4/lightning_indexer.py:945-1036, where the block sort runs
 * on the logits the Cube unit just produced).  Rows of fewer than 2 k groups,
 * or whose groups reaching the bound are too many, fall back to reading the
 * whole row; the result equals dsa_topk_f32's.
 */
int dsa_topk_f32_group_max(const float* scores, int64_t rows, int64_t cols, int64_t ld,
                           const int32_t* row_len, const float* group_max, int64_t ld_g, int32_t k,
                           int32_t pad_invalid, int32_t* out_idx, float* out_val, void* stream);

/*
 * Lightning-indexer logits, fp8 e4m3 q and k with a per-key fp32 scale.
 * Replaces the Cube QK + ReLU and Vector weight/head-reduce/mask stages of the
 * `call` built by make_lightning_indexer_kernel
 * (examples/deepseek_v4/lightning_indexer.py:661-795,868-944; golden :303-314).
 *
 * q [B, S1, N1, D] fp8, k [B, S2, D] fp8 (one key head), key_scale [B, S2] fp32 or
 * NULL (= 1), weights [B, S1, N1] fp32, act_q / act_k [B] int32 per-batch lengths or
 * NULL (= S1 / S2).  sparse_mode 3 = right-down causal, 0 = none.  N1 = 64, D = 128.
 * logits [B * S1, ld] fp32: entry (t, s) is written for s < row_len[t] (masked
 * entries inside computed tiles are -inf; others are left untouched).
 * row_len [B * S1] int32 or NULL: number of keys row t attends to.
 */
int dsa_indexer_logits_fp8(const void* q, const void* k, const float* key_scale,
                           const float* weights, const int32_t* act_q, const int32_t* act_k,
                           int64_t B, int64_t S1, int64_t S2, int32_t N1, int32_t D,
                           int32_t sparse_mode, float* logits, int64_t ld, int32_t* row_len,
                           void* stream);

/*
 * The same logits plus, per query row, the maximum of every group of 16
 * consecutive keys: group_max [B * S1, ld_g] fp32, ld_g >= ceil(S2 / 16) (groups
 * past a row's visible keys hold -inf or are not written).  This is the input
 * of dsa_topk_f32_group_max; dsa_lightning_indexer_fp8 chains the two.
 */
int dsa_indexer_logits_fp8_group_max(const void* q, const void* k, const float* key_scale,
                                     const float* weights, const int32_t* act_q, const int32_t* act_k,
                                     int64_t B, int64_t S1, int64_t S2, int32_t N1, int32_t D,
                                     int32_t sparse_mode, float* logits, int64_t ld, int32_t* row_len,
                                     float* group_max, int64_t ld_g, void* stream);

/*
 * Full lightning indexer: logits (above) then top-`sparse_count` per query row.
 * Replaces the whole `call` of make_lightning_indexer_kernel
 * (examples/deepseek_v4/lightning_indexer.py:338-1199) behind the host wrapper
 * lightning_indexer (:1202-1376) for the BSND layout with N2 = 1.
 * indices [B, S1, sparse_count] int32, values [B, S1, sparse_count] fp32 or NULL.
 * workspace: dsa_lightning_indexer_workspace_bytes(B, S1, S2) bytes.
 */
size_t dsa_lightning_indexer_workspace_bytes(int64_t B, int64_t S1, int64_t S2);
int dsa_lightning_indexer_fp8(const void* q, const void* k, const float* key_scale,
                              const float* weights, const int32_t* act_q, const int32_t* act_k,
                              int64_t B, int64_t S1, int64_t S2, int32_t N1, int32_t D,
                              int32_t sparse_count, int32_t sparse_mode, int32_t* indices,
                              float* values, void* workspace, size_t workspace_bytes,
                              void* stream);

/*
 * Indexer logits for the reference's other key / query layouts
 * (examples/deepseek_v4/lightning_indexer.py:1256-1302 with its conversions
 * :48-193), read in place instead of converted:
 *   seq_q: per-batch query lengths (seq_q_cumulative = 0; rows b * S1 + t, the
 *          BSND layout) or their prefix sums (= 1; rows seq_q[b-1] + t, the TND
 *          layout [T, N1, D]); NULL = S1 for every batch.
 *   seq_k: per-batch key lengths or prefix sums (TND keys [T2, D]); NULL = S2.
 *   block_table [B, max_blocks] or NULL: keys (and key_scale) live in a page pool
 *          of pool_rows = blocks * block_size rows (the PA_BSND layout
 *          [blocks, block_size, 1, D]); key s of batch b is pool row
 *          block_table[b, s / block_size] * block_size + s % block_size.  Takes
 *          per-batch key lengths.
 * S1 / S2 are the largest per-batch query / key lengths (larger lengths are
 * clipped to them); prefix sums must end at T, so that every query row belongs to
 * a batch.  logits has one row per query row (B * S1 padded, or T for prefix
 * sums); row_len likewise, as above.
 */
int dsa_indexer_logits_fp8_varlen(const void* q, const void* k, const float* key_scale,
                                  const float* weights, const int32_t* seq_q, int32_t seq_q_cumulative,
                                  const int32_t* seq_k, int32_t seq_k_cumulative,
                                  const int32_t* block_table, int32_t block_size, int32_t max_blocks,
                                  int64_t pool_rows, int64_t B, int64_t S1, int64_t S2, int32_t N1,
                                  int32_t D, int32_t sparse_mode, float* logits, int64_t ld,
                                  int32_t* row_len, void* stream);

/*
 * Full lightning indexer for those layouts: the logits above, then the top
 * `sparse_count` of each of the q_rows query rows (q_rows = B * S1 for padded
 * rows, T for prefix sums).  indices [q_rows, sparse_count] int32 (the TND output
 * [T, 1, K] of lightning_indexer.py:1365-1368 for prefix sums), values likewise
 * or NULL.  workspace: dsa_lightning_indexer_varlen_workspace_bytes(q_rows, S2).
 */
size_t dsa_lightning_indexer_varlen_workspace_bytes(int64_t q_rows, int64_t S2);
int dsa_lightning_indexer_fp8_varlen(const void* q, const void* k, const float* key_scale,
                                     const float* weights, const int32_t* seq_q, int32_t seq_q_cumulative,
                                     const int32_t* seq_k, int32_t seq_k_cumulative,
                                     const int32_t* block_table, int32_t block_size, int32_t max_blocks,
                                     int64_t pool_rows, int64_t B, int64_t S1, int64_t S2, int64_t q_rows,
                                     int32_t N1, int32_t D, int32_t sparse_count, int32_t sparse_mode,
                                     int32_t* indices, float* values, void* workspace,
                                     size_t workspace_bytes, void* stream);

/*
 * The same full indexer for the reference wrapper's own input dtypes: q
 * [q_rows, N1, 128] and k fp16 (is_f16 = 1) or bf16 (0), 1 <= N1 <= 64 heads,
 * weights [q_rows, N1] fp32 (lightning_indexer.py:1250-1255, 1284-1285).  q.k
 * accumulates the exact 16-bit products in fp32 (16-bit MFMA), as the golden
 * cpu_lightning_indexer computes in fp32 (:272-305).  key_scale (per key row) is
 * optional, as above; layouts, lengths, outputs and workspace as
 * dsa_lightning_indexer_fp8_varlen.  q and k must be 16-byte aligned.
 */
int dsa_lightning_indexer_h16_varlen(const void* q, const void* k, const float* key_scale,
                                     const float* weights, const int32_t* seq_q, int32_t seq_q_cumulative,
                                     const int32_t* seq_k, int32_t seq_k_cumulative,
                                     const int32_t* block_table, int32_t block_size, int32_t max_blocks,
                                     int64_t pool_rows, int64_t B, int64_t S1, int64_t S2, int64_t q_rows,
                                     int32_t N1, int32_t D, int32_t is_f16, int32_t sparse_count,
                                     int32_t sparse_mode, int32_t* indices, float* values, void* workspace,
                                     size_t workspace_bytes, void* stream);

/*
 * Sparse MLA forward: bf16 q [B, S, H, d_qk], one latent KV head, d_v = 512.
 * Replaces the `call` of sparse_attention_fwd
 * (examples/sparse_flash_attention/example_sparse_flash_attn.py:18-243, main(Q, KV,
 * Indices, Output, workspace_1..5)) and of the paged variant
 * (examples/sparse_flash_attention/bench_sfa/sparse_flash_attn_pa_no_cv_pipeline.py:27-377),
 * and adds the LSE output of the DeepSeek-V4 sparse flash MLA
 * (examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_kernel.py:2120-2131).
 *
 * kv: contiguous [B, skv, 1, d_qk] bf16 when block_table is NULL, else a page pool
 *     [num_blocks, block_size, 1, d_qk] addressed through block_table [B, max_blocks];
 *     then skv = num_blocks * block_size (pages outside the pool are skipped).
 * indices [B, S, 1, topk] int32; entries < 0, >= kv_len[b] (NULL: skv or
 *     max_blocks*block_size), on a page < 0, or (is_causal) > q_start[b] + s
 *     (q_start NULL: kv_len[b] - S) are skipped.
 * attn_sink [H] fp32 or NULL.  d_qk in {576, 512}.
 * out [B, S, H, 512] bf16, lse [B, S, H] fp32 (natural log) or NULL.
 * num_splits: index-list splits per token (0 = automatic); with more than one
 *     split the workspace must hold dsa_sparse_mla_workspace_bytes(...) bytes.
 */
size_t dsa_sparse_mla_workspace_bytes(int64_t B, int64_t S, int32_t H, int32_t topk,
                                      int32_t num_splits);
int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* indices,
                       const int32_t* block_table, const int32_t* kv_len, const int32_t* q_start,
                       const float* attn_sink, int64_t B, int64_t S, int32_t H, int32_t d_qk,
                       int32_t d_v, int64_t skv, int32_t block_size, int32_t max_blocks,
                       int32_t topk, float sm_scale, int32_t is_causal, int32_t num_splits,
                       void* out, float* lse, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * dsa_sparse_mla_fwd for fp16 q / kv, out [B, S, H, 512] fp16 (fp16 MFMA, the
 * probabilities rounded to fp16 before P.V).  Replaces the same calls as
 * dsa_sparse_mla_fwd built for the reference factory's default dtype, fp16
 * (examples/sparse_flash_attention/example_sparse_flash_attn.py:49, output
 * cast :292, driver :296).  Same arguments, rules and workspace otherwise.
 */
int dsa_sparse_mla_fwd_f16(const void* q, const void* kv, const int32_t* indices,
                           const int32_t* block_table, const int32_t* kv_len, const int32_t* q_start,
                           const float* attn_sink, int64_t B, int64_t S, int32_t H, int32_t d_qk,
                           int32_t d_v, int64_t skv, int32_t block_size, int32_t max_blocks,
                           int32_t topk, float sm_scale, int32_t is_causal, int32_t num_splits,
                           void* out, float* lse, void* workspace, size_t workspace_bytes,
                           void* stream);

/*
 * dsa_sparse_mla_fwd without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, results and kernels as dsa_sparse_mla_fwd; the
 * split partials go to a fixed array of DSA_SPARSE_MLA_SCRATCH_BYTES per GPU,
 * resident from the library's first call on that GPU until the process ends.
 * Calls whose partials need more (dsa_sparse_mla_workspace_bytes(...) above the
 * limit) return DSA_E_WORKSPACE_TOO_SMALL.  Every call on one GPU shares that
 * array, which keeps the last call's contents (each call writes every partial it
 * reads, so nothing needs clearing): calls that overlap on one GPU (concurrent
 * streams or threads) race and must be serialised by the caller.
 */
#define DSA_SPARSE_MLA_SCRATCH_BYTES ((size_t)64 << 20)
int dsa_sparse_mla_fwd_noalloc(const void* q, const void* kv, const int32_t* indices,
                               const int32_t* block_table, const int32_t* kv_len, const int32_t* q_start,
                               const float* attn_sink, int64_t B, int64_t S, int32_t H, int32_t d_qk,
                               int32_t d_v, int64_t skv, int32_t block_size, int32_t max_blocks,
                               int32_t topk, float sm_scale, int32_t is_causal, int32_t num_splits,
                               void* out, float* lse, void* stream);

/*
 * Block-sparse indexer logits (the HISA second stage): replaces the call of
 * paged_block_sparse_mqa_attn_return_logits
 * (examples/HISA/paged_block_sparse_mqa_attn_expert.py:54-422; reference
 * ref_paged_block_sparse_mqa_attn :425-468).
 *   q [batch * seq_len, heads, 128], weights [batch * seq_len, heads] (fp16, or
 *   bf16 with is_bf16 = 1); kv_cache [num_phys_blocks, kv_block_size, 1, 128];
 *   topk_block_indices [batch * seq_len, topk] logical blocks, block_tables
 *   [batch, max_blocks], context_lens [batch] int32.
 *   logits [batch * seq_len, topk, kv_block_size] fp32:
 *   sum_h w_h ReLU(q_h . k_j), -inf at positions >= context_lens[b] (and for a
 *   block id outside the table or a missing page).  heads in {16, 32, 48, 64},
 *   kv_block_size a multiple of 16.
 */
int dsa_block_sparse_indexer_logits(const void* q, const void* kv_cache, const int32_t* topk_block_indices,
                                    const void* weights, const int32_t* context_lens, const int32_t* block_tables,
                                    int64_t batch, int64_t seq_len, int32_t heads, int32_t index_dim, int32_t topk,
                                    int64_t num_phys_blocks, int32_t kv_block_size, int32_t max_blocks,
                                    int32_t is_bf16, float* logits, void* stream);

/*
 * DeepSeek-V4 sparse flash MLA: sliding window over the original KV plus the
 * compressed KV, with sinks.  Replaces the call behind sparse_flash_mla
 * (examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_api.py:94-253; kernel
 * sparse_flash_mla_kernel.py:1099-2166) with the golden's semantics
 * (sparse_flash_mla_golden.py:56-153).
 *   q [T, N1, 512] bf16; query row s of batch b is row q_prefix[b] + s for
 *     s < act_q_lens[b] (TND: q_prefix = cu_seqlens_q[:-1]; BSND: b * S);
 *     its position is seqused_kv[b] - act_q_lens[b] + s.
 *   ori_kv [ori_blocks, ori_block_size, 1, 512] bf16 + ori_block_table [B, ori_table_len]:
 *     the window of ori_win_left + 1 positions ending at the row's position.
 *   cmp_kv [cmp_blocks, cmp_block_size, 1, 512] + cmp_block_table, or NULL (window only):
 *     with cmp_sparse_indices [T, topk_cmp] int32 ("csa", n_cmp = topk_cmp) the
 *     listed compressed positions below floor((position + 1) / cmp_ratio), read
 *     up to the first -1; without ("hca") all compressed positions below it,
 *     n_cmp >= the largest such count (max(seqused_kv) / cmp_ratio).
 *   sinks [N1] fp32; K = V; out [T, N1, 512] bf16, lse [T, N1] fp32 (natural log)
 *   or NULL.  Rows outside every batch get out = 0.
 * workspace: dsa_sparse_flash_mla_workspace_bytes(T, N1, ori_win_left, n_cmp).
 */
size_t dsa_sparse_flash_mla_workspace_bytes(int64_t T, int32_t N1, int32_t ori_win_left, int32_t n_cmp);
int dsa_sparse_flash_mla(const void* q, int64_t T, int32_t N1, int32_t D, const int32_t* q_prefix,
                         const int32_t* act_q_lens, const int32_t* seqused_kv, int64_t B, const void* ori_kv,
                         int64_t ori_blocks, int32_t ori_block_size, const int32_t* ori_block_table,
                         int32_t ori_table_len, const void* cmp_kv, int64_t cmp_blocks, int32_t cmp_block_size,
                         const int32_t* cmp_block_table, int32_t cmp_table_len,
                         const int32_t* cmp_sparse_indices, int32_t topk_cmp, int32_t n_cmp, int32_t cmp_ratio,
                         const float* sinks, float softmax_scale, int32_t ori_win_left, void* out, float* lse,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * dsa_sparse_flash_mla for fp16 q / ori_kv / cmp_kv and an fp16 out (the API's
 * fp16 mapping, sparse_flash_mla_api.py:16-21).  Same arguments otherwise.
 */
int dsa_sparse_flash_mla_f16(const void* q, int64_t T, int32_t N1, int32_t D, const int32_t* q_prefix,
                             const int32_t* act_q_lens, const int32_t* seqused_kv, int64_t B, const void* ori_kv,
                             int64_t ori_blocks, int32_t ori_block_size, const int32_t* ori_block_table,
                             int32_t ori_table_len, const void* cmp_kv, int64_t cmp_blocks, int32_t cmp_block_size,
                             const int32_t* cmp_block_table, int32_t cmp_table_len,
                             const int32_t* cmp_sparse_indices, int32_t topk_cmp, int32_t n_cmp, int32_t cmp_ratio,
                             const float* sinks, float softmax_scale, int32_t ori_win_left, void* out, float* lse,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Row quantisation (the step before the indexer).  x is bf16 [rows, cols],
 * cols a multiple of 8, x 16-byte and y 8-byte aligned; one scale per row.
 *
 * dsa_act_quant_int8 replaces the call of act_quant_kernel_int8_optimized
 * (examples/deepseek_v4/act_quant.py:25-90, outputs Y [M, N] int8 and S [M] fp32)
 * with the golden's rule (act_quant_torch, :110-149): s = max(absmax, 1e-4) / 127
 * (round_scale = 1: 2^ceil(log2 of it), the fast_round_scale bit rule of
 * :93-107), y = round_half_even(clamp(x / s, -127, 127)).
 *
 * dsa_quant_fp8_rows: s = max(absmax / 448, FLT_MIN), y = e4m3fn(x / s) rounded
 * to nearest even — the per-key fp8 quantisation whose scale is the indexer's
 * key_scale (the fp8 producer of the lightning indexer,
 * examples/deepseek_v4/lightning_indexer.py:199-335 consumes its dequantised form).
 */
int dsa_act_quant_int8(const void* x, int64_t M, int64_t N, int32_t round_scale, int8_t* y,
                       float* scale, void* stream);
int dsa_quant_fp8_rows(const void* x, int64_t rows, int64_t cols, void* y, float* scale,
                       void* stream);

/*
 * Quantise-on-append for a paged fp8 key cache in the indexer's PA_BSND layout
 * (pool [blocks, block_size, 1, D] + key_scale [blocks, block_size],
 * lightning_indexer.py:271-292): new bf16 keys k [T, D] are quantised with the
 * dsa_quant_fp8_rows rule and written to pool row slots[t] (= page * block_size
 * + offset; -1 or >= pool_rows: dropped) together with their scale, in one pass.
 */
int dsa_indexer_k_append_fp8(const void* k, int64_t T, int32_t D, const int64_t* slots,
                             int64_t pool_rows, void* pool, float* pool_scale, void* stream);

/*
 * Indexer query producer: bf16 q [T, N1, D] -> fp8 q8 [T, N1, D] with one scale
 * per (token, head), folded into the head weights: weights_out[t, h] =
 * weights[t, h] * s[t, h] (exact for the ReLU score, since
 * w * ReLU(s * q8 . k) = (w * s) * ReLU(q8 . k) for s > 0), so the indexer takes
 * q8 and weights_out unchanged (lightning_indexer.py:199-335).
 */
int dsa_indexer_q_quant_fp8(const void* q, const float* weights, int64_t T, int32_t N1, int32_t D,
                            void* q8, float* weights_out, void* stream);

/*
 * dsa_quant_fp8_rows and dsa_indexer_q_quant_fp8 for fp16 inputs (same rules,
 * same outputs).  They let the lightning indexer take the reference's fp16 q / k
 * (lightning_indexer.py:1250-1255) by quantising them on the device.
 */
int dsa_quant_fp8_rows_f16(const void* x, int64_t rows, int64_t cols, void* y, float* scale, void* stream);
int dsa_indexer_q_quant_fp8_f16(const void* q, const float* weights, int64_t T, int32_t N1, int32_t D,
                                void* q8, float* weights_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_MI355X_H_ */
