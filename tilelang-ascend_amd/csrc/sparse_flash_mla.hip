// DeepSeek-V4 sparse flash MLA on gfx950: sliding-window attention over the
// original KV cache plus attention over compressed KV tokens, with sinks
// (examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_api.py:94-253, golden
// sparse_flash_mla_golden.py:56-153).
//
// For query row s of batch b (s_global = seqused_kv[b] - act_q[b] + s) the keys are
//   * the window: original positions max(s_global - win_left, 0) .. s_global;
//   * compressed positions (t = floor((s_global + 1) / cmp_ratio)):
//       scenario 2 ("hca"): all of 0 .. t - 1;
//       scenario 3 ("csa"): the first min(K, t) entries of its top-k list, up to
//       the first -1, each kept when < t and < floor(seqused_kv / cmp_ratio);
// each cache paged through its own block table.  K = V (D = 512), one KV head
// shared by N1 query heads, a per-head sink in the softmax denominator, and
// LSE = m + ln(sum).
//
// The sparse MLA core generates each query row's key slots itself (window slots,
// then compressed slots), applies the rules and the two page tables while it
// resolves them to physical rows (bit 30 marks the compressed pool), and gathers
// those rows straight into LDS as it does for any index list: one launch, no
// index list in memory.
#include "dsa_common.h"
#include "mla_run.h"

extern "C" size_t dsa_sparse_flash_mla_workspace_bytes(int64_t T, int32_t N1, int32_t ori_win_left,
                                                       int32_t n_cmp) {
  if (T <= 0 || ori_win_left < 0 || n_cmp < 0) return 0;
  return dsa::sparse_mla_split_bytes(T, N1, ori_win_left + 1 + n_cmp, 0);
}

namespace {

int flash_mla_entry(const void* q, int64_t T, int32_t N1, int32_t D, const int32_t* q_prefix,
                    const int32_t* act_q_lens, const int32_t* seqused_kv, int64_t B, const void* ori_kv,
                    int64_t ori_blocks, int32_t ori_block_size, const int32_t* ori_block_table, int32_t ori_table_len,
                    const void* cmp_kv, int64_t cmp_blocks, int32_t cmp_block_size, const int32_t* cmp_block_table,
                    int32_t cmp_table_len, const int32_t* cmp_sparse_indices, int32_t topk_cmp, int32_t n_cmp,
                    int32_t cmp_ratio, const float* sinks, float softmax_scale, int32_t ori_win_left, void* out,
                    float* lse, void* workspace, size_t workspace_bytes, void* stream, int32_t f16,
                    const char* what) {
  using namespace dsa;
  if (D != 512) return set_error(kUnsupported, "%s: only D = 512 is built (got %d)", what, D);
  if (T < 0 || B < 0 || N1 <= 0 || ori_win_left < 0 || n_cmp < 0)
    return set_error(kInvalidArgument, "%s: bad sizes", what);
  const int scenario = cmp_kv == nullptr ? 1 : (cmp_sparse_indices == nullptr ? 2 : 3);
  if (scenario == 1) n_cmp = 0;
  if (scenario == 3 && (topk_cmp <= 0 || n_cmp != topk_cmp))
    return set_error(kInvalidArgument, "%s: selected compressed keys need n_cmp = topk_cmp > 0", what);
  if (scenario >= 2 && (cmp_ratio <= 0 || cmp_block_table == nullptr || cmp_block_size <= 0 || cmp_table_len <= 0))
    return set_error(kInvalidArgument, "%s: compressed KV needs cmp_ratio, a block table and a block size", what);
  if (ori_block_table == nullptr || ori_block_size <= 0 || ori_table_len <= 0 || ori_kv == nullptr)
    return set_error(kInvalidArgument, "%s: the original KV needs a block table and a block size", what);
  if (T == 0 || B == 0) return kOk;
  if (q == nullptr || q_prefix == nullptr || act_q_lens == nullptr || seqused_kv == nullptr || out == nullptr ||
      sinks == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", what);
  if (T > 0x7fffffff || B > 0x7fffffff) return set_error(kUnsupported, "%s: too many rows", what);
  const int64_t L64 = (int64_t)ori_win_left + 1 + n_cmp;
  if (L64 > 0x7fffffff) return set_error(kUnsupported, "%s: key list too long", what);
  const int L = (int)L64;
  const size_t need = dsa_sparse_flash_mla_workspace_bytes(T, N1, ori_win_left, n_cmp);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return set_error(kWorkspaceTooSmall, "%s: workspace of %zu bytes needed, %zu given", what, need,
                     workspace_bytes);
  const int64_t ori_rows = ori_blocks * ori_block_size, cmp_rows = scenario >= 2 ? cmp_blocks * cmp_block_size : 0;
  if (ori_rows > kRowTag2 || cmp_rows > kRowTag2)
    return set_error(kUnsupported, "%s: pools of more than 2^30 rows", what);

  V4Keys v;
  v.q_prefix = q_prefix;
  v.act_q = act_q_lens;
  v.seqused_kv = seqused_kv;
  v.ori_bt = ori_block_table;
  v.cmp_bt = cmp_block_table;
  v.cmp_idx = cmp_sparse_indices;
  v.ori_rows = ori_rows;
  v.cmp_rows = cmp_rows;
  v.ori_bs = ori_block_size;
  v.ori_tl = ori_table_len;
  v.cmp_bs = cmp_block_size;
  v.cmp_tl = cmp_table_len;
  v.B = (int)B;
  v.K = scenario == 3 ? topk_cmp : 0;
  v.n_cmp = n_cmp;
  v.scenario = scenario;
  v.cmp_ratio = cmp_ratio > 0 ? cmp_ratio : 1;
  v.win = ori_win_left + 1;

  MlaRun r{};
  r.q = q;
  r.kv = ori_kv;
  r.kv2 = cmp_kv;
  r.pool_rows2 = cmp_rows;
  r.direct = 1;
  r.v4 = &v;
  r.indices = nullptr;
  r.attn_sink = sinks;
  r.B = 1;
  r.S = T;
  r.H = N1;
  r.d_qk = 512;
  r.d_v = 512;
  r.skv = ori_rows;
  r.topk = L;
  r.sm_scale = softmax_scale;
  r.is_causal = 0;
  r.num_splits = 0;
  r.out = out;
  r.lse = lse;
  r.workspace = workspace;
  r.workspace_bytes = workspace_bytes;
  r.stream = stream;
  r.f16 = f16;
  return sparse_mla_run(r, what);
}

}  // namespace

extern "C" int dsa_sparse_flash_mla(const void* q, int64_t T, int32_t N1, int32_t D, const int32_t* q_prefix,
                                    const int32_t* act_q_lens, const int32_t* seqused_kv, int64_t B,
                                    const void* ori_kv, int64_t ori_blocks, int32_t ori_block_size,
                                    const int32_t* ori_block_table, int32_t ori_table_len, const void* cmp_kv,
                                    int64_t cmp_blocks, int32_t cmp_block_size, const int32_t* cmp_block_table,
                                    int32_t cmp_table_len, const int32_t* cmp_sparse_indices, int32_t topk_cmp,
                                    int32_t n_cmp, int32_t cmp_ratio, const float* sinks, float softmax_scale,
                                    int32_t ori_win_left, void* out, float* lse, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  return flash_mla_entry(q, T, N1, D, q_prefix, act_q_lens, seqused_kv, B, ori_kv, ori_blocks, ori_block_size,
                         ori_block_table, ori_table_len, cmp_kv, cmp_blocks, cmp_block_size, cmp_block_table,
                         cmp_table_len, cmp_sparse_indices, topk_cmp, n_cmp, cmp_ratio, sinks, softmax_scale,
                         ori_win_left, out, lse, workspace, workspace_bytes, stream, 0, "dsa_sparse_flash_mla");
}

extern "C" int dsa_sparse_flash_mla_f16(const void* q, int64_t T, int32_t N1, int32_t D, const int32_t* q_prefix,
                                        const int32_t* act_q_lens, const int32_t* seqused_kv, int64_t B,
                                        const void* ori_kv, int64_t ori_blocks, int32_t ori_block_size,
                                        const int32_t* ori_block_table, int32_t ori_table_len, const void* cmp_kv,
                                        int64_t cmp_blocks, int32_t cmp_block_size, const int32_t* cmp_block_table,
                                        int32_t cmp_table_len, const int32_t* cmp_sparse_indices, int32_t topk_cmp,
                                        int32_t n_cmp, int32_t cmp_ratio, const float* sinks, float softmax_scale,
                                        int32_t ori_win_left, void* out, float* lse, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return flash_mla_entry(q, T, N1, D, q_prefix, act_q_lens, seqused_kv, B, ori_kv, ori_blocks, ori_block_size,
                         ori_block_table, ori_table_len, cmp_kv, cmp_blocks, cmp_block_size, cmp_block_table,
                         cmp_table_len, cmp_sparse_indices, topk_cmp, n_cmp, cmp_ratio, sinks, softmax_scale,
                         ori_win_left, out, lse, workspace, workspace_bytes, stream, 1, "dsa_sparse_flash_mla_f16");
}
