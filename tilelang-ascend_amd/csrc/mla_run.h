// Internal entry of the sparse MLA forward shared by the C-ABI functions that
// reach it (plain / paged indices, and lists of already resolved pool rows).
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace dsa {

// In a list of resolved rows, this bit marks a row of the second pool.
constexpr int kRowTag2 = 1 << 30;

// DeepSeek-V4 key sets (sliding window over the original cache + compressed
// keys), generated per query row inside the sparse MLA kernel instead of read
// from an index list: slot j < win is original position max(sg - win + 1, 0) + j
// (sg = the row's position), slot win + i is compressed position i (scenario 2,
// all below floor((sg + 1) / cmp_ratio)) or the i-th entry of the row's list
// (scenario 3, read up to its first -1 and the first min(K, threshold) entries,
// kept when below the threshold and floor(seqused_kv / cmp_ratio)).
struct V4Keys {
  const int32_t* q_prefix;    // [B] first query row of each batch
  const int32_t* act_q;       // [B] query rows of each batch
  const int32_t* seqused_kv;  // [B] original KV length of each batch
  const int32_t* ori_bt;      // [B, ori_tl]
  const int32_t* cmp_bt;      // [B, cmp_tl] or null
  const int32_t* cmp_idx;     // [T, K] or null
  int64_t ori_rows, cmp_rows;
  int ori_bs, ori_tl, cmp_bs, cmp_tl;
  int B, K, n_cmp, scenario, cmp_ratio, win;
};

#ifdef __HIPCC__
__device__ __forceinline__ int v4_floordiv(int a, int b) {
  const int q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

__device__ __forceinline__ int32_t v4_page_row(const int32_t* bt, int tl, int bs, int64_t pool_rows, int b,
                                               int pos) {
  const int blk = pos / bs;
  const int page = blk < tl ? bt[(int64_t)b * tl + blk] : -1;
  const int64_t r = (int64_t)page * bs + pos % bs;
  return (page >= 0 && r < pool_rows) ? (int32_t)r : -1;
}

// Batch of query row t (the last with q_prefix <= t, prefixes ascending), or -1
// when t lies in no batch's rows.
__device__ __forceinline__ int v4_batch(const V4Keys& v, int64_t t) {
  int lo = 0, hi = v.B - 1, b = -1;
  while (lo <= hi) {
    const int mid = (lo + hi) >> 1;
    if (v.q_prefix[mid] <= t) {
      b = mid;
      lo = mid + 1;
    } else {
      hi = mid - 1;
    }
  }
  if (b >= 0 && t >= (int64_t)v.q_prefix[b] + v.act_q[b]) b = -1;
  return b;
}

// Resolved row of key slot j of query row t (batch b), or -1.  `stop`: position
// of the first -1 in the row's compressed list (scenario 3).
__device__ __forceinline__ int32_t v4_row(const V4Keys& v, int64_t t, int b, int j, int stop) {
  const int act_q = v.act_q[b], act_kv = v.seqused_kv[b];
  const int sg = act_kv - act_q + (int)(t - v.q_prefix[b]);
  if (j < v.win) {
    const int pos = (sg - (v.win - 1) > 0 ? sg - (v.win - 1) : 0) + j;
    return pos <= sg ? v4_page_row(v.ori_bt, v.ori_tl, v.ori_bs, v.ori_rows, b, pos) : -1;
  }
  const int i = j - v.win;
  if (v.scenario == 1 || i >= v.n_cmp) return -1;
  const int thr = v4_floordiv(sg + 1, v.cmp_ratio);
  int pos = -1;
  if (v.scenario == 2) {
    pos = i < thr ? i : -1;
  } else {
    const int n = min(min(v.K, thr > 0 ? thr : 0), stop);
    if (i < n) {
      const int e = v.cmp_idx[t * v.K + i];
      if (e >= 0 && e < thr && e < v4_floordiv(act_kv, v.cmp_ratio)) pos = e;
    }
  }
  if (pos < 0) return -1;
  const int32_t r = v4_page_row(v.cmp_bt, v.cmp_tl, v.cmp_bs, v.cmp_rows, b, pos);
  return r >= 0 ? (r | kRowTag2) : -1;
}
#endif

struct MlaRun {
  const void* q;               // [B * S, H, d_qk], bf16 (fp16 when f16)
  const void* kv;              // rows [*, d_qk] (batch rows, a page pool, or pool 1), q's type
  const int32_t* indices;      // [B * S, topk]
  const int32_t* block_table;  // [B, max_blocks] or null
  const int32_t* kv_len;       // [B] or null
  const int32_t* q_start;      // [B] or null
  const float* attn_sink;      // [H] or null
  const V4Keys* v4;            // key sets generated per row (indices unused), or null
  const void* kv2;             // pool 2 of resolved rows, or null
  int64_t pool_rows2;
  int direct;                  // indices are resolved rows (kRowTag2 selects pool 2)
  int64_t B, S;
  int32_t H, d_qk, d_v;
  int64_t skv;                 // rows per batch, or rows in the (first) pool
  int32_t block_size, max_blocks, topk;
  float sm_scale;
  int32_t is_causal, num_splits;
  int32_t f16;                 // q, kv and out are IEEE half instead of bfloat16
  void* out;
  float* lse;
  void* workspace;
  size_t workspace_bytes;
  void* stream;
};

int sparse_mla_run(const MlaRun& r, const char* what);
size_t sparse_mla_split_bytes(int64_t T, int32_t H, int32_t topk, int32_t num_splits);

}  // namespace dsa
