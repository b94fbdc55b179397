// Block-sparse indexer logits on gfx950 (the HISA second stage): for every query
// token and each of its top-k logical key blocks, the lightning-indexer score of
// every key in the block,
//   logits[t, i, j] = sum_h w[t, h] * ReLU(q[t, h, :] . K[page, j, :])
//   page = block_tables[b, blk[t, i]],  -inf where blk * block_size + j >= context_lens[b]
// (examples/HISA/paged_block_sparse_mqa_attn_expert.py:54-424, reference
// ref_paged_block_sparse_mqa_attn :425-468).  fp16 or bf16 q / keys / weights,
// fp32 accumulation and output.
//
// One workgroup (4 waves) per token and up to four of its blocks (fewer when the
// grid would drop under 256 workgroups); wave w takes each
// block's 16-key tiles w, w + 4, ... and loads its keys of the next block before
// scoring the current one.  Per tile and 16-head group, four v_mfma_f32_16x16x32
// (A = q rows of 16 heads, B = K^T of 16 keys, K = 128 dims) leave lane (g, c)
// with heads 4g .. 4g + 3 of key c; ReLU * w is summed over the lane's heads and
// head groups, then over the four lane groups with permlane swaps.  Keys are
// read straight from HBM into registers (each key row is used by every head
// group of the wave, never by another wave), q and w once per workgroup.  The
// kernel is HBM bound: 2 * index_dim bytes per key in, 4 bytes per key out.
#include "dsa_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kDim = 128;

typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;

struct BsParams {
  const uint16_t* q;        // [T, H, 128]
  const uint16_t* kv;       // [num_blocks, bs, 1, 128]
  const int32_t* blk;       // [T, topk] logical block ids
  const uint16_t* w;        // [T, H]
  const int32_t* ctx;       // [batch]
  const int32_t* bt;        // [batch, max_blocks]
  float* out;               // [T, topk, bs]
  int64_t num_blocks;
  int seq_len, topk, bs, max_blocks;
  int spg;                  // blocks of one token per workgroup (1, 2 or 4)
};

template <bool BF16>
__device__ __forceinline__ float to_f32(uint16_t h) {
  if constexpr (BF16) return __uint_as_float((uint32_t)h << 16);
  else return (float)__builtin_bit_cast(_Float16, h);
}

template <bool BF16>
__device__ __forceinline__ dsa::f32x4 mfma(const dsa::i32x4& a, const dsa::i32x4& b, const dsa::f32x4& c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dsa::bf16x8, a), __builtin_bit_cast(dsa::bf16x8, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int HG, bool BF16>
__global__ __launch_bounds__(kWaves * 64) void block_sparse_indexer_kernel(BsParams p) {
  // workgroup -> (token, up to spg consecutive block slots); a wave's keys of the
  // next block are loaded before the current block is scored
  const int ngroups = (p.topk + p.spg - 1) / p.spg;
  const int64_t t = blockIdx.x / ngroups;
  const int slot0 = (int)(blockIdx.x % ngroups) * p.spg;
  const int nslots = min(p.spg, p.topk - slot0);
  const int b = (int)(t / p.seq_len);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int ntiles = p.bs >> 4;
  const int ctx = p.ctx[b];

  // q rows (A operands): head group hg, k-step ks -> head 16 hg + c, dims 32 ks + 8 g .. + 7
  dsa::i32x4 qa[HG][4];
  float wv[HG][4];
  const uint16_t* qt = p.q + t * (int64_t)(16 * HG) * kDim;
#pragma unroll
  for (int hg = 0; hg < HG; ++hg) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qa[hg][ks] = *reinterpret_cast<const dsa::i32x4*>(qt + (16 * hg + c) * kDim + 32 * ks + 8 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[hg][r] = to_f32<BF16>(p.w[t * (16 * HG) + 16 * hg + 4 * g + r]);
  }

  // page of slot i (-1: no such block)
  auto page_of = [&](int i, int& lb) {
    lb = p.blk[t * p.topk + slot0 + i];
    const int pg = (lb >= 0 && lb < p.max_blocks) ? p.bt[(int64_t)b * p.max_blocks + lb] : -1;
    return (pg >= 0 && pg < p.num_blocks) ? pg : -1;
  };
  // this wave's tiles of a block: kt = wave + kWaves u, u < kTiles (bs <= 16 kWaves kTiles is
  // handled by the outer loop below)
  constexpr int kTiles = 2;
  auto load = [&](dsa::i32x4 (&kf)[kTiles][4], int pg, int kt0) {
    const uint16_t* kb = p.kv + (int64_t)(pg < 0 ? 0 : pg) * p.bs * kDim;
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
      const int kt = kt0 + u * kWaves;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)  // B operands: key 16 kt + c, dims 32 ks + 8 g .. + 7
        kf[u][ks] = (pg >= 0 && kt < ntiles)
                        ? *reinterpret_cast<const dsa::i32x4*>(kb + (16 * kt + c) * kDim + 32 * ks + 8 * g)
                        : dsa::i32x4{0, 0, 0, 0};
    }
  };
  auto score = [&](const dsa::i32x4 (&kf)[kTiles][4], int pg, int lb, int kt0, float* orow) {
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
      const int kt = kt0 + u * kWaves;
      if (kt >= ntiles) break;  // wave-uniform
      const int key = 16 * kt + c;
      if (pg < 0) {
        if (g == 0) orow[key] = -__builtin_inff();
        continue;
      }
      float acc = 0.f;
#pragma unroll
      for (int hg = 0; hg < HG; ++hg) {
        dsa::f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) d = mfma<BF16>(qa[hg][ks], kf[u][ks], d);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc = fmaf(wv[hg][r], fmaxf(d[r], 0.f), acc);
      }
      acc = dsa::xor32_sum(dsa::xor16_sum(acc));
      if (g == 0) orow[key] = (int64_t)lb * p.bs + key < ctx ? acc : -__builtin_inff();
    }
  };

  for (int kt0 = wave; kt0 < ntiles; kt0 += kWaves * kTiles) {
    dsa::i32x4 ka[kTiles][4], kn[kTiles][4];
    int lba, lbn;
    int pga = page_of(0, lba);
    load(ka, pga, kt0);
    for (int i = 0; i < nslots; ++i) {
      int pgn = -1;
      lbn = 0;
      if (i + 1 < nslots) {
        pgn = page_of(i + 1, lbn);
        load(kn, pgn, kt0);
      }
      score(ka, pga, lba, kt0, p.out + (t * p.topk + slot0 + i) * p.bs);
      if (i + 1 < nslots) {
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) ka[u][ks] = kn[u][ks];
        pga = pgn;
        lba = lbn;
      }
    }
  }
}

template <int HG>
int launch_hg(const BsParams& p, int64_t tokens, bool bf16, hipStream_t st) {
  const int64_t grid = tokens * ((p.topk + p.spg - 1) / p.spg);
  if (bf16)
    hipLaunchKernelGGL((block_sparse_indexer_kernel<HG, true>), dim3((unsigned)grid), dim3(kWaves * 64), 0, st, p);
  else
    hipLaunchKernelGGL((block_sparse_indexer_kernel<HG, false>), dim3((unsigned)grid), dim3(kWaves * 64), 0, st, p);
  return dsa::check_launch("dsa_block_sparse_indexer_logits");
}

}  // namespace

extern "C" int dsa_block_sparse_indexer_logits(const void* q, const void* kv_cache, const int32_t* topk_block_indices,
                                               const void* weights, const int32_t* context_lens,
                                               const int32_t* block_tables, int64_t batch, int64_t seq_len,
                                               int32_t heads, int32_t index_dim, int32_t topk, int64_t num_phys_blocks,
                                               int32_t kv_block_size, int32_t max_blocks, int32_t is_bf16,
                                               float* logits, void* stream) {
  using namespace dsa;
  const char* what = "dsa_block_sparse_indexer_logits";
  if (index_dim != kDim) return set_error(kUnsupported, "%s: index_dim must be 128 (got %d)", what, index_dim);
  if (heads <= 0 || heads % 16 != 0 || heads > 64)
    return set_error(kUnsupported, "%s: heads must be 16, 32, 48 or 64 (got %d)", what, heads);
  if (kv_block_size <= 0 || kv_block_size % 16 != 0)
    return set_error(kInvalidArgument, "%s: kv_block_size must be a positive multiple of 16 (got %d)", what,
                     kv_block_size);
  if (batch < 0 || seq_len < 0 || topk < 0 || max_blocks <= 0 || num_phys_blocks < 0)
    return set_error(kInvalidArgument, "%s: bad sizes", what);
  const int64_t items = batch * seq_len * topk;
  if (items == 0) return kOk;
  if (items > 0x7fffffff) return set_error(kUnsupported, "%s: too many (token, block) pairs", what);
  if (q == nullptr || kv_cache == nullptr || topk_block_indices == nullptr || weights == nullptr ||
      context_lens == nullptr || block_tables == nullptr || logits == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", what);
  BsParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.kv = static_cast<const uint16_t*>(kv_cache);
  p.blk = topk_block_indices;
  p.w = static_cast<const uint16_t*>(weights);
  p.ctx = context_lens;
  p.bt = block_tables;
  p.out = logits;
  p.num_blocks = num_phys_blocks;
  p.seq_len = (int)seq_len;
  p.topk = topk;
  p.bs = kv_block_size;
  p.max_blocks = max_blocks;
  hipStream_t st = (hipStream_t)stream;
  const int64_t tokens = batch * seq_len;
  // four blocks per workgroup unless that leaves fewer than 256 workgroups (one
  // token's 64 blocks: 4.5 us as 64 workgroups, 8.7 us as 16)
  p.spg = 1;
  while (p.spg < 4 && tokens * ((topk + 2 * p.spg - 1) / (2 * p.spg)) >= 256) p.spg *= 2;
  switch (heads / 16) {
    case 1: return launch_hg<1>(p, tokens, is_bf16 != 0, st);
    case 2: return launch_hg<2>(p, tokens, is_bf16 != 0, st);
    case 3: return launch_hg<3>(p, tokens, is_bf16 != 0, st);
    default: return launch_hg<4>(p, tokens, is_bf16 != 0, st);
  }
}
