// Lightning-indexer logits on gfx950 fp8 MFMA.
//
//   logits[b, t, s] = key_scale[b, s] * sum_h w[b, t, h] * ReLU(q[b, t, h, :] . k[b, s, :])
//
// with the causal rule of the reference golden (examples/deepseek_v4/lightning_indexer.py:303-314):
// for sparse_mode 3 row t sees keys s < ak - aq + t + 1, and a row whose causal
// length is <= 0 sees all ak keys; sparse_mode 0 sees all ak keys; rows t >= aq
// see none.  q and k are fp8 e4m3 (OCP, torch.float8_e4m3fn); the per-key fp32
// scale is applied after the head sum, which is exact because scale > 0.
//
// Work decomposition.  One workgroup = 8 waves = 16 query tokens of one batch
// row x one chunk of keys.  Each wave holds the A operands of its 2 tokens
// (64 heads x 128 dims each) in registers and streams 64-key tiles of K from a
// double-buffered LDS ring.  One v_mfma_scale_f32_16x16x128_f8f6f4 computes a
// 16-head x 16-key block over the whole 128-dim head, so the ReLU, the head
// weight and the head sum are applied to the accumulator registers directly and
// only the final fp32 logit is written to HBM.  Workgroups that share a key
// chunk are placed on the same XCD so the chunk stays in that XCD's L2.
#include "dsa_common.h"

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kTokPerWave = 2;
constexpr int kTokPerBlock = kWaves * kTokPerWave;  // 16
constexpr int kHeads = 64;
constexpr int kDim = 128;
constexpr int kKeyTile = 64;
constexpr int kRowBytes = kDim + 16;  // padded LDS row: conflict-free 16-byte reads

struct IndexerParams {
  const uint8_t* q;        // [B, S1, 64, 128] fp8
  const uint8_t* k;        // [B, S2, 128] fp8
  const float* key_scale;  // [B, S2] or null
  const float* w;          // [B, S1, 64]
  const int32_t* act_q;    // [B] or null
  const int32_t* act_k;    // [B] or null
  float* logits;           // [B * S1, ld]
  int32_t* row_len;        // [B * S1] or null
  int64_t ld;
  int B, S1, S2, sparse_mode;
  int chunk, ntb, nkc;
};

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Number of leading keys row t of a batch with (aq, ak) attends to.
__device__ __forceinline__ int visible_keys(int t, int aq, int ak, int sparse_mode) {
  if (t >= aq) return 0;
  if (sparse_mode == 3) {
    int cl = ak - aq + t + 1;
    return cl > 0 ? cl : ak;
  }
  return ak;
}

__global__ __launch_bounds__(kThreads) void indexer_fp8_kernel(IndexerParams p) {
  __shared__ __align__(16) uint8_t ktile[2][kKeyTile * kRowBytes];
  __shared__ float kscale[2][kKeyTile];

  // XCD-aware mapping: key groups (b, chunk) are dealt to XCDs, all token blocks
  // of one key group run on the same XCD.
  const int bid = blockIdx.x;
  const int xcd = bid % dsa::kNumXcd, r = bid / dsa::kNumXcd;
  const int kg = xcd + dsa::kNumXcd * (r / p.ntb);
  const int tb = r % p.ntb;
  if (kg >= p.B * p.nkc) return;
  const int b = kg / p.nkc, kc = kg % p.nkc;

  const int aq = p.act_q ? clampi(p.act_q[b], 0, p.S1) : p.S1;
  const int ak = p.act_k ? clampi(p.act_k[b], 0, p.S2) : p.S2;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;

  // Key range of this workgroup: its chunk, clipped to what its tokens can see.
  int lmax = 0;
#pragma unroll
  for (int i = 0; i < kTokPerBlock; ++i) {
    const int t = tb * kTokPerBlock + i;
    if (t < p.S1) lmax = max(lmax, visible_keys(t, aq, ak, p.sparse_mode));
  }
  const int k0 = kc * p.chunk;
  const int kend = min(k0 + p.chunk, p.S2);  // last key this workgroup may write
  const int k1 = min(kend, lmax);            // last key any token needs

  int tok[kTokPerWave], L[kTokPerWave];
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    tok[j] = tb * kTokPerBlock + wave * kTokPerWave + j;
    L[j] = tok[j] < p.S1 ? visible_keys(tok[j], aq, ak, p.sparse_mode) : 0;
  }
  if (kc == 0 && p.row_len != nullptr && lane == 0) {
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j)
      if (tok[j] < p.S1) p.row_len[(int64_t)b * p.S1 + tok[j]] = L[j];
  }
  if (k0 >= k1) return;

  // A operands: lane (g, c) holds head 16*mt + c, bytes [32g, 32g+32) of the head.
  dsa::i32x8 qa[kTokPerWave][4];
  float wt[kTokPerWave][4][4];
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    const bool ok = tok[j] < p.S1;
    const int64_t trow = (int64_t)b * p.S1 + (ok ? tok[j] : 0);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const dsa::i32x4* src =
          reinterpret_cast<const dsa::i32x4*>(p.q + (trow * kHeads + 16 * mt + c) * kDim + 32 * g);
      dsa::i32x4 lo = ok ? src[0] : dsa::i32x4{0, 0, 0, 0};
      dsa::i32x4 hi = ok ? src[1] : dsa::i32x4{0, 0, 0, 0};
      qa[j][mt] = dsa::i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int i = 0; i < 4; ++i) wt[j][mt][i] = ok ? p.w[trow * kHeads + 16 * mt + 4 * g + i] : 0.f;
    }
  }

  // Staging: thread tid copies 16 bytes of key (tid / 8), part (tid % 8).
  const int skey = tid >> 3, spart = tid & 7;
  const uint8_t* kbase = p.k + (int64_t)b * p.S2 * kDim;
  const float* sbase = p.key_scale ? p.key_scale + (int64_t)b * p.S2 : nullptr;
  auto load_tile = [&](int kt0, dsa::i32x4& v, float& sc) {
    const int key = kt0 + skey;
    v = key < k1 ? *reinterpret_cast<const dsa::i32x4*>(kbase + (int64_t)key * kDim + spart * 16)
                 : dsa::i32x4{0, 0, 0, 0};
    sc = 1.f;
    if (tid < kKeyTile) {
      const int key2 = kt0 + tid;
      sc = (sbase && key2 < k1) ? sbase[key2] : 1.f;
    }
  };
  auto store_tile = [&](int buf, const dsa::i32x4& v, float sc) {
    *reinterpret_cast<dsa::i32x4*>(&ktile[buf][skey * kRowBytes + spart * 16]) = v;
    if (tid < kKeyTile) kscale[buf][tid] = sc;
  };

  const int ntiles = (k1 - k0 + kKeyTile - 1) / kKeyTile;
  {
    dsa::i32x4 v;
    float sc;
    load_tile(k0, v, sc);
    store_tile(0, v, sc);
  }
  __syncthreads();

  const dsa::f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    const int kt0 = k0 + it * kKeyTile;
    dsa::i32x4 nv;
    float nsc;
    const bool more = it + 1 < ntiles;
    if (more) load_tile(kt0 + kKeyTile, nv, nsc);

    float res[kTokPerWave][4];
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const uint8_t* rp = &ktile[buf][(blk * 16 + c) * kRowBytes + 32 * g];
      const dsa::i32x4 b0 = *reinterpret_cast<const dsa::i32x4*>(rp);
      const dsa::i32x4 b1 = *reinterpret_cast<const dsa::i32x4*>(rp + 16);
      const dsa::i32x8 bf = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
      for (int j = 0; j < kTokPerWave; ++j) {
        float acc = 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          // D[row = head 16mt + 4g + i][col = key blk*16 + c]
          const dsa::f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              qa[j][mt], bf, zero, 0, 0, 0, 127, 0, 127);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc = fmaf(wt[j][mt][i], fmaxf(d[i], 0.f), acc);
        }
        acc += __shfl_xor(acc, 16, 64);
        acc += __shfl_xor(acc, 32, 64);
        res[j][blk] = acc;
      }
    }

    // lane (g, c) writes key kt0 + 16g + c
    const int s = kt0 + lane;
    const float sc = kscale[buf][lane];
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j) {
      if (tok[j] < p.S1 && s < kend) {
        float v = g == 0 ? res[j][0] : (g == 1 ? res[j][1] : (g == 2 ? res[j][2] : res[j][3]));
        v = s < L[j] ? v * sc : -__builtin_inff();
        __builtin_nontemporal_store(v, p.logits + ((int64_t)b * p.S1 + tok[j]) * p.ld + s);
      }
    }
    if (more) store_tile(buf ^ 1, nv, nsc);
    __syncthreads();
  }
}

}  // namespace

namespace dsa {

int indexer_fp8_launch(const uint8_t* q, const uint8_t* k, const float* key_scale, const float* w,
                       const int32_t* act_q, const int32_t* act_k, int B, int S1, int S2,
                       int sparse_mode, float* logits, int64_t ld, int32_t* row_len,
                       hipStream_t stream) {
  IndexerParams p;
  p.q = q;
  p.k = k;
  p.key_scale = key_scale;
  p.w = w;
  p.act_q = act_q;
  p.act_k = act_k;
  p.logits = logits;
  p.row_len = row_len;
  p.ld = ld;
  p.B = B;
  p.S1 = S1;
  p.S2 = S2;
  p.sparse_mode = sparse_mode;
  p.ntb = (S1 + kTokPerBlock - 1) / kTokPerBlock;
  // Aim for >= 4 workgroups per CU over the whole launch while keeping each
  // workgroup's key chunk a multiple of the LDS tile.
  int chunk = 4096;
  while (chunk > kKeyTile && (int64_t)B * p.ntb * ((S2 + chunk - 1) / chunk) < 1024) chunk >>= 1;
  p.chunk = chunk;
  p.nkc = (S2 + chunk - 1) / chunk;
  const int64_t groups = (int64_t)B * p.nkc;
  const int64_t nblocks = ((groups + kNumXcd - 1) / kNumXcd) * kNumXcd * p.ntb;
  if (nblocks <= 0) return kOk;
  if (nblocks > 0x7fffffff) return set_error(kUnsupported, "indexer: grid too large");
  hipLaunchKernelGGL(indexer_fp8_kernel, dim3((unsigned)nblocks), dim3(kThreads), 0, stream, p);
  return check_launch("dsa_indexer_logits_fp8");
}

}  // namespace dsa

extern "C" int dsa_indexer_logits_fp8(const void* q, const void* k, const float* key_scale,
                                      const float* weights, const int32_t* act_q,
                                      const int32_t* act_k, int64_t B, int64_t S1, int64_t S2,
                                      int32_t N1, int32_t D, int32_t sparse_mode, float* logits,
                                      int64_t ld, int32_t* row_len, void* stream) {
  using namespace dsa;
  if (N1 != kHeads || D != kDim)
    return set_error(kUnsupported,
                     "dsa_indexer_logits_fp8: only 64 index heads x 128 dims are built (got %d x %d)",
                     N1, D);
  if (B < 0 || S1 < 0 || S2 < 0 || ld < S2 || S1 > 0x7fffffff || S2 > 0x7fffffff || B > 0x7fffffff)
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8: bad sizes");
  if (sparse_mode != 0 && sparse_mode != 3)
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8: sparse_mode must be 0 or 3, got %d",
                     sparse_mode);
  if (B == 0 || S1 == 0) return kOk;
  if (q == nullptr || k == nullptr || weights == nullptr || logits == nullptr)
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8: null pointer");
  return indexer_fp8_launch(static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(k),
                            key_scale, weights, act_q, act_k, (int)B, (int)S1, (int)S2,
                            sparse_mode, logits, ld, row_len, (hipStream_t)stream);
}

namespace dsa {
int topk_launch(const float* x, int64_t rows, int64_t cols, int64_t ld, const int32_t* row_len,
                int32_t K, int32_t pad_invalid, int32_t* out_idx, float* out_val,
                hipStream_t stream);
}

extern "C" size_t dsa_lightning_indexer_workspace_bytes(int64_t B, int64_t S1, int64_t S2) {
  const size_t rows = (size_t)(B < 0 ? 0 : B) * (size_t)(S1 < 0 ? 0 : S1);
  const size_t logits = rows * (size_t)(S2 < 0 ? 0 : S2) * sizeof(float);
  return ((logits + 255) & ~size_t(255)) + rows * sizeof(int32_t);
}

extern "C" int dsa_lightning_indexer_fp8(const void* q, const void* k, const float* key_scale,
                                         const float* weights, const int32_t* act_q,
                                         const int32_t* act_k, int64_t B, int64_t S1, int64_t S2,
                                         int32_t N1, int32_t D, int32_t sparse_count,
                                         int32_t sparse_mode, int32_t* indices, float* values,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  using namespace dsa;
  if (sparse_count < 1 || sparse_count > 8192)
    return set_error(kInvalidArgument, "dsa_lightning_indexer_fp8: sparse_count must be in [1, 8192], got %d",
                     sparse_count);
  if (B < 0 || S1 < 0 || S2 < 0) return set_error(kInvalidArgument, "dsa_lightning_indexer_fp8: bad sizes");
  const size_t need = dsa_lightning_indexer_workspace_bytes(B, S1, S2);
  if (B * S1 == 0) return kOk;
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(kWorkspaceTooSmall, "dsa_lightning_indexer_fp8: workspace of %zu bytes needed, %zu given",
                     need, workspace_bytes);
  if (indices == nullptr) return set_error(kInvalidArgument, "dsa_lightning_indexer_fp8: null indices");
  float* logits = static_cast<float*>(workspace);
  const size_t logit_bytes = (size_t)B * S1 * S2 * sizeof(float);
  int32_t* row_len = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + ((logit_bytes + 255) & ~size_t(255)));
  hipStream_t st = (hipStream_t)stream;
  if (S2 == 0)  // no keys: every row is all -1, the top-k kernel handles cols == 0
    return topk_launch(logits, B * S1, 0, 0, nullptr, sparse_count, 1, indices, values, st);
  int rc = dsa_indexer_logits_fp8(q, k, key_scale, weights, act_q, act_k, B, S1, S2, N1, D,
                                  sparse_mode, logits, S2, row_len, stream);
  if (rc != kOk) return rc;
  return topk_launch(logits, B * S1, S2, S2, row_len, sparse_count, 1, indices, values, st);
}
