// Sparse MLA forward on gfx950 bf16 MFMA.
//
// For every query token and head h:
//   s_j   = sm_scale * q[h, :Dqk] . kv[idx_j, :Dqk]        over the valid indices j
//   out_h = sum_j softmax(s)_j * kv[idx_j, :512]           (bf16 out, fp32 accumulate)
//   lse_h = m + ln(sum_j exp(s_j - m))                      (fp32, natural log)
// The single latent KV head is shared by all heads (d_qk = 576 = 512 latent +
// 64 rope, or 512; d_v = 512).  Index j is valid when 0 <= idx < kv_len[b],
// the page it maps to exists, and (causal) idx <= q_start[b] + s.  Invalid
// entries (-1 padding, the out-of-range sentinel) take no part; a row with no
// valid index yields out = 0, lse = -inf.  An optional per-head sink adds
// exp(sink - m) to the denominator (sparse_flash_mla_golden.py:115-149).
//
// Work decomposition.  One workgroup (8 waves) handles one token, up to 128
// heads (one 16-head group per wave; waves past H only help with the gather)
// and one slice ("split") of the token's index list.
// Each step gathers 32 indexed KV rows (one 1152-byte row per key) into LDS:
// row-major for the score product and transposed (V^T) for the PV product, the
// transpose being done while writing LDS.  Per wave and step:
//   S^T[32 keys x 16 heads] = K[32 x Dqk] . Q^T        (v_mfma_f32_16x16x32_bf16)
//   O^T[512 x 16 heads]    += V^T[512 x 32] . P^T     (same instruction)
// Computing S^T rather than S leaves each lane holding exactly the 8
// probabilities (one head, 8 keys) that the PV instruction wants as its B
// operand, so P never leaves registers.  The online softmax runs in the exp2
// domain in registers.  The next step's rows are fetched into registers while
// the current step computes.  With more than one split the workgroups write
// normalised partial outputs plus their LSE, and a combine kernel merges them.
#include "dsa_common.h"

namespace {

constexpr int kKT = 32;          // keys per step
constexpr int kDV = 512;         // value dim
constexpr int kVtStride = 80;    // bytes per V^T row in LDS (32 keys * 2 + 16 pad)
constexpr int kMaxKeysPerSplit = 2048;

struct MlaParams {
  const uint16_t* q;            // [T, H, Dqk]
  const uint16_t* kv;           // [B, Skv, Dqk] or page pool [blocks * bs, Dqk]
  const int32_t* indices;       // [T, topk]
  const int32_t* block_table;   // [B, max_blocks] or null
  const int32_t* kv_len;        // [B] or null
  const int32_t* q_start;       // [B] or null
  const float* sink;            // [H] or null
  uint16_t* out;                // [T, H, 512]
  float* lse;                   // [T, H] or null
  float* part_o;                // [T, nsplit, H, 512]
  float* part_lse;              // [T, nsplit, H]
  int64_t skv;                  // keys per batch row (non-paged) or max_blocks * bs
  int64_t pool_rows;            // rows in the page pool (paged)
  int B, S, H, topk;
  int block_size, max_blocks;
  int nsplit, keys_per_split, nhg;
  float scale_log2;
  int causal;
};

// Slot of key k (0..31) in a V^T row: slot 8g + j holds key 16*(j/4) + 4g + j%4,
// the order in which lane group g holds its 8 probabilities.
__device__ __forceinline__ int vt_slot(int k) {
  const int g = (k & 15) >> 2;
  const int j = 4 * (k >> 4) + (k & 3);
  return 8 * g + j;
}

constexpr int kWaves = 8;
constexpr int kHeadsPerGroup = 16 * kWaves;

template <int DQK>
__global__ __launch_bounds__(kWaves * 64) void sparse_mla_kernel(MlaParams p) {
  constexpr int NT = kWaves * 64;
  constexpr int KSTEPS = DQK / 32;          // MFMA k-steps of the score product
  constexpr int NCH = DQK / 8;              // 16-byte chunks per KV row
  constexpr int KROW = DQK * 2 + 16;        // padded LDS row (bytes)
  constexpr int NTASK = 16 * NCH;           // (key pair, chunk) copy tasks per step
  constexpr int NITER = (NTASK + NT - 1) / NT;

  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* ktile = smem;                                   // [32][KROW]
  unsigned char* vt = smem + kKT * KROW;                         // [512][kVtStride]
  int64_t* rows = reinterpret_cast<int64_t*>(vt + kDV * kVtStride);  // [keys_per_split]

  // ---- workgroup -> (token, head group, split); head groups of one (token,
  // split) share an XCD so the second gather of the same rows hits L2.
  const int bid = blockIdx.x;
  const int xcd = bid % dsa::kNumXcd, r = bid / dsa::kNumXcd;
  const int hg = r % p.nhg;
  const int64_t x = (int64_t)(r / p.nhg) * dsa::kNumXcd + xcd;
  const int64_t T = (int64_t)p.B * p.S;
  if (x >= T * p.nsplit) return;
  const int64_t token = x / p.nsplit;
  const int split = (int)(x % p.nsplit);
  const int b = (int)(token / p.S), s = (int)(token % p.S);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int head = hg * kHeadsPerGroup + wave * 16 + c;
  const bool head_ok = head < p.H;
  const bool wave_active = hg * kHeadsPerGroup + wave * 16 < p.H;

  const int kbeg = split * p.keys_per_split;
  const int nkeys = max(0, min(p.keys_per_split, p.topk - kbeg));

  // ---- resolve this split's indices to physical rows (-1 = skip) ----
  {
    const int kvl = p.kv_len ? p.kv_len[b] : (int)(p.skv < 0x7fffffff ? p.skv : 0x7fffffff);
    const int qs = p.q_start ? p.q_start[b] : kvl - p.S;
    const int32_t* ip = p.indices + token * p.topk + kbeg;
    for (int j = tid; j < nkeys; j += NT) {
      const int idx = ip[j];
      int64_t row = -1;
      bool ok = idx >= 0 && idx < kvl && (int64_t)idx < p.skv;
      if (ok && p.causal) ok = idx <= qs + s;
      if (ok) {
        if (p.block_table) {
          const int blk = idx / p.block_size;
          const int page = blk < p.max_blocks ? p.block_table[(int64_t)b * p.max_blocks + blk] : -1;
          const int64_t rr = (int64_t)page * p.block_size + idx % p.block_size;
          if (page >= 0 && rr < p.pool_rows) row = rr;
        } else {
          row = (int64_t)b * p.skv + idx;
        }
      }
      rows[j] = row;
    }
  }

  // ---- Q^T operand for this wave's 16 heads: lane (g, c) = head c, dims 32ks + 8g .. +8
  dsa::bf16x8 qf[KSTEPS];
  {
    const uint16_t* qp = p.q + (token * p.H + (head_ok ? head : 0)) * DQK + 8 * g;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      dsa::i32x4 v = head_ok ? *reinterpret_cast<const dsa::i32x4*>(qp + 32 * ks)
                             : dsa::i32x4{0, 0, 0, 0};
      qf[ks] = __builtin_bit_cast(dsa::bf16x8, v);
    }
  }
  __syncthreads();  // rows[] ready

  // ---- gather helpers: task q -> key pair m = q % 16, chunk ch = q / 16
  dsa::i32x4 pf[NITER][2];
  auto fetch = [&](int step) {
#pragma unroll
    for (int it = 0; it < NITER; ++it) {
      const int t = tid + it * NT;
      const int m = t & 15, ch = t >> 4;
      const int kk = step * kKT + 2 * m;
      dsa::i32x4 v0 = {0, 0, 0, 0}, v1 = {0, 0, 0, 0};
      if (t < NTASK) {
        const int64_t r0 = kk < nkeys ? rows[kk] : -1;
        const int64_t r1 = kk + 1 < nkeys ? rows[kk + 1] : -1;
        if (r0 >= 0) v0 = *reinterpret_cast<const dsa::i32x4*>(p.kv + r0 * DQK + 8 * ch);
        if (r1 >= 0) v1 = *reinterpret_cast<const dsa::i32x4*>(p.kv + r1 * DQK + 8 * ch);
      }
      pf[it][0] = v0;
      pf[it][1] = v1;
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int it = 0; it < NITER; ++it) {
      const int t = tid + it * NT;
      if (t < NTASK) {
        const int m = t & 15, ch = t >> 4;
        const int k0 = 2 * m;
        *reinterpret_cast<dsa::i32x4*>(ktile + k0 * KROW + 16 * ch) = pf[it][0];
        *reinterpret_cast<dsa::i32x4*>(ktile + (k0 + 1) * KROW + 16 * ch) = pf[it][1];
        if (ch < kDV / 8) {
          const int slot = vt_slot(k0);  // k0 + 1 sits in slot + 1
          unsigned char* dst = vt + (8 * ch) * kVtStride + 2 * slot;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t a = (uint32_t)pf[it][0][e], bb = (uint32_t)pf[it][1][e];
            // element 2e (low halves) and 2e + 1 (high halves) of both keys
            *reinterpret_cast<uint32_t*>(dst + (2 * e) * kVtStride) = (a & 0xffffu) | (bb << 16);
            *reinterpret_cast<uint32_t*>(dst + (2 * e + 1) * kVtStride) = (a >> 16) | (bb & 0xffff0000u);
          }
        }
      }
    }
  };

  // ---- online-softmax state: lane (g, c) owns head c
  float m_run = -__builtin_inff();
  float l_run = 0.f;
  if (p.sink != nullptr && split == 0 && head_ok) {
    m_run = p.sink[head] * dsa::kLog2e;
    l_run = g == 0 ? 1.f : 0.f;
  }
  dsa::f32x4 o[kDV / 16];
#pragma unroll
  for (int dt = 0; dt < kDV / 16; ++dt) o[dt] = dsa::f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = (nkeys + kKT - 1) / kKT;
  if (nsteps > 0) {
    fetch(0);
    stash();
  }
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const bool more = step + 1 < nsteps;
    if (more) fetch(step + 1);

    if (wave_active) {
    // S^T = K . Q^T : acc[kt][i] = score(key 16kt + 4g + i, head c)
    dsa::f32x4 acc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      acc[kt] = dsa::f32x4{0.f, 0.f, 0.f, 0.f};
      const unsigned char* kp = ktile + (16 * kt + c) * KROW + 16 * g;
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const dsa::bf16x8 a = __builtin_bit_cast(dsa::bf16x8, *reinterpret_cast<const dsa::i32x4*>(kp + 64 * ks));
        acc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[ks], acc[kt], 0, 0, 0);
      }
    }

    // mask + scale (log2 domain) and the tile max per head
    float sv[2][4];
    float tmax = -__builtin_inff();
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = step * kKT + 16 * kt + 4 * g + i;
        const bool ok = kk < nkeys && rows[kk] >= 0;
        sv[kt][i] = ok ? acc[kt][i] * p.scale_log2 : -__builtin_inff();
        tmax = fmaxf(tmax, sv[kt][i]);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    float alpha = 1.f;
    float pr[2][4];
    if (m_new == -__builtin_inff()) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[kt][i] = 0.f;
    } else {
      alpha = exp2f(m_run - m_new);
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[kt][i] = exp2f(sv[kt][i] - m_new);
          psum += pr[kt][i];
        }
      l_run = l_run * alpha + psum;
    }
    m_run = m_new;
    if (!__all(alpha == 1.f)) {
#pragma unroll
      for (int dt = 0; dt < kDV / 16; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[dt][i] *= alpha;
    }

    // P^T operand: slots 0..3 = keys 4g..4g+3, slots 4..7 = keys 16+4g..16+4g+3
    dsa::i32x4 pb;
    pb[0] = (int)dsa::pack_bf16x2(pr[0][0], pr[0][1]);
    pb[1] = (int)dsa::pack_bf16x2(pr[0][2], pr[0][3]);
    pb[2] = (int)dsa::pack_bf16x2(pr[1][0], pr[1][1]);
    pb[3] = (int)dsa::pack_bf16x2(pr[1][2], pr[1][3]);
    const dsa::bf16x8 pbf = __builtin_bit_cast(dsa::bf16x8, pb);

    // O^T[d, head] += V^T[d, slots] . P^T[slots, head]
    const unsigned char* vp = vt + c * kVtStride + 16 * g;
#pragma unroll
    for (int dt = 0; dt < kDV / 16; ++dt) {
      const dsa::bf16x8 a = __builtin_bit_cast(dsa::bf16x8, *reinterpret_cast<const dsa::i32x4*>(vp + dt * 16 * kVtStride));
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pbf, o[dt], 0, 0, 0);
    }
    }  // wave_active

    __syncthreads();
    if (more) stash();
    __syncthreads();
  }

  // ---- epilogue: lane (g, c) holds O^T[16dt + 4g + i][head c]
  float l_tot = l_run;
  l_tot += __shfl_xor(l_tot, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  const bool has = l_tot > 0.f;
  const float inv = has ? 1.f / l_tot : 0.f;
  const float lse_v = has ? (m_run + log2f(l_tot)) * dsa::kLn2 : -__builtin_inff();
  if (!head_ok) return;
  if (p.nsplit == 1) {
    uint16_t* op = p.out + (token * p.H + head) * kDV + 4 * g;
#pragma unroll
    for (int dt = 0; dt < kDV / 16; ++dt) {
      dsa::i32x2 v;
      v[0] = (int)dsa::pack_bf16x2(o[dt][0] * inv, o[dt][1] * inv);
      v[1] = (int)dsa::pack_bf16x2(o[dt][2] * inv, o[dt][3] * inv);
      *reinterpret_cast<dsa::i32x2*>(op + 16 * dt) = v;
    }
    if (g == 0 && p.lse) p.lse[token * p.H + head] = lse_v;
  } else {
    const int64_t prow = (token * p.nsplit + split) * p.H + head;
    float* op = p.part_o + prow * kDV + 4 * g;
#pragma unroll
    for (int dt = 0; dt < kDV / 16; ++dt) {
      dsa::f32x4 v = {o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv};
      *reinterpret_cast<dsa::f32x4*>(op + 16 * dt) = v;
    }
    if (g == 0) p.part_lse[prow] = lse_v;
  }
}

// Merge split partials: lse = logsumexp_p lse_p, out = sum_p exp(lse_p - lse) out_p.
// One 128-thread group per (token, head); each thread owns 4 consecutive dims.
__global__ __launch_bounds__(256) void mla_combine_kernel(const float* __restrict__ part_o,
                                                          const float* __restrict__ part_lse,
                                                          int64_t rows, int H, int nsplit,
                                                          uint16_t* __restrict__ out,
                                                          float* __restrict__ lse) {
  const int64_t rh = (int64_t)blockIdx.x * 2 + (threadIdx.x >> 7);
  if (rh >= rows) return;
  const int d4 = threadIdx.x & 127;
  const int64_t token = rh / H;
  const int head = (int)(rh % H);
  float mx = -__builtin_inff();
  for (int sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, part_lse[(token * nsplit + sp) * H + head]);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  if (mx != -__builtin_inff()) {
    for (int sp = 0; sp < nsplit; ++sp) {
      const int64_t prow = (token * nsplit + sp) * H + head;
      const float wgt = __expf(part_lse[prow] - mx);
      den += wgt;
      const dsa::f32x4 v = *reinterpret_cast<const dsa::f32x4*>(part_o + prow * kDV + 4 * d4);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += wgt * v[i];
    }
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  dsa::i32x2 v;
  v[0] = (int)dsa::pack_bf16x2(acc[0] * inv, acc[1] * inv);
  v[1] = (int)dsa::pack_bf16x2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<dsa::i32x2*>(out + rh * kDV + 4 * d4) = v;
  if (d4 == 0 && lse) lse[rh] = den > 0.f ? mx + __logf(den) : -__builtin_inff();
}

template <int DQK>
int launch_mla(const MlaParams& p, int64_t nblocks, hipStream_t stream) {
  constexpr int KROW = DQK * 2 + 16;
  const size_t smem = (size_t)kKT * KROW + (size_t)kDV * kVtStride + sizeof(int64_t) * (size_t)p.keys_per_split;
  auto fn = sparse_mla_kernel<DQK>;
  hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  if (e != hipSuccess)
    return dsa::set_error(dsa::kHipError, "sparse_mla: cannot reserve %zu bytes of LDS: %s", smem,
                          hipGetErrorString(e));
  hipLaunchKernelGGL(fn, dim3((unsigned)nblocks), dim3(kWaves * 64), smem, stream, p);
  return dsa::check_launch("dsa_sparse_mla_fwd");
}

int choose_splits(int64_t tokens, int nhg, int topk) {
  // enough workgroups to cover the 256 CUs about twice; keep >= 256 keys per split
  int ns = 1;
  while (tokens * nhg * ns < 512 && (topk + 2 * ns - 1) / (2 * ns) >= 256) ns *= 2;
  while ((topk + ns - 1) / ns > kMaxKeysPerSplit) ++ns;
  return ns;
}

}  // namespace

extern "C" size_t dsa_sparse_mla_workspace_bytes(int64_t B, int64_t S, int32_t H, int32_t topk,
                                                 int32_t num_splits) {
  const int64_t T = B * S;
  const int nhg = (H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  const int ns = num_splits > 0 ? num_splits : choose_splits(T, nhg, topk);
  if (ns <= 1) return 0;
  return (size_t)T * ns * H * (kDV + 1) * sizeof(float);
}

extern "C" int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* indices,
                                  const int32_t* block_table, const int32_t* kv_len,
                                  const int32_t* q_start, const float* attn_sink, int64_t B,
                                  int64_t S, int32_t H, int32_t d_qk, int32_t d_v, int64_t skv,
                                  int32_t block_size, int32_t max_blocks, int32_t topk,
                                  float sm_scale, int32_t is_causal, int32_t num_splits, void* out,
                                  float* lse, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  using namespace dsa;
  if (d_v != kDV)
    return set_error(kUnsupported, "dsa_sparse_mla_fwd: d_v must be 512 (got %d)", d_v);
  if (d_qk != 576 && d_qk != 512)
    return set_error(kUnsupported, "dsa_sparse_mla_fwd: d_qk must be 576 or 512 (got %d)", d_qk);
  if (B < 0 || S < 0 || H <= 0 || topk < 0 || skv < 0)
    return set_error(kInvalidArgument, "dsa_sparse_mla_fwd: bad sizes");
  if (block_table != nullptr && (block_size <= 0 || max_blocks <= 0))
    return set_error(kInvalidArgument, "dsa_sparse_mla_fwd: paged KV needs block_size > 0 and max_blocks > 0");
  const int64_t T = B * S;
  if (T == 0) return kOk;
  if (q == nullptr || kv == nullptr || indices == nullptr || out == nullptr)
    return set_error(kInvalidArgument, "dsa_sparse_mla_fwd: null pointer");

  MlaParams p;
  p.q = static_cast<const uint16_t*>(q);
  p.kv = static_cast<const uint16_t*>(kv);
  p.indices = indices;
  p.block_table = block_table;
  p.kv_len = kv_len;
  p.q_start = q_start;
  p.sink = attn_sink;
  p.out = static_cast<uint16_t*>(out);
  p.lse = lse;
  p.skv = block_table ? (int64_t)max_blocks * block_size : skv;
  p.pool_rows = skv;
  p.B = (int)B;
  p.S = (int)S;
  p.H = H;
  p.topk = topk;
  p.block_size = block_size;
  p.max_blocks = max_blocks;
  p.scale_log2 = sm_scale * kLog2e;
  p.causal = is_causal;

  p.nhg = (H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  int ns = num_splits > 0 ? num_splits : choose_splits(T, p.nhg, topk);
  if (topk == 0) ns = 1;
  const int kps = topk > 0 ? (topk + ns - 1) / ns : 0;
  if (kps > kMaxKeysPerSplit)
    return set_error(kInvalidArgument, "dsa_sparse_mla_fwd: %d keys per split exceeds %d; raise num_splits",
                     kps, kMaxKeysPerSplit);
  p.nsplit = ns;
  p.keys_per_split = kps;
  if (ns > 1) {
    const size_t need = (size_t)T * ns * H * (kDV + 1) * sizeof(float);
    if (workspace == nullptr || workspace_bytes < need)
      return set_error(kWorkspaceTooSmall, "dsa_sparse_mla_fwd: workspace of %zu bytes needed, %zu given",
                       need, workspace_bytes);
    p.part_o = static_cast<float*>(workspace);
    p.part_lse = p.part_o + (size_t)T * ns * H * kDV;
  } else {
    p.part_o = nullptr;
    p.part_lse = nullptr;
  }
  const int64_t units = T * ns;
  const int64_t nblocks = ((units + kNumXcd - 1) / kNumXcd) * kNumXcd * p.nhg;
  if (nblocks > 0x7fffffff) return set_error(kUnsupported, "dsa_sparse_mla_fwd: grid too large");
  hipStream_t st = (hipStream_t)stream;
  const int rc = d_qk == 576 ? launch_mla<576>(p, nblocks, st) : launch_mla<512>(p, nblocks, st);
  if (rc != kOk || ns == 1) return rc;
  const int64_t rows = T * H;
  hipLaunchKernelGGL(mla_combine_kernel, dim3((unsigned)((rows + 1) / 2)), dim3(256), 0, st,
                     p.part_o, p.part_lse, rows, H, ns, p.out, lse);
  return check_launch("dsa_sparse_mla_fwd(combine)");
}
