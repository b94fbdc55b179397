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
// Work decomposition.  One workgroup (8 waves, two per SIMD) handles one token,
// up to 128 heads (one 16-head MFMA tile per wave; waves past H only help with
// the gather) and one slice ("split") of the token's index list.  The indexed
// KV rows (1152 bytes each) are gathered 32 at a time straight into an LDS ring
// with global_load_lds (no staging registers): 3 stages (two steps in flight
// while one is computed) for short lists, 2 stages for long ones (measured
// faster there) and for the 4-wave workgroups, two of which share a CU so that
// one's prologue and epilogue overlap the other's steps.  A stage is 36 blocks
// of 1 KB; block (key group kg, chunk group cg) at (cg * 4 + kg) * 1024 holds
// keys 8kg .. 8kg+7 x 16-byte chunks
// 8cg .. 8cg+7, key-major, with chunk c of key k (in-block indices) stored at
// slot k * 8 + (c ^ k ^ (kg & 1)).  One global_load_lds then fetches whole
// 128-byte lines (8 chunks of one key per 8 lanes), and the XOR swizzle keeps
// both LDS read patterns below free of bank conflicts.  Per wave and step:
//   S^T[32 keys x 16 heads] = K[32 x Dqk] . Q^T        (v_mfma_f32_16x16x32_bf16)
//   O^T[512 x 16 heads]    += V^T[512 x 32] . P^T
// Computing S^T leaves each lane holding exactly the 8 probabilities (one head,
// 8 keys) that the PV instruction takes as its B operand, so P never leaves
// registers.  The V^T operand is read from the same tile with the transposing
// LDS load ds_read_b64_tr_b16, so V is never copied.  The softmax keeps a
// reference maximum per head and rescales O only when a score exceeds it by
// more than 2^8.  With more than one split the workgroups write normalised
// partial outputs plus their LSE, and a combine kernel merges them.
#include <mutex>

#include "dsa_common.h"
#include "mla_run.h"

namespace {

constexpr int kKT = 32;          // keys per step
constexpr int kDV = 512;         // value dim
constexpr int kWaves = 8;                        // waves of the 128-head workgroup
constexpr int kHeadsPerGroup = 16 * kWaves;      // heads per head group (grid and workspace sizing)
constexpr int kStagesWide = 3;  // ring stages for short lists (3 measured 2 % faster than 4 at decode)
constexpr int kStagesPair = 2;  // ring stages for long lists and for 4-wave workgroups
constexpr int kMaxKeysPerSplit = 2048;
constexpr float kSlack = 8.f;    // log2 headroom of the reference maximum

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short i16x8;

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
  uint16_t* part_o;             // fp16 [T, nsplit, H, 512]: the normalised partial output / part_scale
  float* part_lse;              // [T, nsplit, H]
  float* part_scale;            // [T, nsplit, H]: a power of two >= the row's largest |output|
  int64_t skv;                  // keys per batch row (non-paged) or max_blocks * bs
  int64_t pool_rows;            // rows in the page pool (paged)
  const uint16_t* kv2;          // second row pool (direct rows with the kRowTag2 bit) or null
  int64_t pool_rows2;           // rows in the second pool
  int direct;                   // indices are physical rows (kRowTag2: row of kv2), already resolved
  int v4_on;                    // key sets generated from v4 (no index list)
  dsa::V4Keys v4;
  int B, S, H, topk;
  int block_size, max_blocks;
  int nsplit, keys_per_split, nhg;
  float scale_log2;
  int causal;
};

using dsa::IntC;
using dsa::lds_read_b128;
using dsa::lds_read_tr16;
using dsa::lds_wait;
using dsa::lds_wait1;
using dsa::static_for;
using dsa::wait_vmcnt;
using dsa::xor16_max;
using dsa::xor16_sum;
using dsa::xor32_max;
using dsa::xor32_sum;

// Source of the gathers for invalid keys: always in bounds, always zero.
__device__ __align__(16) uint16_t g_zero_row[576];

// WAVES = 8: 128 heads per workgroup, one workgroup per CU.  WAVES = 4 (H <= 64,
// e.g. DeepSeek-V4's 64 heads): 64 heads per workgroup and a 2-stage ring, so two
// workgroups share a CU (2 waves per SIMD, <= 80 KB of LDS each) and one's
// prologue / epilogue runs beside the other's steps instead of leaving half the
// waves of a 128-head workgroup without heads.
template <int DQK, int kStages, int WAVES>
__global__ __launch_bounds__(WAVES * 64, 8 / WAVES) void sparse_mla_kernel(MlaParams p) {
  constexpr int NT = WAVES * 64;
  constexpr int HPG = 16 * WAVES;  // heads per workgroup
  constexpr int KSTEPS = DQK / 32;          // MFMA k-steps of the score product
  constexpr int NCH = DQK / 8;              // 16-byte chunks per KV row
  constexpr int STAGE = kKT * DQK * 2;      // bytes per ring stage
  // wave w's i-th load fills block (kg = w % 4, cg = CGS i + w / 4): with 8 waves,
  // waves 0-3 own the even chunk groups and waves 4-7 the odd ones; with 4 waves
  // each wave loads every chunk group of its 8 keys
  static_assert(NCH % 8 == 0, "whole chunk groups");
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
  constexpr int CGS = WAVES / 4;                  // chunk-group stride of a wave's loads
  constexpr int NCG = NCH / 8;                    // chunk groups: 9 (576) or 8 (512)
  constexpr int LOADS_HI = (NCG + CGS - 1) / CGS; // loads per step of waves 0-3
  constexpr int LOADS_LO = NCG / CGS;             // loads per step of waves 4-7
  static_assert(2 * LOADS_HI < 64, "vmcnt range");

  extern __shared__ __align__(16) unsigned char smem[];
  int32_t* rows = reinterpret_cast<int32_t*>(smem + kStages * STAGE);  // [keys_per_split]

  // ---- workgroup -> (token, head group, split).  Workgroup ids are dealt to
  // the 8 XCDs round-robin; XCD x takes a contiguous range of (token, split)
  // units, so the head groups and splits of one token share that XCD's L2 (q is
  // fetched once per token, a second gather of the same rows hits, the partial
  // results stay close to the combine) and neighbouring tokens, whose index
  // sets overlap, do too.
  const int bid = blockIdx.x;
  const int xcd = bid % dsa::kNumXcd, r = bid / dsa::kNumXcd;
  const int hg = r % p.nhg;
  const int64_t T = (int64_t)p.B * p.S;
  const int64_t units = T * p.nsplit;
  const int64_t per_xcd = (units + dsa::kNumXcd - 1) / dsa::kNumXcd;
  const int64_t x = (int64_t)xcd * per_xcd + r / p.nhg;
  if (x >= units || r / p.nhg >= per_xcd) return;
  const int64_t token = x / p.nsplit;
  const int split = (int)(x % p.nsplit);
  const int b = (int)(token / p.S), s = (int)(token % p.S);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int head = hg * HPG + wave * 16 + c;
  const bool head_ok = head < p.H;
  const bool wave_active = hg * HPG + wave * 16 < p.H;

  const int kbeg = split * p.keys_per_split;
  const int nkeys = max(0, min(p.keys_per_split, p.topk - kbeg));

  // ---- Q^T operand: lane (g, c) holds head c, dims 64(ks/2) + 16g + 8(ks%2) .. +8,
  // i.e. 16-byte chunk 8(ks/2) + 2g + ks%2 (the chunk order the K reads use; any
  // order shared by both operands gives the same dot product)
  dsa::bf16x8 qf[KSTEPS];
  {
    const uint16_t* qp = p.q + (token * p.H + (head_ok ? head : 0)) * DQK + 16 * g;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      dsa::i32x4 v = head_ok ? *reinterpret_cast<const dsa::i32x4*>(qp + 64 * (ks >> 1) + 8 * (ks & 1))
                             : dsa::i32x4{0, 0, 0, 0};
      qf[ks] = __builtin_bit_cast(dsa::bf16x8, v);
    }
  }

  // ---- resolve this split's indices to physical rows (-1 = skip) ----
  if (p.v4_on) {
    __shared__ int v4_sh[2];  // batch of this row, first -1 of its compressed list
    if (tid == 0) {
      v4_sh[0] = dsa::v4_batch(p.v4, token);
      v4_sh[1] = p.v4.K;
    }
    __syncthreads();
    const int vb = v4_sh[0];
    if (vb >= 0 && p.v4.scenario == 3) {
      const int32_t* ci = p.v4.cmp_idx + token * p.v4.K;
      for (int j = tid; j < p.v4.K; j += NT)
        if (ci[j] == -1) atomicMin(&v4_sh[1], j);
      __syncthreads();
    }
    const int stop = v4_sh[1];
    for (int j = tid; j < nkeys; j += NT) rows[j] = vb >= 0 ? dsa::v4_row(p.v4, token, vb, kbeg + j, stop) : -1;
  } else {
    const int kvl = p.kv_len ? p.kv_len[b] : (int)(p.skv < 0x7fffffff ? p.skv : 0x7fffffff);
    const int qs = p.q_start ? p.q_start[b] : kvl - p.S;
    const int32_t* ip = p.indices + token * p.topk + kbeg;
    for (int j = tid; j < nkeys; j += NT) {
      const int idx = ip[j];
      int32_t row = -1;
      if (p.direct) {
        // resolved rows: bit 30 selects the second pool
        const int r = idx & ~dsa::kRowTag2;
        if (idx >= 0 && (int64_t)r < ((idx & dsa::kRowTag2) ? p.pool_rows2 : p.pool_rows)) row = idx;
        rows[j] = row;
        continue;
      }
      bool ok = idx >= 0 && idx < kvl && (int64_t)idx < p.skv;
      if (ok && p.causal) ok = idx <= qs + s;
      if (ok) {
        if (p.block_table) {
          const int blk = idx / p.block_size;
          const int page = blk < p.max_blocks ? p.block_table[(int64_t)b * p.max_blocks + blk] : -1;
          const int64_t rr = (int64_t)page * p.block_size + idx % p.block_size;
          if (page >= 0 && rr < p.pool_rows) row = (int32_t)rr;
        } else {
          row = (int32_t)((int64_t)b * p.skv + idx);
        }
      }
      rows[j] = row;
    }
  }
  wait_vmcnt<0>();  // Q operands are in registers before any gather is queued
  __syncthreads();  // rows[] ready

  // ---- gather of step `step` into ring stage step % kStages.  Wave w fills the
  // blocks (kg = w % 4, cg = CGS i + w / 4), i = 0, 1, ...; lane l loads in-block
  // key l / 8 and chunk (l % 8) ^ (l / 8) ^ (kg & 1), so it lands in slot l.
  const int gkg = wave & 3;
  const int gkey = 8 * gkg + (lane >> 3);
  const int gch0 = 8 * (wave >> 2) + ((lane & 7) ^ (lane >> 3) ^ (gkg & 1));
  const bool many = (wave >> 2) == 0;  // waves 0-3 issue LOADS_HI loads per step
  auto issue = [&](int step) {
    unsigned char* sb = smem + (step % kStages) * STAGE;
    const int kk = step * kKT + gkey;
    const int32_t rr = kk < nkeys ? rows[kk] : -1;
    const uint16_t* src = (rr >= 0 ? ((rr & dsa::kRowTag2) ? p.kv2 + (int64_t)(rr & ~dsa::kRowTag2) * DQK
                                                           : p.kv + (int64_t)rr * DQK)
                                   : g_zero_row) +
                          8 * gch0;
#pragma unroll
    for (int i = 0; i < LOADS_HI; ++i) {
      if (i < LOADS_LO || many)
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + 64 * CGS * i),
                                         (DSA_LDS void*)(sb + (i * WAVES + wave) * 1024), 16, 0, 0);
    }
  };

  // ---- softmax state: lane (g, c) owns head c
  float m_ref = -__builtin_inff();
  float l_run = 0.f;
  if (p.sink != nullptr && split == 0 && head_ok) {
    m_ref = p.sink[head] * dsa::kLog2e;
    l_run = g == 0 ? 1.f : 0.f;
  }
  dsa::f32x4 o[kDV / 16];
#pragma unroll
  for (int dt = 0; dt < kDV / 16; ++dt) o[dt] = dsa::f32x4{0.f, 0.f, 0.f, 0.f};

  const int nsteps = (nkeys + kKT - 1) / kKT;
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st)
    if (st < nsteps) issue(st);

  for (int step = 0; step < nsteps; ++step) {
    // this wave's gathers for `step` are done once at most the younger ones
    // (up to kStages - 2 steps) are outstanding; the barrier publishes all waves'
    const int younger = min(kStages - 2, nsteps - 1 - step);
    if (many) {
      if (younger >= 2) wait_vmcnt<2 * LOADS_HI>();
      else if (younger == 1) wait_vmcnt<LOADS_HI>();
      else wait_vmcnt<0>();
    } else {
      if (younger >= 2) wait_vmcnt<2 * LOADS_LO>();
      else if (younger == 1) wait_vmcnt<LOADS_LO>();
      else wait_vmcnt<0>();
    }
    __builtin_amdgcn_s_barrier();
    // the stage read in the previous step is free for step + kStages - 1
    if (step + kStages - 1 < nsteps) issue(step + kStages - 1);

    if (wave_active) {
      const unsigned char* sb = smem + (step % kStages) * STAGE;
      // S^T = K . Q^T : acc[kt][i] = score(key 16kt + 4g + i, head c); the A
      // fragment of (kt, ks) is chunk 8(ks/2) + 2g + ks%2 of key 16kt + c.  Reads
      // run kPre fragments ahead of the MFMAs that consume them.
      dsa::f32x4 acc[2] = {dsa::f32x4{0.f, 0.f, 0.f, 0.f}, dsa::f32x4{0.f, 0.f, 0.f, 0.f}};
      // A fragment (kt, ks) = chunk 8(ks/2) + 2g + ks%2 of key 16kt + c: block
      // (kg = 2kt + c/8, cg = ks/2), in-block key c%8, in-block chunk 2g + ks%2
      //   ->  byte offset (ks/2) 4096 + kt 2048 + (ks%2 ? kq1 : kq0).
      // (Group g reading chunks 2g, 2g+1 keeps the 16 rows x 4 groups of one
      // ds_read_b128 conflict-free, measured; the order 4(ks%2) + g halves the rate.)
      const int qkin = c & 7, qkg1 = (c >> 3) & 1;
      const int qm = qkin ^ qkg1;  // swizzle of this lane's key
      const unsigned char* qrow = sb + qkg1 * 1024 + qkin * 128;
      const uint32_t kq0 = (uint32_t)(size_t)(DSA_LDS unsigned char*)(qrow + 16 * ((2 * g) ^ qm));
      const uint32_t kq1 = (uint32_t)(size_t)(DSA_LDS unsigned char*)(qrow + 16 * ((2 * g + 1) ^ qm));
      // fragment f = 2 ks + kt; kPre fragments in flight
      constexpr int kPre = 4;
      dsa::i32x4 kfr[kPre];
      // fragment f: ks = f / 2, kt = f % 2
      static_for<0, kPre>([&](auto F) {
        constexpr int f = decltype(F)::value;
        kfr[f] = lds_read_b128<(f >> 2) * 4096 + (f & 1) * 2048>((f >> 1) & 1 ? kq1 : kq0);
      });
      static_for<0, 2 * KSTEPS>([&](auto F) {
        constexpr int f = decltype(F)::value;
        constexpr int younger = (2 * KSTEPS - 1 - f) < (kPre - 1) ? (2 * KSTEPS - 1 - f) : (kPre - 1);
        lds_wait1<younger>(kfr[f % kPre]);
        const dsa::i32x4 cur = kfr[f % kPre];
        constexpr int fn = f + kPre;
        if constexpr (fn < 2 * KSTEPS)
          kfr[f % kPre] = lds_read_b128<(fn >> 2) * 4096 + (fn & 1) * 2048>((fn >> 1) & 1 ? kq1 : kq0);
        acc[f & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dsa::bf16x8, cur), qf[f >> 1],
                                                             acc[f & 1], 0, 0, 0);
        // keep the pipeline as written: fragment f + kPre's read, then MFMA f
        // (the compiler's own order measured ~2 % slower)
        __builtin_amdgcn_sched_barrier(0);
      });

      // validity of the step's 32 keys as a wave-uniform bit mask
      const int mk = step * kKT + (lane & 31);
      const uint32_t vmask = (uint32_t)__ballot(mk < nkeys && rows[mk] >= 0);
      float sv[2][4];
      float tmax = -__builtin_inff();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sv[kt][i] = acc[kt][i];
          tmax = fmaxf(tmax, sv[kt][i]);
        }
      if (vmask != 0xffffffffu) {
        tmax = -__builtin_inff();
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (!((vmask >> (16 * kt + 4 * g + i)) & 1u)) sv[kt][i] = -__builtin_inff();
            tmax = fmaxf(tmax, sv[kt][i]);
          }
      }
      // scores stay raw (unscaled) until the exponent: s * scale_log2 - m_ref
      tmax = xor32_max(xor16_max(tmax)) * p.scale_log2;
      // m_ref is a reference maximum, not the running one: probabilities are
      // exp2(s - m_ref) and may reach 2^kSlack before O and l move to a new
      // reference.  Exact in fp32 / bf16 (relative precision is unchanged) and
      // it turns the per-step rescale of O into a rare event.
      if (__any(tmax > m_ref + kSlack)) {
        const float m_new = fmaxf(m_ref, tmax);
        const float alpha = m_new == -__builtin_inff() ? 1.f : __builtin_amdgcn_exp2f(m_ref - m_new);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < kDV / 16; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[dt][i] *= alpha;
        m_ref = m_new;
      }
      const float mref = m_ref == -__builtin_inff() ? 0.f : m_ref;
      float pr[2][4];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[kt][i] = __builtin_amdgcn_exp2f(fmaf(sv[kt][i], p.scale_log2, -mref));
          l_run += pr[kt][i];
        }
      // P^T operand: element 4kt + i = key 16kt + 4g + i
      dsa::i32x4 pb;
      pb[0] = (int)dsa::pack_bf16x2(pr[0][0], pr[0][1]);
      pb[1] = (int)dsa::pack_bf16x2(pr[0][2], pr[0][3]);
      pb[2] = (int)dsa::pack_bf16x2(pr[1][0], pr[1][1]);
      pb[3] = (int)dsa::pack_bf16x2(pr[1][2], pr[1][3]);
      const dsa::bf16x8 pbf = __builtin_bit_cast(dsa::bf16x8, pb);

      // O^T[d, head] += V^T[d, keys] . P^T[keys, head].  The transposing load:
      // lane s of group g points at V[16r + 4g + s/4][16dt + 4(s%4)] (chunk
      // 2dt + (s%4)/2, byte 8 (s%2)) and lane o receives V[16r + 4g + j][16dt + o]
      // for j = 0..3 (elements 4r + j).
      // transposing read r of d-tile dt, lane (g, s = c): key 16r + 4g + s/4 -> block
      // kg = 2r + g/2, in-block key k = 4(g%2) + s/4; chunk 2dt + h (h = (s%4)/2) ->
      // cg = dt/4, in-block chunk 2(dt%4) + h; byte 8(s%2).  With m = k ^ (kg & 1):
      //   offset = (dt/4) 4096 + r 2048 + vq[dt % 4],  vq[e] = vbase + 32 (e ^ (m / 2))
      const int sub = c & 3;
      const int vk = 4 * (g & 1) + (c >> 2);
      const int vm = vk ^ ((g >> 1) & 1);
      const uint32_t vbase = (uint32_t)(size_t)(DSA_LDS unsigned char*)(sb + (g >> 1) * 1024 + vk * 128 + 16 * ((sub >> 1) ^ (vm & 1)) + 8 * (sub & 1));
      uint32_t vq[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) vq[e] = vbase + 32 * (e ^ (vm >> 1));
      // kVPre fragment pairs in flight; pair dt is complete once at most the
      // younger pairs (2 reads each) are outstanding
      constexpr int kVPre = 4;
      dsa::i32x2 vfr[kVPre][2];
      static_for<0, kVPre>([&](auto F) {
        constexpr int f = decltype(F)::value;
        vfr[f][0] = lds_read_tr16<(f >> 2) * 4096>(vq[f & 3]);
        vfr[f][1] = lds_read_tr16<(f >> 2) * 4096 + 2048>(vq[f & 3]);
      });
      static_for<0, kDV / 16>([&](auto D) {
        constexpr int dt = decltype(D)::value;
        constexpr int younger = (kDV / 16 - 1 - dt) < (kVPre - 1) ? (kDV / 16 - 1 - dt) : (kVPre - 1);
        lds_wait<2 * younger>(vfr[dt % kVPre][0], vfr[dt % kVPre][1]);
        const dsa::i32x2 v0 = vfr[dt % kVPre][0], v1 = vfr[dt % kVPre][1];
        constexpr int dn = dt + kVPre;
        if constexpr (dn < kDV / 16) {
          vfr[dt % kVPre][0] = lds_read_tr16<(dn >> 2) * 4096>(vq[dn & 3]);
          vfr[dt % kVPre][1] = lds_read_tr16<(dn >> 2) * 4096 + 2048>(vq[dn & 3]);
        }
        const dsa::i32x4 av = {v0[0], v0[1], v1[0], v1[1]};
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dsa::bf16x8, av), pbf, o[dt], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      });
    }
  }

  // ---- epilogue: lane (g, c) holds O^T[16dt + 4g + i][head c]
  const float l_tot = xor32_sum(xor16_sum(l_run));
  const bool has = l_tot > 0.f;
  const float inv = has ? 1.f / l_tot : 0.f;
  const float lse_v = has ? (m_ref + __builtin_amdgcn_logf(l_tot)) * dsa::kLn2 : -__builtin_inff();
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
    // fp16 partials scaled by a power of two per (token, head): 2 bytes per value
    // instead of 4 and a relative error of 2^-12 of the row's largest entry
    const int64_t prow = (token * p.nsplit + split) * p.H + head;
    float amax = 0.f;
#pragma unroll
    for (int dt = 0; dt < kDV / 16; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(o[dt][i]));
    amax = xor32_max(xor16_max(amax)) * inv;
    int e = 0;
    if (amax > 0.f) (void)frexpf(amax, &e);  // amax = m 2^e, m in [0.5, 1)
    const float down = ldexpf(inv, -e);       // o * inv / 2^e
    uint16_t* op = p.part_o + prow * kDV + 4 * g;
#pragma unroll
    for (int dt = 0; dt < kDV / 16; ++dt) {
      const _Float16 h0 = (_Float16)(o[dt][0] * down), h1 = (_Float16)(o[dt][1] * down);
      const _Float16 h2 = (_Float16)(o[dt][2] * down), h3 = (_Float16)(o[dt][3] * down);
      dsa::i32x2 v;
      v[0] = (int)((uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16));
      v[1] = (int)((uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16));
      *reinterpret_cast<dsa::i32x2*>(op + 16 * dt) = v;
    }
    if (g == 0) {
      p.part_lse[prow] = lse_v;
      p.part_scale[prow] = ldexpf(1.f, e);
    }
  }
}

// Merge split partials: lse = logsumexp_p lse_p, out = sum_p exp(lse_p - lse) out_p.
// 64 threads per (token, head) row, 8 dims (16 bytes of fp16) each, four rows per
// block.  The lse, scale and slice of kCombineU splits are all loaded before any
// is used, so a row costs one round trip per kCombineU splits; chunks beyond the
// first are merged online (the running sums rescaled to the new maximum).
constexpr int kCombineU = 8;
constexpr int kCombineRows = 4;  // rows per 256-thread block

__global__ __launch_bounds__(256) void mla_combine_kernel(const uint16_t* __restrict__ part_o,
                                                          const float* __restrict__ part_lse,
                                                          const float* __restrict__ part_scale,
                                                          int64_t rows, int H, int nsplit,
                                                          uint16_t* __restrict__ out,
                                                          float* __restrict__ lse) {
  const int64_t rh = (int64_t)blockIdx.x * kCombineRows + (threadIdx.x >> 6);
  if (rh >= rows) return;
  const int d8 = threadIdx.x & 63;
  const int64_t token = rh / H;
  const int head = (int)(rh % H);
  const int64_t row0 = token * nsplit * H + head;  // partial row of split 0
  float mx = -__builtin_inff(), den = 0.f;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int s0 = 0; s0 < nsplit; s0 += kCombineU) {
    float l[kCombineU], sc[kCombineU];
    dsa::i32x4 v[kCombineU];
#pragma unroll
    for (int u = 0; u < kCombineU; ++u) {
      const bool ok = s0 + u < nsplit;
      const int64_t prow = row0 + (int64_t)(s0 + u) * H;
      l[u] = ok ? part_lse[prow] : -__builtin_inff();
      sc[u] = ok ? part_scale[prow] : 0.f;
      v[u] = ok ? *reinterpret_cast<const dsa::i32x4*>(part_o + prow * kDV + 8 * d8) : dsa::i32x4{0, 0, 0, 0};
    }
    float cm = mx;
#pragma unroll
    for (int u = 0; u < kCombineU; ++u) cm = fmaxf(cm, l[u]);
    if (cm == -__builtin_inff()) continue;  // nothing valid so far
    const float r = mx == -__builtin_inff() ? 0.f : __expf(mx - cm);
    den *= r;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= r;
#pragma unroll
    for (int u = 0; u < kCombineU; ++u) {
      const float w = l[u] == -__builtin_inff() ? 0.f : __expf(l[u] - cm);
      den += w;
      const float ws = w * sc[u];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w2 = (uint32_t)v[u][e >> 1];
        const uint16_t h = (uint16_t)((e & 1) ? (w2 >> 16) : (w2 & 0xffffu));
        acc[e] = fmaf(ws, (float)__builtin_bit_cast(_Float16, h), acc[e]);
      }
    }
    mx = cm;
  }
  const float f = den > 0.f ? 1.f / den : 0.f;
  dsa::i32x4 ov;
#pragma unroll
  for (int e = 0; e < 4; ++e) ov[e] = (int)dsa::pack_bf16x2(acc[2 * e] * f, acc[2 * e + 1] * f);
  *reinterpret_cast<dsa::i32x4*>(out + rh * kDV + 8 * d8) = ov;
  if (d8 == 0 && lse) lse[rh] = den > 0.f ? mx + __logf(den) : -__builtin_inff();
}

template <int DQK, int STAGES, int WAVES>
int launch_mla_stages(const MlaParams& p, int64_t nblocks, hipStream_t stream) {
  const size_t smem = (size_t)STAGES * kKT * DQK * 2 + sizeof(int32_t) * (size_t)p.keys_per_split;
  auto fn = sparse_mla_kernel<DQK, STAGES, WAVES>;
  static std::atomic<int> lds_reserved[dsa::kMaxDevices];
  const int rc = dsa::reserve_lds((const void*)fn, smem, lds_reserved, "sparse_mla");
  if (rc != dsa::kOk) return rc;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblocks), dim3(WAVES * 64), smem, stream, p);
  return dsa::check_launch("dsa_sparse_mla_fwd");
}

// Ring depth and workgroup form.  An 8-wave workgroup (256 VGPRs per wave) fills
// a CU's register file, so it runs alone on its CU: long index lists (prefill)
// use a 2-stage ring (measured faster than 3 or 4 there), short ones (decode
// splits, dominated by gather latency) a 3-stage ring (2 % faster than 4).  4-wave workgroups pair up on a CU
// with 2-stage rings (<= 80 KB of LDS each) and overlap one's prologue and
// epilogue with the other's steps.
template <int DQK>
int launch_mla(const MlaParams& p, int64_t nblocks, hipStream_t stream) {
  // 64 or fewer heads: 4-wave workgroups, when two of them fit in a CU's 160 KB
  // of LDS (not at d_qk = 576 with 2048-key lists: the 128-head form then).
  // Two 64-head workgroups per CU measured slower than one of 128 heads for H = 128.
  const size_t lds4 = (size_t)kStagesPair * kKT * DQK * 2 + sizeof(int32_t) * (size_t)p.keys_per_split + 64;
  if (p.H <= 64 && 2 * lds4 <= 160 * 1024) return launch_mla_stages<DQK, kStagesPair, 4>(p, nblocks, stream);
  if (nblocks >= 1024 && p.keys_per_split > 512)
    return launch_mla_stages<DQK, kStagesPair, kWaves>(p, nblocks, stream);
  return launch_mla_stages<DQK, kStagesWide, kWaves>(p, nblocks, stream);
}

int choose_splits(int64_t tokens, int nhg, int topk) {
  // split the index list until the 256 CUs are covered, keeping >= 256 keys per
  // split (more splits cost more fp32 partials than the extra CUs return); a
  // handful of rows (single-token decode) is latency bound instead, and splits
  // down to 128 keys (below that the combine costs more than it saves)
  const int min_keys = tokens * nhg >= 16 ? 256 : 128;
  int ns = 1;
  while (tokens * nhg * ns < 256 && (topk + 2 * ns - 1) / (2 * ns) >= min_keys) ns *= 2;
  while ((topk + ns - 1) / ns > kMaxKeysPerSplit) ++ns;
  return ns;
}

}  // namespace

namespace dsa {

size_t sparse_mla_split_bytes(int64_t T, int32_t H, int32_t topk, int32_t num_splits) {
  const int nhg = (H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  const int ns = num_splits > 0 ? num_splits : choose_splits(T, nhg, topk);
  if (ns <= 1) return 0;
  return (size_t)T * ns * H * (kDV * sizeof(uint16_t) + 2 * sizeof(float));
}

int sparse_mla_run(const MlaRun& r, const char* what) {
  if (r.d_v != kDV) return set_error(kUnsupported, "%s: d_v must be 512 (got %d)", what, r.d_v);
  if (r.d_qk != 576 && r.d_qk != 512)
    return set_error(kUnsupported, "%s: d_qk must be 576 or 512 (got %d)", what, r.d_qk);
  if (r.B < 0 || r.S < 0 || r.H <= 0 || r.topk < 0 || r.skv < 0)
    return set_error(kInvalidArgument, "%s: bad sizes", what);
  if (!(r.sm_scale > 0.f) || r.sm_scale == __builtin_inff())
    return set_error(kInvalidArgument, "%s: sm_scale must be positive and finite", what);
  if (r.block_table != nullptr && (r.block_size <= 0 || r.max_blocks <= 0))
    return set_error(kInvalidArgument, "%s: paged KV needs block_size > 0 and max_blocks > 0", what);
  const int64_t T = r.B * r.S;
  if (T == 0) return kOk;
  if (r.q == nullptr || r.kv == nullptr || (r.indices == nullptr && r.v4 == nullptr) || r.out == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", what);
  if (r.direct) {
    if (r.skv > kRowTag2 || r.pool_rows2 > kRowTag2 || (r.pool_rows2 > 0 && r.kv2 == nullptr))
      return set_error(kUnsupported, "%s: resolved rows need pools of at most 2^30 rows", what);
  } else if ((r.block_table ? r.skv : r.B * r.skv) >= ((int64_t)1 << 31)) {
    return set_error(kUnsupported, "%s: more than 2^31 - 1 KV rows", what);
  }

  MlaParams p;
  p.q = static_cast<const uint16_t*>(r.q);
  p.kv = static_cast<const uint16_t*>(r.kv);
  p.indices = r.indices;
  p.block_table = r.block_table;
  p.kv_len = r.kv_len;
  p.q_start = r.q_start;
  p.sink = r.attn_sink;
  p.out = static_cast<uint16_t*>(r.out);
  p.lse = r.lse;
  p.skv = r.block_table ? (int64_t)r.max_blocks * r.block_size : r.skv;
  p.pool_rows = r.skv;
  p.kv2 = static_cast<const uint16_t*>(r.kv2);
  p.pool_rows2 = r.pool_rows2;
  p.direct = r.direct;
  p.v4_on = r.v4 != nullptr;
  if (r.v4 != nullptr) p.v4 = *r.v4;
  p.B = (int)r.B;
  p.S = (int)r.S;
  p.H = r.H;
  p.topk = r.topk;
  p.block_size = r.block_size;
  p.max_blocks = r.max_blocks;
  p.scale_log2 = r.sm_scale * kLog2e;
  p.causal = r.is_causal;

  p.nhg = (r.H + kHeadsPerGroup - 1) / kHeadsPerGroup;
  int ns = r.num_splits > 0 ? r.num_splits : choose_splits(T, p.nhg, r.topk);
  if (r.topk == 0) ns = 1;
  const int kps = r.topk > 0 ? (r.topk + ns - 1) / ns : 0;
  if (kps > kMaxKeysPerSplit)
    return set_error(kInvalidArgument, "%s: %d keys per split exceeds %d; raise num_splits", what, kps,
                     kMaxKeysPerSplit);
  p.nsplit = ns;
  p.keys_per_split = kps;
  if (ns > 1) {
    const size_t need = (size_t)T * ns * r.H * (kDV * sizeof(uint16_t) + 2 * sizeof(float));
    if (r.workspace == nullptr || r.workspace_bytes < need)
      return set_error(kWorkspaceTooSmall, "%s: workspace of %zu bytes needed, %zu given", what, need,
                       r.workspace_bytes);
    p.part_o = static_cast<uint16_t*>(r.workspace);
    p.part_lse = reinterpret_cast<float*>(p.part_o + (size_t)T * ns * r.H * kDV);
    p.part_scale = p.part_lse + (size_t)T * ns * r.H;
  } else {
    p.part_o = nullptr;
    p.part_lse = nullptr;
    p.part_scale = nullptr;
  }
  const int64_t units = T * ns;
  const int64_t nblocks = ((units + kNumXcd - 1) / kNumXcd) * kNumXcd * p.nhg;
  if (nblocks > 0x7fffffff) return set_error(kUnsupported, "%s: grid too large", what);
  hipStream_t st = (hipStream_t)r.stream;
  const int rc = r.d_qk == 576 ? launch_mla<576>(p, nblocks, st) : launch_mla<512>(p, nblocks, st);
  if (rc != kOk || ns == 1) return rc;
  const int64_t rows = T * r.H;
  hipLaunchKernelGGL(mla_combine_kernel, dim3((unsigned)((rows + kCombineRows - 1) / kCombineRows)), dim3(256), 0, st,
                     p.part_o, p.part_lse, p.part_scale, rows, r.H, ns, p.out, r.lse);
  return check_launch("dsa_sparse_mla_fwd(combine)");
}

}  // namespace dsa

// ---- the allocation-free entry point: split partials in a fixed device array ----
namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;  // DSA_SPARSE_MLA_SCRATCH_BYTES

// Split partials of dsa_sparse_mla_fwd_noalloc.  In host code this name is a
// host-side stand-in, not a device address: only the pointer that
// hipGetSymbolAddress returns for the current device may be passed to kernels or
// memory calls.
__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[dsa::kMaxDevices];  // device address of `scratch`, per device

// Address of this device's copy of `scratch`, looked up on the first call on the
// device (with that device current) and kept for the process's lifetime.
int scratch_for_current_device(void** out, const char* what) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) return dsa::set_error(dsa::kHipError, "%s: hipGetDevice: %s", what, hipGetErrorString(ge));
  if (dev < 0 || dev >= dsa::kMaxDevices)
    return dsa::set_error(dsa::kUnsupported, "%s: device %d is beyond the %d supported", what, dev, dsa::kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return dsa::set_error(dsa::kHipError, "%s: hipGetSymbolAddress(scratch): %s", what, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return dsa::kOk;
}

}  // namespace

extern "C" size_t dsa_sparse_mla_workspace_bytes(int64_t B, int64_t S, int32_t H, int32_t topk,
                                                 int32_t num_splits) {
  return dsa::sparse_mla_split_bytes(B * S, H, topk, num_splits);
}

extern "C" int dsa_sparse_mla_fwd_noalloc(const void* q, const void* kv, const int32_t* indices,
                                          const int32_t* block_table, const int32_t* kv_len,
                                          const int32_t* q_start, const float* attn_sink, int64_t B,
                                          int64_t S, int32_t H, int32_t d_qk, int32_t d_v, int64_t skv,
                                          int32_t block_size, int32_t max_blocks, int32_t topk,
                                          float sm_scale, int32_t is_causal, int32_t num_splits, void* out,
                                          float* lse, void* stream) {
  const char* what = "dsa_sparse_mla_fwd_noalloc";
  if (B < 0 || S < 0 || H <= 0 || topk < 0) return dsa::set_error(dsa::kInvalidArgument, "%s: bad sizes", what);
  const size_t need = dsa::sparse_mla_split_bytes(B * S, H, topk, num_splits);
  if (need > kScratchBytes)
    return dsa::set_error(dsa::kWorkspaceTooSmall,
                          "%s: the split partials need %zu bytes, above the fixed %zu-byte scratch; "
                          "use fewer tokens or splits per call, or dsa_sparse_mla_fwd with a workspace",
                          what, need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_for_current_device(&ws, what);
    if (rc != dsa::kOk) return rc;
  }
  dsa::MlaRun r{};
  r.q = q;
  r.kv = kv;
  r.indices = indices;
  r.block_table = block_table;
  r.kv_len = kv_len;
  r.q_start = q_start;
  r.attn_sink = attn_sink;
  r.B = B;
  r.S = S;
  r.H = H;
  r.d_qk = d_qk;
  r.d_v = d_v;
  r.skv = skv;
  r.block_size = block_size;
  r.max_blocks = max_blocks;
  r.topk = topk;
  r.sm_scale = sm_scale;
  r.is_causal = is_causal;
  r.num_splits = num_splits;
  r.out = out;
  r.lse = lse;
  r.workspace = ws;
  r.workspace_bytes = need > 0 ? kScratchBytes : 0;
  r.stream = stream;
  return dsa::sparse_mla_run(r, what);
}

extern "C" int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* indices,
                                  const int32_t* block_table, const int32_t* kv_len,
                                  const int32_t* q_start, const float* attn_sink, int64_t B,
                                  int64_t S, int32_t H, int32_t d_qk, int32_t d_v, int64_t skv,
                                  int32_t block_size, int32_t max_blocks, int32_t topk,
                                  float sm_scale, int32_t is_causal, int32_t num_splits, void* out,
                                  float* lse, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  dsa::MlaRun r{};
  r.q = q;
  r.kv = kv;
  r.indices = indices;
  r.block_table = block_table;
  r.kv_len = kv_len;
  r.q_start = q_start;
  r.attn_sink = attn_sink;
  r.B = B;
  r.S = S;
  r.H = H;
  r.d_qk = d_qk;
  r.d_v = d_v;
  r.skv = skv;
  r.block_size = block_size;
  r.max_blocks = max_blocks;
  r.topk = topk;
  r.sm_scale = sm_scale;
  r.is_causal = is_causal;
  r.num_splits = num_splits;
  r.out = out;
  r.lse = lse;
  r.workspace = workspace;
  r.workspace_bytes = workspace_bytes;
  r.stream = stream;
  return dsa::sparse_mla_run(r, "dsa_sparse_mla_fwd");
}
