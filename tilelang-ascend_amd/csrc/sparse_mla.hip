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
// Work decomposition.  One workgroup handles one token, up to 128 heads (a
// "head group") and one slice ("split") of the token's index list.  The indexed
// KV rows (1152 bytes each) are gathered 32 at a time ("steps") straight into an
// LDS ring with global_load_lds (no staging registers), and both products run on
// MFMA with the single KV tile read from LDS by every head:
//   S^T[32 keys x heads] = K[32 x Dqk] . Q^T
//   O^T[512 x heads]    += V^T[512 x 32] . P^T
// Computing S^T leaves each lane holding exactly the probabilities (one head, 8
// keys) that the P.V instruction takes as its B operand, so P never leaves
// registers, and the V^T operand is read from the same tile with the transposing
// LDS load ds_read_b64_tr_b16, so V is never copied.  The softmax keeps a
// reference maximum per head and rescales O only when a score exceeds it by
// more than 2^8.  With more than one split the workgroups write fp16 partial
// outputs plus their LSE, and a combine kernel merges them.
//
// Two workgroup forms (launch_mla):
//  * more than 64 heads: 4 waves of 32 heads, one wave per SIMD holding Q^T and
//    O^T in registers, v_mfma_f32_32x32x16_bf16, a 4-stage ring (mla_w4_kernel);
//  * 64 heads or fewer: 4 waves of 16 heads (v_mfma_f32_16x16x32_bf16), a
//    2-stage ring, two workgroups per CU (sparse_mla_kernel).
#include <mutex>

#include "dsa_common.h"
#include "mla_run.h"

namespace {

constexpr int kKT = 32;          // keys per step
constexpr int kDV = 512;         // value dim
constexpr int kHeadsPerGroup = 128;  // heads per head group (grid and workspace sizing)
constexpr int kStagesPair = 2;       // ring stages of the paired 64-head workgroups
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
  int balance;                  // token order balanced for short causal rows (balanced_token)
  int order;                    // the 4-wave form gathers each list's rows in row-range order (order_rows)
  uint32_t buf_records;         // 16-byte records of the KV pool (buffer-addressed gathers of the 4-wave form)
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

// 16x16x32 MFMA on 16-bit operands held as raw dwords (F16: IEEE half, else bf16).
template <bool F16>
__device__ __forceinline__ dsa::f32x4 mfma16x16x32(dsa::i32x4 a, dsa::i32x4 b, dsa::f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(dsa::f16x8, a), __builtin_bit_cast(dsa::f16x8, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dsa::bf16x8, a),
                                                   __builtin_bit_cast(dsa::bf16x8, b), c, 0, 0, 0);
}

// Source of the gathers for invalid keys: always in bounds, always zero.
__device__ __align__(16) uint16_t g_zero_row[576];

// Physical row of each index of this split (-1 = skip): rows[j] for key kbeg + j of
// the token's list, after the validity rules (range, page, causal) or the
// DeepSeek-V4 key-set generation.  All NT threads of the workgroup take part.
// Returns the largest j this thread wrote with a valid row (-1: none), so that
// the caller can stop after the last valid key instead of stepping through the
// -1 padding of a short list.  rmin / rmax take the smallest and largest key
// this thread wrote with a valid row (unchanged when it wrote none): the list's
// index for contiguous and paged lists, the row otherwise; with lidx (not null)
// those two kinds also write each entry's index to lidx[j].
// mid() runs once the list's own loads (indices, lengths, page table) are issued,
// so loads it issues (the query operands) overlap the resolution without
// delaying it: memory results retire in issue order, so a query load issued
// ahead of a page-table load would make the table wait for the query.
struct NoMid {
  __device__ void operator()() const {}
};
// Kinds of index list.  A kernel compiled for one kind has no branch join between
// the kinds' row resolutions: at such a join the compiler waited for every load
// in flight, the query operands included, before the first gathers could issue.
constexpr int kListAny = 0;     // decided at run time (DeepSeek-V4 key sets, resolved rows, paged, contiguous)
constexpr int kListContig = 1;  // indices into one contiguous KV sequence per batch row
constexpr int kListPaged = 2;   // indices through a block table into a page pool
template <int NT, int KIND = kListAny, typename Mid = NoMid>
__device__ __forceinline__ int resolve_rows(const MlaParams& p, int64_t token, int b, int s, int kbeg, int nkeys,
                                             int32_t* rows, int tid, Mid mid, int& rmin, int& rmax,
                                             int32_t* lidx = nullptr) {
  auto seen = [&](int32_t row) {
    rmin = min(rmin, (int)row);
    rmax = max(rmax, (int)row);
  };
  if (KIND == kListAny && p.v4_on) {
    mid();
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
    int last = -1;
    for (int j = tid; j < nkeys; j += NT) {
      const int32_t row = vb >= 0 ? dsa::v4_row(p.v4, token, vb, kbeg + j, stop) : -1;
      rows[j] = row;
      if (row >= 0) {
        last = j;
        seen(row);
      }
    }
    return last;
  } else {
    // every index load of the thread is issued before any is used, then every
    // page-table load: two memory round trips for the whole list instead of one
    // or two per 2048 / NT keys
    constexpr int R = kMaxKeysPerSplit / NT;  // list entries per thread
    const int kvl = p.kv_len ? p.kv_len[b] : (int)(p.skv < 0x7fffffff ? p.skv : 0x7fffffff);
    const int qs = p.q_start ? p.q_start[b] : kvl - p.S;
    // loads at clamped positions, without a branch per load (an empty list
    // reads nothing), then selects
    const int32_t* ip = p.indices + token * p.topk;
    int idx[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      idx[r] = p.topk > 0 ? __builtin_nontemporal_load(ip + min(kbeg + tid + r * NT, p.topk - 1)) : -1;
#pragma unroll
    for (int r = 0; r < R; ++r) idx[r] = tid + r * NT < nkeys ? idx[r] : -1;
    // the compiler may not hoist mid()'s loads above the list's loads
    asm volatile("" ::: "memory");
    int last = -1;
    if (KIND == kListAny && p.direct) {
      mid();
      // resolved rows: bit 30 selects the second pool
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = tid + r * NT;
        const int rr = idx[r] & ~dsa::kRowTag2;
        const bool ok = idx[r] >= 0 && (int64_t)rr < ((idx[r] & dsa::kRowTag2) ? p.pool_rows2 : p.pool_rows);
        if (j < nkeys) rows[j] = ok ? idx[r] : -1;
        if (j < nkeys && ok) {
          last = j;
          seen(idx[r]);
        }
      }
      return last;
    }
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ok[r] = idx[r] >= 0 && idx[r] < kvl && (int64_t)idx[r] < p.skv;
      if (p.causal) ok[r] = ok[r] && idx[r] <= qs + s;
    }
    if (KIND == kListPaged || (KIND == kListAny && p.block_table)) {
      // table entries at clamped positions (max_blocks > 0), loaded without a
      // branch per load, ahead of mid()'s loads; their values are taken only
      // after mid() (a wait for them is not hoisted above its loads)
      const int32_t* bt = p.block_table + (int64_t)b * p.max_blocks;
      int page[R];
#pragma unroll
      for (int r = 0; r < R; ++r) page[r] = bt[min(max(idx[r], 0) / p.block_size, p.max_blocks - 1)];
      asm volatile("" ::: "memory");
      mid();
#pragma unroll
      for (int r = 0; r < R; ++r) asm volatile("" : "+v"(page[r]) : : "memory");
#pragma unroll
      for (int r = 0; r < R; ++r) page[r] = ok[r] && idx[r] / p.block_size < p.max_blocks ? page[r] : -1;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = tid + r * NT;
        const int64_t rr = (int64_t)page[r] * p.block_size + idx[r] % p.block_size;
        const bool okr = page[r] >= 0 && rr < p.pool_rows;
        if (j < nkeys) rows[j] = okr ? (int32_t)rr : -1;
        if (lidx != nullptr && j < nkeys) lidx[j] = idx[r];
        if (j < nkeys && okr) {
          last = j;
          seen(idx[r]);
        }
      }
    } else {
      mid();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = tid + r * NT;
        if (j < nkeys) rows[j] = ok[r] ? (int32_t)((int64_t)b * p.skv + idx[r]) : -1;
        if (lidx != nullptr && j < nkeys) lidx[j] = idx[r];
        if (j < nkeys && ok[r]) {
          last = j;
          seen(idx[r]);
        }
      }
    }
    return last;
  }
}

// Reorders the valid rows of rows[0, nlist) by 64 buckets of their list index
// lidx[j], bucket (lidx[j] - lo) >> sh with sh the smallest shift that maps
// hi - lo below 64, keeping list order within a bucket, and drops the invalid
// (-1) rows; returns the number of valid rows, which then fill rows[0, n).
// Neighbouring tokens of a prefill on one XCD, whose lists are gathered step by
// step in parallel, then sweep the sequence in the same direction at the same
// pace, so the rows they share are fetched once into that XCD's L2 and DRAM
// pages are read in order; the sums are taken in another order, which changes
// only their rounding.  The order is a function of the list alone (ballot
// ranks, no atomics; the same for a contiguous and a paged copy of the
// sequence), so results are reproducible.  tab: 2304 ints of free LDS.  All NT
// threads take part.
template <int NT>
__device__ __forceinline__ int order_rows(int32_t* rows, const int32_t* lidx, int nlist, int lo, int hi,
                                          int32_t* tab, int tid) {
  constexpr int R = kMaxKeysPerSplit / NT;  // list entries per thread: j = tid + r NT
  constexpr int NW = NT / 64;
  constexpr int NB = 64;
  const int lane = tid & 63, wave = tid >> 6;
  const int span = hi - lo;
  const int sh = max(0, (32 - __builtin_clz((uint32_t)span | 1u)) - 6);  // span >> sh < 64
  // phase 1: group g = r NW + wave (list entries 256 r + 64 wave .. + 63, so group
  // order is list order): each entry's rank among the group's entries of its
  // bucket (a ballot match on the bucket's 7 bits) and each bucket's count in
  // tab[g][bucket].  One wave's LDS writes land in issue order, so its zeros
  // precede its counts without a barrier.
  int32_t v[R];
  uint32_t key[R];  // bucket (NB: invalid) | rank << 8
#pragma unroll
  for (int r = 0; r < R; ++r) tab[(r * NW + wave) * NB + lane] = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int j = tid + r * NT;
    v[r] = j < nlist ? rows[j] : -1;
    const int bk = v[r] >= 0 ? (lidx[j] - lo) >> sh : NB;
    // lanes whose bucket agrees with this lane's in every bit: per bit, the
    // ballot of the bit, inverted (flip = ~0) where this lane's bit is 0
    uint32_t mlo = ~0u, mhi = ~0u;
#pragma unroll
    for (int k = 0; k < 7; ++k) {
      const uint32_t bit = ((uint32_t)bk >> k) & 1u;
      const uint64_t bal = __ballot(bit);
      const uint32_t flip = bit - 1u;
      mlo &= (uint32_t)bal ^ flip;
      mhi &= (uint32_t)(bal >> 32) ^ flip;
    }
    const int rank = (int)__builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u));
    if (rank == 0 && bk < NB) tab[(r * NW + wave) * NB + bk] = __popc(mlo) + __popc(mhi);
    key[r] = (uint32_t)bk | ((uint32_t)rank << 8);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  // phase 2: lane b of wave w sums bucket b over groups R w .. R w + R - 1, then
  // the offsets of every (group, bucket): the bucket's start (an exclusive scan
  // over buckets, one bucket per lane) + the counts of earlier groups
  int c[R], run = 0;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    c[i] = run;
    run += tab[(wave * R + i) * NB + lane];
  }
  int32_t* const part = tab + R * NW * NB;  // [NW][NB]
  part[wave * NB + lane] = run;
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  int pre = 0, tot = 0;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) {
    const int t = part[w2 * NB + lane];
    tot += t;
    pre += w2 < wave ? t : 0;
  }
  const int inc = (int)dsa::wave_inclusive_scan((uint32_t)tot);
  const int nvalid = __builtin_amdgcn_readlane(inc, 63);
#pragma unroll
  for (int i = 0; i < R; ++i) tab[(wave * R + i) * NB + lane] = inc - tot + pre + c[i];
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  // phase 3: every valid row to its place
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int bk = (int)(key[r] & 0xffu);
    if (bk < NB) rows[tab[(r * NW + wave) * NB + bk] + (int)(key[r] >> 8)] = v[r];
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  return nvalid;
}

// Token of workgroup (xcd, rq) when p.balance is set (one sequence, one split, one
// head group, causal).  Token s of the chunk has at most min(topk, qs + s + 1)
// valid keys, so the first s_short = clamp(topk - 1 - qs, 0, S) tokens have short
// lists, which the kernel ends after their last valid key.  The long tokens are
// cut into 8 equal contiguous ranges, one per XCD (neighbouring tokens' index sets
// overlap in one L2), and the short ones are dealt round-robin after them, so the
// XCDs get equal work.  -1: no token (the grid has up to 8 spare workgroups).
__device__ __forceinline__ int64_t balanced_token(const MlaParams& p, int xcd, int rq) {
  const int64_t kvl = p.kv_len ? (int64_t)p.kv_len[0] : p.skv;
  const int64_t qs = p.q_start ? (int64_t)p.q_start[0] : kvl - p.S;
  const int s_short = (int)min((int64_t)p.S, max((int64_t)0, (int64_t)p.topk - 1 - qs));
  const int nl = p.S - s_short;
  const int per_l = (nl + dsa::kNumXcd - 1) / dsa::kNumXcd;
  const int nlx = max(0, min(per_l, nl - xcd * per_l));
  if (rq < nlx) return (int64_t)s_short + (int64_t)xcd * per_l + rq;
  const int64_t sh = (int64_t)dsa::kNumXcd * (rq - nlx) + xcd;
  return sh < s_short ? sh : -1;
}

// 16-head-per-wave form.  A ring stage is 36 (or 32) blocks of 1 KB; block (key
// group kg, chunk group cg) at (cg * 4 + kg) * 1024 holds keys 8kg .. 8kg+7 x
// 16-byte chunks 8cg .. 8cg+7, key-major, with chunk c of key k (in-block
// indices) stored at slot k * 8 + (c ^ k ^ (kg & 1)).  One global_load_lds then
// fetches whole 128-byte lines (8 chunks of one key per 8 lanes), and the XOR
// swizzle keeps both LDS read patterns free of bank conflicts.
//
// 16 heads per wave, WAVES waves per workgroup.  The library runs it with
// WAVES = 4 for H <= 64 (e.g. DeepSeek-V4's 64 heads): 64 heads per workgroup and
// a 2-stage ring, so two workgroups share a CU (2 waves per SIMD, <= 80 KB of LDS
// each) and one's prologue / epilogue runs beside the other's steps.  (WAVES = 8,
// one 128-head workgroup per CU, measured slower than the 4-wave 128-head form
// below and is not launched.)
template <int DQK, int kStages, int WAVES, bool F16>
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
  const int nlist = max(0, min(p.keys_per_split, p.topk - kbeg));  // list entries of this split

  // ---- Q^T operand: lane (g, c) holds head c, dims 64(ks/2) + 16g + 8(ks%2) .. +8,
  // i.e. 16-byte chunk 8(ks/2) + 2g + ks%2 (the chunk order the K reads use; any
  // order shared by both operands gives the same dot product)
  dsa::i32x4 qf[KSTEPS];
  {
    const uint16_t* qp = p.q + (token * p.H + (head_ok ? head : 0)) * DQK + 16 * g;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks)
      qf[ks] = head_ok ? *reinterpret_cast<const dsa::i32x4*>(qp + 64 * (ks >> 1) + 8 * (ks & 1))
                       : dsa::i32x4{0, 0, 0, 0};
  }

  // ---- resolve this split's indices to physical rows (-1 = skip); the list
  // ends after its last valid key (steps past it would add exactly nothing) ----
  int rmin = 0x7fffffff, rmax = -1;  // (unused here)
  int last_ok = resolve_rows<NT, kListAny>(p, token, b, s, kbeg, nlist, rows, tid, NoMid{}, rmin, rmax);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) last_ok = max(last_ok, __shfl_xor(last_ok, o));
  int32_t* const last_slot = rows + p.keys_per_split;  // one per wave
  if (lane == 0) last_slot[wave] = last_ok;
  wait_vmcnt<0>();  // Q operands are in registers before any gather is queued
  __syncthreads();  // rows[] and last_slot[] ready
  int nk = -1;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) nk = max(nk, last_slot[w]);
  const int nkeys = __builtin_amdgcn_readfirstlane(nk + 1);

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
        acc[f & 1] = mfma16x16x32<F16>(cur, qf[f >> 1], acc[f & 1]);
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
        const uint32_t m = vmask >> (4 * g);  // one variable shift; constant bit tests below
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (!((m >> (16 * kt + i)) & 1u)) sv[kt][i] = -__builtin_inff();
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
      pb[0] = (int)dsa::pack_half2<F16>(pr[0][0], pr[0][1]);
      pb[1] = (int)dsa::pack_half2<F16>(pr[0][2], pr[0][3]);
      pb[2] = (int)dsa::pack_half2<F16>(pr[1][0], pr[1][1]);
      pb[3] = (int)dsa::pack_half2<F16>(pr[1][2], pr[1][3]);

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
        o[dt] = mfma16x16x32<F16>(av, pb, o[dt]);
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
      v[0] = (int)dsa::pack_half2<F16>(o[dt][0] * inv, o[dt][1] * inv);
      v[1] = (int)dsa::pack_half2<F16>(o[dt][2] * inv, o[dt][3] * inv);
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

// ---------------------------------------------------------------------------
// 128-head form (H > 64): four waves, one per SIMD, 32 heads each, on
// v_mfma_f32_32x32x16_bf16.  Per wave and 32-key step:
//   S^T[32 keys x 32 heads]  = sum over 36 k-steps of K[32 x 16] . Q^T[16 x 32]
//   O^T[512 x 32 heads]     += V^T[512 x 32] . P^T[32 x 32]   (16 d-tiles x 2 k-steps)
// A 32-head wave reads each K / V fragment once for 32 heads, half the LDS bytes
// per MFMA of the 16-head form, and one wave per SIMD owns the whole register
// file: Q^T (144 VGPRs at d_qk 576) and O^T (256 accumulators) stay resident.
// With no second wave on the SIMD to fill the softmax gap, the loop is software
// pipelined: step j runs the score MFMAs of key step j, then the P.V MFMAs of
// step j - 1 with the softmax of step j spread between them.  A 4-stage LDS ring (3 steps of
// gathers in flight) keeps one step for P.V, one for the scores and two loading.
//
// Register layouts (lane l, hh = l / 32, l32 = l % 32):
//   32x32 result (S^T and O^T tiles), element r: row 8 (r / 4) + 4 hh + r % 4, column l32
//   A operand: row l32, k-elements 8 hh .. 8 hh + 7;  B operand: column l32, same k
// so the lane holding head l32's scores of keys {8 (r / 4) + 4 hh + r % 4} passes
// exactly those as P^T for the k-slots 8 hh .. 8 hh + 7 of two P.V k-steps, with
// k-slot i of k-step kk standing for key 16 kk + 8 (i / 4) + 4 hh + i % 4; the
// V^T operand is read for the same keys with two transposing reads (4 keys each).
// ---------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kW4Stages = 4;  // ring stages of the 4-wave form
// LDS fragment reads in flight per wave.  With one wave per SIMD nothing else
// covers a read's latency; 6 / 5 measured 0.3-1 % faster than 4 / 4 at 128K and
// at config 4 (the kernel then holds 252 VGPRs), 7 was slower and 7 / 6 spills.
constexpr int kW4KPre = 6;    // score A fragments in flight
constexpr int kW4VPre = 5;    // P.V A fragments (two reads each) in flight

// The MFMAs of this form are issued as inline asm so that the register file stays
// partitioned as designed.  The 256 O^T accumulators are not C++ values at all:
// d-tile DT lives in a[16 DT .. 16 DT + 15], named in the asm text, and every
// asm statement of the kernel that issues an MFMA or touches the AGPRs lists all
// 256 AGPRs as clobbered, so the compiler neither places a value of its own
// there nor leaves them out of the kernel's register count.  (As C++ values the
// accumulators were copied into VGPRs around every MFMA and Q^T spilled.)  The
// score accumulators, Q^T and the working set are ordinary VGPR values.  The
// compiler does not insert MFMA hazard wait states for inline asm; the kernel
// places them itself (mfma_drain) where a VALU instruction or a store reads an
// MFMA result soon after it was written.  Chained MFMAs on one accumulator
// (exactly overlapping srcC / vdst) need none.
#define DSA_A10(p) \
  "a" #p "0", "a" #p "1", "a" #p "2", "a" #p "3", "a" #p "4", "a" #p "5", "a" #p "6", "a" #p "7", "a" #p "8", "a" #p "9"
#define DSA_AGPRS                                                                                                  \
  "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8", "a9", DSA_A10(1), DSA_A10(2), DSA_A10(3), DSA_A10(4),        \
      DSA_A10(5), DSA_A10(6), DSA_A10(7), DSA_A10(8), DSA_A10(9), DSA_A10(10), DSA_A10(11), DSA_A10(12), DSA_A10(13), \
      DSA_A10(14), DSA_A10(15), DSA_A10(16), DSA_A10(17), DSA_A10(18), DSA_A10(19), DSA_A10(20), DSA_A10(21),        \
      DSA_A10(22), DSA_A10(23), DSA_A10(24), "a250", "a251", "a252", "a253", "a254", "a255"

// S^T = K . Q^T (first k-step) and S^T += K . Q^T, in VGPRs (F16: IEEE half
// operands, else bf16)
template <bool F16>
__device__ __forceinline__ void mfma32_v0(f32x16& acc, dsa::i32x4 a, dsa::i32x4 b) {
  if constexpr (F16) asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b) : DSA_AGPRS);
  else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc) : "v"(a), "v"(b) : DSA_AGPRS);
}
template <bool F16>
__device__ __forceinline__ void mfma32_v(f32x16& acc, dsa::i32x4 a, dsa::i32x4 b) {
  if constexpr (F16) asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b) : DSA_AGPRS);
  else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b) : DSA_AGPRS);
}
// O^T d-tile DT += V^T . P^T
template <int DT, bool F16>
__device__ __forceinline__ void mfma32_o(dsa::i32x4 a, dsa::i32x4 b) {
  if constexpr (F16)
    asm volatile("v_mfma_f32_32x32x16_f16 a[%2:%3], %0, %1, a[%2:%3]"
                 :
                 : "v"(a), "v"(b), "i"(16 * DT), "i"(16 * DT + 15)
                 : DSA_AGPRS);
  else
    asm volatile("v_mfma_f32_32x32x16_bf16 a[%2:%3], %0, %1, a[%2:%3]"
                 :
                 : "v"(a), "v"(b), "i"(16 * DT), "i"(16 * DT + 15)
                 : DSA_AGPRS);
}
// O^T = 0
__device__ __forceinline__ void zero_o() {
  asm volatile(
      ".set .Ldsa_acc, 0\n"
      ".rept 256\n"
      "v_accvgpr_write_b32 a[.Ldsa_acc], 0\n"
      ".set .Ldsa_acc, .Ldsa_acc + 1\n"
      ".endr" ::
          : DSA_AGPRS);
}
// O^T *= alpha, one register at a time through one VGPR (the rescale is rare)
__device__ __forceinline__ void scale_o(float alpha) {
  float t;
  asm volatile(
      ".set .Ldsa_acc, 0\n"
      ".rept 256\n"
      "v_accvgpr_read_b32 %0, a[.Ldsa_acc]\n"
      "v_mul_f32 %0, %0, %1\n"
      "v_accvgpr_write_b32 a[.Ldsa_acc], %0\n"
      ".set .Ldsa_acc, .Ldsa_acc + 1\n"
      ".endr"
      : "=&v"(t)
      : "v"(alpha)
      : DSA_AGPRS);
}
// the 16 values of O^T d-tile DT
template <int DT>
__device__ __forceinline__ void read_o(float (&t)[16]) {
  asm volatile(
      ".set .Ldsa_acc, %16\n"
      "v_accvgpr_read_b32 %0, a[.Ldsa_acc]\n"
      "v_accvgpr_read_b32 %1, a[.Ldsa_acc + 1]\n"
      "v_accvgpr_read_b32 %2, a[.Ldsa_acc + 2]\n"
      "v_accvgpr_read_b32 %3, a[.Ldsa_acc + 3]\n"
      "v_accvgpr_read_b32 %4, a[.Ldsa_acc + 4]\n"
      "v_accvgpr_read_b32 %5, a[.Ldsa_acc + 5]\n"
      "v_accvgpr_read_b32 %6, a[.Ldsa_acc + 6]\n"
      "v_accvgpr_read_b32 %7, a[.Ldsa_acc + 7]\n"
      "v_accvgpr_read_b32 %8, a[.Ldsa_acc + 8]\n"
      "v_accvgpr_read_b32 %9, a[.Ldsa_acc + 9]\n"
      "v_accvgpr_read_b32 %10, a[.Ldsa_acc + 10]\n"
      "v_accvgpr_read_b32 %11, a[.Ldsa_acc + 11]\n"
      "v_accvgpr_read_b32 %12, a[.Ldsa_acc + 12]\n"
      "v_accvgpr_read_b32 %13, a[.Ldsa_acc + 13]\n"
      "v_accvgpr_read_b32 %14, a[.Ldsa_acc + 14]\n"
      "v_accvgpr_read_b32 %15, a[.Ldsa_acc + 15]"
      : "=v"(t[0]), "=v"(t[1]), "=v"(t[2]), "=v"(t[3]), "=v"(t[4]), "=v"(t[5]), "=v"(t[6]), "=v"(t[7]), "=v"(t[8]),
        "=v"(t[9]), "=v"(t[10]), "=v"(t[11]), "=v"(t[12]), "=v"(t[13]), "=v"(t[14]), "=v"(t[15])
      : "i"(16 * DT));
}
// max(a, b, c) without the quieting the compiler adds around fmaxf of asm outputs
__device__ __forceinline__ float max3(float a, float b, float c) {
  float r;
  asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Pins the computation of v ahead of this point of the (volatile) asm stream:
// without it the compiler sinks the softmax arithmetic past the P.V MFMAs it is
// meant to hide behind.
__device__ __forceinline__ void pin(float& v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void pin(int& v) { asm volatile("" ::"v"(v)); }

// Wait states between a 16-pass MFMA's write and a VALU / memory read of its
// result (more than the 18 the ISA requires).
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 7\n s_nop 7\n s_nop 7" ::: "memory"); }
// VALU write -> MFMA source read.
__device__ __forceinline__ void valu_to_mfma() { asm volatile("s_nop 3" ::: "memory"); }

// Ring layout of the 4-wave form.  A stage holds 32 keys x d_qk as one 1 KB block
// per chunk pair cp (16-byte chunks 2 cp and 2 cp + 1, i.e. dims 16 cp .. 16 cp + 15)
// at cp * 1024.  Key k's 32-byte piece sits at position k ^ 4 (cp % 2), its two
// chunks swapped when k / 8 is odd:
//   offset = cp * 1024 + (k ^ 4 (cp % 2)) * 32 + 16 ((chunk % 2) ^ (k / 8 % 2)).
// Then (a) one 64-lane load fills one block (lane l: 16-byte slot l), (b) the score
// A fragments (chunk pair ks, one 16-lane group per 16 keys) hit 16 distinct 16-byte
// bank groups, and (c) every 16-lane group of a transposing P.V read takes one
// contiguous 128-byte tile (4 keys x 16 dims), the dense pattern ds_read_b64_tr_b16
// serves near its peak rate (about 2.8x the rate measured for 4 rows at a 128-byte
// stride), the two groups read together falling in disjoint bank halves.
__device__ __forceinline__ uint32_t w4_pos(int k, int cp, int c1) {
  return (uint32_t)(cp * 1024 + ((k ^ (4 * (cp & 1))) * 32) + 16 * (c1 ^ ((k >> 3) & 1)));
}

// 16-byte LDS-direct load of record `idx` of a buffer of 16-byte records (zeros
// past the buffer's end); OFF applies to both the global and the LDS address,
// soff to the global address only.
template <int OFF>
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, DSA_LDS void* lds, uint32_t idx,
                                                  uint32_t soff) {
  __builtin_amdgcn_struct_ptr_buffer_load_lds(rsrc, lds, 16, idx, 0, soff, OFF, 0);
}

// One 32-bit LDS read issued as inline asm (it joins the counted stream of the
// kernel's own LDS reads instead of drawing a compiler lgkmcnt(0) wait).
__device__ __forceinline__ int32_t lds_read_b32(uint32_t addr) {
  int32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// BUF: the gathers address the KV pool as a buffer of 16-byte records (a 32-bit
// record index per lane; an index past the pool reads zeros), which issues in about
// a fifth of the time of a 64-bit per-lane address.  The hardware forms the byte
// offset in 32 bits, so this is for pools of at most 4 GiB with rows from one pool.
template <int DQK, bool F16, bool BUF, int KIND>
__global__ __launch_bounds__(256, 1) void mla_w4_kernel(MlaParams p) {
  constexpr int NT = 256;
  constexpr int KS = DQK / 16;          // score k-steps: 36 (576) or 32 (512)
  constexpr int NCG = DQK / 64;         // 128-byte chunk groups per KV row: 9 or 8
  constexpr int STAGE = kKT * DQK * 2;  // bytes per ring stage
  constexpr int ND = kDV / 32;          // P.V d-tiles
  static_assert(2 * NCG < 64, "vmcnt range");
  static_assert(KS >= 23, "the softmax is spread over 23 score MFMAs");

  extern __shared__ __align__(16) unsigned char smem[];
  int32_t* rows = reinterpret_cast<int32_t*>(smem + kW4Stages * STAGE);

  // ---- workgroup -> (token, head group, split), contiguous (token, split)
  // ranges per XCD as in the 8-wave form
  const int bid = blockIdx.x;
  const int xcd = bid % dsa::kNumXcd, rq = bid / dsa::kNumXcd;
  const int hg = rq % p.nhg;
  const int64_t T = (int64_t)p.B * p.S;
  const int64_t units = T * p.nsplit;
  const int64_t per_xcd = (units + dsa::kNumXcd - 1) / dsa::kNumXcd;
  int64_t x;
  if (p.balance) {
    x = balanced_token(p, xcd, rq);
    if (x < 0) return;
  } else {
    x = (int64_t)xcd * per_xcd + rq / p.nhg;
    if (x >= units || rq / p.nhg >= per_xcd) return;
  }
  const int64_t token = x / p.nsplit;
  const int split = (int)(x % p.nsplit);
  const int b = (int)(token / p.S), s = (int)(token % p.S);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS-DMA bases stay scalar
  const int hh = lane >> 5, l32 = lane & 31;
  const int head = hg * kHeadsPerGroup + wave * 32 + l32;
  const bool head_ok = head < p.H;
  const bool wave_active = hg * kHeadsPerGroup + wave * 32 < p.H;
  const int kbeg = split * p.keys_per_split;
  const int nlist = max(0, min(p.keys_per_split, p.topk - kbeg));  // list entries of this split

  // O^T = 0 and the sink load before any other memory operation: the compiler
  // waits for every load in flight ahead of an asm block naming the accumulation
  // registers, and for all earlier loads ahead of a load's first use.
  zero_o();
  const float sink_log2 =
      p.sink != nullptr && split == 0 && head_ok ? p.sink[head] * dsa::kLog2e : -__builtin_inff();

  // ---- Q^T operand of k-step ks: head l32, dims 16 ks + 8 hh .. + 8.  Loaded
  // behind the index loads of the list and ahead of their use, so the query
  // fetch overlaps the row resolution and the first gathers; the first score
  // MFMA waits for it together with the gathers of step 0.
  dsa::i32x4 qf[KS];
  // with p.order the list's indices go to the (empty) ring for order_rows
  int32_t* const lidx = reinterpret_cast<int32_t*>(smem + 16384);
  int rmin = 0x7fffffff, rmax = -1;
  int last_ok = resolve_rows<NT, KIND>(
      p, token, b, s, kbeg, nlist, rows, tid,
      [&]() {
        const uint16_t* qp = p.q + (token * p.H + (head_ok ? head : 0)) * DQK + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const dsa::i32x4*>(qp + 16 * ks);
      },
      rmin, rmax, p.order ? lidx : nullptr);
  // (a lane past the last head computes with head 0's query; its column of S, P
  // and O is never written out, and no other head's column depends on it)
  // The list ends after its last valid key: the steps past it (the -1 padding of
  // a short causal row) would add exactly nothing.
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    last_ok = max(last_ok, __shfl_xor(last_ok, o));
    rmin = min(rmin, __shfl_xor(rmin, o));
    rmax = max(rmax, __shfl_xor(rmax, o));
  }
  // one slot per wave: its last valid key, then its smallest and largest row
  int32_t* const last_slot = rows + p.keys_per_split;
  if (lane == 0) {
    last_slot[wave] = last_ok;
    last_slot[4 + wave] = rmin;
    last_slot[8 + wave] = rmax;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // rows[] and last_slot[] written
  __builtin_amdgcn_s_barrier();                        // ... by every wave
  int nkeys = __builtin_amdgcn_readfirstlane(
      max(max(last_slot[0], last_slot[1]), max(last_slot[2], last_slot[3])) + 1);
  if (p.order && nkeys > 0) {
    const int lo = min(min(last_slot[4], last_slot[5]), min(last_slot[6], last_slot[7]));
    const int hi = max(max(last_slot[8], last_slot[9]), max(last_slot[10], last_slot[11]));
    // the (empty) ring holds the ordering's tables
    static_assert(16384 + 4 * kMaxKeysPerSplit <= STAGE, "tables and indices fit the first ring stage");
    nkeys = __builtin_amdgcn_readfirstlane(order_rows<NT>(rows, lidx, nlist, __builtin_amdgcn_readfirstlane(lo),
                                                          __builtin_amdgcn_readfirstlane(hi),
                                                          reinterpret_cast<int32_t*>(smem), tid));
  }

  // ---- gathers: wave w fills chunk pairs w, w + 4, .. of every step; lane l of a
  // block load writes 16-byte slot l of the block, i.e. key gk = (l / 2) ^ 4 (w % 2),
  // chunk gc1 = (l % 2) ^ (gk / 8 % 2) of the pair.  The load's immediate offset
  // (32 cp bytes) applies to the LDS address too, so M0 is pre-biased by -32 cp.
  const int gk = (lane >> 1) ^ (4 * (wave & 1));
  const int gc1 = (lane & 1) ^ ((gk >> 3) & 1);
  const uint32_t lds0 = (uint32_t)(size_t)(DSA_LDS unsigned char*)smem;
  const uint32_t rows_lds = lds0 + kW4Stages * STAGE;
  const int last_key = max(nkeys - 1, 0);
  // rows[] entry of this lane's gather key in step `step` (clamped inside the list)
  auto row_read = [&](int step) -> int32_t { return lds_read_b32(rows_lds + 4 * min(step * kKT + gk, last_key)); };
  auto row_ok = [&](int step, int32_t raw) -> int32_t { return step * kKT + gk < nkeys ? raw : -1; };
  constexpr int R16 = DQK / 8;  // 16-byte records per KV row
  const __amdgpu_buffer_rsrc_t kv_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.kv, (short)16, (int)p.buf_records, 0x00020000);
  const uint16_t* const zero_src = g_zero_row + 8 * gc1;
  const uint16_t* const kv_src = p.kv + 8 * gc1;
  const uint16_t* const kv2_src = (p.kv2 ? p.kv2 : p.kv) + 8 * gc1;
  // the load operand of row rr (-1: zeros): a record index (BUF) or a pointer
  auto gather_src = [&](int32_t rr) {
    if constexpr (BUF) {
      return rr >= 0 ? (uint32_t)rr * (uint32_t)R16 + (uint32_t)gc1 : 0xffffffffu;
    } else {
      const uint16_t* base = (rr & dsa::kRowTag2) ? kv2_src : kv_src;
      const uint16_t* src = base + (int64_t)(rr & ~dsa::kRowTag2) * DQK;
      return rr >= 0 ? src : zero_src;
    }
  };
  using GSrc = decltype(gather_src(0));
  const GSrc no_src = gather_src(-1);
  auto issue_one = [&](int step, GSrc src, auto C) {
    constexpr int cp = 4 * decltype(C)::value;  // + wave
    unsigned char* sb = smem + (step % kW4Stages) * STAGE + wave * 1024;
    if constexpr (BUF)
      buffer_load_lds16<32 * cp>(kv_rsrc, (DSA_LDS void*)(sb + cp * (1024 - 32)), src, 32 * wave);
    else
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + 16 * wave),
                                       (DSA_LDS void*)(sb + cp * (1024 - 32)), 16, 32 * cp, 0);
  };
  auto issue = [&](int step, GSrc src) {
    static_for<0, NCG>([&](auto C) { issue_one(step, src, C); });
  };
  // rows[] entry of key l32 of step `step`, for its validity bit (clamped)
  auto mask_read = [&](int step) -> int32_t { return lds_read_b32(rows_lds + 4 * min(step * kKT + l32, last_key)); };
  auto mask_of = [&](int step, int32_t raw) -> uint32_t {
    return (uint32_t)__ballot(step * kKT + l32 < nkeys && raw >= 0);
  };

  // ---- LDS read addresses (bytes from the start of a stage)
  // score A fragment of k-step ks: key l32, chunk 2 ks + hh (pair ks), at kq[ks % 2] + ks * 1024
  uint32_t kq[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) kq[e] = w4_pos(l32, e, hh) - 1024 * e;
  // P.V A fragment (d-tile dt, k-step kk), transposing read r (keys +8r): group
  // g = lane / 16 and lane sl = lane % 16 point at key 16 kk + 8 r + 4 hh + sl / 4,
  // dims 32 dt + 16 (g % 2) + 4 (sl % 4) .. + 4, i.e. chunk pair 2 dt + g % 2, at
  // vq[r] + dt * 2048 + kk * 512
  uint32_t vq[2];
  {
    const int g = (lane >> 4) & 3, sl = lane & 15;
#pragma unroll
    for (int r2 = 0; r2 < 2; ++r2)
      vq[r2] = w4_pos(8 * r2 + 4 * hh + (sl >> 2), g & 1, (sl & 3) >> 1) + 8 * (sl & 1);
  }

  // ---- softmax state: lanes l32 and l32 + 32 share head l32 (the sink was
  // loaded first thing: a load issued after the query loads would hold its use,
  // and the ring fill behind it, until the query had arrived)
  float m_ref = sink_log2;
  float l_run = m_ref == -__builtin_inff() ? 0.f : (hh == 0 ? 1.f : 0.f);

  // P.V A fragments in flight: fragment f = 2 dt + kk, two transposing reads
  dsa::i32x2 vfr[kW4VPre][2];
  auto v_read = [&](uint32_t vbase, auto F) {
    constexpr int f = decltype(F)::value;
    constexpr int dt = f >> 1, kk = f & 1;
    vfr[f % kW4VPre][0] = lds_read_tr16<dt * 2048 + kk * 512>(vbase + vq[0]);
    vfr[f % kW4VPre][1] = lds_read_tr16<dt * 2048 + kk * 512>(vbase + vq[1]);
  };

  // score product of the step in `sbase`: S^T = K . Q^T over KS k-steps, kW4KPre
  // fragment reads in flight; hook(IntC<f>) runs after MFMA f.  With VPF the
  // first kW4VPre P.V fragments (of the stage at `vbase`) are read during the last
  // score MFMAs, whose K reads are already issued, so the P.V phase starts with
  // its operands in flight.
  // Score accumulators by step parity (the scores of step j accumulate while the
  // exponentials of step j - 1 are taken) and P^T of the step whose P.V is next.
  f32x16 sacc[2];
  dsa::i32x4 pbuf[2];  // the B operands of the two P.V k-steps
  auto scores = [&](f32x16& acc, uint32_t sbase, uint32_t vbase, auto VPF, auto&& hook) {
    constexpr bool vpf = decltype(VPF)::value != 0;
    static_assert(kW4VPre <= kW4KPre, "the V prefetch uses the K-read slots of the last MFMAs");
    dsa::i32x4 kfr[kW4KPre];
    static_for<0, kW4KPre>([&](auto F) {
      constexpr int f = decltype(F)::value;
      kfr[f] = lds_read_b128<f * 1024>(sbase + kq[f & 1]);
    });
    static_for<0, KS>([&](auto F) {
      constexpr int f = decltype(F)::value;
      constexpr int ky = (KS - 1 - f) < (kW4KPre - 1) ? (KS - 1 - f) : (kW4KPre - 1);
      constexpr int tail0 = KS - kW4KPre;  // first MFMA without a K read to issue
      constexpr int vissued = vpf && f > tail0 ? (f - tail0 < kW4VPre ? f - tail0 : kW4VPre) : 0;
      lds_wait1<ky + 2 * vissued>(kfr[f % kW4KPre]);
      const dsa::i32x4 cur = kfr[f % kW4KPre];
      constexpr int fn = f + kW4KPre;
      if constexpr (fn < KS) kfr[f % kW4KPre] = lds_read_b128<fn * 1024>(sbase + kq[fn & 1]);
      if constexpr (f == 0) mfma32_v0<F16>(acc, cur, qf[f]);
      else mfma32_v<F16>(acc, cur, qf[f]);
      if constexpr (vpf && f >= tail0 && f - tail0 < kW4VPre) v_read(vbase, IntC<f - tail0>{});
      hook(IntC<f>{});
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // The softmax in pieces sized to the issue slots an MFMA leaves its wave: one
  // 32-cycle MFMA window holds about two VALU operations beside a score MFMA and
  // its fragment read, one beside a P.V MFMA and its two transposing reads (a
  // transcendental counts twice).  Per step S:
  //  * max_piece m = 0 .. 10, in the P.V windows of the step that computed S:
  //    0-7 the lane's maximum (one v_max3 each), 8 the other half-wave's, 9 the
  //    scale, 10 the reference update (which scales l_run and records alpha);
  //  * exp_piece e = 0 .. 32, in the score windows of the next step: e = 2k takes
  //    s_k * scale - mref (and, k even, packs exponentials k - 2, k - 1), e = 2k + 1
  //    the exponential of k, e = 32 packs 14, 15;
  //  * sum_piece k = 0 .. 15, in the P.V windows of the next step: l_run += p_k.
  // A raised reference records alpha only: O is rescaled once the P.V in flight
  // (the previous step's, on the old reference) is done.
  constexpr int kMaxPieces = 11, kExpPieces = 33;
  float tmax = 0.f, mref = 0.f, alpha = 1.f;
  bool rescale = false;
  auto max_piece = [&](f32x16& sc, auto M) {
    constexpr int m = decltype(M)::value;
    if constexpr (m == 0) {
      tmax = max3(sc[0], sc[1], sc[2]);
      pin(tmax);
    } else if constexpr (m >= 1 && m <= 6) {
      tmax = max3(tmax, sc[2 * m + 1], sc[2 * m + 2]);
      pin(tmax);
    } else if constexpr (m == 7) {
      tmax = max3(tmax, sc[15], sc[15]);
      pin(tmax);
    } else if constexpr (m == 8) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
      tmax = max3(__uint_as_float(r[0]), __uint_as_float(r[1]), __uint_as_float(r[1]));
      pin(tmax);
    } else if constexpr (m == 9) {
      tmax *= p.scale_log2;
      pin(tmax);
    } else if constexpr (m == 10) {
      // m_ref is a reference maximum, raised only when a score passes it by more
      // than 2^kSlack: probabilities exp2(s - m_ref) may reach 2^kSlack, which fp32
      // and bf16 carry with unchanged relative precision
      if (__any(tmax > m_ref + kSlack)) {
        const float m_new = fmaxf(m_ref, tmax);
        alpha = m_ref == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(m_ref - m_new);
        l_run *= alpha;
        rescale = __any(alpha != 1.f && m_ref != -__builtin_inff());
        m_ref = m_new;
      }
      mref = m_ref == -__builtin_inff() ? 0.f : m_ref;
      pin(mref);
    }
  };
  auto pack = [&](f32x16& sc, dsa::i32x4 (&pb)[2], auto A) {
    constexpr int a = decltype(A)::value;
    int w = (int)dsa::pack_half2<F16>(sc[a], sc[a + 1]);
    pin(w);
    pb[a >> 3][(a & 7) >> 1] = w;
  };
  auto exp_piece = [&](f32x16& sc, dsa::i32x4 (&pb)[2], auto E) {
    constexpr int e = decltype(E)::value;
    constexpr int k = e >> 1;
    if constexpr (e < 32 && (e & 1) == 0) {
      if constexpr (k >= 2 && (k & 1) == 0) pack(sc, pb, IntC<k - 2>{});
      float x = fmaf(sc[k], p.scale_log2, -mref);
      pin(x);
      sc[k] = x;
    } else if constexpr (e < 32) {
      float x = __builtin_amdgcn_exp2f(sc[k]);
      pin(x);
      sc[k] = x;
    } else if constexpr (e == 32) {
      pack(sc, pb, IntC<14>{});
    }
  };
  auto sum_piece = [&](f32x16& sc, auto K) {
    l_run += sc[decltype(K)::value];
    pin(l_run);
  };
  auto max_range = [&](f32x16& sc) { static_for<0, kMaxPieces>([&](auto M) { max_piece(sc, M); }); };
  auto exp_range = [&](f32x16& sc, dsa::i32x4 (&pb)[2], auto LO) {
    static_for<decltype(LO)::value, kExpPieces>([&](auto E) { exp_piece(sc, pb, E); });
  };
  auto sum_range = [&](f32x16& sc) { static_for<0, 16>([&](auto K) { sum_piece(sc, K); }); };
  // invalid keys (a partial step, -1 or masked indices; rare) score -inf.
  // Element r of this lane is key 8 (r / 4) + 4 hh + r % 4 of the step.
  auto apply_mask = [&](f32x16& sc, uint32_t vmask) {
    if (vmask != 0xffffffffu) {
      const uint32_t m = vmask >> (4 * hh);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (!((m >> (8 * (r >> 2) + (r & 3))) & 1u)) sc[r] = -__builtin_inff();
    }
  };
  auto apply_rescale = [&]() {
    if (rescale) {
      mfma_drain();
      scale_o(alpha);
      rescale = false;
    }
  };

  // P.V of the step in `sbase` with P^T = pp: 32 MFMAs (d-tile dt, k-step kk),
  // fragment f = 2 dt + kk; hook(IntC<f>) after MFMA f.  The first kW4VPre
  // fragments are in flight already (read by the score loop) unless `fresh`.
  auto pv = [&](uint32_t sbase, const dsa::i32x4 (&pp)[2], bool fresh, auto&& hook) {
    if (fresh) static_for<0, kW4VPre>([&](auto F) { v_read(sbase, F); });
    static_for<0, 2 * ND>([&](auto F) {
      constexpr int f = decltype(F)::value;
      constexpr int dt = f >> 1, kk = f & 1;
      constexpr int younger = (2 * ND - 1 - f) < (kW4VPre - 1) ? (2 * ND - 1 - f) : (kW4VPre - 1);
      lds_wait<2 * younger>(vfr[f % kW4VPre][0], vfr[f % kW4VPre][1]);
      const dsa::i32x4 av = {vfr[f % kW4VPre][0][0], vfr[f % kW4VPre][0][1], vfr[f % kW4VPre][1][0],
                             vfr[f % kW4VPre][1][1]};
      constexpr int fn = f + kW4VPre;
      if constexpr (fn < 2 * ND) {
        constexpr int dn = fn >> 1, kn = fn & 1;
        vfr[f % kW4VPre][0] = lds_read_tr16<dn * 2048 + kn * 512>(sbase + vq[0]);
        vfr[f % kW4VPre][1] = lds_read_tr16<dn * 2048 + kn * 512>(sbase + vq[1]);
      }
      mfma32_o<dt, F16>(av, pp[kk]);
      hook(IntC<f>{});
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  const int nsteps = (nkeys + kKT - 1) / kKT;
  auto gather_wait = [&](int younger) {  // this wave's gathers done but `younger` steps
    if (younger >= 2) wait_vmcnt<2 * NCG>();
    else if (younger == 1) wait_vmcnt<NCG>();
    else wait_vmcnt<0>();
  };

  // ---- schedule.  Step j: wait for the gathers of step j, then the barrier
  // (stage j complete in every wave; stage j - 2 released by every wave), the
  // scores of j with the gathers of step j + 2 issued one chunk group every four
  // MFMAs (a burst of loads stalls the issuing wave) and the exponentials of
  // j - 1, then the P.V of j - 1 with the sums of j - 1 and the maximum of j.
  // Stages in use at step j: j - 1 (P.V), j (scores), j + 1 and j + 2 (loading).
  // The rows[] entries a step needs (its validity mask, the gather rows two steps
  // ahead) are read one step early, ahead of the fragment reads whose waits cover
  // them.  The loop is unrolled by two so that the parity buffers are registers.
  int32_t row_raw = 0, mask_raw = 0;
  if (nsteps > 0) {
    int32_t r0 = row_read(0), r1 = row_read(1);
    row_raw = row_read(2);
    mask_raw = mask_read(0);
    // tied to the wait: no use of the four values may be scheduled before it
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r0), "+v"(r1), "+v"(row_raw), "+v"(mask_raw)::"memory");
    issue(0, gather_src(row_ok(0, r0)));
    if (nsteps > 1) issue(1, gather_src(row_ok(1, r1)));
  }
  auto step = [&](int j, auto PAR) {
    constexpr int P = decltype(PAR)::value, Q = 1 - P;  // buffers of step j and of step j - 1
    gather_wait(min(1, nsteps - 1 - j));
    __builtin_amdgcn_s_barrier();
    const int32_t row_next = row_read(j + 3);
    const int32_t mask_next = mask_read(j + 1);
    const uint32_t vmask = mask_of(j, mask_raw);
    // the last two steps load the zero row into idle stages instead of branching
    // around each load
    const bool more = j + 2 < nsteps;
    const GSrc src = more ? gather_src(row_ok(j + 2, row_raw)) : no_src;
    if (wave_active) {
      const uint32_t sbase = lds0 + (j % kW4Stages) * STAGE;
      const uint32_t vbase = lds0 + ((j + kW4Stages - 1) % kW4Stages) * STAGE;  // stage of step j - 1
      if (j == 0) {
        scores(sacc[P], sbase, 0u, IntC<0>{}, [&](auto F) {
          constexpr int f = decltype(F)::value;
          if constexpr ((f & 3) == 1 && (f >> 2) < NCG) issue_one(j + 2, src, IntC<(f >> 2)>{});
        });
        mfma_drain();
        apply_mask(sacc[P], vmask);
        max_range(sacc[P]);
        rescale = false;  // O is still zero
      } else {
        // gathers at MFMAs 1, 5, 9, ..; exponential pieces of j - 1 after every MFMA
        scores(sacc[P], sbase, vbase, IntC<1>{}, [&](auto F) {
          constexpr int f = decltype(F)::value;
          if constexpr ((f & 3) == 1 && (f >> 2) < NCG) issue_one(j + 2, src, IntC<(f >> 2)>{});
          if constexpr (f < kExpPieces) exp_piece(sacc[Q], pbuf, IntC<f>{});
        });
        // pieces the score MFMAs had no room for (d_qk = 512)
        constexpr int placed = KS < kExpPieces ? KS : kExpPieces;
        exp_range(sacc[Q], pbuf, IntC<placed>{});
        mfma_drain();
        apply_mask(sacc[P], vmask);
        // sums of j - 1 at MFMAs 0 .. 15, the maximum of j at 16 .. 26
        pv(vbase, pbuf, false, [&](auto F) {
          constexpr int f = decltype(F)::value;
          if constexpr (f < 16) sum_piece(sacc[Q], IntC<f>{});
          if constexpr (f >= 16 && f - 16 < kMaxPieces) max_piece(sacc[P], IntC<f - 16>{});
        });
        static_assert(16 + kMaxPieces <= 2 * ND, "the softmax pieces fit the P.V MFMAs");
        apply_rescale();
      }
    } else {
      issue(j + 2, src);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // The two rows[] reads land in their registers asynchronously, after the
    // fragment waits above; a use here keeps the compiler from handing those
    // registers to other values before then (in the last steps the entries
    // themselves are not needed).
    asm volatile("" ::"v"(row_next), "v"(mask_next));
    row_raw = row_next;
    mask_raw = mask_next;
  };
  auto last = [&](auto PAR) {  // the step nsteps - 1 has parity PAR
    constexpr int P = decltype(PAR)::value;
    exp_range(sacc[P], pbuf, IntC<0>{});
    valu_to_mfma();
    pv(lds0 + ((nsteps - 1) % kW4Stages) * STAGE, pbuf, true, [&](auto F) {
      constexpr int f = decltype(F)::value;
      if constexpr (f < 16) sum_piece(sacc[P], IntC<f>{});
    });
  };
  if (nsteps > 0) step(0, IntC<0>{});
  int j = 1;
  for (; j + 1 < nsteps; j += 2) {
    step(j, IntC<1>{});
    step(j + 1, IntC<0>{});
  }
  if (j < nsteps) step(j, IntC<1>{});
  if (nsteps > 0 && wave_active) {
    if ((nsteps - 1) & 1) last(IntC<1>{});
    else last(IntC<0>{});
  }

  // ---- epilogue: lane (hh, l32) holds O^T[32 dt + 8 (r / 4) + 4 hh + r % 4][head l32]
  mfma_drain();
  const float l_tot = xor32_sum(l_run);
  const bool has = l_tot > 0.f;
  const float inv = has ? 1.f / l_tot : 0.f;
  const float lse_v = has ? (m_ref + __builtin_amdgcn_logf(l_tot)) * dsa::kLn2 : -__builtin_inff();

  // O^T leaves through LDS so that every global store writes a whole 1 KB output
  // row (one head, 64 lanes x 16 bytes) instead of 32 scattered 16-byte pieces.
  // Wave w's 32 rows sit at w * 32 KB of the (now idle) ring: 8-dim chunk c of
  // head h at h * 1024 + 16 (c ^ (h % 16)), its two 8-byte halves swapped for
  // h >= 16, which keeps both the 8-byte writes (32 heads of one half-wave) and
  // the 16-byte row reads free of bank conflicts.
  static_assert(32 * kDV * 2 * 4 <= kW4Stages * STAGE, "O staging fits the ring");
  __syncthreads();  // every wave is done with the ring
  unsigned char* const ob = smem + wave * (32 * kDV * 2);
  const int oh_sw = l32 & 15, ohalf = hh ^ ((l32 >> 4) & 1);
  auto o_put = [&](int c, dsa::i32x2 v) {
    *reinterpret_cast<dsa::i32x2*>(ob + l32 * (kDV * 2) + 16 * (c ^ oh_sw) + 8 * ohalf) = v;
  };
  auto o_flush = [&](uint16_t* rows_out) {  // rows_out: row of this wave's first head
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int nh = min(32, p.H - (hg * kHeadsPerGroup + wave * 32));
#pragma unroll 8
    for (int i = 0; i < 32; ++i) {
      if (i >= nh) break;
      dsa::i32x4 v = *reinterpret_cast<const dsa::i32x4*>(ob + i * (kDV * 2) + 16 * (lane ^ (i & 15)));
      if (i & 16) v = dsa::i32x4{v[2], v[3], v[0], v[1]};
      *reinterpret_cast<dsa::i32x4*>(rows_out + (int64_t)i * kDV + 8 * lane) = v;
    }
  };
  const int64_t head0 = hg * kHeadsPerGroup + wave * 32;  // this wave's first head
  if (p.nsplit == 1) {
    static_for<0, ND>([&](auto D) {
      constexpr int dt = decltype(D)::value;
      float t[16];
      read_o<dt>(t);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        dsa::i32x2 v;
        v[0] = (int)dsa::pack_half2<F16>(t[4 * q4] * inv, t[4 * q4 + 1] * inv);
        v[1] = (int)dsa::pack_half2<F16>(t[4 * q4 + 2] * inv, t[4 * q4 + 3] * inv);
        o_put(4 * dt + q4, v);
      }
    });
    if (wave_active) o_flush(p.out + (token * p.H + head0) * kDV);
    if (head_ok && hh == 0 && p.lse) p.lse[token * p.H + head] = lse_v;
  } else {
    // fp16 partials scaled by a power of two per (token, head), as the 8-wave form
    const int64_t prow0 = (token * p.nsplit + split) * p.H;
    float amax = 0.f;
    static_for<0, ND>([&](auto D) {
      float t[16];
      read_o<decltype(D)::value>(t);
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(t[i]));
    });
    amax = xor32_max(amax) * inv;
    int e = 0;
    if (amax > 0.f) (void)frexpf(amax, &e);
    const float down = ldexpf(inv, -e);
    static_for<0, ND>([&](auto D) {
      constexpr int dt = decltype(D)::value;
      float t[16];
      read_o<dt>(t);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const _Float16 h0 = (_Float16)(t[4 * q4] * down), h1 = (_Float16)(t[4 * q4 + 1] * down);
        const _Float16 h2 = (_Float16)(t[4 * q4 + 2] * down), h3 = (_Float16)(t[4 * q4 + 3] * down);
        dsa::i32x2 v;
        v[0] = (int)((uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16));
        v[1] = (int)((uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16));
        o_put(4 * dt + q4, v);
      }
    });
    if (wave_active) o_flush(p.part_o + (prow0 + head0) * kDV);
    if (head_ok && hh == 0) {
      p.part_lse[prow0 + head] = lse_v;
      p.part_scale[prow0 + head] = ldexpf(1.f, e);
    }
  }
}

// Merge split partials: lse = logsumexp_p lse_p, out = sum_p exp(lse_p - lse) out_p.
// 64 threads per (token, head) row, 8 dims (16 bytes of fp16) each, four rows per
// block.  The lse, scale and slice of kCombineU splits are all loaded before any
// is used, so a row costs one round trip per kCombineU splits; chunks beyond the
// first are merged online (the running sums rescaled to the new maximum).
// kCombineU is 4 for up to 4 splits (no idle load slots: config-3 decode 59.6 ->
// 58.0 us, bit-identical), else 8 (16 or 32 measured no faster at 32 splits).
constexpr int kCombineRows = 4;  // rows per 256-thread block

template <bool F16, int kCombineU>
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
  for (int e = 0; e < 4; ++e) ov[e] = (int)dsa::pack_half2<F16>(acc[2 * e] * f, acc[2 * e + 1] * f);
  *reinterpret_cast<dsa::i32x4*>(out + rh * kDV + 8 * d8) = ov;
  if (d8 == 0 && lse) lse[rh] = den > 0.f ? mx + __logf(den) : -__builtin_inff();
}

template <int DQK, int STAGES, int WAVES, bool F16>
int launch_mla_stages(const MlaParams& p, int64_t nblocks, hipStream_t stream) {
  // ring, the rows[] list, one last-valid-key slot per wave
  const size_t smem = (size_t)STAGES * kKT * DQK * 2 + sizeof(int32_t) * ((size_t)p.keys_per_split + WAVES);
  auto fn = sparse_mla_kernel<DQK, STAGES, WAVES, F16>;
  static std::atomic<int> lds_reserved[dsa::kMaxDevices];
  const int rc = dsa::reserve_lds((const void*)fn, smem, lds_reserved, "sparse_mla");
  if (rc != dsa::kOk) return rc;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblocks), dim3(WAVES * 64), smem, stream, p);
  return dsa::check_launch("dsa_sparse_mla_fwd");
}

template <int DQK, bool F16, bool BUF, int KIND>
int launch_mla_w4_as(const MlaParams& p, int64_t nblocks, hipStream_t stream) {
  // ring, the rows[] list, one last-valid-key slot and a row range per wave
  const size_t smem = (size_t)kW4Stages * kKT * DQK * 2 + sizeof(int32_t) * ((size_t)p.keys_per_split + 12);
  auto fn = mla_w4_kernel<DQK, F16, BUF, KIND>;
  static std::atomic<int> lds_reserved[dsa::kMaxDevices];
  const int rc = dsa::reserve_lds((const void*)fn, smem, lds_reserved, "sparse_mla");
  if (rc != dsa::kOk) return rc;
  hipLaunchKernelGGL(fn, dim3((unsigned)nblocks), dim3(256), smem, stream, p);
  return dsa::check_launch("dsa_sparse_mla_fwd");
}

template <int DQK, bool F16>
int launch_mla_w4(MlaParams p, int64_t nblocks, hipStream_t stream) {
  // one causal sequence in one split: short rows spread over the XCDs
  // (balanced_token), whose grid needs up to 8 more workgroups
  if (p.B == 1 && p.nsplit == 1 && p.nhg == 1 && p.causal && !p.v4_on && !p.direct && p.topk > 0) {
    p.balance = 1;
    nblocks = ((int64_t)p.S + dsa::kNumXcd - 1) / dsa::kNumXcd * dsa::kNumXcd + dsa::kNumXcd;
  }
  // rows of the pool: a page pool (or resolved rows), or B sequences of skv rows
  const int64_t rows = (p.block_table || p.direct) ? p.pool_rows : (int64_t)p.B * p.skv;
  // the buffer's byte offsets are 32-bit: pools of at most 4 GiB
  const int64_t records = rows * (DQK / 8);
  if (p.kv2 == nullptr && records * 16 <= ((int64_t)1 << 32)) {
    p.buf_records = (uint32_t)records;
    // the bf16, d_qk 576 path of DeepSeek's layers has kernels per list kind
    if constexpr (DQK == 576 && !F16) {
      if (!p.v4_on && !p.direct)
        return p.block_table ? launch_mla_w4_as<DQK, F16, true, kListPaged>(p, nblocks, stream)
                             : launch_mla_w4_as<DQK, F16, true, kListContig>(p, nblocks, stream);
    }
    return launch_mla_w4_as<DQK, F16, true, kListAny>(p, nblocks, stream);
  }
  p.buf_records = 0u;
  return launch_mla_w4_as<DQK, F16, false, kListAny>(p, nblocks, stream);
}

// Workgroup form.  More than 64 heads: the 4-wave, 128-head form (one
// workgroup per CU, a 4-stage ring, O in the accumulation registers).  64 or
// fewer heads: 4-wave, 64-head workgroups with 2-stage rings (<= 80 KB of LDS
// each) that pair up on a CU, so one's prologue and epilogue runs beside the
// other's steps -- when two of them fit in the CU's 160 KB of LDS.
template <int DQK, bool F16>
int launch_mla(const MlaParams& p, int64_t nblocks, hipStream_t stream) {
  const size_t lds4 = (size_t)kStagesPair * kKT * DQK * 2 + sizeof(int32_t) * (size_t)p.keys_per_split + 64;
  if (p.H <= 64 && 2 * lds4 <= 160 * 1024) return launch_mla_stages<DQK, kStagesPair, 4, F16>(p, nblocks, stream);
  return launch_mla_w4<DQK, F16>(p, nblocks, stream);
}

int choose_splits(int64_t tokens, int nhg, int topk) {
  // split the index list until the 256 CUs are covered, keeping >= 256 keys per
  // split (more splits cost more partials than the extra CUs return).  A handful
  // of rows (single-token decode) is latency bound instead: each halving saves
  // key steps down to splits of 64 keys (two steps; beyond that the combine's
  // extra rounds cost more), but the first split, which adds the combine launch,
  // pays only for lists of more than 128 keys.  Single-token decode, one
  // MI355X: top-2048 16 -> 32 splits 29.6 -> 27.9 us, V4 csa 4 -> 8 splits
  // 21.3 -> 18.9 us, a 128-key list 1 -> 2 splits 15.8 -> 16.1 us.
  const bool few = tokens * nhg < 16;
  const int min_keys = few ? 64 : 256;
  int ns = 1;
  if (!few || topk > 128)
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
  p.balance = 0;
  // index order of the gathers where neighbouring query tokens of a sequence
  // share rows (a prefill, contiguous or paged)
  p.order = r.S > 1 && !r.direct && r.v4 == nullptr;

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
  const int rc = r.f16 ? (r.d_qk == 576 ? launch_mla<576, true>(p, nblocks, st) : launch_mla<512, true>(p, nblocks, st))
                       : (r.d_qk == 576 ? launch_mla<576, false>(p, nblocks, st) : launch_mla<512, false>(p, nblocks, st));
  if (rc != kOk || ns == 1) return rc;
  const int64_t rows = T * r.H;
  const dim3 cgrid((unsigned)((rows + kCombineRows - 1) / kCombineRows));
  auto combine = [&](auto U) {
    constexpr int u = decltype(U)::value;
    if (r.f16)
      hipLaunchKernelGGL((mla_combine_kernel<true, u>), cgrid, dim3(256), 0, st, p.part_o, p.part_lse, p.part_scale,
                         rows, r.H, ns, p.out, r.lse);
    else
      hipLaunchKernelGGL((mla_combine_kernel<false, u>), cgrid, dim3(256), 0, st, p.part_o, p.part_lse, p.part_scale,
                         rows, r.H, ns, p.out, r.lse);
  };
  if (ns <= 4) combine(IntC<4>{});
  else combine(IntC<8>{});
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

namespace {

int mla_fwd_entry(const void* q, const void* kv, const int32_t* indices, const int32_t* block_table,
                  const int32_t* kv_len, const int32_t* q_start, const float* attn_sink, int64_t B, int64_t S,
                  int32_t H, int32_t d_qk, int32_t d_v, int64_t skv, int32_t block_size, int32_t max_blocks,
                  int32_t topk, float sm_scale, int32_t is_causal, int32_t num_splits, void* out, float* lse,
                  void* workspace, size_t workspace_bytes, void* stream, int32_t f16, const char* what) {
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
  r.f16 = f16;
  r.out = out;
  r.lse = lse;
  r.workspace = workspace;
  r.workspace_bytes = workspace_bytes;
  r.stream = stream;
  return dsa::sparse_mla_run(r, what);
}

}  // namespace

extern "C" int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* indices,
                                  const int32_t* block_table, const int32_t* kv_len,
                                  const int32_t* q_start, const float* attn_sink, int64_t B,
                                  int64_t S, int32_t H, int32_t d_qk, int32_t d_v, int64_t skv,
                                  int32_t block_size, int32_t max_blocks, int32_t topk,
                                  float sm_scale, int32_t is_causal, int32_t num_splits, void* out,
                                  float* lse, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  return mla_fwd_entry(q, kv, indices, block_table, kv_len, q_start, attn_sink, B, S, H, d_qk, d_v, skv, block_size,
                       max_blocks, topk, sm_scale, is_causal, num_splits, out, lse, workspace, workspace_bytes, stream,
                       0, "dsa_sparse_mla_fwd");
}

extern "C" int dsa_sparse_mla_fwd_f16(const void* q, const void* kv, const int32_t* indices,
                                      const int32_t* block_table, const int32_t* kv_len,
                                      const int32_t* q_start, const float* attn_sink, int64_t B,
                                      int64_t S, int32_t H, int32_t d_qk, int32_t d_v, int64_t skv,
                                      int32_t block_size, int32_t max_blocks, int32_t topk,
                                      float sm_scale, int32_t is_causal, int32_t num_splits, void* out,
                                      float* lse, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  return mla_fwd_entry(q, kv, indices, block_table, kv_len, q_start, attn_sink, B, S, H, d_qk, d_v, skv, block_size,
                       max_blocks, topk, sm_scale, is_causal, num_splits, out, lse, workspace, workspace_bytes, stream,
                       1, "dsa_sparse_mla_fwd_f16");
}
