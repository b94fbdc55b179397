// Lightning-indexer logits for fp16 / bf16 q and k (the reference wrapper's own
// input dtypes, examples/deepseek_v4/lightning_indexer.py:1250-1255) on gfx950
// 16-bit MFMA:
//
//   logits[row, s] = key_scale[s] * sum_{h < N1} w[row, h] * ReLU(q[row, h, :] . k[s, :])
//
// with the rows, causal rule, layouts (BSND / TND query rows; BSND / TND / paged
// keys), row lengths and -inf convention of the fp8 kernel (indexer.hip) and of
// the golden cpu_lightning_indexer (:199-335).  q.k is accumulated in fp32 from
// the exact 16-bit products, as the golden computes it, but the head sum is formed
// as (sum_h w_h d_h + sum_h w_h |d_h|) / 2 rather than sum_h w_h ReLU(d_h): the
// negative heads' terms cancel between the two sums, so a logit's rounding error
// is bounded by a few fp32 ulps of sum_h |w_h d_h| (not of the logit itself), and
// a logit much smaller than that sum carries a larger relative error than the
// golden's own rounding.  N1 <= 64 heads (the missing heads count as zero).
//
// Work decomposition.  One workgroup = 8 waves = 8 query tokens (one per wave, two
// waves per SIMD) of one batch row x one chunk of keys.  A wave holds its token's
// q as MFMA A operands (64 heads x 128 dims, 64 VGPRs) and its head weights.  Key
// tiles of 64 x 128 16-bit values stream through a 3-stage LDS ring with
// global_load_lds, chunk c of key s stored at slot c ^ (s % 16) so that the 32
// keys of one B-operand read hit distinct banks.  Per 32-key block a wave issues
// 16 v_mfma_f32_32x32x16 (2 head tiles x 8 k-steps; one tile when N1 <= 32); a
// lane then holds 16 heads' q.k of one key per tile and applies ReLU and the
// weights, one block behind, its FMAs interleaved with the next block's MFMAs
// (two accumulator sets).  Once per
// 64-key tile one permlane swap adds the other half of the heads for both blocks,
// and the tile's logits (and, for long rows, the maxima of its four 16-key groups,
// which the top-k uses as on the fp8 path) are stored.
#include "dsa_common.h"

#include <type_traits>

namespace {

constexpr int kHWaves = 8;
constexpr int kHThreads = kHWaves * 64;
constexpr int kHTokPerBlock = kHWaves;  // one query token per wave
constexpr int kHHeads = 64;
constexpr int kHDim = 128;
constexpr int kHTile = 64;                      // keys per LDS tile
constexpr int kHStages = 3;
constexpr int kHTileBytes = kHTile * kHDim * 2;  // 16 KB
constexpr int kHLoadsPerTile = kHTileBytes / 1024 / kHWaves;  // 1 KB loads per wave and tile: 2
constexpr int kHMaxChunk = 131072;
constexpr int kHMaxChunkPaged = 16384;  // the chunk's pool rows are held in LDS

struct H16Params {
  const uint16_t* q;          // [q rows, N1, 128]
  const uint16_t* k;          // [B * S2 or T2 or pool rows, 128]
  const float* key_scale;     // per key row, or null
  const float* w;             // [q rows, N1] fp32
  const int32_t* act_q;       // [B] per-batch query lengths or null
  const int32_t* act_k;       // [B] per-batch key lengths or null
  const int32_t* cum_q;       // [B] prefix sums of the query lengths or null
  const int32_t* cum_k;       // [B] prefix sums of the key lengths or null
  const int32_t* block_table;  // [B, max_blocks] or null
  int64_t pool_rows;
  int block_size, max_blocks;
  float* logits;      // [q rows, ld]
  int32_t* row_len;   // [q rows] or null
  float* gmax;        // [q rows, ld_g] maxima of 16-key groups, or null
  int64_t ld;
  int64_t ld_g;
  int B, S1, S2, N1, sparse_mode;
  int chunk, ntb, nkc;
  int64_t per_xcd;
};

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

__device__ __forceinline__ int visible_keys(int t, int aq, int ak, int sparse_mode) {
  if (t >= aq) return 0;
  if (sparse_mode == 3) {
    const int cl = ak - aq + t + 1;
    return cl > 0 ? cl : ak;
  }
  return ak;
}

// s_waitcnt vmcnt(n) for a small run-time n (one immediate form per case).
__device__ __forceinline__ void wait_vmcnt_rt(int n) {
  switch (n) {
    case 0: dsa::wait_vmcnt<0>(); break;
    case 1: dsa::wait_vmcnt<1>(); break;
    case 2: dsa::wait_vmcnt<2>(); break;
    case 3: dsa::wait_vmcnt<3>(); break;
    case 4: dsa::wait_vmcnt<4>(); break;
    case 5: dsa::wait_vmcnt<5>(); break;
    case 6: dsa::wait_vmcnt<6>(); break;
    case 7: dsa::wait_vmcnt<7>(); break;
    case 8: dsa::wait_vmcnt<8>(); break;
    case 9: dsa::wait_vmcnt<9>(); break;
    case 10: dsa::wait_vmcnt<10>(); break;
    default: dsa::wait_vmcnt<11>(); break;
  }
}

template <bool F16>
__device__ __forceinline__ dsa::f32x16 mfma32(dsa::i32x4 a, dsa::i32x4 b, dsa::f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(dsa::f16x8, a), __builtin_bit_cast(dsa::f16x8, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(dsa::bf16x8, a),
                                                   __builtin_bit_cast(dsa::bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ int32_t lds_read_i32(uint32_t addr) {
  int32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// Source of the key loads for pages outside the pool (never scored).
__device__ __align__(16) uint16_t g_zero_key16[kHDim];
__device__ float g_zero_scale16[kHTile];

// HT: 32-head tiles computed (1 when N1 <= 32: the second tile's heads are all
// zero and would only add zeros).
template <bool F16, bool PAGED, bool GMAX, int HT>
__global__ __launch_bounds__(kHThreads) void indexer_h16_kernel(H16Params p) {
  static_assert(HT == 1 || HT == 2, "one or two head tiles");
  __shared__ __align__(1024) uint8_t ktile[kHStages][kHTileBytes];
  __shared__ __align__(256) float kscale[kHStages][kHTile];
  __shared__ int32_t krows[PAGED ? kHMaxChunkPaged : 1];

  // work item (key group (b, chunk), token block), key group major, 8 contiguous
  // ranges dealt to the 8 XCDs (the workgroups of one key chunk share an L2)
  const int bid = blockIdx.x;
  const int xcd = bid % dsa::kNumXcd, r = bid / dsa::kNumXcd;
  const int64_t witem = (int64_t)xcd * p.per_xcd + r;
  if (r >= p.per_xcd || witem >= (int64_t)p.B * p.nkc * p.ntb) return;
  const int kg = (int)(witem / p.ntb), tb = (int)(witem % p.ntb);
  const int b = kg / p.nkc, kc = kg % p.nkc;

  int aq, ak;
  int64_t qbase, kbase_row;
  if (p.cum_q) {
    qbase = b > 0 ? p.cum_q[b - 1] : 0;
    aq = clampi(p.cum_q[b] - (int)qbase, 0, p.S1);
  } else {
    qbase = (int64_t)b * p.S1;
    aq = p.act_q ? clampi(p.act_q[b], 0, p.S1) : p.S1;
  }
  if (p.cum_k) {
    kbase_row = b > 0 ? p.cum_k[b - 1] : 0;
    ak = clampi(p.cum_k[b] - (int)kbase_row, 0, p.S2);
  } else {
    kbase_row = (int64_t)b * p.S2;
    ak = p.act_k ? clampi(p.act_k[b], 0, p.S2) : p.S2;
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = lane >> 5, l32 = lane & 31;

  // visible_keys is ak over a leading run of tokens (mode 3, cl <= 0), then
  // nondecreasing up to aq, then 0, so its maximum over the block's tokens
  // [t0, t1) lies at t0 or t1 - 1
  const int t0 = tb * kHTokPerBlock;
  const int t1 = min(min(t0 + kHTokPerBlock, p.S1), aq);
  const int lmax =
      t0 < t1 ? max(visible_keys(t0, aq, ak, p.sparse_mode), visible_keys(t1 - 1, aq, ak, p.sparse_mode)) : 0;
  const int k0 = kc * p.chunk;
  const int kend = min(k0 + p.chunk, p.S2);
  const int k1 = min(kend, lmax);

  const int tok = tb * kHTokPerBlock + wave;
  const bool tok_ok = p.cum_q ? tok < aq : tok < p.S1;
  const int L = tok_ok ? visible_keys(tok, aq, ak, p.sparse_mode) : 0;
  if (kc == 0 && p.row_len != nullptr && lane == 0 && tok_ok) p.row_len[qbase + tok] = L;
  if (k0 >= k1) return;  // workgroup-uniform
  const int64_t trow = qbase + (tok_ok ? tok : 0);

  // ---- per-token operands: A of head tile t, k-step ks = head 32 t + l32, dims
  // 16 ks + 8 hh .. + 8; the weight of result element r of tile t (head
  // 32 t + 8 (r / 4) + 4 hh + r % 4); heads >= N1 are zero
  dsa::i32x4 qa[HT][8];
  float wv[HT][16];
#pragma unroll
  for (int t = 0; t < HT; ++t) {
    const int head = 32 * t + l32;
    const bool ok = tok_ok && head < p.N1;
    const uint16_t* qp = p.q + (trow * p.N1 + (ok ? head : 0)) * kHDim + 8 * hh;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qa[t][ks] = ok ? *reinterpret_cast<const dsa::i32x4*>(qp + 16 * ks) : dsa::i32x4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int hr = 32 * t + 8 * (e >> 2) + 4 * hh + (e & 3);
      wv[t][e] = (tok_ok && hr < p.N1) ? p.w[trow * p.N1 + hr] : 0.f;
    }
  }
  if constexpr (PAGED) {
    for (int i = tid; i < k1 - k0; i += kHThreads) {
      const int key = k0 + i;
      const int blk = key / p.block_size;
      const int pg = blk < p.max_blocks ? p.block_table[(int64_t)b * p.max_blocks + blk] : -1;
      const int64_t row = (int64_t)pg * p.block_size + key % p.block_size;
      krows[i] = (pg >= 0 && row < p.pool_rows) ? (int32_t)row : -1;
    }
  }
  // without key scales the scale ring holds 1.0 for good (no scale loads are issued)
  if (p.key_scale == nullptr && tid < kHStages * kHTile) (&kscale[0][0])[tid] = 1.f;
  dsa::wait_vmcnt<0>();  // operands in registers before the ring's loads are counted
  __syncthreads();       // krows[] (and the scale ring) ready

  // ---- key tiles: wave w's load i fills 1 KB block 2 w + i of the tile: lane l
  // loads key 4 (2 w + i) + l / 16, 16-byte slot l % 16 holding chunk
  // (l % 16) ^ (key % 16); wave 0 also loads the tile's 64 key scales
  const int ntiles = (k1 - k0 + kHTile - 1) / kHTile;
  const uint16_t* kbase = PAGED ? p.k : p.k + kbase_row * kHDim;
  const float* sbase = p.key_scale ? (PAGED ? p.key_scale : p.key_scale + kbase_row) : nullptr;
  const int nload = kHLoadsPerTile + ((wave == 0 && sbase != nullptr) ? 1 : 0);
  // Contiguous keys are read through buffer descriptors over the batch row's
  // keys [0, k1): 16-byte records for the keys (record 16 s + chunk), 4-byte
  // records for the scales; a key at or past k1 (the tail of the last tile, or a
  // tile past the end, issued so that the ring's counts hold) reads zeros, and
  // no lane computes a 64-bit address.
  const __amdgpu_buffer_rsrc_t krsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)16, PAGED ? 0 : k1 * (kHDim / 8), 0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(sbase != nullptr ? sbase : g_zero_scale16), (short)4, PAGED || sbase == nullptr ? 0 : k1, 0x00020000);
  auto issue = [&](int tile) {
    unsigned char* dst = &ktile[tile % kHStages][0];
    if constexpr (PAGED) {
      const int t = tile < ntiles ? tile : ntiles - 1;  // past the end: the last tile again (never read)
      const int kt0 = k0 + t * kHTile;
#pragma unroll
      for (int i = 0; i < kHLoadsPerTile; ++i) {
        const int kk = 4 * (kHLoadsPerTile * wave + i) + (lane >> 4);
        const int key = min(kt0 + kk, k1 - 1);
        const int row = krows[key - k0];
        const int c = (lane & 15) ^ (kk & 15);
        const uint16_t* src = row >= 0 ? kbase + (int64_t)row * kHDim + 8 * c : g_zero_key16 + 8 * c;
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                         (DSA_LDS void*)(dst + 1024 * (kHLoadsPerTile * wave + i)), 16, 0, 0);
      }
      if (wave == 0 && sbase != nullptr) {
        const int key = min(kt0 + lane, k1 - 1);
        const int row = krows[key - k0];
        const float* src = row >= 0 ? sbase + row : g_zero_scale16 + lane;
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), (DSA_LDS void*)&kscale[tile % kHStages][0],
                                         4, 0, 0);
      }
    } else {
      const uint32_t kt0 = (uint32_t)(k0 + tile * kHTile);
#pragma unroll
      for (int i = 0; i < kHLoadsPerTile; ++i) {
        const int kk = 4 * (kHLoadsPerTile * wave + i) + (lane >> 4);
        const uint32_t rec = (uint32_t)(kk * (kHDim / 8) + ((lane & 15) ^ (kk & 15)));
        __builtin_amdgcn_struct_ptr_buffer_load_lds(krsrc, (DSA_LDS void*)(dst + 1024 * (kHLoadsPerTile * wave + i)),
                                                    16, kt0 * (kHDim / 8) + rec, 0, 0, 0, 0);
      }
      if (wave == 0 && sbase != nullptr)
        __builtin_amdgcn_struct_ptr_buffer_load_lds(srsrc, (DSA_LDS void*)&kscale[tile % kHStages][0], 4,
                                                    kt0 + (uint32_t)lane, 0, 0, 0, 0);
    }
  };

  // B-operand reads: key 32 blk + l32 of the tile, chunk 2 ks + hh
  const uint32_t tile0 = (uint32_t)(size_t)(DSA_LDS unsigned char*)&ktile[0][0];
  const uint32_t sc0 = (uint32_t)(size_t)(DSA_LDS unsigned char*)&kscale[0][0];

  // logit stores through a buffer descriptor over this row's part of the chunk:
  // stores past it (keys >= kend, an absent token, the lanes of the second head
  // half) are dropped by the hardware
  float* orow = p.logits + trow * p.ld + k0;
  const __amdgpu_buffer_rsrc_t ost =
      __builtin_amdgcn_make_buffer_rsrc(orow, (short)0, tok_ok ? (kend - k0) * 4 : 0, 0x00020000);
  // group maxima: one float per 16 keys (the chunk start is a multiple of 64)
  const __amdgpu_buffer_rsrc_t gst = __builtin_amdgcn_make_buffer_rsrc(
      GMAX ? p.gmax + trow * p.ld_g + k0 / 16 : p.logits, (short)0,
      (GMAX && tok_ok) ? ((kend - k0 + 15) / 16) * 4 : 0, 0x00020000);
  // stores per tile: a logit (and a group-maxima) store
  constexpr int kStoresPerTile = GMAX ? 2 : 1;

#pragma unroll
  for (int i = 0; i < kHStages - 1; ++i) issue(i);

  // Block b's FMAs run beside block b + 1's MFMAs (the accumulators alternate
  // between two sets by block parity), and a tile's epilogue runs once its second
  // block's FMAs are done, in the next tile: a permlane swap adds the two head
  // halves of both blocks at once, leaving block 0's logits in lanes 0-31 and
  // block 1's in lanes 32-63 (lane l holds key l of the tile), so the tile takes
  // one key-scale read, one 256-byte logit store and one group-maxima pass.  The
  // first tile's "previous" epilogue stores to offsets the buffer range drops.
  dsa::f32x16 acc[2][2] = {};  // [block parity][head tile]; tile 1 unused when HT == 1
  float hA = 0.f;  // this lane's half-head sum of block 0 of the current tile
  float tksc = 0.f;  // the previous tile's key scale, key and store offsets
  int tkey = 0, toff = 0x40000000, tgoff = 0x40000000;
  // sum_h w_h ReLU(d_h) = (sum_h w_h d_h + sum_h w_h |d_h|) / 2 (|.| is a free
  // source modifier; max would also need a canonicalising instruction), element e
  // of the head tiles
  auto fma_pair = [&](const dsa::f32x16& a0, const dsa::f32x16& a1, int e, float& s1, float& s2) {
    s1 = fmaf(wv[0][e], a0[e], s1);
    s2 = fmaf(wv[0][e], fabsf(a0[e]), s2);
    if constexpr (HT == 2) {
      s1 = fmaf(wv[HT - 1][e], a1[e], s1);
      s2 = fmaf(wv[HT - 1][e], fabsf(a1[e]), s2);
    }
  };
  // a / b: the half-head sums of the tile's blocks 0 and 1 (lane l < 32: heads of
  // the lower half, l >= 32: the upper half, key l % 32)
  auto finish_tile = [&](float a, float b, float ksc, int key, int off, int goff) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    const float s = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    const float v = key < L ? s * ksc : -__builtin_inff();
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ost, off, 0, 0);
    if constexpr (GMAX) {
      // max over each row of 16 lanes (16 consecutive keys): v_max_f32 with DPP
      // quad swaps, then half-row and row mirrors (each DPP source written two
      // wait states earlier).  v_max_f32 returns the non-NaN operand, and the
      // top-k orders NaN last, so a NaN logit never raises a group's maximum.
      float m = v;
      asm volatile(
          "s_nop 1\n"
          "v_max_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n"
          "s_nop 1\n"
          "v_max_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n"
          "s_nop 1\n"
          "v_max_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n"
          "s_nop 1\n"
          "v_max_f32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf"
          : "+v"(m));
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m), gst, goff, 0, 0);
    }
  };
  for (int it = 0; it < ntiles; ++it) {
    // tile it's loads are done once the younger ones may remain: the next tile's
    // loads and the stores of each of the (at most two) tiles finished since
    wait_vmcnt_rt(nload + (it == 0 ? 0 : (it == 1 ? kStoresPerTile : 2 * kStoresPerTile)));
    // a bare barrier: __syncthreads() would also drain the prefetched tiles
    __builtin_amdgcn_s_barrier();
    issue(it + kHStages - 1);
    const int st = it % kHStages;
    const uint32_t tb0 = tile0 + st * kHTileBytes;
    dsa::static_for<0, 2>([&](auto BLK) {
      constexpr int blk = decltype(BLK)::value;
      constexpr int pb = 1 - blk;  // the previous block's set
      // the B fragments (and in block 1 the tile's 64 key scales, read first and
      // complete once the first fragment is) as asm reads with counted waits: a
      // compiler-issued LDS read would first wait for every LDS-DMA load in
      // flight, the prefetched tiles included.  The scales are read before the
      // next tile's loads can overwrite their ring stage.
      const uint32_t rowa = tb0 + (32 * blk + l32) * (kHDim * 2);
      int32_t raw = 0;
      if constexpr (blk == 1) raw = lds_read_i32(sc0 + 4 * (st * kHTile + lane));
      dsa::i32x4 kb[8];
      dsa::static_for<0, 8>([&](auto KS) {
        constexpr int ks = decltype(KS)::value;
        kb[ks] = dsa::lds_read_b128<0>(rowa + 16 * ((2 * ks + hh) ^ (l32 & 15)));
      });
      dsa::f32x16 a0 = {}, a1 = {};
      float s1 = 0.f, s2 = 0.f;
      dsa::static_for<0, 8>([&](auto KS) {
        constexpr int ks = decltype(KS)::value;
        if constexpr (ks == 0 && blk == 1)
          asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(kb[0]), "+v"(raw));
        else
          dsa::lds_wait1<7 - ks>(kb[ks]);
        a0 = mfma32<F16>(qa[0][ks], kb[ks], a0);
        if constexpr (HT == 2) a1 = mfma32<F16>(qa[HT - 1][ks], kb[ks], a1);
        fma_pair(acc[pb][0], acc[pb][1], 2 * ks, s1, s2);
        fma_pair(acc[pb][0], acc[pb][1], 2 * ks + 1, s1, s2);
        __builtin_amdgcn_sched_barrier(0);
      });
      acc[blk][0] = a0;
      acc[blk][1] = a1;
      if constexpr (blk == 0) {
        // the FMAs just done were block 1 of the previous tile: its epilogue
        finish_tile(hA, 0.5f * (s1 + s2), tksc, tkey, toff, tgoff);
      } else {
        hA = 0.5f * (s1 + s2);  // block 0 of this tile
        tksc = __int_as_float(raw);
        tkey = k0 + it * kHTile + lane;
        toff = (it * kHTile + lane) * 4;
        // lanes 0, 16, 32 and 48 store the tile's four groups
        tgoff = (lane & 15) == 0 ? (it * (kHTile / 16) + (lane >> 4)) * 4 : 0x40000000;
      }
    });
  }
  {
    // the last tile's block 1 and epilogue
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) fma_pair(acc[1][0], acc[1][1], e, s1, s2);
    finish_tile(hA, 0.5f * (s1 + s2), tksc, tkey, toff, tgoff);
  }
  // no LDS DMA may still be in flight when the workgroup's LDS is released
  dsa::wait_vmcnt<0>();
}

}  // namespace

namespace dsa {

int topk_launch(const float* x, int64_t rows, int64_t cols, int64_t ld, const int32_t* row_len,
                const float* gmax, int64_t ld_g, int32_t K, int32_t pad_invalid, int32_t* out_idx,
                float* out_val, hipStream_t stream);

}  // namespace dsa

namespace {

int indexer_h16_launch(const H16Params& base, bool f16, hipStream_t stream) {
  using namespace dsa;
  H16Params p = base;
  p.ntb = (p.S1 + kHTokPerBlock - 1) / kHTokPerBlock;
  int chunk = p.block_table != nullptr ? kHMaxChunkPaged : kHMaxChunk;
  while (chunk > kHTile && (int64_t)p.B * p.ntb * ((p.S2 + chunk - 1) / chunk) < 256) chunk >>= 1;
  p.chunk = chunk;
  p.nkc = (p.S2 + chunk - 1) / chunk;
  const int64_t work = (int64_t)p.B * p.nkc * p.ntb;
  p.per_xcd = (work + kNumXcd - 1) / kNumXcd;
  const int64_t nblocks = p.per_xcd * kNumXcd;
  if (nblocks <= 0) return kOk;
  if (nblocks > 0x7fffffff) return set_error(kUnsupported, "indexer (16-bit): grid too large");
  const dim3 grid((unsigned)nblocks), blk(kHThreads);
  const bool paged = p.block_table != nullptr, gm = p.gmax != nullptr;
  const bool one_tile = p.N1 <= 32;
  auto go = [&](auto F16C, auto PAGEDC, auto GMAXC) {
    constexpr bool kF16 = decltype(F16C)::value, kPaged = decltype(PAGEDC)::value, kGmax = decltype(GMAXC)::value;
    if (one_tile) hipLaunchKernelGGL((indexer_h16_kernel<kF16, kPaged, kGmax, 1>), grid, blk, 0, stream, p);
    else hipLaunchKernelGGL((indexer_h16_kernel<kF16, kPaged, kGmax, 2>), grid, blk, 0, stream, p);
  };
  using T = std::true_type;
  using F = std::false_type;
  if (f16) {
    if (paged) gm ? go(T{}, T{}, T{}) : go(T{}, T{}, F{});
    else gm ? go(T{}, F{}, T{}) : go(T{}, F{}, F{});
  } else {
    if (paged) gm ? go(F{}, T{}, T{}) : go(F{}, T{}, F{});
    else gm ? go(F{}, F{}, T{}) : go(F{}, F{}, F{});
  }
  return check_launch("dsa_lightning_indexer_h16_varlen");
}


}  // namespace

extern "C" size_t dsa_lightning_indexer_varlen_workspace_bytes(int64_t q_rows, int64_t S2);

extern "C" int dsa_lightning_indexer_h16_varlen(const void* q, const void* k, const float* key_scale,
                                                const float* weights, const int32_t* seq_q,
                                                int32_t seq_q_cumulative, const int32_t* seq_k,
                                                int32_t seq_k_cumulative, const int32_t* block_table,
                                                int32_t block_size, int32_t max_blocks, int64_t pool_rows,
                                                int64_t B, int64_t S1, int64_t S2, int64_t q_rows, int32_t N1,
                                                int32_t D, int32_t is_f16, int32_t sparse_count,
                                                int32_t sparse_mode, int32_t* indices, float* values,
                                                void* workspace, size_t workspace_bytes, void* stream) {
  using namespace dsa;
  const char* what = "dsa_lightning_indexer_h16_varlen";
  if (sparse_count < 1 || sparse_count > 8192)
    return set_error(kInvalidArgument, "%s: sparse_count must be in [1, 8192], got %d", what, sparse_count);
  if (N1 < 1 || N1 > kHHeads || D != kHDim)
    return set_error(kUnsupported, "%s: 1..64 index heads x 128 dims are built (got %d x %d)", what, N1, D);
  if (B < 0 || S1 < 0 || S2 < 0 || q_rows < 0 || S1 > 0x7fffffff || S2 > 0x7fffffff || B > 0x7fffffff)
    return set_error(kInvalidArgument, "%s: bad sizes", what);
  if (sparse_mode != 0 && sparse_mode != 3)
    return set_error(kInvalidArgument, "%s: sparse_mode must be 0 or 3, got %d", what, sparse_mode);
  if (!seq_q_cumulative && q_rows != B * S1)
    return set_error(kInvalidArgument, "%s: padded query rows need q_rows = B * S1", what);
  if ((seq_q_cumulative && seq_q == nullptr) || (seq_k_cumulative && seq_k == nullptr))
    return set_error(kInvalidArgument, "%s: cumulative lengths need a length array", what);
  if (block_table != nullptr) {
    if (block_size <= 0 || max_blocks <= 0 || pool_rows < 0 || pool_rows > 0x7fffffff)
      return set_error(kInvalidArgument, "%s: paged keys need block_size > 0, max_blocks > 0 and pool_rows in "
                                         "[0, 2^31)", what);
    if (seq_k_cumulative)
      return set_error(kInvalidArgument, "%s: paged keys take per-batch key lengths, not prefix sums", what);
  }
  if (q_rows == 0) return kOk;
  const size_t need = dsa_lightning_indexer_varlen_workspace_bytes(q_rows, S2);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(kWorkspaceTooSmall, "%s: workspace of %zu bytes needed, %zu given", what, need, workspace_bytes);
  if (indices == nullptr) return set_error(kInvalidArgument, "%s: null indices", what);
  // the fp8 entry points' workspace layout (logits | row lengths | group maxima)
  const IndexerWorkspace wl = indexer_workspace(q_rows, S2);
  float* logits = static_cast<float*>(workspace);
  int32_t* row_len = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + wl.rowlen_off);
  float* gmax = use_group_max(S2, sparse_count) ? reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.gmax_off)
                                                : nullptr;
  hipStream_t st = (hipStream_t)stream;
  if (S2 == 0 || B == 0 || S1 == 0)  // no keys (or no rows to score): every row is all -1
    return topk_launch(logits, q_rows, 0, 0, nullptr, nullptr, 0, sparse_count, 1, indices, values, st);
  if (q == nullptr || k == nullptr || weights == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", what);
  if ((reinterpret_cast<uintptr_t>(q) & 15u) != 0 || (reinterpret_cast<uintptr_t>(k) & 15u) != 0)
    return set_error(kInvalidArgument, "%s: q and k must be 16-byte aligned", what);
  // the kernel writes every row's length (the chunk-0 workgroup of its token block)
  H16Params p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.key_scale = key_scale;
  p.w = weights;
  p.act_q = seq_q_cumulative ? nullptr : seq_q;
  p.cum_q = seq_q_cumulative ? seq_q : nullptr;
  p.act_k = seq_k_cumulative ? nullptr : seq_k;
  p.cum_k = seq_k_cumulative ? seq_k : nullptr;
  p.block_table = block_table;
  p.block_size = block_size;
  p.max_blocks = max_blocks;
  p.pool_rows = pool_rows;
  p.logits = logits;
  p.row_len = row_len;
  p.gmax = gmax;
  p.ld = S2;
  p.ld_g = wl.ld_g;
  p.B = (int)B;
  p.S1 = (int)S1;
  p.S2 = (int)S2;
  p.N1 = N1;
  p.sparse_mode = sparse_mode;
  const int rc = indexer_h16_launch(p, is_f16 != 0, st);
  if (rc != kOk) return rc;
  return topk_launch(logits, q_rows, S2, S2, row_len, gmax, wl.ld_g, sparse_count, 1, indices, values, st);
}
