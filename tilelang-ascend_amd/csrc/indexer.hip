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
// Formulation.  ReLU(d) = (d + |d|) / 2, so with u_t = sum_h w[t, h] q[t, h, :]
//   sum_h w_h ReLU(q_h . k) = ( sum_h w_h |q_h . k|  +  u_t . k ) / 2.
// The first sum costs one FMA per (head, key) with the |.| source modifier.  The
// second is an fp8 MFMA whose A rows hold u split into four fp8 pieces with
// power-of-two scales (E8M0 block scales of the MFMA), u = sum_s 2^(e-4s) u_s,
// exact to 2^-17 of max|u|; its 16 rows carry the pieces of 4 tokens, so one
// MFMA per 16 keys serves 4 waves.  Both terms keep fp32-level accuracy; q.k is
// never rounded to a narrower type.
//
// Work decomposition.  One workgroup = 16 waves = 16 query tokens (one per wave)
// of one batch row x one chunk of keys.  A wave holds its token's A operands
// (64 heads x 128 dims of fp8 plus the u pieces) in registers.  K streams through
// an 8-stage LDS ring of 64-key tiles filled with global_load_lds, consumed in
// pairs of tiles with one workgroup barrier per pair (four tiles in flight while
// a pair is computed; one barrier per tile cost ~2 % more at 128K keys); a tile
// stores 16-byte chunk j of key s at slot j ^ (s & 7) ^ ((s >> 3) & 1), which
// keeps the B-operand reads (16 keys x one chunk, 128-byte rows) on distinct
// banks for both 8- and 16-lane LDS phases.  Per 16-key block a wave issues 4 fp8
// MFMAs (v_mfma_scale_f32_16x16x128_f8f6f4) and 16 FMAs, and once per tile the u
// MFMA for one block of its group of 4 waves (the results pass through LDS).  The
// 4 lane groups then exchange their partial sums with permlane swaps (a
// reduce-scatter) so that lane l ends up with key 64-tile + l and the tile is one
// coalesced 256-byte store.  That reduce-scatter of tile i runs in tile i+1 and
// the rest of its epilogue (u.k, scale, store) in tile i+2, behind the barrier
// that publishes tile i's u.k and behind the first MFMAs of the tile, so the
// waves released by a barrier start with matrix work rather than all doing VALU
// work at once.  Workgroups that share a key chunk are placed on the same XCD so
// the chunk stays in that XCD's L2.
#include "dsa_common.h"

namespace {

constexpr int kWaves = 16;
constexpr int kThreads = kWaves * 64;
constexpr int kTokPerBlock = kWaves;  // one query token per wave
constexpr int kHeads = 64;
constexpr int kDim = 128;
constexpr int kKeyTile = 64;
constexpr int kStages = 8;  // ring of key tiles; one barrier per pair of tiles
constexpr int kTileBytes = kKeyTile * kDim;      // 8 KB
constexpr int kKeyLoaders = kTileBytes / 1024;   // 1 KB loads per tile (waves 0..7 or 8..15)
constexpr int kSplits = 4;                       // fp8 pieces of u
constexpr int kE4m3Max = 448;
constexpr int kMaxChunk = 131072;                // keys per workgroup at most
constexpr int kMaxChunkPaged = 16384;            // paged keys: the chunk's pool rows are held in LDS

struct IndexerParams {
  const uint8_t* q;        // [B, S1, 64, 128] fp8
  const uint8_t* k;        // [B, S2, 128] fp8
  const float* key_scale;  // [B, S2] or null
  const float* w;          // [B, S1, 64]
  const int32_t* act_q;    // [B] per-batch query lengths or null
  const int32_t* act_k;    // [B] per-batch key lengths or null
  const int32_t* cum_q;    // [B] prefix sums of the query lengths (varlen rows) or null
  const int32_t* cum_k;    // [B] prefix sums of the key lengths (varlen keys) or null
  const int32_t* block_table;  // [B, max_blocks] pages of the key pool (paged keys) or null
  int64_t pool_rows;       // keys in the page pool
  int block_size, max_blocks;
  float* logits;           // [B * S1, ld]
  int32_t* row_len;        // [B * S1] or null
  float* gmax;             // [B * S1, ld_g] maxima of 16-key groups of the logits, or null
  int64_t ld;
  int64_t ld_g;
  int B, S1, S2, sparse_mode;
  int chunk, ntb, nkc;
  int64_t per_xcd;        // work items (key group, token block) per XCD
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

// Maximum over the 64 lanes of a wave, in every lane: DPP quad permutes and
// row mirrors within each row of 16 lanes, then the permlane swaps across rows
// (no LDS round trip; max is exact, so the combining order does not matter).
template <int CTL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));   // quad_perm [1,0,3,2]
  x = fmaxf(x, dpp_f32<0x4E>(x));   // quad_perm [2,3,0,1]
  x = fmaxf(x, dpp_f32<0x141>(x));  // row_half_mirror
  x = fmaxf(x, dpp_f32<0x140>(x));  // row_mirror
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
}

// u/2 = sum_h (w_h / 2) q_h of one token, for the u MFMA.  token_u_load issues
// the query loads: lane (r, cc) = (lane >> 4, lane & 15) takes heads 16r ..
// 16r+15, bytes 8cc .. 8cc+7 of each (sixteen 8-byte loads, all in flight).
// token_u_sum forms the partial sums of those heads for the 8 dims with the
// token's weights (wl: its 64 weights, staged in LDS), and a reduce-scatter over
// the four lane rows (permlane swaps) leaves lane (r, cc) the totals of dims
// 8cc + 2r and 8cc + 2r + 1, returned in u0, u1 (the function returns that
// first dim).  Every dim's total is (rows 0 + 2) + (rows 1 + 3).  The sums are
// taken as sum_h w_h q_h and halved at the end, which rounds exactly as the
// sum of (w_h / 2) q_h does (a power-of-two scale commutes with rounding,
// subnormal results aside).
__device__ __forceinline__ void token_u_load(const uint8_t* qtok, int lane, dsa::i32x2 (&qv)[16]) {
  const uint8_t* qp = qtok + 16 * (lane >> 4) * kDim + 8 * (lane & 15);
#pragma unroll
  for (int j = 0; j < 16; ++j) qv[j] = *reinterpret_cast<const dsa::i32x2*>(qp + j * kDim);
}

__device__ __forceinline__ int token_u_sum(const dsa::i32x2 (&qv)[16], const float* wl, int lane, float& u0,
                                           float& u1) {
  const int r = lane >> 4, cc = lane & 15;
  dsa::f32x4 wv[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) wv[k] = *reinterpret_cast<const dsa::f32x4*>(wl + 16 * r + 4 * k);
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float w = wv[j >> 2][j & 3];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(qv[j][hf], false);  // bytes 0, 1
      const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(qv[j][hf], true);   // bytes 2, 3
      a[4 * hf + 0] = fmaf(w, lo[0], a[4 * hf + 0]);
      a[4 * hf + 1] = fmaf(w, lo[1], a[4 * hf + 1]);
      a[4 * hf + 2] = fmaf(w, hi[0], a[4 * hf + 2]);
      a[4 * hf + 3] = fmaf(w, hi[1], a[4 * hf + 3]);
    }
  }
  // rows 0, 1 keep dims 0..3 of their 8, rows 2, 3 dims 4..7 (pairs of rows 0-2, 1-3)
  float b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[i]), __float_as_uint(a[4 + i]), false, false);
    b[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  // row r keeps dims 2r, 2r + 1 (pairs of rows 0-1, 2-3)
  float t[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(b[i]), __float_as_uint(b[2 + i]), false, false);
    t[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  u0 = 0.5f * t[0];
  u1 = 0.5f * t[1];
  return 8 * cc + 2 * r;
}

// Makes this wave's LDS writes visible to its own later LDS reads of other
// lanes' entries (the compiler may not move such reads above the writes).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Waits until at most n of this wave's vector-memory operations are in flight
// (n is a small run-time value; each case is an immediate s_waitcnt).
__device__ __forceinline__ void wait_vmcnt_upto(int n) {
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
    default: dsa::wait_vmcnt<10>(); break;
  }
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(size_t)(const DSA_LDS unsigned char*)p;
}

// s_waitcnt lgkmcnt(N) tied to both halves of a B fragment.
template <int N>
__device__ __forceinline__ void lds_wait2(dsa::i32x4& a, dsa::i32x4& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}

template <int OFF>
__device__ __forceinline__ float lds_read_f32(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}

// Source of the key loads for pages outside the pool (never scored: such keys
// only occur in malformed block tables, which the host wrapper rejects).
__device__ __align__(16) uint8_t g_zero_key[kDim];
__device__ float g_zero_scale[kKeyTile];

// PAGED: keys live in a page pool [blocks * block_size, D] addressed through
// p.block_table; the physical rows of this workgroup's key chunk are resolved
// once into LDS.  GMAX: the maxima of 16-key groups are emitted (p.gmax); as a
// template parameter it costs the loop nothing when they are not wanted.
template <bool PAGED, bool GMAX>
__global__ __launch_bounds__(kThreads) void indexer_fp8_kernel(IndexerParams p) {
  __shared__ __align__(1024) uint8_t ktile[kStages][kTileBytes];
  __shared__ int32_t krows[PAGED ? kMaxChunkPaged : 1];
  __shared__ __align__(256) float kscale[kStages][kKeyTile];
  // u pieces, rows padded to 144 B so the 16 rows one MFMA operand read touches
  // fall on distinct banks
  __shared__ __align__(16) uint8_t usplit[kWaves][kSplits][kDim + 16];
  __shared__ int uexp[kWaves];
  __shared__ __align__(16) float wsh[kWaves][kHeads];  // each token's weights
  __shared__ __align__(16) float lin[4][kWaves][kKeyTile];  // u.k per token and key, four tiles

  // XCD-aware mapping: the work items (key group (b, chunk), token block), key
  // group major, are cut into 8 equal contiguous ranges, one per XCD (workgroup
  // ids are dealt to the XCDs round-robin), so the XCDs get equal work and the
  // workgroups sharing a key chunk run on one XCD, its keys in that XCD's L2.
  const int bid = blockIdx.x;
  const int xcd = bid % dsa::kNumXcd, r = bid / dsa::kNumXcd;
  const int64_t witem = (int64_t)xcd * p.per_xcd + r;
  if (r >= p.per_xcd || witem >= (int64_t)p.B * p.nkc * p.ntb) return;
  // the host bounds the grid (hence witem) below 2^31: 32-bit division
  const int kg = (int)witem / p.ntb, tb = (int)witem % p.ntb;
  const int b = kg / p.nkc, kc = kg % p.nkc;

  // Rows of batch b: varlen (prefix sums) or padded [B, S1] / [B, S2].
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
  const int g = lane >> 4, c = lane & 15;

  // Key range of this workgroup: its chunk, clipped to what its tokens can see.
  // visible_keys is ak over a leading run of tokens (mode 3, cl <= 0), then
  // nondecreasing up to aq, then 0, so its maximum over the block's tokens
  // [t0, t1) lies at t0 or t1 - 1
  const int t0 = tb * kTokPerBlock;
  const int t1 = min(min(t0 + kTokPerBlock, p.S1), aq);
  const int lmax =
      t0 < t1 ? max(visible_keys(t0, aq, ak, p.sparse_mode), visible_keys(t1 - 1, aq, ak, p.sparse_mode)) : 0;
  const int k0 = kc * p.chunk;
  const int kend = min(k0 + p.chunk, p.S2);  // last key this workgroup may write
  const int k1 = min(kend, lmax);            // last key any token needs

  const int tok = tb * kTokPerBlock + wave;
  // varlen rows past the batch's length do not exist; padded rows do (row_len 0)
  const bool tok_ok = p.cum_q ? tok < aq : tok < p.S1;
  const int L = tok_ok ? visible_keys(tok, aq, ak, p.sparse_mode) : 0;
  if (kc == 0 && p.row_len != nullptr && lane == 0 && tok_ok) p.row_len[qbase + tok] = L;
  if (k0 >= k1) return;
  const int64_t trow = qbase + (tok_ok ? tok : 0);

  // ---- key tiles ------------------------------------------------------------
  const int ntiles = (k1 - k0 + kKeyTile - 1) / kKeyTile;
  const uint8_t* kbase = PAGED ? p.k : p.k + kbase_row * kDim;
  const float* sbase = p.key_scale ? (PAGED ? p.key_scale : p.key_scale + kbase_row) : nullptr;
  // The ring is filled a pair of tiles at a time, and every wave issues exactly
  // one 1 KB load per pair: waves 0-7 fill the pair's first tile, waves 8-15 its
  // second, so the loads' address work does not make some waves late at the
  // pair barrier.  Lane l of wave w fills LDS bytes [(w % 8) KB + 16 l, +16) of
  // its tile: key s = 8 (w % 8) + l/8, slot l%8, which holds the key's chunk
  // (l%8) ^ swz(s).  Waves 7 and 15 also load their tile's 64 key scales.
  const int lslice = wave & 7, lhalf = wave >> 3;
  const int lkey = 8 * lslice + (lane >> 3);
  const int lchunk = (lane & 7) ^ (lkey & 7) ^ ((lkey >> 3) & 1);
  const bool scale_loader = lslice == kKeyLoaders - 1 && sbase != nullptr;
  // Contiguous keys are read through buffer descriptors over the batch row's
  // keys [0, k1): 16-byte records for the keys (record 8 s + chunk), 4-byte
  // records for the scales.  A key at or past k1 (the tail of the last tile, or
  // a tile past the end, issued so that every pair has its one load) reads
  // zeros, and no lane computes a 64-bit address.
  const __amdgpu_buffer_rsrc_t krsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)16, PAGED ? 0 : k1 * (kDim / 16), 0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(sbase != nullptr ? sbase : g_zero_scale), (short)4, PAGED || sbase == nullptr ? 0 : k1, 0x00020000);
  const uint32_t krec = (uint32_t)(lkey * (kDim / 16) + lchunk);
  // the loads of the pair (tile0, tile0 + 1); tile0 is even
  auto issue = [=](int tile0) {
    const int t = tile0 + lhalf;
    const int kt0 = k0 + t * kKeyTile;
    DSA_LDS void* kdst = (DSA_LDS void*)&ktile[t & (kStages - 1)][1024 * lslice];
    DSA_LDS void* sdst = (DSA_LDS void*)&kscale[t & (kStages - 1)][0];
    if constexpr (PAGED) {
      // past the end: the last tile's keys again, into a free ring slot (never read)
      const int tt = t < ntiles ? t : ntiles - 1;
      const int key = min(k0 + tt * kKeyTile + lkey, k1 - 1);
      const int row = krows[key - k0];
      const uint8_t* src = row >= 0 ? kbase + (int64_t)row * kDim + 16 * lchunk : g_zero_key + 16 * lchunk;
      __builtin_amdgcn_global_load_lds(src, kdst, 16, 0, 0);
      if (scale_loader) {
        const int skey = min(k0 + tt * kKeyTile + lane, k1 - 1);
        const int srow = krows[skey - k0];
        const float* ssrc = srow >= 0 ? sbase + srow : g_zero_scale + lane;
        __builtin_amdgcn_global_load_lds(ssrc, sdst, 4, 0, 0);
      }
    } else {
      __builtin_amdgcn_struct_ptr_buffer_load_lds(krsrc, kdst, 16, (uint32_t)kt0 * (kDim / 16) + krec, 0, 0, 0, 0);
      if (scale_loader)
        __builtin_amdgcn_struct_ptr_buffer_load_lds(srsrc, sdst, 4, (uint32_t)(kt0 + lane), 0, 0, 0, 0);
    }
  };
  // ---- per-token operands -------------------------------------------------
  // Row trow exists (a workgroup that reaches this point has a valid token, so
  // its batch has row qbase): every load below is issued unconditionally, and a
  // wave past the batch's tokens zeroes its weights and A operands once they
  // arrive (loads behind a wave-uniform condition would become branches that
  // each wait for their load).  First the u sums' operands (the token's 64
  // weights, one per lane, copied into LDS, and the query bytes in the u sums'
  // layout); the ring's first tiles and the A operands are requested while the
  // sums are formed.
  const int qkeep = tok_ok ? -1 : 0;
  __builtin_amdgcn_global_load_lds(p.w + trow * kHeads + lane, (DSA_LDS void*)&wsh[wave][0], 4, 0, 0);
  dsa::i32x2 qv[16];
  token_u_load(p.q + trow * kHeads * kDim, lane, qv);
  dsa::wait_vmcnt<0>();
  wave_lds_sync();
  // u/2 = sum_h (w_h / 2) q_h: lane (r, cc) ends with dims udim and udim + 1.
  float u0 = 0.f, u1 = 0.f;
  int udim = 2 * lane;
  if (tok_ok) udim = token_u_sum(qv, &wsh[wave][0], lane, u0, u1);
  // w/2 for the heads whose |q.k| this lane's accumulators hold (16mt + 4g + i).
  float wh[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const dsa::f32x4 v = *reinterpret_cast<const dsa::f32x4*>(&wsh[wave][16 * mt + 4 * g]);
#pragma unroll
    for (int i = 0; i < 4; ++i) wh[mt][i] = __int_as_float(__float_as_int(0.5f * v[i]) & qkeep);
  }
  // Contiguous keys: the ring's first tiles (paged keys need the chunk's rows
  // first, below).
  if constexpr (!PAGED) {
#pragma unroll
    for (int i = 0; i < kStages - 2; i += 2) issue(i);
  }
  // q: lane (g, c) holds head 16*mt + c, bytes [32g, 32g+32) of the head.
  dsa::i32x8 qa[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const dsa::i32x4* src =
        reinterpret_cast<const dsa::i32x4*>(p.q + (trow * kHeads + 16 * mt + c) * kDim + 32 * g);
    const dsa::i32x4 lo = src[0], hi = src[1];
    qa[mt] = dsa::i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  // Power-of-two split of u: sigma_s = 2^(e - 4s) with max|u| / 2^e in (224, 448].
  const float umax = wave_max(fmaxf(fabsf(u0), fabsf(u1)));
  int e = -100;
  if (umax > 0.f) {
    int ex;
    (void)frexpf(umax / (float)kE4m3Max, &ex);  // umax/448 = f * 2^ex, f in [0.5, 1)
    e = clampi(ex, -100, 100);
  }
  if (lane == 0) uexp[wave] = e;
  if constexpr (PAGED) {
    // physical pool row of every key of the chunk (-1: page outside the pool)
    for (int i = tid; i < k1 - k0; i += kThreads) {
      const int key = k0 + i;
      const int blk = key / p.block_size;
      const int pg = blk < p.max_blocks ? p.block_table[(int64_t)b * p.max_blocks + blk] : -1;
      const int64_t row = (int64_t)pg * p.block_size + key % p.block_size;
      krows[i] = (pg >= 0 && row < p.pool_rows) ? (int32_t)row : -1;
    }
  }
  {
    float r0 = u0, r1 = u1;
#pragma unroll
    for (int sp = 0; sp < kSplits; ++sp) {
      const float inv = ldexpf(1.f, 4 * sp - e), sig = ldexpf(1.f, e - 4 * sp);
      const int pk = __builtin_amdgcn_cvt_pk_fp8_f32(r0 * inv, r1 * inv, 0, false);
      *reinterpret_cast<uint16_t*>(&usplit[wave][sp][udim]) = (uint16_t)pk;
      r0 = fmaf(-sig, __builtin_amdgcn_cvt_f32_fp8(pk, 0), r0);
      r1 = fmaf(-sig, __builtin_amdgcn_cvt_f32_fp8(pk, 1), r1);
    }
  }
  // without key scales the scale ring holds 1.0 for good (no scale loads are issued)
  if (sbase == nullptr && tid < kStages * kKeyTile) (&kscale[0][0])[tid] = 1.f;
  __syncthreads();
  // u pieces of the group's 4 tokens as A rows: row 4*tq + sp = piece sp of token
  // grp0 + tq; lane (g, c) holds row c, bytes 32g..32g+31.  In the result, lane
  // (g, c) then holds the 4 pieces (rows 4g..4g+3) of token grp0 + g for key c.
  // The operand stays in LDS (read once per tile, where it is used).
  const int grp0 = wave & ~3, ublk = wave & 3;
  const uint32_t ua_addr = lds_addr(&usplit[grp0 + (c >> 2)][c & 3][32 * g]);
  const int uscale = clampi(127 + uexp[grp0 + (c >> 2)] - 4 * (c & 3), 1, 254);

  // B-operand reads: lane (g, c) reads key 16blk + c, chunks 2g and 2g+1.
  const int rslot = (2 * g) ^ (c & 7) ^ (c >> 3);
  const uint32_t rd0 = lds_addr(&ktile[0][0]) + c * kDim + 16 * rslot;
  const uint32_t rd1 = lds_addr(&ktile[0][0]) + c * kDim + 16 * (rslot ^ 1);
  const uint32_t sc_addr = lds_addr(&kscale[0][0]) + 4 * lane;
  const uint32_t ub_rd0 = rd0 + (wave & 3) * 2048, ub_rd1 = rd1 + (wave & 3) * 2048;  // block ublk

  // Logit stores: a buffer descriptor over this row's part of the chunk; stores
  // past it (keys >= kend, or an out-of-range token) are dropped by the hardware,
  // so every wave issues exactly one store per tile.
  float* orow = p.logits + trow * p.ld + k0;
  const __amdgpu_buffer_rsrc_t ost = __builtin_amdgcn_make_buffer_rsrc(
      orow, (short)0, tok_ok ? (kend - k0) * 4 : 0, 0x00020000);
  // Group maxima: one float per 16 keys (the chunk start is a multiple of 64).
  constexpr bool want_gmax = GMAX;
  // Group maxima of four consecutive tiles are gathered in one register (lane
  // 16 j + s holds group j of tile 4 b + s) and stored together.
  const int gslot_lane = lane & 15;
  float gacc = 0.f;
  const __amdgpu_buffer_rsrc_t gst = __builtin_amdgcn_make_buffer_rsrc(
      want_gmax ? p.gmax + trow * p.ld_g + k0 / 16 : p.logits, (short)0,
      (want_gmax && tok_ok) ? ((kend - k0 + 15) / 16) * 4 : 0, 0x00020000);

#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int j = 0; j < 8; ++j) qa[mt][j] &= qkeep;
  // the u pieces' A operand, read once (loop invariant)
  dsa::i32x8 ua;
  {
    dsa::i32x4 u0 = dsa::lds_read_b128<0>(ua_addr), u1 = dsa::lds_read_b128<16>(ua_addr);
    lds_wait2<0>(u0, u1);
    ua = dsa::i32x8{u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
  }
  // The operand loads above complete before the loop (their values were used,
  // and loads complete in issue order), so the only vector memory operations in
  // flight inside the loop are the ring's and the stores.
  if constexpr (PAGED) {
    dsa::wait_vmcnt<0>();
#pragma unroll
    for (int i = 0; i < kStages - 2; i += 2) issue(i);
  }

  // u.k hand-off: this wave writes block ublk of its group's 4 tokens, reads its own token.
  const uint32_t lin_wr = lds_addr(&lin[0][grp0 + g][16 * ublk + c]);
  const uint32_t lin_rd = lds_addr(&lin[0][wave][lane]);
  constexpr uint32_t kLinBuf = kWaves * kKeyTile * 4;

  // Epilogue of a finished tile: reduce-scatter of the partial sums, plus u.k,
  // times the key scale, masked, stored.  tile < 0 issues a store that the
  // buffer range check drops, so every iteration has exactly one store.
  // lk: this lane's u.k of the tile (read from LDS by the caller, already waited for).
  auto reduce = [&](const float (&ap)[4]) {
    float r02, r13;
    {
      const auto s0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ap[0]), __float_as_uint(ap[2]), false, false);
      r02 = __uint_as_float(s0[0]) + __uint_as_float(s0[1]);
      const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ap[1]), __float_as_uint(ap[3]), false, false);
      r13 = __uint_as_float(s1[0]) + __uint_as_float(s1[1]);
    }
    const auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(r02), __float_as_uint(r13), false, false);
    return __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
  };
  auto finish = [&](float sum, float ksp, float lk, int tile, auto SLOT) {
    constexpr int kSlot = decltype(SLOT)::value;  // tile % 4, or -1: the last tiles (run-time slot)
    // A tile < 0 (the first pair has no finished tile) has a negative offset,
    // which the descriptor's range check drops as a huge unsigned one.
    sum += lk;
    if (k0 + (tile + 1) * kKeyTile <= L) {  // the whole tile is visible (wave-uniform)
      sum *= ksp;
    } else {
      const int key = k0 + tile * kKeyTile + lane;
      sum = key < L ? sum * ksp : -__builtin_inff();
    }
    const int voff = (tile * kKeyTile + lane) * 4;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sum), ost, voff, 0, 0);
    if constexpr (want_gmax) {
      // max over each row of 16 lanes (16 consecutive keys): v_max_f32 with DPP
      // quad swaps, then half-row and row mirrors (each DPP source written two
      // wait states earlier).  v_max_f32 returns the non-NaN operand, and the
      // top-k orders NaN last, so a NaN logit never raises a group's maximum.
      float m = sum;
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
      const int slot = kSlot >= 0 ? kSlot : (tile & 3);
      gacc = gslot_lane == slot ? m : gacc;
      if (kSlot == 3 || kSlot < 0) {
        // lanes 16 j + s, s <= slot, store group j of tile (tile - slot + s); the
        // other lanes' offsets are out of range (dropped), as are tiles < 0
        const int t = tile - slot + gslot_lane;
        const int goff = (gslot_lane <= slot && t >= 0) ? (t * 4 + (lane >> 4)) * 4 : 0x40000000;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(gacc), gst, goff, 0, 0);
      }
    }
  };

  const dsa::f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  // ap / ksp: partial sums and key scale of the previous tile; s2 / k2: the
  // reduced sums and key scale of the tile before it
  float ap[4] = {0.f, 0.f, 0.f, 0.f};
  float ksp = 1.f, s2 = 0.f, k2 = 1.f;
  // One tile; ST = it % kStages is a compile-time ring slot, so every LDS offset
  // below is an instruction immediate.  Tiles go in pairs (it even, it + 1) with
  // one barrier per pair; a tile's epilogue runs two tiles later, in the next
  // pair, behind the barrier that publishes its u.k.
  auto step = [&](int it, auto STC) {
    constexpr int ST = decltype(STC)::value;
    constexpr int SUB = ST & 1;
    constexpr uint32_t so = ST * kTileBytes;
    if constexpr (SUB == 0) {
      // This wave's load for the pair (it, it + 1) is done once at most
      // min(2 + it, 8) newer memory operations are in flight: it was issued at
      // pair it - 6 (or in the prologue, followed by the prologue's later
      // loads), and each pair since issued one load and one logit store per
      // tile; a group-maxima store every fourth tile, or a scale load (waves 7
      // and 15, after their key load), only adds to them, so the bound stays
      // safe.  Its LDS writes and reads of the previous pair are complete.
      wait_vmcnt_upto(min(2 + it, 8));
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ksp), "+v"(k2));
      __builtin_amdgcn_s_barrier();
      // The four waves of a SIMD are served oldest-first; a wave lowers its
      // priority as it gets through the pair, so the four finish it together
      // instead of the oldest idling at the next barrier.
      __builtin_amdgcn_s_setprio(3);
      issue(it + kStages - 2);
    }

    const float ksc = lds_read_f32<ST * kKeyTile * 4>(sc_addr);
    // u.k of tile it - 2 (written in the previous pair); issued ahead of the B
    // fragments so that their first wait covers it
    float lkp = lds_read_f32<((ST + 2) & 3) * kLinBuf>(lin_rd);
    float a[4];
    // B fragments of block blk (16 keys x 128 B); the next block's read is in
    // flight while the current block's MFMAs run.
    dsa::i32x4 nb0 = dsa::lds_read_b128<so>(rd0), nb1 = dsa::lds_read_b128<so>(rd1);
    dsa::static_for<0, 4>([&](auto BLK) {
      constexpr int blk = decltype(BLK)::value;
      dsa::i32x4 b0 = nb0, b1 = nb1;
      if constexpr (blk < 3) {
        nb0 = dsa::lds_read_b128<so + (blk + 1) * 2048>(rd0);
        nb1 = dsa::lds_read_b128<so + (blk + 1) * 2048>(rd1);
        if constexpr (blk == 0)
          asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(b0), "+v"(b1), "+v"(lkp));
        else
          lds_wait2<2>(b0, b1);
      } else {
        lds_wait2<0>(b0, b1);
      }
      const dsa::i32x8 bf = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
      dsa::f32x4 d[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)  // D[row = head 16mt + 4g + i][col = key 16blk + c]
        d[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[mt], bf, zero, 0, 0, 0, 127, 0, 127);
      if constexpr (blk == 0) {
        const float s1 = reduce(ap);  // tile it - 1
        finish(s2, k2, lkp, it - 2, dsa::IntC<(ST + 2) & 3>{});
        s2 = s1;
        k2 = ksp;
      }
      float acc = 0.f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = fmaf(wh[mt][i], fabsf(d[mt][i]), acc);
      a[blk] = acc;
      constexpr int prio = 3 - ((4 * SUB + blk + 1) * 3) / 8;
      __builtin_amdgcn_s_setprio(prio);
    });
    {
      // u.k of block ublk for the group's 4 tokens -> LDS (read two tiles later).
      dsa::i32x4 k0v = dsa::lds_read_b128<so>(ub_rd0), k1v = dsa::lds_read_b128<so>(ub_rd1);
      lds_wait2<0>(k0v, k1v);
      const dsa::i32x8 ub = {k0v[0], k0v[1], k0v[2], k0v[3], k1v[0], k1v[1], k1v[2], k1v[3]};
      const dsa::f32x4 du = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ua, ub, zero, 0, 0, 0, uscale, 0, 127);
      const float lv = (du[0] + du[1]) + (du[2] + du[3]);
      asm volatile("ds_write_b32 %0, %1 offset:%2" : : "v"(lin_wr), "v"(lv), "i"((ST & 3) * kLinBuf) : "memory");
    }
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) ap[blk] = a[blk];
    ksp = ksc;
  };
  for (int it = 0; it < ntiles; it += kStages) {
    step(it, dsa::IntC<0>{});
    if (it + 1 < ntiles) step(it + 1, dsa::IntC<1>{});
    if (it + 2 < ntiles) step(it + 2, dsa::IntC<2>{});
    if (it + 3 < ntiles) step(it + 3, dsa::IntC<3>{});
    if (it + 4 < ntiles) step(it + 4, dsa::IntC<4>{});
    if (it + 5 < ntiles) step(it + 5, dsa::IntC<5>{});
    if (it + 6 < ntiles) step(it + 6, dsa::IntC<6>{});
    if (it + 7 < ntiles) step(it + 7, dsa::IntC<7>{});
  }
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ksp), "+v"(k2));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_s_setprio(0);
  // the epilogues of the last two tiles
  auto lin_of = [&](int t) {
    float lk;
    switch (t & 3) {
      case 0: lk = lds_read_f32<0>(lin_rd); break;
      case 1: lk = lds_read_f32<kLinBuf>(lin_rd); break;
      case 2: lk = lds_read_f32<2 * kLinBuf>(lin_rd); break;
      default: lk = lds_read_f32<3 * kLinBuf>(lin_rd); break;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lk));
    return lk;
  };
  if (ntiles >= 2) finish(s2, k2, lin_of(ntiles - 2), ntiles - 2, dsa::IntC<-1>{});
  finish(reduce(ap), ksp, lin_of(ntiles - 1), ntiles - 1, dsa::IntC<-1>{});
  // No LDS DMA may still be in flight when the workgroup's LDS is released.
  dsa::wait_vmcnt<0>();
}

// ---- decode form: batch rows of at most kDecMaxTok query tokens ---------------
// The kernel above shares each LDS key tile among the 16 tokens of a workgroup;
// with one token per batch row (decode) 15 of its 16 waves would idle.  Here every
// wave is independent: one (batch row, token, key chunk) per wave, its token's A
// operands and u pieces in registers, its keys loaded straight from global memory
// into B-operand registers, two 64-key tiles in flight, no LDS ring and no
// barriers.  Per 16-key block: the same 4 + 1 fp8 MFMAs and 16 FMAs as above, the
// same operand bytes and the same order of additions (the u MFMA repeats the four
// pieces in every row group, so each lane group receives u.k of the block and
// lane 16 j + c keeps block j's), so both forms write bit-identical logits; then
// the same reduce-scatter, key scale, mask and group maxima.
constexpr int kDecWaves = 4;
constexpr int kDecMaxTok = 4;
constexpr int kDecRing = 2;  // 3 and 4 measured no faster (the stream runs at ~4.5 TB/s either way)
constexpr int kDecMaxChunk = 2048;

template <bool PAGED, bool SCALED>
__global__ __launch_bounds__(kDecWaves * 64) void indexer_decode_kernel(IndexerParams p) {
  __shared__ __align__(16) uint8_t upieces[kDecWaves][kSplits][kDim];
  __shared__ __align__(16) float dwsh[kDecWaves][kHeads];
  __shared__ int32_t drows[PAGED ? kDecWaves : 1][PAGED ? kDecMaxChunk : 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, c = lane & 15;
  const int64_t unit = (int64_t)blockIdx.x * kDecWaves + wave;  // (b, t, kc), kc fastest
  if (unit >= (int64_t)p.B * p.S1 * p.nkc) return;
  const int kc = (int)(unit % p.nkc);
  const int t = (int)((unit / p.nkc) % p.S1);
  const int b = (int)(unit / ((int64_t)p.nkc * p.S1));

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
  if (p.cum_q && t >= aq) return;  // varlen rows past the batch's length do not exist
  const int L = visible_keys(t, aq, ak, p.sparse_mode);
  const int64_t trow = qbase + t;
  if (kc == 0 && p.row_len != nullptr && lane == 0) p.row_len[trow] = L;
  const int k0 = kc * p.chunk;
  const int kend = min(k0 + p.chunk, p.S2);
  const int k1 = min(kend, L);
  if (k0 >= k1) return;

  // operands as in the kernel above: weights (one per lane, shared through
  // LDS), the u sums' query bytes, then the A operands
  const float wl = p.w[trow * kHeads + lane];
  dsa::i32x2 qv[16];
  token_u_load(p.q + trow * kHeads * kDim, lane, qv);
  // q: lane (g, c) holds head 16 mt + c, bytes [32g, 32g+32).
  dsa::i32x8 qa[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const uint8_t* src = p.q + (trow * kHeads + 16 * mt + c) * kDim + 32 * g;
    const dsa::i32x4 lo = *reinterpret_cast<const dsa::i32x4*>(src);
    const dsa::i32x4 hi = *reinterpret_cast<const dsa::i32x4*>(src + 16);
    qa[mt] = dsa::i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  dwsh[wave][lane] = wl;
  wave_lds_sync();
  float wh[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const dsa::f32x4 v = *reinterpret_cast<const dsa::f32x4*>(&dwsh[wave][16 * mt + 4 * g]);
#pragma unroll
    for (int i = 0; i < 4; ++i) wh[mt][i] = 0.5f * v[i];
  }

  // u/2 = sum_h (w_h / 2) q_h and its fp8 pieces, as above.
  float u0, u1;
  const int udim = token_u_sum(qv, &dwsh[wave][0], lane, u0, u1);
  const float umax = wave_max(fmaxf(fabsf(u0), fabsf(u1)));
  int e = -100;
  if (umax > 0.f) {
    int ex;
    (void)frexpf(umax / (float)kE4m3Max, &ex);
    e = clampi(ex, -100, 100);
  }
  {
    float r0 = u0, r1 = u1;
#pragma unroll
    for (int sp = 0; sp < kSplits; ++sp) {
      const float inv = ldexpf(1.f, 4 * sp - e), sig = ldexpf(1.f, e - 4 * sp);
      const int pk = __builtin_amdgcn_cvt_pk_fp8_f32(r0 * inv, r1 * inv, 0, false);
      *reinterpret_cast<uint16_t*>(&upieces[wave][sp][udim]) = (uint16_t)pk;
      r0 = fmaf(-sig, __builtin_amdgcn_cvt_f32_fp8(pk, 0), r0);
      r1 = fmaf(-sig, __builtin_amdgcn_cvt_f32_fp8(pk, 1), r1);
    }
  }
  const uint8_t* kbase = PAGED ? p.k : p.k + kbase_row * kDim;
  const float* sbase = SCALED ? (PAGED ? p.key_scale : p.key_scale + kbase_row) : nullptr;
  if constexpr (PAGED) {
    for (int i = lane; i < k1 - k0; i += 64) {
      const int key = k0 + i;
      const int blk = key / p.block_size;
      const int pg = blk < p.max_blocks ? p.block_table[(int64_t)b * p.max_blocks + blk] : -1;
      const int64_t row = (int64_t)pg * p.block_size + key % p.block_size;
      drows[wave][i] = (pg >= 0 && row < p.pool_rows) ? (int32_t)row : -1;
    }
  }
  // this wave's LDS writes (u pieces, rows) are read back by other lanes of the wave
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // u pieces as A rows: row r holds piece r % 4 (scale 2^(e - 4 (r % 4))), so lane
  // (g, c) of the result holds the four pieces of u.k for key c in every group g
  dsa::i32x8 ua;
  {
    const dsa::i32x4 lo = *reinterpret_cast<const dsa::i32x4*>(&upieces[wave][c & 3][32 * g]);
    const dsa::i32x4 hi = *reinterpret_cast<const dsa::i32x4*>(&upieces[wave][c & 3][32 * g + 16]);
    ua = dsa::i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  const int uscale = clampi(127 + e - 4 * (c & 3), 1, 254);

  auto row_of = [&](int key) -> int {  // physical row of key in [k0, k1), -1 outside the pool
    if constexpr (PAGED) return drows[wave][key - k0];
    else return key;
  };
  const int ntiles = (k1 - k0 + kKeyTile - 1) / kKeyTile;
  dsa::i32x4 kb[kDecRing][4][2];
  float ks[kDecRing];
  auto issue = [&](int tile, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    const int tt = tile < ntiles ? tile : ntiles - 1;  // past the end: reload the last tile (never used)
    const int kt0 = k0 + tt * kKeyTile;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const int row = row_of(min(kt0 + 16 * blk + c, k1 - 1));
      const uint8_t* src = (row >= 0 ? kbase + (int64_t)row * kDim : g_zero_key) + 32 * g;
      kb[sl][blk][0] = *reinterpret_cast<const dsa::i32x4*>(src);
      kb[sl][blk][1] = *reinterpret_cast<const dsa::i32x4*>(src + 16);
    }
    if constexpr (SCALED) {
      const int row = row_of(min(kt0 + lane, k1 - 1));
      ks[sl] = row >= 0 ? sbase[row] : 0.f;
    } else {
      ks[sl] = 1.f;
    }
  };

  float* orow = p.logits + trow * p.ld + k0;
  const __amdgpu_buffer_rsrc_t ost = __builtin_amdgcn_make_buffer_rsrc(orow, (short)0, (kend - k0) * 4, 0x00020000);
  const bool want_gmax = p.gmax != nullptr;
  const __amdgpu_buffer_rsrc_t gst = __builtin_amdgcn_make_buffer_rsrc(
      want_gmax ? p.gmax + trow * p.ld_g + k0 / 16 : p.logits, (short)0,
      want_gmax ? ((kend - k0 + 15) / 16) * 4 : 0, 0x00020000);
  const dsa::f32x4 zero = {0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int tile, auto SLOT) {
    constexpr int sl = decltype(SLOT)::value;
    float ap[4], lin = 0.f;
#pragma unroll
    for (int blk = 0; blk < 4; ++blk) {
      const dsa::i32x8 bf = {kb[sl][blk][0][0], kb[sl][blk][0][1], kb[sl][blk][0][2], kb[sl][blk][0][3],
                             kb[sl][blk][1][0], kb[sl][blk][1][1], kb[sl][blk][1][2], kb[sl][blk][1][3]};
      dsa::f32x4 d[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        d[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[mt], bf, zero, 0, 0, 0, 127, 0, 127);
      const dsa::f32x4 du = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ua, bf, zero, 0, 0, 0, uscale, 0, 127);
      if (g == blk) lin = (du[0] + du[1]) + (du[2] + du[3]);  // u.k of key 16 blk + c
      float acc = 0.f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = fmaf(wh[mt][i], fabsf(d[mt][i]), acc);
      ap[blk] = acc;
    }
    // reduce-scatter over the 4 lane groups: lane l ends with key kt0 + l
    float r02, r13;
    {
      const auto s0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ap[0]), __float_as_uint(ap[2]), false, false);
      r02 = __uint_as_float(s0[0]) + __uint_as_float(s0[1]);
      const auto s1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ap[1]), __float_as_uint(ap[3]), false, false);
      r13 = __uint_as_float(s1[0]) + __uint_as_float(s1[1]);
    }
    const auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(r02), __float_as_uint(r13), false, false);
    float sum = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
    sum += lin;
    const int key = k0 + tile * kKeyTile + lane;
    sum = key < L ? sum * ks[sl] : -__builtin_inff();
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sum), ost, (tile * kKeyTile + lane) * 4, 0, 0);
    if (want_gmax) {
      float m = sum;  // max over each 16-lane row, as in the kernel above
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
      const int goff = c == 0 ? (tile * 4 + g) * 4 : 0x40000000;  // one lane per group; others dropped
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m), gst, goff, 0, 0);
    }
  };

  issue(0, dsa::IntC<0>{});
  for (int it = 0; it < ntiles; it += kDecRing) {
    issue(it + 1, dsa::IntC<1>{});
    compute(it, dsa::IntC<0>{});
    if (it + 1 >= ntiles) break;
    issue(it + 2, dsa::IntC<0>{});
    compute(it + 1, dsa::IntC<1>{});
  }
}

}  // namespace

namespace dsa {

int indexer_fp8_launch(const uint8_t* q, const uint8_t* k, const float* key_scale, const float* w,
                       const int32_t* act_q, const int32_t* act_k, const int32_t* cum_q,
                       const int32_t* cum_k, const int32_t* block_table, int block_size,
                       int max_blocks, int64_t pool_rows, int B, int S1, int S2,
                       int sparse_mode, float* logits, int64_t ld, int32_t* row_len,
                       float* gmax, int64_t ld_g, hipStream_t stream) {
  IndexerParams p;
  p.q = q;
  p.k = k;
  p.key_scale = key_scale;
  p.w = w;
  p.act_q = act_q;
  p.act_k = act_k;
  p.cum_q = cum_q;
  p.cum_k = cum_k;
  p.block_table = block_table;
  p.block_size = block_size;
  p.max_blocks = max_blocks;
  p.pool_rows = pool_rows;
  p.logits = logits;
  p.row_len = row_len;
  p.gmax = gmax;
  p.ld = ld;
  p.ld_g = ld_g;
  p.B = B;
  p.S1 = S1;
  p.S2 = S2;
  p.sparse_mode = sparse_mode;
  p.ntb = (S1 + kTokPerBlock - 1) / kTokPerBlock;
  if (S1 <= kDecMaxTok) {
    // decode form: one wave per (batch row, token, key chunk); chunks shrink to
    // 256 keys until the launch has 2048 waves (8 per CU)
    int dchunk = kDecMaxChunk;
    while (dchunk > 4 * kKeyTile && (int64_t)B * S1 * ((S2 + dchunk - 1) / dchunk) < 2048) dchunk >>= 1;
    p.chunk = dchunk;
    p.nkc = (S2 + dchunk - 1) / dchunk;
    p.ntb = 1;
    p.per_xcd = 0;
    const int64_t units = (int64_t)B * S1 * p.nkc;
    const int64_t nwg = (units + kDecWaves - 1) / kDecWaves;
    if (nwg <= 0) return kOk;
    if (nwg > 0x7fffffff) return set_error(kUnsupported, "indexer: grid too large");
    const bool paged = block_table != nullptr, scaled = key_scale != nullptr;
    const dim3 grid((unsigned)nwg), blk(kDecWaves * 64);
    if (paged && scaled) hipLaunchKernelGGL((indexer_decode_kernel<true, true>), grid, blk, 0, stream, p);
    else if (paged) hipLaunchKernelGGL((indexer_decode_kernel<true, false>), grid, blk, 0, stream, p);
    else if (scaled) hipLaunchKernelGGL((indexer_decode_kernel<false, true>), grid, blk, 0, stream, p);
    else hipLaunchKernelGGL((indexer_decode_kernel<false, false>), grid, blk, 0, stream, p);
    return check_launch("dsa_indexer_logits_fp8(decode)");
  }
  // Shrink the key chunk (a multiple of the LDS tile) until the launch has one
  // workgroup per CU.  A workgroup's fixed cost (A operands, ring fill, the
  // group-maxima flush) is worth amortising over a longer chunk: with 32 query
  // rows x 128K keys, 256 workgroups of 1024 keys take 39 us where 1024 of 256
  // keys took 70.
  // Long chunks also cut the re-reads of the query block (read once per chunk)
  // and the workgroups' fixed costs: at 128K keys, 16384-key chunks take 3.44 ms
  // against 3.61 with 4096; 32768, 65536 and 131072-key chunks 3304, 3271 and
  // 3244 us (one workgroup per token block and CU).
  int chunk = block_table != nullptr ? kMaxChunkPaged : kMaxChunk;
  while (chunk > kKeyTile && (int64_t)B * p.ntb * ((S2 + chunk - 1) / chunk) < 256) chunk >>= 1;
  p.chunk = chunk;
  p.nkc = (S2 + chunk - 1) / chunk;
  const int64_t work = (int64_t)B * p.nkc * p.ntb;
  p.per_xcd = (work + kNumXcd - 1) / kNumXcd;
  const int64_t nblocks = p.per_xcd * kNumXcd;
  if (nblocks <= 0) return kOk;
  if (nblocks > 0x7fffffff) return set_error(kUnsupported, "indexer: grid too large");
  const dim3 grid((unsigned)nblocks), block(kThreads);
  if (block_table != nullptr) {
    if (p.gmax != nullptr) hipLaunchKernelGGL((indexer_fp8_kernel<true, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((indexer_fp8_kernel<true, false>), grid, block, 0, stream, p);
  } else {
    if (p.gmax != nullptr) hipLaunchKernelGGL((indexer_fp8_kernel<false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((indexer_fp8_kernel<false, false>), grid, block, 0, stream, p);
  }
  return check_launch("dsa_indexer_logits_fp8");
}

}  // namespace dsa

namespace {
int indexer_logits_impl(const void* q, const void* k, const float* key_scale, const float* weights,
                        const int32_t* act_q, const int32_t* act_k, int64_t B, int64_t S1, int64_t S2,
                        int32_t N1, int32_t D, int32_t sparse_mode, float* logits, int64_t ld,
                        int32_t* row_len, float* gmax, int64_t ld_g, void* stream) {
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
                            key_scale, weights, act_q, act_k, nullptr, nullptr, nullptr, 0, 0, 0,
                            (int)B, (int)S1, (int)S2, sparse_mode, logits, ld, row_len, gmax, ld_g,
                            (hipStream_t)stream);
}
}  // namespace

extern "C" int dsa_indexer_logits_fp8(const void* q, const void* k, const float* key_scale,
                                      const float* weights, const int32_t* act_q,
                                      const int32_t* act_k, int64_t B, int64_t S1, int64_t S2,
                                      int32_t N1, int32_t D, int32_t sparse_mode, float* logits,
                                      int64_t ld, int32_t* row_len, void* stream) {
  return indexer_logits_impl(q, k, key_scale, weights, act_q, act_k, B, S1, S2, N1, D, sparse_mode, logits,
                             ld, row_len, nullptr, 0, stream);
}

extern "C" int dsa_indexer_logits_fp8_group_max(const void* q, const void* k, const float* key_scale,
                                                const float* weights, const int32_t* act_q,
                                                const int32_t* act_k, int64_t B, int64_t S1, int64_t S2,
                                                int32_t N1, int32_t D, int32_t sparse_mode, float* logits,
                                                int64_t ld, int32_t* row_len, float* group_max, int64_t ld_g,
                                                void* stream) {
  using namespace dsa;
  if (group_max == nullptr || ld_g < (S2 + 15) / 16)
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8_group_max: group_max with ld_g >= ceil(S2 / 16) needed");
  return indexer_logits_impl(q, k, key_scale, weights, act_q, act_k, B, S1, S2, N1, D, sparse_mode, logits,
                             ld, row_len, group_max, ld_g, stream);
}

namespace dsa {
int topk_launch(const float* x, int64_t rows, int64_t cols, int64_t ld, const int32_t* row_len,
                const float* gmax, int64_t ld_g, int32_t K, int32_t pad_invalid, int32_t* out_idx,
                float* out_val, hipStream_t stream);
}

using dsa::IndexerWorkspace;
using dsa::indexer_workspace;
using dsa::use_group_max;

extern "C" size_t dsa_lightning_indexer_workspace_bytes(int64_t B, int64_t S1, int64_t S2) {
  return indexer_workspace((B < 0 ? 0 : B) * (S1 < 0 ? 0 : S1), S2).bytes;
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
  const IndexerWorkspace wl = indexer_workspace(B * S1, S2);
  float* logits = static_cast<float*>(workspace);
  int32_t* row_len = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + wl.rowlen_off);
  float* gmax = use_group_max(S2, sparse_count) ? reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.gmax_off)
                                                : nullptr;
  hipStream_t st = (hipStream_t)stream;
  if (S2 == 0)  // no keys: every row is all -1, the top-k kernel handles cols == 0
    return topk_launch(logits, B * S1, 0, 0, nullptr, nullptr, 0, sparse_count, 1, indices, values, st);
  int rc = indexer_logits_impl(q, k, key_scale, weights, act_q, act_k, B, S1, S2, N1, D, sparse_mode, logits,
                               S2, row_len, gmax, wl.ld_g, stream);
  if (rc != kOk) return rc;
  return topk_launch(logits, B * S1, S2, S2, row_len, gmax, wl.ld_g, sparse_count, 1, indices, values, st);
}

namespace {
int indexer_logits_varlen_impl(const void* q, const void* k, const float* key_scale, const float* weights,
                               const int32_t* seq_q, int32_t seq_q_cumulative, const int32_t* seq_k,
                               int32_t seq_k_cumulative, const int32_t* block_table, int32_t block_size,
                               int32_t max_blocks, int64_t pool_rows, int64_t B, int64_t S1, int64_t S2,
                               int32_t N1, int32_t D, int32_t sparse_mode, float* logits, int64_t ld,
                               int32_t* row_len, float* gmax, int64_t ld_g, void* stream) {
  using namespace dsa;
  if (N1 != kHeads || D != kDim)
    return set_error(kUnsupported,
                     "dsa_indexer_logits_fp8_varlen: only 64 index heads x 128 dims are built (got %d x %d)", N1, D);
  if (B < 0 || S1 < 0 || S2 < 0 || ld < S2 || S1 > 0x7fffffff || S2 > 0x7fffffff || B > 0x7fffffff)
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8_varlen: bad sizes");
  if (sparse_mode != 0 && sparse_mode != 3)
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8_varlen: sparse_mode must be 0 or 3, got %d",
                     sparse_mode);
  if ((seq_q_cumulative && seq_q == nullptr) || (seq_k_cumulative && seq_k == nullptr))
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8_varlen: cumulative lengths need a length array");
  if (block_table != nullptr) {
    if (block_size <= 0 || max_blocks <= 0 || pool_rows < 0 || pool_rows > 0x7fffffff)
      return set_error(kInvalidArgument,
                       "dsa_indexer_logits_fp8_varlen: paged keys need block_size > 0, max_blocks > 0 and "
                       "pool_rows in [0, 2^31)");
    if (seq_k_cumulative)
      return set_error(kInvalidArgument,
                       "dsa_indexer_logits_fp8_varlen: paged keys take per-batch key lengths, not prefix sums");
  }
  if (B == 0 || S1 == 0) return kOk;
  if (q == nullptr || k == nullptr || weights == nullptr || logits == nullptr)
    return set_error(kInvalidArgument, "dsa_indexer_logits_fp8_varlen: null pointer");
  const int32_t* act_q = seq_q_cumulative ? nullptr : seq_q;
  const int32_t* cum_q = seq_q_cumulative ? seq_q : nullptr;
  const int32_t* act_k = seq_k_cumulative ? nullptr : seq_k;
  const int32_t* cum_k = seq_k_cumulative ? seq_k : nullptr;
  return indexer_fp8_launch(static_cast<const uint8_t*>(q), static_cast<const uint8_t*>(k), key_scale,
                            weights, act_q, act_k, cum_q, cum_k, block_table, block_size, max_blocks,
                            pool_rows, (int)B, (int)S1, (int)S2, sparse_mode, logits, ld, row_len, gmax,
                            ld_g, (hipStream_t)stream);
}
}  // namespace

extern "C" int dsa_indexer_logits_fp8_varlen(const void* q, const void* k, const float* key_scale,
                                             const float* weights, const int32_t* seq_q,
                                             int32_t seq_q_cumulative, const int32_t* seq_k,
                                             int32_t seq_k_cumulative, const int32_t* block_table,
                                             int32_t block_size, int32_t max_blocks, int64_t pool_rows,
                                             int64_t B, int64_t S1, int64_t S2, int32_t N1, int32_t D,
                                             int32_t sparse_mode, float* logits, int64_t ld,
                                             int32_t* row_len, void* stream) {
  return indexer_logits_varlen_impl(q, k, key_scale, weights, seq_q, seq_q_cumulative, seq_k, seq_k_cumulative,
                                    block_table, block_size, max_blocks, pool_rows, B, S1, S2, N1, D,
                                    sparse_mode, logits, ld, row_len, nullptr, 0, stream);
}

extern "C" size_t dsa_lightning_indexer_varlen_workspace_bytes(int64_t q_rows, int64_t S2) {
  return indexer_workspace(q_rows, S2).bytes;
}

extern "C" int dsa_lightning_indexer_fp8_varlen(const void* q, const void* k, const float* key_scale,
                                                const float* weights, const int32_t* seq_q,
                                                int32_t seq_q_cumulative, const int32_t* seq_k,
                                                int32_t seq_k_cumulative, const int32_t* block_table,
                                                int32_t block_size, int32_t max_blocks, int64_t pool_rows,
                                                int64_t B, int64_t S1, int64_t S2, int64_t q_rows,
                                                int32_t N1, int32_t D, int32_t sparse_count,
                                                int32_t sparse_mode, int32_t* indices, float* values,
                                                void* workspace, size_t workspace_bytes, void* stream) {
  using namespace dsa;
  if (sparse_count < 1 || sparse_count > 8192)
    return set_error(kInvalidArgument,
                     "dsa_lightning_indexer_fp8_varlen: sparse_count must be in [1, 8192], got %d", sparse_count);
  if (B < 0 || S1 < 0 || S2 < 0 || q_rows < 0)
    return set_error(kInvalidArgument, "dsa_lightning_indexer_fp8_varlen: bad sizes");
  if (!seq_q_cumulative && q_rows != B * S1)
    return set_error(kInvalidArgument, "dsa_lightning_indexer_fp8_varlen: padded query rows need q_rows = B * S1");
  if (q_rows == 0) return kOk;
  const size_t need = dsa_lightning_indexer_varlen_workspace_bytes(q_rows, S2);
  if (workspace == nullptr || workspace_bytes < need)
    return set_error(kWorkspaceTooSmall,
                     "dsa_lightning_indexer_fp8_varlen: workspace of %zu bytes needed, %zu given", need,
                     workspace_bytes);
  if (indices == nullptr) return set_error(kInvalidArgument, "dsa_lightning_indexer_fp8_varlen: null indices");
  const IndexerWorkspace wl = indexer_workspace(q_rows, S2);
  float* logits = static_cast<float*>(workspace);
  int32_t* row_len = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + wl.rowlen_off);
  float* gmax = use_group_max(S2, sparse_count) ? reinterpret_cast<float*>(static_cast<char*>(workspace) + wl.gmax_off)
                                                : nullptr;
  hipStream_t st = (hipStream_t)stream;
  if (S2 == 0 || B == 0 || S1 == 0)  // no keys (or no rows to score): every row is all -1
    return topk_launch(logits, q_rows, 0, 0, nullptr, nullptr, 0, sparse_count, 1, indices, values, st);
  int rc = indexer_logits_varlen_impl(q, k, key_scale, weights, seq_q, seq_q_cumulative, seq_k, seq_k_cumulative,
                                      block_table, block_size, max_blocks, pool_rows, B, S1, S2, N1, D,
                                      sparse_mode, logits, S2, row_len, gmax, wl.ld_g, stream);
  if (rc != kOk) return rc;
  return topk_launch(logits, q_rows, S2, S2, row_len, gmax, wl.ld_g, sparse_count, 1, indices, values, st);
}
