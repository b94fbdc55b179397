// Row-wise top-k over fp32 scores for gfx950: exact radix select + LDS sort.
//
// Contract (the lightning indexer golden, examples/deepseek_v4/lightning_indexer.py:316-325):
//   out[r, :] = argsort(-x[r, :L_r], stable=True)[:K]  (descending value, ties to
//   the lower index); entries whose value is <= -1e30 become -1 when pad_invalid;
//   positions past min(K, L_r) are -1 (value -inf).
//
// Method.  Every element gets a 64-bit composite key
//   C = (ordered(x) << 32) | ~index
// where ordered() maps fp32 onto uint32 monotonically (-0.0 folded onto +0.0 so
// they tie, NaN placed below -inf as torch.sort places it last).  All C are
// distinct and "C larger" == "earlier in the stable descending order", so the
// top-K set is exactly {C >= C_K} for the K-th largest composite C_K.  C_K is
// found digit by digit (12-bit digits) with LDS histograms; each pass narrows
// the group that holds C_K.  Once the group is small it is copied to LDS and the
// remaining digits are resolved there, so a row is read from HBM once (rows up
// to 32K are held in registers) or twice (longer rows, streamed).  The K chosen
// composites are then bitonic-sorted in LDS (descending) and written out.
#include "dsa_common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kHistBits = 12;
constexpr int kBins = 1 << kHistBits;
constexpr int kCandCap = 4096;

__device__ __forceinline__ uint32_t ordered_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) == 0u) u = 0u;                                       // -0.0 -> +0.0
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0u) return 0u;  // NaN: last
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t idx) {
  return ((uint64_t)key << 32) | (uint64_t)(~idx);
}

struct Shared {
  uint32_t hist[kBins];
  uint32_t wsum[kWaves];
  uint32_t nsel;
  uint32_t ncand;
  uint32_t res_bucket;
  uint32_t res_above;
  uint32_t res_count;
};

// Exclusive prefix sum over the 1024 threads of the block.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wsum) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wid] = x;
  __syncthreads();
  uint32_t pre = 0;
  for (int w = 0; w < wid; ++w) pre += wsum[w];
  __syncthreads();
  return pre + x - v;
}

// Find the bucket b* (scanning from the top bin down) that holds the need-th
// largest element of the histogram.  Publishes b*, the count strictly above it
// and its own count through the shared struct.
__device__ __forceinline__ void find_bucket(Shared& sh, uint32_t need) {
  const int t = threadIdx.x;
  const int top = kBins - 1 - 4 * t;  // this thread owns bins top, top-1, top-2, top-3
  uint32_t h0 = sh.hist[top], h1 = sh.hist[top - 1], h2 = sh.hist[top - 2], h3 = sh.hist[top - 3];
  uint32_t local = h0 + h1 + h2 + h3;
  uint32_t before = block_exclusive_scan(local, sh.wsum);
  if (before < need && need <= before + local) {
    uint32_t acc = before;
    uint32_t hs[4] = {h0, h1, h2, h3};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (acc + hs[i] >= need) {
        sh.res_bucket = (uint32_t)(top - i);
        sh.res_above = acc;
        sh.res_count = hs[i];
        break;
      }
      acc += hs[i];
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void clear_hist(Shared& sh) {
  for (int i = threadIdx.x; i < kBins; i += kThreads) sh.hist[i] = 0u;
}

// Bitonic sort of buf[0..n) into descending order (n padded to a power of two
// with zeros, the smallest composite).
__device__ void sort_desc(uint64_t* buf, int n, int p2) {
  for (int i = n + threadIdx.x; i < p2; i += kThreads) buf[i] = 0ull;
  __syncthreads();
  for (int size = 2; size <= p2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < (p2 >> 1); t += kThreads) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        uint64_t a = buf[i], b = buf[j];
        if ((a < b) == desc) {
          buf[i] = b;
          buf[j] = a;
        }
      }
      __syncthreads();
    }
  }
}

// ITEMS > 0: the row (length <= ITEMS * 1024) lives in registers, element
// e = j * 1024 + tid for j < ITEMS.  ITEMS == 0: the row is re-read from global
// memory on every pass.
template <int ITEMS>
__global__ __launch_bounds__(kThreads) void topk_rows_kernel(
    const float* __restrict__ x, int64_t ld, int32_t cols, const int32_t* __restrict__ row_len,
    int32_t K, int32_t p2, int32_t pad_invalid, int32_t* __restrict__ out_idx,
    float* __restrict__ out_val) {
  extern __shared__ __align__(16) unsigned char smem[];
  Shared& sh = *reinterpret_cast<Shared*>(smem);
  uint64_t* sel = reinterpret_cast<uint64_t*>(smem + ((sizeof(Shared) + 15) & ~size_t(15)));
  uint64_t* cand = sel + p2;

  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ld;
  int L = cols;
  if (row_len != nullptr) {
    int r = row_len[row];
    L = r < 0 ? 0 : (r < cols ? r : cols);
  }
  if (tid == 0) {
    sh.nsel = 0u;
    sh.ncand = 0u;
  }

  uint32_t keys[ITEMS > 0 ? ITEMS : 1];
  if constexpr (ITEMS > 0) {
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
      const int e = j * kThreads + tid;
      keys[j] = e < L ? ordered_key(__builtin_nontemporal_load(xr + e)) : 0u;
    }
  }

  int nsel_final;
  if (L <= K) {
    // Everything is selected.
    __syncthreads();
    if constexpr (ITEMS > 0) {
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        const int e = j * kThreads + tid;
        if (e < L) sel[e] = composite(keys[j], (uint32_t)e);
      }
    } else {
      for (int e = tid; e < L; e += kThreads) sel[e] = composite(ordered_key(xr[e]), (uint32_t)e);
    }
    nsel_final = L;
    __syncthreads();
  } else {
    // ---- pass 1: top 12 bits of the value key ----
    clear_hist(sh);
    __syncthreads();
    if constexpr (ITEMS > 0) {
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        const int e = j * kThreads + tid;
        if (e < L) atomicAdd(&sh.hist[keys[j] >> 20], 1u);
      }
    } else {
      for (int e = tid; e < L; e += kThreads) atomicAdd(&sh.hist[ordered_key(xr[e]) >> 20], 1u);
    }
    __syncthreads();
    uint32_t need = (uint32_t)K;
    find_bucket(sh, need);
    uint64_t P = sh.res_bucket;
    int s = 64 - kHistBits;
    need -= sh.res_above;
    uint32_t cnt = sh.res_count;
    bool done = (cnt == need);
    __syncthreads();

    // ---- further passes over the row while the group is too large for LDS ----
    while (!done && s > 0 && cnt > (uint32_t)kCandCap) {
      const int w = s < kHistBits ? s : kHistBits;
      const int s2 = s - w;
      const uint64_t dmask = (1ull << w) - 1ull;
      clear_hist(sh);
      __syncthreads();
      if constexpr (ITEMS > 0) {
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
          const int e = j * kThreads + tid;
          if (e < L) {
            const uint64_t C = composite(keys[j], (uint32_t)e);
            if ((C >> s) == P) atomicAdd(&sh.hist[(uint32_t)((C >> s2) & dmask)], 1u);
          }
        }
      } else {
        for (int e = tid; e < L; e += kThreads) {
          const uint64_t C = composite(ordered_key(xr[e]), (uint32_t)e);
          if ((C >> s) == P) atomicAdd(&sh.hist[(uint32_t)((C >> s2) & dmask)], 1u);
        }
      }
      __syncthreads();
      find_bucket(sh, need);
      P = (P << w) | sh.res_bucket;
      s = s2;
      need -= sh.res_above;
      cnt = sh.res_count;
      done = (cnt == need);
      __syncthreads();
    }

    // ---- collect: strictly-above elements are selected; the group goes to LDS ----
    auto collect = [&](uint64_t C) {
      const uint64_t hi = C >> s;
      if (hi > P || (done && hi == P)) {
        sel[atomicAdd(&sh.nsel, 1u)] = C;
      } else if (hi == P) {
        cand[atomicAdd(&sh.ncand, 1u)] = C;
      }
    };
    if constexpr (ITEMS > 0) {
#pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        const int e = j * kThreads + tid;
        if (e < L) collect(composite(keys[j], (uint32_t)e));
      }
    } else {
      for (int e = tid; e < L; e += kThreads) collect(composite(ordered_key(xr[e]), (uint32_t)e));
    }
    __syncthreads();
    const int ncand = (int)sh.ncand;

    // ---- resolve the remaining digits inside the LDS candidate group ----
    // (composites are distinct, so the group shrinks to the single C_K by s == 0)
    while (!done && s > 0) {
      const int w = s < kHistBits ? s : kHistBits;
      const int s2 = s - w;
      const uint64_t dmask = (1ull << w) - 1ull;
      clear_hist(sh);
      __syncthreads();
      for (int i = tid; i < ncand; i += kThreads) {
        const uint64_t C = cand[i];
        if ((C >> s) == P) atomicAdd(&sh.hist[(uint32_t)((C >> s2) & dmask)], 1u);
      }
      __syncthreads();
      find_bucket(sh, need);
      P = (P << w) | sh.res_bucket;
      s = s2;
      need -= sh.res_above;
      cnt = sh.res_count;
      done = (cnt == need);
      __syncthreads();
    }
    for (int i = tid; i < ncand; i += kThreads) {
      const uint64_t C = cand[i];
      if ((C >> s) >= P) sel[atomicAdd(&sh.nsel, 1u)] = C;
    }
    __syncthreads();
    nsel_final = K;
  }

  sort_desc(sel, nsel_final, p2);

  int32_t* orow = out_idx + row * (int64_t)K;
  float* vrow = out_val ? out_val + row * (int64_t)K : nullptr;
  for (int p = tid; p < K; p += kThreads) {
    int32_t idx = -1;
    float val = -__builtin_inff();
    if (p < nsel_final) {
      const uint64_t C = sel[p];
      val = key_value((uint32_t)(C >> 32));
      idx = (int32_t)(~(uint32_t)C);
      if (pad_invalid && val <= -1e30f) idx = -1;
    }
    orow[p] = idx;
    if (vrow) vrow[p] = val;
  }
}

int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

}  // namespace

namespace dsa {

size_t topk_smem_bytes(int K) {
  const int p2 = next_pow2(K < 1 ? 1 : K);
  return ((sizeof(Shared) + 15) & ~size_t(15)) + sizeof(uint64_t) * (size_t)(p2 + kCandCap);
}

int topk_launch(const float* x, int64_t rows, int64_t cols, int64_t ld, const int32_t* row_len,
                int32_t K, int32_t pad_invalid, int32_t* out_idx, float* out_val,
                hipStream_t stream) {
  if (rows == 0 || K == 0) return kOk;
  const int p2 = next_pow2(K);
  const size_t smem = topk_smem_bytes(K);
  const dim3 grid((unsigned)rows), block(kThreads);
  const int c = (int)cols;
#define DSA_TOPK_LAUNCH(ITEMS)                                                                 \
  do {                                                                                         \
    auto fn = topk_rows_kernel<ITEMS>;                                                         \
    if (smem > 64 * 1024)                                                                      \
      (void)hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize,   \
                                (int)smem);                                                    \
    hipLaunchKernelGGL(fn, grid, block, smem, stream, x, ld, c, row_len, K, p2, pad_invalid,   \
                       out_idx, out_val);                                                      \
  } while (0)
  if (cols <= 4 * kThreads) {
    DSA_TOPK_LAUNCH(4);
  } else if (cols <= 8 * kThreads) {
    DSA_TOPK_LAUNCH(8);
  } else if (cols <= 16 * kThreads) {
    DSA_TOPK_LAUNCH(16);
  } else if (cols <= 32 * kThreads) {
    DSA_TOPK_LAUNCH(32);
  } else {
    DSA_TOPK_LAUNCH(0);
  }
#undef DSA_TOPK_LAUNCH
  return check_launch("dsa_topk_f32");
}

}  // namespace dsa

extern "C" int dsa_topk_f32(const float* scores, int64_t rows, int64_t cols, int64_t ld,
                            const int32_t* row_len, int32_t k, int32_t pad_invalid,
                            int32_t* out_idx, float* out_val, void* stream) {
  using namespace dsa;
  if (rows < 0 || cols < 0 || ld < cols || k < 0)
    return set_error(kInvalidArgument, "dsa_topk_f32: bad sizes rows=%lld cols=%lld ld=%lld k=%d",
                     (long long)rows, (long long)cols, (long long)ld, k);
  if (k > 8192)
    return set_error(kUnsupported, "dsa_topk_f32: k=%d exceeds the supported maximum 8192", k);
  if (cols >= (int64_t)1 << 31)
    return set_error(kUnsupported, "dsa_topk_f32: cols=%lld exceeds 2^31-1", (long long)cols);
  if (rows > 0 && k > 0 && (scores == nullptr || out_idx == nullptr))
    return set_error(kInvalidArgument, "dsa_topk_f32: null scores or out_idx");
  return topk_launch(scores, rows, cols, ld, row_len, k, pad_invalid, out_idx, out_val,
                     (hipStream_t)stream);
}
