// Row quantisation on gfx950: the producer of the indexer's fp8 operands and the
// int8 activation quantiser of the DeepSeek-V4 examples.
//
// Every row of x (bf16, or fp16 through the _f16 entry points) is scaled by its
// own absolute maximum:
//   fp8  : s = max(absmax / 448, FLT_MIN),            y = e4m3fn(x / s)
//   int8 : s = max(absmax, 1e-4) / 127,               y = rne(clamp(x / s, +-127))
//   int8 with power-of-two scales: s = 2^ceil(log2(max(absmax, 1e-4) / 127)).
// x / s is an IEEE division and the conversions round to nearest even, so the
// outputs equal the torch goldens bit for bit
// (examples/deepseek_v4/act_quant.py:110-149 for int8; the fp8 rule is the key
// quantisation the indexer's key_scale describes).
//
// Layout of the work: LPR lanes own one row (LPR = the power of two covering
// cols / 8, between 8 and 64), so a wave handles 64 / LPR rows and each lane
// moves 16 bytes of bf16 per step.  Rows of one step (cols <= 512) are taken
// four per lane group with the loads issued together; for longer rows up to 8
// steps per lane stay in registers for the second (convert) pass, and rows
// longer than that are read again (from L2).  The kernel is
// HBM bound: 2 bytes read and 1 byte written per element plus 4 bytes per row.
//
// An optional row map sends input row r to output row dst_rows[r] (-1 or out of
// range: dropped), which is how new keys are appended to a paged fp8 key cache
// (pool row = page * block_size + offset) in the same pass that quantises them.
// An optional per-row factor multiplies the written scale: the indexer's query
// scale is folded into its head weights that way, since
// w * ReLU(s * q8 . k) = (w * s) * ReLU(q8 . k) for s > 0.
#include <hip/hip_runtime.h>
#include <float.h>

#include "dsa_common.h"

namespace {

enum Mode : int { kFp8 = 0, kInt8 = 1, kInt8Pow2 = 2 };

constexpr int kThreads = 256;
constexpr int kCache = 8;  // 16-byte steps per lane kept in registers

struct QuantArgs {
  const uint16_t* x;        // bf16 or fp16 [rows, ld_x]
  int64_t rows, cols, ld_x;
  const int64_t* dst_rows;  // [rows] or null (row r -> r)
  int64_t dst_capacity;     // rows of y / scale
  uint8_t* y;               // fp8 e4m3fn or int8 [dst_capacity, ld_y]
  int64_t ld_y;
  float* scale;             // [dst_capacity]
  const float* fold;        // [rows] or null: scale[dst] = fold[r] * s
};

// The two 16-bit inputs of a dword as fp32 (exact for both types).
template <bool F16>
__device__ __forceinline__ float in_lo(uint32_t w) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  else return __uint_as_float(w << 16);
}
template <bool F16>
__device__ __forceinline__ float in_hi(uint32_t w) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  else return __uint_as_float(w & 0xffff0000u);
}

template <bool F16>
__device__ __forceinline__ float absmax8(const dsa::i32x4& v) {
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = (uint32_t)v[i];
    m = fmaxf(m, fmaxf(fabsf(in_lo<F16>(w)), fabsf(in_hi<F16>(w))));
  }
  return m;
}

// 2^ceil(log2(v)) for a positive normal v, from its bits (exponent, plus one when
// any mantissa bit is set).
__device__ __forceinline__ float pow2_ceil(float v) {
  const uint32_t b = __float_as_uint(v);
  const int e = (int)((b >> 23) & 0xffu) - 127 + ((b & 0x7fffffu) != 0u ? 1 : 0);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

template <int MODE>
__device__ __forceinline__ uint32_t quant4(float a, float b, float c, float d, float s) {
  a = __fdiv_rn(a, s);
  b = __fdiv_rn(b, s);
  c = __fdiv_rn(c, s);
  d = __fdiv_rn(d, s);
  if constexpr (MODE == kFp8) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
  } else {
    auto q = [](float v) -> uint32_t {
      return (uint32_t)(int)rintf(fminf(fmaxf(v, -127.0f), 127.0f)) & 0xffu;
    };
    return q(a) | (q(b) << 8) | (q(c) << 16) | (q(d) << 24);
  }
}

template <int MODE>
__device__ __forceinline__ float row_scale(float amax) {
  if constexpr (MODE == kFp8) {
    return fmaxf(amax / 448.0f, FLT_MIN);
  } else {
    const float s = fmaxf(amax, 1e-4f) / 127.0f;
    if constexpr (MODE == kInt8Pow2) return pow2_ceil(s);
    return s;
  }
}

template <int MODE, bool F16>
__device__ __forceinline__ void store8(uint8_t* dst, const dsa::i32x4& v, float s) {
  const uint32_t w0 = (uint32_t)v[0], w1 = (uint32_t)v[1], w2 = (uint32_t)v[2], w3 = (uint32_t)v[3];
  const uint32_t lo = quant4<MODE>(in_lo<F16>(w0), in_hi<F16>(w0), in_lo<F16>(w1), in_hi<F16>(w1), s);
  const uint32_t hi = quant4<MODE>(in_lo<F16>(w2), in_hi<F16>(w2), in_lo<F16>(w3), in_hi<F16>(w3), s);
  *reinterpret_cast<dsa::i32x2*>(dst) = dsa::i32x2{(int)lo, (int)hi};
}

// Rows of at most 8 * LPR columns (one 16-byte load per lane and row): each lane
// group takes R rows, 64 / LPR rows apart (so every load instruction of a wave
// reads 64 / LPR consecutive rows), and issues all R loads before reducing any,
// to keep enough bytes in flight per CU.
template <int LPR, int MODE, int R, bool F16>
__global__ __launch_bounds__(kThreads) void quant_short_rows_kernel(QuantArgs a) {
  constexpr int kRowsPerWave = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int sl = lane % LPR;
  const int64_t base =
      ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * kRowsPerWave * R + lane / LPR;
  const int64_t col = (int64_t)sl * 8;
  const bool col_ok = col < a.cols;
  dsa::i32x4 v[R];
  int64_t drow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = base + (int64_t)r * kRowsPerWave;
    v[r] = dsa::i32x4{0, 0, 0, 0};
    if (row < a.rows && col_ok) v[r] = *reinterpret_cast<const dsa::i32x4*>(a.x + row * a.ld_x + col);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = base + (int64_t)r * kRowsPerWave;
    drow[r] = -1;
    if (row < a.rows) {
      drow[r] = a.dst_rows ? a.dst_rows[row] : row;
      if (drow[r] >= a.dst_capacity) drow[r] = -1;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float amax = absmax8<F16>(v[r]);
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float s = row_scale<MODE>(amax);
    if (drow[r] >= 0) {
      if (col_ok) store8<MODE, F16>(a.y + drow[r] * a.ld_y + col, v[r], s);
      if (sl == 0) {
        const int64_t row = base + (int64_t)r * kRowsPerWave;
        a.scale[drow[r]] = a.fold ? a.fold[row] * s : s;
      }
    }
  }
}

template <int LPR, int MODE, bool F16>
__global__ __launch_bounds__(kThreads) void quant_rows_kernel(QuantArgs a) {
  constexpr int kRowsPerWave = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int sl = lane % LPR;
  const int64_t row = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * kRowsPerWave + lane / LPR;
  const bool live = row < a.rows;
  int64_t drow = -1;
  if (live) {
    drow = a.dst_rows ? a.dst_rows[row] : row;
    if (drow >= a.dst_capacity) drow = -1;
  }
  const int steps = (int)((a.cols + 8 * LPR - 1) / (8 * LPR));
  const dsa::i32x4* xr = reinterpret_cast<const dsa::i32x4*>(a.x + (live ? row : 0) * a.ld_x);

  // pass 1: absolute maximum of the row (the first kCache steps stay in registers)
  dsa::i32x4 cache[kCache];
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < kCache; ++c) {
    const int64_t col = ((int64_t)c * LPR + sl) * 8;
    cache[c] = dsa::i32x4{0, 0, 0, 0};
    if (c < steps && live && col < a.cols) {
      cache[c] = xr[col / 8];
      amax = fmaxf(amax, absmax8<F16>(cache[c]));
    }
  }
  for (int c = kCache; c < steps; ++c) {
    const int64_t col = ((int64_t)c * LPR + sl) * 8;
    if (live && col < a.cols) amax = fmaxf(amax, absmax8<F16>(xr[col / 8]));
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));

  const float s = row_scale<MODE>(amax);
  if (drow < 0) return;  // nothing below is shared across lanes

  // pass 2: scale, round, store 8 bytes per lane and step
  uint8_t* yr = a.y + drow * a.ld_y;
  auto emit = [&](int c, const dsa::i32x4& v) { store8<MODE, F16>(yr + ((int64_t)c * LPR + sl) * 8, v, s); };
#pragma unroll
  for (int c = 0; c < kCache; ++c) {
    const int64_t col = ((int64_t)c * LPR + sl) * 8;
    if (c < steps && col < a.cols) emit(c, cache[c]);
  }
  for (int c = kCache; c < steps; ++c) {
    const int64_t col = ((int64_t)c * LPR + sl) * 8;
    if (col < a.cols) emit(c, xr[col / 8]);
  }
  if (sl == 0) a.scale[drow] = a.fold ? a.fold[row] * s : s;
}

template <int MODE, int R, bool F16>
int launch_short(const QuantArgs& a, int lpr, hipStream_t st, const char* what) {
  const int64_t rows_per_block = (kThreads / 64) * (64 / lpr) * R;
  const int64_t grid = (a.rows + rows_per_block - 1) / rows_per_block;
  if (grid > 0x7fffffff) return dsa::set_error(dsa::kInvalidArgument, "%s: too many rows", what);
  switch (lpr) {
    case 8: quant_short_rows_kernel<8, MODE, R, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
    case 16: quant_short_rows_kernel<16, MODE, R, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
    case 32: quant_short_rows_kernel<32, MODE, R, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
    default: quant_short_rows_kernel<64, MODE, R, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
  }
  return dsa::check_launch(what);
}

template <int MODE, bool F16>
int launch_mode(const QuantArgs& a, hipStream_t st, const char* what) {
  int lpr = 8;
  while (lpr < 64 && (int64_t)lpr * 8 < a.cols) lpr *= 2;
  if (a.cols <= 8 * lpr) {
    // one load per lane and row; R rows per lane group: 2 up to 2^25 elements
    // (128K-key cache 15.4 -> 12.9 us, 4096-token query 25.0 -> 21.6 us against 4),
    // 4 above (1M rows: 73.9 us against 78.8)
    if (a.rows * a.cols <= ((int64_t)1 << 25)) return launch_short<MODE, 2, F16>(a, lpr, st, what);
    return launch_short<MODE, 4, F16>(a, lpr, st, what);
  }
  const int64_t rows_per_block = (kThreads / 64) * (64 / lpr);
  const int64_t grid = (a.rows + rows_per_block - 1) / rows_per_block;
  if (grid > 0x7fffffff) return dsa::set_error(dsa::kInvalidArgument, "%s: too many rows", what);
  switch (lpr) {
    case 8: quant_rows_kernel<8, MODE, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
    case 16: quant_rows_kernel<16, MODE, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
    case 32: quant_rows_kernel<32, MODE, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
    default: quant_rows_kernel<64, MODE, F16><<<(unsigned)grid, kThreads, 0, st>>>(a); break;
  }
  return dsa::check_launch(what);
}

int quant_launch(int mode, const QuantArgs& a, void* stream, const char* what, bool f16 = false) {
  if (a.rows < 0 || a.cols <= 0 || a.cols % 8 != 0 || a.ld_x < a.cols || a.ld_x % 8 != 0 ||
      a.ld_y < a.cols || a.ld_y % 8 != 0)
    return dsa::set_error(dsa::kInvalidArgument,
                          "%s: cols must be a positive multiple of 8 and the leading dimensions multiples of 8 "
                          "no smaller than cols (rows %lld, cols %lld, ld_x %lld, ld_y %lld)",
                          what, (long long)a.rows, (long long)a.cols, (long long)a.ld_x, (long long)a.ld_y);
  if (a.rows == 0) return dsa::kOk;
  if (a.x == nullptr || a.y == nullptr || a.scale == nullptr)
    return dsa::set_error(dsa::kInvalidArgument, "%s: null pointer", what);
  if ((reinterpret_cast<uintptr_t>(a.x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(a.y) & 7u) != 0)
    return dsa::set_error(dsa::kInvalidArgument, "%s: x must be 16-byte and y 8-byte aligned", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (f16) return launch_mode<kFp8, true>(a, st, what);  // fp16 inputs: the fp8 producers only
  switch (mode) {
    case kFp8: return launch_mode<kFp8, false>(a, st, what);
    case kInt8: return launch_mode<kInt8, false>(a, st, what);
    default: return launch_mode<kInt8Pow2, false>(a, st, what);
  }
}

}  // namespace

extern "C" int dsa_quant_fp8_rows(const void* x, int64_t rows, int64_t cols, void* y, float* scale,
                                  void* stream) {
  QuantArgs a{static_cast<const uint16_t*>(x), rows, cols, cols, nullptr, rows,
              static_cast<uint8_t*>(y), cols, scale, nullptr};
  return quant_launch(kFp8, a, stream, "dsa_quant_fp8_rows");
}

extern "C" int dsa_act_quant_int8(const void* x, int64_t M, int64_t N, int32_t round_scale, int8_t* y,
                                  float* scale, void* stream) {
  QuantArgs a{static_cast<const uint16_t*>(x), M, N, N, nullptr, M, reinterpret_cast<uint8_t*>(y), N,
              scale, nullptr};
  return quant_launch(round_scale ? kInt8Pow2 : kInt8, a, stream, "dsa_act_quant_int8");
}

extern "C" int dsa_indexer_k_append_fp8(const void* k, int64_t T, int32_t D, const int64_t* slots,
                                        int64_t pool_rows, void* pool, float* pool_scale, void* stream) {
  if (T > 0 && slots == nullptr)
    return dsa::set_error(dsa::kInvalidArgument, "dsa_indexer_k_append_fp8: null slot map");
  if (pool_rows < 0)
    return dsa::set_error(dsa::kInvalidArgument, "dsa_indexer_k_append_fp8: negative pool size");
  QuantArgs a{static_cast<const uint16_t*>(k), T, D, D, slots, pool_rows, static_cast<uint8_t*>(pool), D,
              pool_scale, nullptr};
  return quant_launch(kFp8, a, stream, "dsa_indexer_k_append_fp8");
}

extern "C" int dsa_indexer_q_quant_fp8(const void* q, const float* weights, int64_t T, int32_t N1, int32_t D,
                                       void* q8, float* weights_out, void* stream) {
  if (N1 <= 0 || T < 0)
    return dsa::set_error(dsa::kInvalidArgument, "dsa_indexer_q_quant_fp8: bad sizes (T %lld, N1 %d)",
                          (long long)T, N1);
  if (T > 0 && weights == nullptr)
    return dsa::set_error(dsa::kInvalidArgument, "dsa_indexer_q_quant_fp8: null weights");
  QuantArgs a{static_cast<const uint16_t*>(q), T * N1, D, D, nullptr, T * N1, static_cast<uint8_t*>(q8), D,
              weights_out, weights};
  return quant_launch(kFp8, a, stream, "dsa_indexer_q_quant_fp8");
}

extern "C" int dsa_quant_fp8_rows_f16(const void* x, int64_t rows, int64_t cols, void* y, float* scale,
                                      void* stream) {
  QuantArgs a{static_cast<const uint16_t*>(x), rows, cols, cols, nullptr, rows,
              static_cast<uint8_t*>(y), cols, scale, nullptr};
  return quant_launch(kFp8, a, stream, "dsa_quant_fp8_rows_f16", true);
}

extern "C" int dsa_indexer_q_quant_fp8_f16(const void* q, const float* weights, int64_t T, int32_t N1, int32_t D,
                                           void* q8, float* weights_out, void* stream) {
  if (N1 <= 0 || T < 0)
    return dsa::set_error(dsa::kInvalidArgument, "dsa_indexer_q_quant_fp8_f16: bad sizes (T %lld, N1 %d)",
                          (long long)T, N1);
  if (T > 0 && weights == nullptr)
    return dsa::set_error(dsa::kInvalidArgument, "dsa_indexer_q_quant_fp8_f16: null weights");
  QuantArgs a{static_cast<const uint16_t*>(q), T * N1, D, D, nullptr, T * N1, static_cast<uint8_t*>(q8), D,
              weights_out, weights};
  return quant_launch(kFp8, a, stream, "dsa_indexer_q_quant_fp8_f16", true);
}
