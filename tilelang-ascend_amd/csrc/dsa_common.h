// Shared helpers for the DSA (DeepSeek Sparse Attention) gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <atomic>

namespace dsa {

// Records a printf-style message as this thread's last error (read back through
// dsa_last_error()).  Always returns the error code it is given.
int set_error(int code, const char* fmt, ...);

// Checks the launch that was just made; on failure records `what` plus the HIP
// error string and returns a non-zero code.
int check_launch(const char* what);

// Devices whose per-kernel LDS reservations are cached (more are served uncached).
constexpr int kMaxDevices = 64;

// Raises kernel `fn`'s dynamic LDS limit to at least `bytes` on the current
// device.  `per_device` (one slot per device, zero-initialised, owned by the
// kernel instance) remembers the largest reservation made, so the attribute call
// runs once per kernel, device and size increase rather than on every launch.
int reserve_lds(const void* fn, size_t bytes, std::atomic<int>* per_device, const char* what);

enum Code : int {
  kOk = 0,
  kInvalidArgument = 1,
  kWorkspaceTooSmall = 2,
  kUnsupported = 3,
  kHipError = 4,
};

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Workspace of the full lightning indexer (both the fp8 and the 16-bit entry
// points): fp32 logits [rows, S2] | int32 row_len [rows] | fp32 maxima of 16-key
// groups [rows, ceil(S2 / 16)], each part 256-byte aligned.
struct IndexerWorkspace {
  size_t rowlen_off, gmax_off, bytes;
  int64_t ld_g;
};

inline IndexerWorkspace indexer_workspace(int64_t rows_in, int64_t S2_in) {
  const size_t rows = (size_t)(rows_in < 0 ? 0 : rows_in);
  const size_t S2 = (size_t)(S2_in < 0 ? 0 : S2_in);
  auto up = [](size_t x) { return (x + 255) & ~size_t(255); };
  IndexerWorkspace w;
  w.ld_g = (int64_t)((S2 + 15) / 16);
  w.rowlen_off = up(rows * S2 * sizeof(float));
  w.gmax_off = w.rowlen_off + up(rows * sizeof(int32_t));
  w.bytes = w.gmax_off + rows * (size_t)w.ld_g * sizeof(float);
  return w;
}

// The top-k reads the group maxima (and only the groups that can hold a top-K
// element) when a row has at least 2 K groups; below that it streams the row.
inline bool use_group_max(int64_t S2, int32_t K) { return (S2 + 15) / 16 >= 2 * (int64_t)K; }

// The MI355X has 8 XCDs; consecutive workgroup ids are dealt round-robin to
// them.  Kernels that want related workgroups to share one XCD's L2 regroup
// their linear id with this constant.
constexpr int kNumXcd = 8;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 (round to nearest even) for two values, low half = lo
// (one v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;

// fp32 -> fp16 (round to nearest even) for two values, low half = lo
// (one v_cvt_pk_f16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const f16x2_t v = __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

// Two fp32 values packed as the 16-bit element type of the MLA kernels (F16:
// IEEE half, else bfloat16).
template <bool F16>
__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
  if constexpr (F16) return pack_f16x2(lo, hi);
  else return pack_bf16x2(lo, hi);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  uint32_t a = __float_as_uint(x);
  if ((a & 0x7f800000u) == 0x7f800000u && (a & 0x7fffffu)) return 0x7fc0u;  // NaN
  a += 0x7fffu + ((a >> 16) & 1u);
  return (uint16_t)(a >> 16);
}

#define DSA_LDS __attribute__((address_space(3)))

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Transposing LDS read (ds_read_b64_tr_b16) issued as inline asm.  The builtin
// form makes the compiler drain every in-flight global_load_lds (vmcnt(0))
// before it, since it cannot tell the two apart; here the caller orders the
// read after the step's barrier and waits for its result with lds_wait<N>.
template <int OFF>
__device__ __forceinline__ dsa::i32x2 lds_read_tr16(uint32_t addr) {
  dsa::i32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
// 16-byte LDS read issued as inline asm, for the same reason: it pins how far
// ahead of their MFMAs the reads run.
template <int OFF>
__device__ __forceinline__ dsa::i32x4 lds_read_b128(uint32_t addr) {
  dsa::i32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}
template <int N>
__device__ __forceinline__ void lds_wait1(dsa::i32x4& a) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(N));
}
// s_waitcnt lgkmcnt(N); the registers passed in are tied to the wait so that no
// use of them is scheduled before it.
template <int N>
__device__ __forceinline__ void lds_wait(dsa::i32x2& a, dsa::i32x2& b) {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}

template <int V>
struct IntC {
  static constexpr int value = V;
};
// Compile-time loop: f(IntC<B>{}), ..., f(IntC<E - 1>{}).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(IntC<B>{});
    static_for<B + 1, E>(f);
  }
}

// Inclusive prefix sum over the 64 lanes of a wave, VALU only: DPP row shifts
// by 1, 2, 4, 8 scan each row of 16 lanes, then row broadcasts of lanes 15 and
// 31 carry the row totals into the rows above (lanes of masked rows add 0).
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t x) {
  int v = (int)x;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return (uint32_t)v;
}

// Cross-lane reductions over the lane groups l ^ 16 and l ^ 32 (gfx950 permlane swaps).
__device__ __forceinline__ float xor16_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace dsa
