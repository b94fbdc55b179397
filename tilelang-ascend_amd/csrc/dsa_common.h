// Shared helpers for the DSA (DeepSeek Sparse Attention) gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace dsa {

// Records a printf-style message as this thread's last error (read back through
// dsa_last_error()).  Always returns the error code it is given.
int set_error(int code, const char* fmt, ...);

// Checks the launch that was just made; on failure records `what` plus the HIP
// error string and returns a non-zero code.
int check_launch(const char* what);

enum Code : int {
  kOk = 0,
  kInvalidArgument = 1,
  kWorkspaceTooSmall = 2,
  kUnsupported = 3,
  kHipError = 4,
};

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

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

__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  uint32_t a = __float_as_uint(x);
  if ((a & 0x7f800000u) == 0x7f800000u && (a & 0x7fffffu)) return 0x7fc0u;  // NaN
  a += 0x7fffu + ((a >> 16) & 1u);
  return (uint16_t)(a >> 16);
}

}  // namespace dsa
