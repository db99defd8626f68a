// Shared device and host helpers for the gfx950 MoE dispatch kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/moe_dispatch.h"

namespace moe {

// ---------------------------------------------------------------- host side

// Records `msg` as the calling thread's last error and returns `status`.
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks hipGetLastError() after a launch; maps a failure to MOE_ERR_LAUNCH.
int check_launch(const char *what);

inline bool is_aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- device side

constexpr int kWave = 64;  // CDNA wavefront width

// 16-byte vector of the memory kernels (a clang vector, so the non-temporal
// builtins accept it).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// fp32 -> bf16, round to nearest even on the dropped 16 mantissa bits; NaN
// becomes the canonical quiet NaN 0x7FC0 (what torch's .to(bfloat16) stores).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Packs two fp32 values into one dword of two RNE bf16 (lo = first).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_rne(lo) | (f32_to_bf16_rne(hi) << 16);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Number of set bits of `mask` below the calling lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
}

// Reads a 64-bit value from `lane` (lane must be wave-uniform).
__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
  uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), lane);
  uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32), lane);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// A wave-uniform 64-bit value as scalar registers.  Each half goes through
// uint32_t: the builtin returns int, and OR-ing that int into a 64-bit value
// would sign-extend a low half with bit 31 set across the high half.
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), lane));
}

// Loads map entry `i` of an int32 or int64 map as int64.
template <bool kI64>
__device__ __forceinline__ int64_t load_idx(const void *map, int64_t i) {
  if constexpr (kI64) {
    return static_cast<const int64_t *>(map)[i];
  } else {
    return static_cast<int64_t>(static_cast<const int32_t *>(map)[i]);
  }
}

}  // namespace moe
