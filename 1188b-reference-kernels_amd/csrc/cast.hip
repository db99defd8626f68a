// Element casts of the router backward: bf16 -> fp32 (exact) and fp32 -> bf16
// (round to nearest even).
//
// Math: kernel_cases/case11_router_bwd_cast_bf16_to_fp32.py:43-44
// (x.to(torch.float32)) and kernel_cases/case25_ref_unary_cast_fp32_to_bf16.py:
// 56-66 (round_bf16_rne: add 0x7FFF + the kept LSB to the fp32 bits, keep the
// high half).  NaN becomes the quiet NaN 0x7FC0 (torch's scalar conversion;
// the case's bit formula, written for finite inputs, would wrap a NaN's bits).
// The timed op is inp.to(torch.bfloat16) (case25...py:107).
//
// HBM-bound streaming, grid-stride over the array: fp32 -> bf16 converts 8
// elements per thread and iteration (32-byte fp32 in, non-temporal loads;
// 16-byte bf16 out), bf16 -> fp32 4 (8-byte bf16 in, plain loads; 16-byte fp32
// out); a scalar tail covers the last elements and unaligned pointers.
#include <algorithm>

#include "moe_common.h"

namespace moe {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void f32_to_bf16_vec(const float *src, int64_t nvec, uint16_t *dst) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < nvec; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src) + 2 * i);
    const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src) + 2 * i + 1);
    u32x4 o;
    o.x = pack_bf16x2(__uint_as_float(a.x), __uint_as_float(a.y));
    o.y = pack_bf16x2(__uint_as_float(a.z), __uint_as_float(a.w));
    o.z = pack_bf16x2(__uint_as_float(b.x), __uint_as_float(b.y));
    o.w = pack_bf16x2(__uint_as_float(b.z), __uint_as_float(b.w));
    *(reinterpret_cast<u32x4 *>(dst) + i) = o;
  }
}

// 4 elements per thread: an 8-byte load (plain: the output is twice the input, and non-temporal loads
// measured 11% slower here) and one 16-byte store, both contiguous across the wavefront.
__global__ __launch_bounds__(kThreads) void bf16_to_f32_vec(const uint16_t *src, int64_t nvec, float *dst) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < nvec; i += stride) {
    const u32x2 v = *(reinterpret_cast<const u32x2 *>(src) + i);
    const u32x4 a = {v.x << 16, v.x & 0xffff0000u, v.y << 16, v.y & 0xffff0000u};
    *(reinterpret_cast<u32x4 *>(dst) + i) = a;
  }
}

__global__ __launch_bounds__(kThreads) void f32_to_bf16_scalar(const float *src, int64_t begin, int64_t n, uint16_t *dst) {
  const int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) dst[i] = static_cast<uint16_t>(f32_to_bf16_rne(src[i]));
}

__global__ __launch_bounds__(kThreads) void bf16_to_f32_scalar(const uint16_t *src, int64_t begin, int64_t n, float *dst) {
  const int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) dst[i] = bf16_to_f32(src[i]);
}

int64_t vec_grid(int64_t nvec) {
  // One vector per thread up to 2^20 workgroups (measured faster than fewer
  // workgroups looping); grid-stride beyond.
  return std::max<int64_t>(1, std::min<int64_t>(ceil_div(nvec, kThreads), int64_t(1) << 20));
}

}  // namespace
}  // namespace moe

extern "C" {

int moe_cast_f32_to_bf16(const float *src, int64_t n, moe_bf16_t *dst, void *stream) {
  using namespace moe;
  if (n < 0) return fail(MOE_ERR_SHAPE, "moe_cast_f32_to_bf16: negative n=%lld", (long long)n);
  if (n == 0) return MOE_OK;
  if (src == nullptr || dst == nullptr) return fail(MOE_ERR_INVALID_ARG, "moe_cast_f32_to_bf16: null src or dst");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = is_aligned(src, 32) && is_aligned(dst, 16);
  const int64_t nvec = vec ? n / 8 : 0;
  if (nvec > 0) f32_to_bf16_vec<<<dim3(vec_grid(nvec)), dim3(kThreads), 0, s>>>(src, nvec, dst);
  const int64_t rest = n - nvec * 8;
  if (rest > 0) {
    const int64_t g = ceil_div(rest, kThreads);
    if (g > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "moe_cast_f32_to_bf16: n=%lld too large for the scalar path", (long long)n);
    f32_to_bf16_scalar<<<dim3(g), dim3(kThreads), 0, s>>>(src, nvec * 8, n, dst);
  }
  return check_launch("moe_cast_f32_to_bf16");
}

int moe_cast_bf16_to_f32(const moe_bf16_t *src, int64_t n, float *dst, void *stream) {
  using namespace moe;
  if (n < 0) return fail(MOE_ERR_SHAPE, "moe_cast_bf16_to_f32: negative n=%lld", (long long)n);
  if (n == 0) return MOE_OK;
  if (src == nullptr || dst == nullptr) return fail(MOE_ERR_INVALID_ARG, "moe_cast_bf16_to_f32: null src or dst");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = is_aligned(src, 8) && is_aligned(dst, 16);
  const int64_t nvec = vec ? n / 4 : 0;
  if (nvec > 0) bf16_to_f32_vec<<<dim3(vec_grid(nvec)), dim3(kThreads), 0, s>>>(src, nvec, dst);
  const int64_t rest = n - nvec * 4;
  if (rest > 0) {
    const int64_t g = ceil_div(rest, kThreads);
    if (g > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "moe_cast_bf16_to_f32: n=%lld too large for the scalar path", (long long)n);
    bf16_to_f32_scalar<<<dim3(g), dim3(kThreads), 0, s>>>(src, nvec * 4, n, dst);
  }
  return check_launch("moe_cast_bf16_to_f32");
}

}  // extern "C"
