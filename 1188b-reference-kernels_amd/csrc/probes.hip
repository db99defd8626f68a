// Measurement probes (not part of the dispatch path): the ceilings the kernels'
// roofline fractions are read against, measured on the same GPU.
//
//   moe_probe_mfma: every wavefront issues `iters` rounds of 16 independent
//     v_mfma_f32_16x16x32_bf16 on operands held in registers (no memory traffic
//     inside the loop): the matrix-core issue ceiling at whatever clock the
//     board holds under it.  Two wavefronts per SIMD hide the issue gaps.
//     The operands are pseudo-random bf16 values fixed per lane (the inputs do
//     not change from one MFMA to the next, so this is an upper bound on what
//     streaming real data reaches).
//   moe_probe_stream: 16-byte vectors over n_vec elements, each workgroup a
//     contiguous segment (four vectors per thread and step, loads issued before
//     use), with mode 0 = copy (read src, write dst), 1 = read only (a
//     per-thread XOR of everything read, one 16-byte store per thread at the
//     end), 2 = write only; + 4: non-temporal loads and stores.
#include "../../include/moe_probes.h"
#include "moe_common.h"

namespace moe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void probe_mfma_kernel(int64_t iters, float *sink) {
  const uint32_t lane = threadIdx.x + 256u * blockIdx.x;
  bf16x8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // xorshift-style hash: random signs, exponents near 1, random mantissas
    uint32_t h = lane * 0x9E3779B9u + static_cast<uint32_t>(i) * 0x85EBCA6Bu;
    h ^= h >> 15;
    h *= 0x2C1B3C6Du;
    h ^= h >> 12;
    a[i] = static_cast<__bf16>(__uint_as_float(0x3F000000u | (h & 0x807FFFFFu)));
    b[i] = static_cast<__bf16>(__uint_as_float(0x3F000000u | ((h >> 7) & 0x807FFFFFu)));
  }
  f32x4_t acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  sink[static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x] = s;
}

// Block b streams the contiguous segment [b n / blocks, (b + 1) n / blocks) of the
// vectors, four per thread and step (all loads of a step issued before their use);
// kNt: non-temporal loads and stores.
template <int kMode, bool kNt>
__global__ __launch_bounds__(256) void probe_stream_kernel(const u32x4 *src, u32x4 *dst, int64_t n) {
  constexpr int kU = 4;
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * per;
  const int64_t hi = lo + per < n ? lo + per : n;
  u32x4 x = {0u, 0u, 0u, 0u};
  for (int64_t i = lo + threadIdx.x; i < hi; i += kU * 256) {
    u32x4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t j = i + u * 256;
      if constexpr (kMode != 2) {
        v[u] = j < hi ? (kNt ? __builtin_nontemporal_load(src + j) : src[j]) : u32x4{0u, 0u, 0u, 0u};
      } else {
        v[u] = u32x4{static_cast<uint32_t>(j), 1u, 2u, 3u};
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t j = i + u * 256;
      if constexpr (kMode == 1) {
        x ^= v[u];
      } else if (j < hi) {
        if constexpr (kNt) __builtin_nontemporal_store(v[u], dst + j);
        else dst[j] = v[u];
      }
    }
  }
  if constexpr (kMode == 1) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t < n) dst[t] = x;
  }
}

}  // namespace
}  // namespace moe

extern "C" {

int moe_probe_mfma(int64_t waves, int64_t iters, float *sink, void *stream) {
  using namespace moe;
  if (waves <= 0 || iters <= 0 || waves % 4 != 0) {
    return fail(MOE_ERR_SHAPE, "moe_probe_mfma: waves (%lld) must be a positive multiple of 4, iters (%lld) > 0",
                (long long)waves, (long long)iters);
  }
  if (sink == nullptr) return fail(MOE_ERR_INVALID_ARG, "moe_probe_mfma: null sink");
  probe_mfma_kernel<<<dim3(static_cast<uint32_t>(waves / 4)), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      iters, sink);
  return check_launch("moe_probe_mfma");
}

int moe_probe_stream(int mode, const void *src, void *dst, int64_t n_vec, int64_t blocks, void *stream) {
  using namespace moe;
  if ((mode & 3) == 3 || mode < 0 || mode > 6) {
    return fail(MOE_ERR_INVALID_ARG, "moe_probe_stream: mode %d not 0, 1, 2 (+ 4)", mode);
  }
  if (n_vec <= 0 || blocks <= 0) return fail(MOE_ERR_SHAPE, "moe_probe_stream: n_vec and blocks must be > 0");
  if (dst == nullptr || ((mode & 3) != 2 && src == nullptr)) {
    return fail(MOE_ERR_INVALID_ARG, "moe_probe_stream: null buffer");
  }
  if (!is_aligned(dst, 16) || !is_aligned(src, 16)) return fail(MOE_ERR_ALIGN, "moe_probe_stream: 16-byte alignment");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4 *in = static_cast<const u32x4 *>(src);
  u32x4 *out = static_cast<u32x4 *>(dst);
  const dim3 grid(static_cast<uint32_t>(blocks)), block(256);
  switch (mode) {
    case 0: probe_stream_kernel<0, false><<<grid, block, 0, s>>>(in, out, n_vec); break;
    case 1: probe_stream_kernel<1, false><<<grid, block, 0, s>>>(in, out, n_vec); break;
    case 2: probe_stream_kernel<2, false><<<grid, block, 0, s>>>(in, out, n_vec); break;
    case 4: probe_stream_kernel<0, true><<<grid, block, 0, s>>>(in, out, n_vec); break;
    case 5: probe_stream_kernel<1, true><<<grid, block, 0, s>>>(in, out, n_vec); break;
    default: probe_stream_kernel<2, true><<<grid, block, 0, s>>>(in, out, n_vec); break;
  }
  return check_launch("moe_probe_stream");
}

}  // extern "C"
