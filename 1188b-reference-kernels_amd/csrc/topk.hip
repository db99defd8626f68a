// Router top-k (+ routing mask and merge probs), one wavefront per row; the
// per-row routine and its math citation are in topk_device.h.
#include "topk_device.h"

namespace moe {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

template <int kEPL>
__global__ __launch_bounds__(kThreads) void topk_kernel(const float *logits, int64_t T, int E, int k,
                                                        float *values, int64_t *indices,
                                                        uint8_t *routing_map, float *probs) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (t >= T) return;
  const float *row = logits + t * E;
  topk_row<kEPL>([&](int e) { return row[e]; }, t, E, k, values, indices, routing_map, probs);
}

}  // namespace
}  // namespace moe

extern "C" {

int moe_topk(const float *logits, int64_t T, int64_t E, int64_t k, float *values, int64_t *indices,
             uint8_t *routing_map, float *probs, void *stream) {
  using namespace moe;
  if (T < 0 || E < 0) return fail(MOE_ERR_SHAPE, "moe_topk: negative size (T=%lld E=%lld)", (long long)T, (long long)E);
  if (k < 1 || k > E) return fail(MOE_ERR_SHAPE, "moe_topk: k=%lld out of range for E=%lld", (long long)k, (long long)E);
  if (k > 64) return fail(MOE_ERR_CAPACITY, "moe_topk: k=%lld exceeds the 64 supported", (long long)k);
  if (E > 1024) return fail(MOE_ERR_CAPACITY, "moe_topk: E=%lld exceeds the 1024 supported", (long long)E);
  if (T == 0) return MOE_OK;
  if (logits == nullptr || values == nullptr || indices == nullptr) {
    return fail(MOE_ERR_INVALID_ARG, "moe_topk: null logits, values or indices");
  }
  const int64_t grid = ceil_div(T, kWavesPerBlock);
  if (grid > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "moe_topk: T=%lld too large", (long long)T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int e = static_cast<int>(E), kk = static_cast<int>(k);
  if (E <= 64) topk_kernel<1><<<dim3(grid), dim3(kThreads), 0, s>>>(logits, T, e, kk, values, indices, routing_map, probs);
  else if (E <= 128) topk_kernel<2><<<dim3(grid), dim3(kThreads), 0, s>>>(logits, T, e, kk, values, indices, routing_map, probs);
  else if (E <= 256) topk_kernel<4><<<dim3(grid), dim3(kThreads), 0, s>>>(logits, T, e, kk, values, indices, routing_map, probs);
  else if (E <= 512) topk_kernel<8><<<dim3(grid), dim3(kThreads), 0, s>>>(logits, T, e, kk, values, indices, routing_map, probs);
  else topk_kernel<16><<<dim3(grid), dim3(kThreads), 0, s>>>(logits, T, e, kk, values, indices, routing_map, probs);
  return check_launch("moe_topk");
}

}  // extern "C"
