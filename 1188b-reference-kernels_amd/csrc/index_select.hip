// Row gather along dim 0: out[i, :] = src[index[i], :].
//
// Math: kernel_cases/case06_cp_seq_chunk_index_select.py:38-40 (torch.index_select
// on dim 0 of a bf16 tensor, int32 index); it is also the gather inside the
// permute / unpermute references (case17...:67, case15...:63).
//
// A row is `row_elems` bf16 values.  Each workgroup copies one 64 KiB slice of
// one output row: 256 threads x 16 vectors x 16 bytes, loads issued before
// stores, non-temporal on both sides (every byte is touched exactly once).
// Rows whose length or base is not 16-byte aligned take a 2-byte path.
#include "moe_common.h"

namespace moe {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 16;
constexpr int64_t kSliceVec = static_cast<int64_t>(kThreads) * kUnroll;  // 16-byte vectors per block

template <bool kI64>
__global__ __launch_bounds__(kThreads) void index_select_vec_kernel(const u32x4 *src, int64_t src_rows,
                                                                    int64_t row_vec, const void *index,
                                                                    int64_t blocks_per_row, u32x4 *out) {
  const int64_t row = blockIdx.x / blocks_per_row;
  const int64_t part = blockIdx.x % blocks_per_row;
  const int64_t s = load_idx<kI64>(index, row);
  const bool ok = s >= 0 && s < src_rows;
  const int64_t v0 = part * kSliceVec + threadIdx.x;
  u32x4 buf[kUnroll];
#pragma unroll
  for (int j = 0; j < kUnroll; ++j) {
    const int64_t v = v0 + static_cast<int64_t>(j) * kThreads;
    buf[j] = u32x4{0u, 0u, 0u, 0u};
    if (ok && v < row_vec) buf[j] = __builtin_nontemporal_load(src + s * row_vec + v);
  }
#pragma unroll
  for (int j = 0; j < kUnroll; ++j) {
    const int64_t v = v0 + static_cast<int64_t>(j) * kThreads;
    if (v < row_vec) __builtin_nontemporal_store(buf[j], out + row * row_vec + v);
  }
}

template <bool kI64>
__global__ __launch_bounds__(kThreads) void index_select_scalar_kernel(const uint16_t *src, int64_t src_rows,
                                                                       int64_t row_elems, const void *index,
                                                                       int64_t blocks_per_row, uint16_t *out) {
  const int64_t row = blockIdx.x / blocks_per_row;
  const int64_t part = blockIdx.x % blocks_per_row;
  const int64_t s = load_idx<kI64>(index, row);
  const bool ok = s >= 0 && s < src_rows;
  const int64_t e0 = part * kSliceVec + threadIdx.x;
  for (int j = 0; j < kUnroll; ++j) {
    const int64_t e = e0 + static_cast<int64_t>(j) * kThreads;
    if (e < row_elems) out[row * row_elems + e] = ok ? src[s * row_elems + e] : static_cast<uint16_t>(0);
  }
}

}  // namespace
}  // namespace moe

extern "C" {

int moe_index_select(const moe_bf16_t *src, int64_t src_rows, int64_t row_elems, const void *index,
                     int idx_dtype, int64_t n_index, moe_bf16_t *out, void *stream) {
  using namespace moe;
  if (src_rows < 0 || row_elems < 0 || n_index < 0) {
    return fail(MOE_ERR_SHAPE, "moe_index_select: negative size (src_rows=%lld row_elems=%lld n_index=%lld)",
                (long long)src_rows, (long long)row_elems, (long long)n_index);
  }
  if (idx_dtype != MOE_IDX_I32 && idx_dtype != MOE_IDX_I64) {
    return fail(MOE_ERR_INVALID_ARG, "moe_index_select: idx_dtype %d is not MOE_IDX_I32/I64", idx_dtype);
  }
  if (n_index * row_elems == 0) return MOE_OK;
  if (index == nullptr || out == nullptr || (src == nullptr && src_rows * row_elems > 0)) {
    return fail(MOE_ERR_INVALID_ARG, "moe_index_select: null src, index or out");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = (row_elems % 8 == 0) && is_aligned(src, 16) && is_aligned(out, 16);
  const int64_t units = vec ? row_elems / 8 : row_elems;
  const int64_t bpr = ceil_div(units, kSliceVec);
  const int64_t grid = n_index * bpr;
  if (grid > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "moe_index_select: %lld blocks exceed the grid limit", (long long)grid);
  const bool i64 = idx_dtype == MOE_IDX_I64;
  if (vec) {
    const u32x4 *sv = reinterpret_cast<const u32x4 *>(src);
    u32x4 *ov = reinterpret_cast<u32x4 *>(out);
    if (i64) index_select_vec_kernel<true><<<dim3(grid), dim3(kThreads), 0, s>>>(sv, src_rows, units, index, bpr, ov);
    else index_select_vec_kernel<false><<<dim3(grid), dim3(kThreads), 0, s>>>(sv, src_rows, units, index, bpr, ov);
  } else {
    if (i64) index_select_scalar_kernel<true><<<dim3(grid), dim3(kThreads), 0, s>>>(src, src_rows, units, index, bpr, out);
    else index_select_scalar_kernel<false><<<dim3(grid), dim3(kThreads), 0, s>>>(src, src_rows, units, index, bpr, out);
  }
  return check_launch("moe_index_select");
}

}  // extern "C"
