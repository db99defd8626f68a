// Unpermute (combine) with optional probability-weighted merge, and the
// permute backward (combine of the gradient + permuted-prob gradient gather).
//
// Math:
//   unpermute  kernel_cases/case15_moe_unpermute_mask_fwd.py:58-64 and the
//              int32 variant kernel_cases/case24_ref_moe_unpermute_mask_kernel_false.py:45-68
//                out[t] = bf16( sum_{e ascending, map(t,e) >= 0} float(pin[map(t,e)]) )
//              merge form: the summand is probs[t,e] * float(pin[map(t,e)]).
//   permute bwd kernel_cases/case18_moe_permute_bwd_unpermute_mask.py:68-78 and
//              kernel_cases/case32_ref_moe_unpermute_mask_kernel.py:46-76
//                dact[t] as above (unweighted); dprobs[t,e] = dpp[map(t,e)] or 0.
//
// Bit-exactness: the reference adds with index_add_ in nonzero() order of the
// [E, T] mask, i.e. ascending expert per token, starting from 0.0f.  This
// kernel keeps that order, multiplies then adds (contraction disabled below),
// and rounds once to bf16 with round-to-nearest-even.
//
// Layout of the work: one workgroup of 4 wavefronts per token, each summing
// every 4th 1 KiB slice of the row (256 x 4 measured best of 256-1024 threads
// x 1-4 wavefronts per row at c5).  The token's map entries are
// held in VGPRs (64 experts per register, up to kChunks registers) with their
// ballots; each lane owns 16-byte vectors of the hidden row.  Sources are
// consumed in batches of 8: the wave issues the 8 row loads back to back, then
// accumulates them in ascending expert order.
#include "moe_common.h"

#pragma clang fp contract(off)

namespace moe {
namespace {

#ifndef MOE_UNPERMUTE_THREADS
#define MOE_UNPERMUTE_THREADS 256
#endif
#ifndef MOE_UNPERMUTE_SPLIT
#define MOE_UNPERMUTE_SPLIT 4
#endif
constexpr int kThreads = MOE_UNPERMUTE_THREADS;
constexpr int kSplit = MOE_UNPERMUTE_SPLIT;  // wavefronts sharing one token row
constexpr int kWavesPerBlock = kThreads / kWave / kSplit;  // tokens per workgroup
constexpr int kBatch = 8;

enum Mode { kPlain = 0, kMerge = 1, kBwd = 2 };

struct UnpermuteArgs {
  const uint16_t *pin;
  int64_t R, H, E, T;
  const void *map;
  const float *probs;  // kMerge: merge probs [T, E]; kBwd: dpp [R]
  uint16_t *out;
  float *dprobs;   // kBwd: [T, E]
  float *out_acc;  // optional fp32 accumulator [T, H] (the reference functions return it)
};

template <bool kI64, bool kExpertMajor>
__device__ __forceinline__ int64_t map_at(const UnpermuteArgs &a, int64_t t, int64_t e) {
  return load_idx<kI64>(a.map, kExpertMajor ? e * a.T + t : t * a.E + e);
}

__device__ __forceinline__ void accumulate8(float (&acc)[8], const u32x4 &v, float w, bool weighted) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float lo = bf16_to_f32(d[q] & 0xffffu);
    const float hi = bf16_to_f32(d[q] >> 16);
    if (weighted) {
      acc[2 * q] = acc[2 * q] + w * lo;
      acc[2 * q + 1] = acc[2 * q + 1] + w * hi;
    } else {
      acc[2 * q] = acc[2 * q] + lo;
      acc[2 * q + 1] = acc[2 * q + 1] + hi;
    }
  }
}

template <bool kI64, bool kExpertMajor, int kMode, int kChunks, bool kVec>
__global__ __launch_bounds__(kThreads) void unpermute_kernel(UnpermuteArgs a) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int part = wave % kSplit;  // which share of the row this wave sums
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave / kSplit;
  if (t >= a.T) return;

  // Map entries of this token, 64 experts per chunk, ascending expert order.
  int64_t src[kChunks];
  float w[kChunks];
  uint64_t valid[kChunks];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int64_t e = static_cast<int64_t>(c) * kWave + lane;
    int64_t s = -1;
    if (e < a.E) s = map_at<kI64, kExpertMajor>(a, t, e);
    const bool ok = s >= 0 && s < a.R;
    src[c] = s;
    valid[c] = __ballot(ok);
    w[c] = 0.0f;
    if constexpr (kMode == kMerge) {
      if (ok) w[c] = a.probs[t * a.E + e];
    }
    if constexpr (kMode == kBwd) {
      if (e < a.E && part == 0) a.dprobs[t * a.E + e] = ok ? a.probs[s] : 0.0f;
    }
  }

  if constexpr (kVec) {
    const int64_t nvec = a.H / 8;
    for (int64_t v = part * kWave + lane; v < nvec; v += kWave * kSplit) {
      float acc[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        uint64_t m = valid[c];
        while (m) {
          int64_t rows[kBatch];
          float ws[kBatch];
          int n = 0;
#pragma unroll
          for (int b = 0; b < kBatch; ++b) {
            rows[b] = 0;
            ws[b] = 0.0f;
            if (m) {
              const int bit = __builtin_ctzll(m);
              m &= m - 1;
              rows[b] = readlane64(src[c], bit);
              if constexpr (kMode == kMerge) ws[b] = readlane_f32(w[c], bit);
              n = b + 1;
            }
          }
          u32x4 buf[kBatch];
#pragma unroll
          for (int b = 0; b < kBatch; ++b) {
            if (b < n) buf[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(a.pin + rows[b] * a.H) + v);
          }
#pragma unroll
          for (int b = 0; b < kBatch; ++b) {
            if (b < n) accumulate8(acc, buf[b], ws[b], kMode == kMerge);
          }
        }
      }
      u32x4 o;
      o.x = pack_bf16x2(acc[0], acc[1]);
      o.y = pack_bf16x2(acc[2], acc[3]);
      o.z = pack_bf16x2(acc[4], acc[5]);
      o.w = pack_bf16x2(acc[6], acc[7]);
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4 *>(a.out + t * a.H) + v);
      if (a.out_acc != nullptr) {
        u32x4 lo = {__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]), __float_as_uint(acc[3])};
        u32x4 hi = {__float_as_uint(acc[4]), __float_as_uint(acc[5]), __float_as_uint(acc[6]), __float_as_uint(acc[7])};
        u32x4 *dst = reinterpret_cast<u32x4 *>(a.out_acc + t * a.H) + 2 * v;
        __builtin_nontemporal_store(lo, dst);
        __builtin_nontemporal_store(hi, dst + 1);
      }
    }
  } else {
    for (int64_t i = part * kWave + lane; i < a.H; i += kWave * kSplit) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < kChunks; ++c) {
        uint64_t m = valid[c];
        while (m) {
          const int bit = __builtin_ctzll(m);
          m &= m - 1;
          const int64_t row = readlane64(src[c], bit);
          const float x = bf16_to_f32(a.pin[row * a.H + i]);
          if constexpr (kMode == kMerge) {
            acc = acc + readlane_f32(w[c], bit) * x;
          } else {
            acc = acc + x;
          }
        }
      }
      a.out[t * a.H + i] = static_cast<uint16_t>(f32_to_bf16_rne(acc));
      if (a.out_acc != nullptr) a.out_acc[t * a.H + i] = acc;
    }
  }
}

template <bool kI64, bool kExpertMajor, int kMode, int kChunks>
void launch_4(const UnpermuteArgs &a, bool vec, int64_t grid, hipStream_t s) {
  if (vec) {
    unpermute_kernel<kI64, kExpertMajor, kMode, kChunks, true><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  } else {
    unpermute_kernel<kI64, kExpertMajor, kMode, kChunks, false><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  }
}

template <bool kI64, bool kExpertMajor, int kMode>
void launch_3(const UnpermuteArgs &a, bool vec, int64_t grid, hipStream_t s) {
  if (a.E <= 64) launch_4<kI64, kExpertMajor, kMode, 1>(a, vec, grid, s);
  else if (a.E <= 256) launch_4<kI64, kExpertMajor, kMode, 4>(a, vec, grid, s);
  else launch_4<kI64, kExpertMajor, kMode, 16>(a, vec, grid, s);
}

template <int kMode>
void launch_mode(const UnpermuteArgs &a, bool i64, bool em, bool vec, int64_t grid, hipStream_t s) {
  if (i64 && em) launch_3<true, true, kMode>(a, vec, grid, s);
  else if (i64) launch_3<true, false, kMode>(a, vec, grid, s);
  else if (em) launch_3<false, true, kMode>(a, vec, grid, s);
  else launch_3<false, false, kMode>(a, vec, grid, s);
}

int common_checks(const char *fn, const void *pin, int64_t R, int64_t H, const void *map,
                  int idx_dtype, int map_layout, int64_t E, int64_t T, const void *out) {
  if (R < 0 || H < 0 || E < 0 || T < 0) {
    return fail(MOE_ERR_SHAPE, "%s: negative size (R=%lld H=%lld E=%lld T=%lld)", fn, (long long)R,
                (long long)H, (long long)E, (long long)T);
  }
  if (E > 1024) return fail(MOE_ERR_CAPACITY, "%s: E=%lld exceeds 1024 experts", fn, (long long)E);
  if (idx_dtype != MOE_IDX_I32 && idx_dtype != MOE_IDX_I64) {
    return fail(MOE_ERR_INVALID_ARG, "%s: idx_dtype %d is not MOE_IDX_I32/I64", fn, idx_dtype);
  }
  if (map_layout != MOE_MAP_TOKEN_MAJOR && map_layout != MOE_MAP_EXPERT_MAJOR) {
    return fail(MOE_ERR_INVALID_ARG, "%s: map_layout %d is not a moe_map_layout_t", fn, map_layout);
  }
  if ((R * H > 0 && pin == nullptr) || (T * E > 0 && map == nullptr) || (T * H > 0 && out == nullptr)) {
    return fail(MOE_ERR_INVALID_ARG, "%s: null input, row_id_map or output", fn);
  }
  if (ceil_div(T, kWavesPerBlock) > 0x7fffffff) {
    return fail(MOE_ERR_CAPACITY, "%s: T=%lld too large", fn, (long long)T);
  }
  return MOE_OK;
}

}  // namespace
}  // namespace moe

extern "C" {

int moe_unpermute(const moe_bf16_t *pin, int64_t R, int64_t H, const void *row_id_map,
                  int idx_dtype, int map_layout, int64_t E, int64_t T, const float *merge_probs,
                  moe_bf16_t *out, float *out_acc, void *stream) {
  using namespace moe;
  int st = common_checks("moe_unpermute", pin, R, H, row_id_map, idx_dtype, map_layout, E, T, out);
  if (st != MOE_OK) return st;
  if (T == 0) return MOE_OK;
  UnpermuteArgs a{pin, R, H, E, T, row_id_map, merge_probs, out, nullptr, out_acc};
  const bool vec = (H % 8 == 0) && is_aligned(pin, 16) && is_aligned(out, 16) && is_aligned(out_acc, 16);
  const int64_t grid = ceil_div(T, kWavesPerBlock);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool i64 = idx_dtype == MOE_IDX_I64, em = map_layout == MOE_MAP_EXPERT_MAJOR;
  if (merge_probs != nullptr) launch_mode<kMerge>(a, i64, em, vec, grid, s);
  else launch_mode<kPlain>(a, i64, em, vec, grid, s);
  return check_launch("moe_unpermute");
}

int moe_permute_bwd(const moe_bf16_t *dperm_act, int64_t R, int64_t H, const float *dpp,
                    const void *row_id_map, int idx_dtype, int map_layout, int64_t E, int64_t T,
                    moe_bf16_t *dact, float *dprobs, float *out_acc, void *stream) {
  using namespace moe;
  int st = common_checks("moe_permute_bwd", dperm_act, R, H, row_id_map, idx_dtype, map_layout, E, T,
                         dact);
  if (st != MOE_OK) return st;
  if ((R > 0 && dpp == nullptr) || (T * E > 0 && dprobs == nullptr)) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute_bwd: null dpp or dprobs");
  }
  if (T == 0) return MOE_OK;
  UnpermuteArgs a{dperm_act, R, H, E, T, row_id_map, dpp, dact, dprobs, out_acc};
  const bool vec = (H % 8 == 0) && is_aligned(dperm_act, 16) && is_aligned(dact, 16) && is_aligned(out_acc, 16);
  const int64_t grid = ceil_div(T, kWavesPerBlock);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool i64 = idx_dtype == MOE_IDX_I64, em = map_layout == MOE_MAP_EXPERT_MAJOR;
  launch_mode<kBwd>(a, i64, em, vec, grid, s);
  return check_launch("moe_permute_bwd");
}

}  // extern "C"
