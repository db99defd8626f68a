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
// Layout of the work: each token gets as many wavefronts as its row has 1 KiB
// slices (at most 16), so one pass of 16-byte loads per lane covers the row;
// rows under 4 slices share a 4-wavefront workgroup with other tokens.  At
// H=7168 that is 14 wavefronts per workgroup, measured 11% faster than a fixed
// 4 wavefronts per token walking the row in four passes.
//
// With more than 64 experts the token's map entries are read once per
// workgroup, not once per wavefront: the token's wavefronts split its
// 64-expert chunks and stage the row ids, one validity ballot per chunk and the
// merge weights in LDS; every wavefront then walks the ballots in ascending
// expert order and takes each source row id from LDS (a broadcast read).  At
// E=320 / H=8192 that is 13% faster than every wavefront reading the whole map
// column.  With at most 64 experts each wavefront reads the one chunk itself
// (no barrier, no LDS round trip; 9% faster at c5).  Sources are consumed in
// batches of 8: the wave issues the 8 row loads back to back, then accumulates
// them in ascending expert order.  Workgroups run in launch order: numbering
// them so that each XCD takes a contiguous run of tokens (for L2 sharing of
// expert-major map lines) measured 9% slower at c5, as the concurrently
// running tokens then read and write 8 separate regions.
#include "moe_common.h"

#pragma clang fp contract(off)

namespace moe {
namespace {

constexpr int kMaxThreads = 1024;
constexpr int kMaxE = 4096;                 // the row-id map's limit
constexpr size_t kMaxLds = 160 * 1024;      // gfx950 LDS per workgroup
constexpr int kMaxWavesPerToken = kMaxThreads / kWave;
constexpr int kBatch = 8;

// Launch shape: enough wavefronts per token that each lane owns one 16-byte
// vector (one pass over the row), at most 16; short rows pack several tokens
// into a 4-wavefront workgroup.
struct Shape {
  int waves_per_token, tokens_per_block;
};

Shape pick_shape(int64_t H, bool vec) {
  const int64_t units = vec ? H / 8 : H;
  int64_t w = ceil_div(units, static_cast<int64_t>(kWave));
  w = w < 1 ? 1 : (w > kMaxWavesPerToken ? kMaxWavesPerToken : w);
  const int wpt = static_cast<int>(w);
  return Shape{wpt, wpt >= 4 ? 1 : 4 / wpt};
}

enum Mode { kPlain = 0, kMerge = 1, kBwd = 2 };

struct UnpermuteArgs {
  const uint16_t *pin;
  int64_t R, H, E, T;
  const void *map;
  const float *probs;  // kMerge: merge probs [T, E]; kBwd: dpp [R]
  uint16_t *out;
  float *dprobs;   // kBwd: [T, E]
  float *out_acc;  // optional fp32 accumulator [T, H] (the reference functions return it)
  int waves_per_token, tokens_per_block;
  int nchunks;  // ceil(E / 64)
};

// LDS per token: row ids [nchunks*64] int64, ballots [nchunks] u64, then (merge
// only) weights [nchunks*64] f32.
__host__ __device__ inline size_t lds_bytes_per_token(int nchunks, bool merge) {
  return static_cast<size_t>(nchunks) * (kWave * 8 + 8 + (merge ? kWave * 4 : 0));
}

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

// kStaged: the map goes through LDS (E > 64); otherwise every wavefront reads
// the token's one 64-expert chunk into a register and picks entries with
// readlane, which skips the workgroup barrier and the LDS round trip.
template <bool kI64, bool kExpertMajor, int kMode, bool kVec, bool kStaged>
__global__ __launch_bounds__(kMaxThreads) void unpermute_kernel(UnpermuteArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int split = a.waves_per_token;
  const int part = wave % split;  // which share of the row this wave sums
  const int slot = wave / split;  // which of the workgroup's tokens
  const int nch = kStaged ? a.nchunks : 1;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * a.tokens_per_block + slot;

  unsigned char *tok = smem + slot * lds_bytes_per_token(nch, kMode == kMerge);
  int64_t *s_src = reinterpret_cast<int64_t *>(tok);
  uint64_t *s_valid = reinterpret_cast<uint64_t *>(tok + nch * kWave * 8);
  float *s_w = reinterpret_cast<float *>(tok + nch * (kWave * 8 + 8));
  int64_t r_src = -1;   // !kStaged: this lane's map entry
  float r_w = 0.0f;     // !kStaged: its merge weight
  uint64_t r_valid = 0; // !kStaged: ballot of the valid entries

  // Chunk c of the token's map entries is read by wave (c mod split) when
  // staged, by every wave otherwise.
  if (t < a.T) {
    for (int c = kStaged ? part : 0; c < nch; c += split) {
      const int64_t e = static_cast<int64_t>(c) * kWave + lane;
      int64_t s = -1;
      if (e < a.E) s = map_at<kI64, kExpertMajor>(a, t, e);
      const bool ok = s >= 0 && s < a.R;
      const uint64_t bal = __ballot(ok);
      float w = 0.0f;
      if constexpr (kMode == kMerge) w = ok ? a.probs[t * a.E + e] : 0.0f;
      if constexpr (kMode == kBwd) {
        if (e < a.E && (kStaged || part == 0)) a.dprobs[t * a.E + e] = ok ? a.probs[s] : 0.0f;
      }
      if constexpr (kStaged) {
        s_src[c * kWave + lane] = s;
        if (lane == 0) s_valid[c] = bal;
        if constexpr (kMode == kMerge) s_w[c * kWave + lane] = w;
      } else {
        r_src = s;
        r_valid = bal;
        r_w = w;
      }
    }
  }
  if constexpr (kStaged) __syncthreads();
  if (t >= a.T) return;
  auto valid_of = [&](int c) -> uint64_t { return kStaged ? uniform_u64(s_valid[c]) : r_valid; };
  auto row_of = [&](int c, int bit) -> int64_t {
    return kStaged ? static_cast<int64_t>(uniform_u64(static_cast<uint64_t>(s_src[c * kWave + bit])))
                   : readlane64(r_src, bit);
  };
  auto weight_of = [&](int c, int bit) -> float {
    return kStaged ? __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(s_w[c * kWave + bit])))
                   : readlane_f32(r_w, bit);
  };

  if constexpr (kVec) {
    const int64_t nvec = a.H / 8;
    for (int64_t v = part * kWave + lane; v < nvec; v += kWave * split) {
      float acc[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
      for (int c = 0; c < nch; ++c) {
        uint64_t m = valid_of(c);
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
              rows[b] = row_of(c, bit);
              if constexpr (kMode == kMerge) ws[b] = weight_of(c, bit);
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
    for (int64_t i = part * kWave + lane; i < a.H; i += kWave * split) {
      float acc = 0.0f;
      for (int c = 0; c < nch; ++c) {
        uint64_t m = valid_of(c);
        while (m) {
          const int bit = __builtin_ctzll(m);
          m &= m - 1;
          const int64_t row = row_of(c, bit);
          const float x = bf16_to_f32(a.pin[row * a.H + i]);
          if constexpr (kMode == kMerge) {
            acc = acc + weight_of(c, bit) * x;
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

template <bool kI64, bool kExpertMajor, int kMode>
void launch_3(const UnpermuteArgs &a, bool vec, int64_t grid, hipStream_t s) {
  const int threads = a.waves_per_token * a.tokens_per_block * kWave;
  const bool staged = a.nchunks > 1;
  const size_t lds = staged ? a.tokens_per_block * lds_bytes_per_token(a.nchunks, kMode == kMerge) : 0;
  if (vec && staged) {
    unpermute_kernel<kI64, kExpertMajor, kMode, true, true><<<dim3(grid), dim3(threads), lds, s>>>(a);
  } else if (vec) {
    unpermute_kernel<kI64, kExpertMajor, kMode, true, false><<<dim3(grid), dim3(threads), 0, s>>>(a);
  } else if (staged) {
    unpermute_kernel<kI64, kExpertMajor, kMode, false, true><<<dim3(grid), dim3(threads), lds, s>>>(a);
  } else {
    unpermute_kernel<kI64, kExpertMajor, kMode, false, false><<<dim3(grid), dim3(threads), 0, s>>>(a);
  }
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
  if (E > kMaxE) return fail(MOE_ERR_CAPACITY, "%s: E=%lld exceeds %d experts", fn, (long long)E, kMaxE);
  if (idx_dtype != MOE_IDX_I32 && idx_dtype != MOE_IDX_I64) {
    return fail(MOE_ERR_INVALID_ARG, "%s: idx_dtype %d is not MOE_IDX_I32/I64", fn, idx_dtype);
  }
  if (map_layout != MOE_MAP_TOKEN_MAJOR && map_layout != MOE_MAP_EXPERT_MAJOR) {
    return fail(MOE_ERR_INVALID_ARG, "%s: map_layout %d is not a moe_map_layout_t", fn, map_layout);
  }
  if ((R * H > 0 && pin == nullptr) || (T * E > 0 && map == nullptr) || (T * H > 0 && out == nullptr)) {
    return fail(MOE_ERR_INVALID_ARG, "%s: null input, row_id_map or output", fn);
  }
  if (T > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "%s: T=%lld too large", fn, (long long)T);
  return MOE_OK;
}

// Fills the launch shape into `a` and returns the grid size.
int64_t shape_launch(UnpermuteArgs &a, bool vec) {
  const Shape sh = pick_shape(a.H, vec);
  a.waves_per_token = sh.waves_per_token;
  a.tokens_per_block = sh.tokens_per_block;
  a.nchunks = static_cast<int>(ceil_div(a.E, kWave));
  // Staged map entries of every token of a workgroup must fit the LDS (49 KiB per token
  // at E = 4096): fewer tokens per workgroup for short rows with many experts.
  while (a.tokens_per_block > 1 && a.nchunks > 1 &&
         a.tokens_per_block * lds_bytes_per_token(a.nchunks, true) > kMaxLds) {
    a.tokens_per_block /= 2;
  }
  return ceil_div(a.T, static_cast<int64_t>(a.tokens_per_block));
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
  UnpermuteArgs a{pin, R, H, E, T, row_id_map, merge_probs, out, nullptr, out_acc, 0, 0, 0};
  const bool vec = (H % 8 == 0) && is_aligned(pin, 16) && is_aligned(out, 16) && is_aligned(out_acc, 16);
  const int64_t grid = shape_launch(a, vec);
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
  UnpermuteArgs a{dperm_act, R, H, E, T, row_id_map, dpp, dact, dprobs, out_acc, 0, 0, 0};
  const bool vec = (H % 8 == 0) && is_aligned(dperm_act, 16) && is_aligned(dact, 16) && is_aligned(out_acc, 16);
  const int64_t grid = shape_launch(a, vec);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool i64 = idx_dtype == MOE_IDX_I64, em = map_layout == MOE_MAP_EXPERT_MAJOR;
  launch_mode<kBwd>(a, i64, em, vec, grid, s);
  return check_launch("moe_permute_bwd");
}

}  // extern "C"
