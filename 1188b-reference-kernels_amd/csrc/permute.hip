// Permute (token rows -> expert-major rows) with optional permuted probs.
//
// Math: kernel_cases/case17_moe_permute_with_mask_map.py:58-71 (token-major
// int64 map) and the expert-major variants kernel_cases/case21...:52-68,
// case22...:47-69, case30...:44-58:
//   out[map(t, e)] = x[t];  permuted_probs[map(t, e)] = probs[t, e]   (map >= 0)
//
// Layout of the work: 4 (token-major map) or 2 (expert-major map) wavefronts per
// token, each owning every 4th / 2nd 1 KiB slice of the row (PermShape).  A
// wave reads the token's
// map entries 64 experts at a time, turns "entry >= 0" into a 64-bit ballot,
// loads the x row once into VGPRs as 16-byte vectors (non-temporal loads, plain
// ones when the permuted output is 1 GiB or more), then
// walks the ballot's set bits in ascending expert order and stores the row to
// each destination (plain stores: measured 4-5% faster than non-temporal ones
// at c5 with a 1 GiB flush between calls).  The row is read from HBM once and written k times, which
// is the algorithmic minimum (2TH + 2RH bytes plus the map and probs).
#include <algorithm>

#include "moe_common.h"

namespace moe {
namespace {

// Launch shape per map layout (best of 256-1024 threads x 1-4 wavefronts per
// token row, measured with a 1 GiB flush between calls): a token-major map row
// is one contiguous read, so 4 wavefronts share a row, one token per
// workgroup; an expert-major map is read down a column (stride T entries), so
// 2 wavefronts share a row and a workgroup takes 4 neighbouring tokens, whose
// map entries share cache lines.
template <bool kExpertMajor>
struct PermShape {
  static constexpr int kThreads = kExpertMajor ? 512 : 256;
  static constexpr int kSplit = kExpertMajor ? 2 : 4;  // wavefronts sharing one token row
  static constexpr int kTokensPerBlock = kThreads / kWave / kSplit;
  static constexpr int kMaxVecPerLane = 16 / kSplit;   // 16-byte vectors per lane per pass
};
constexpr int kMinTokensPerBlock = 1;  // of both shapes (sizes the zero-tail workspace)
constexpr int kTailThreads = 256;      // zero-tail kernel

struct PermuteArgs {
  const uint16_t *x;
  int64_t T, H, E;
  const void *map;
  const float *probs;
  uint16_t *out;
  float *pp;
  int64_t num_out;
  int32_t *block_counts;  // per-block number of map entries >= 0 (zero-tail pass), or null
};

template <bool kI64, bool kExpertMajor>
__device__ __forceinline__ int64_t map_at(const PermuteArgs &a, int64_t t, int64_t e) {
  return load_idx<kI64>(a.map, kExpertMajor ? e * a.T + t : t * a.E + e);
}

// kStaged (expert-major map, 64 < E <= kMaxStagedE): the token's map entries are read once per
// workgroup -- the token's wavefronts split its 64-expert chunks, count the
// routed entries, write the permuted probs and stage row ids + ballots in LDS
// -- and every wavefront then walks the staged ballots.  Read per wavefront
// and per chunk inside the store loop, each chunk's map load waits behind the
// previous chunk's row stores (which may alias it): five dependent round trips
// per token at E = 320.
constexpr int kMaxStagedE = 1024;
__host__ __device__ inline int stage_bytes_per_token(int nchunks) { return nchunks * (kWave * 8 + 8); }

// kNtRow: non-temporal loads of the x row (16-byte rows only), else plain loads.
template <bool kI64, bool kExpertMajor, bool kProbs, bool kVec, bool kStaged, bool kNtRow>
__global__ __launch_bounds__(PermShape<kExpertMajor>::kThreads) void permute_kernel(PermuteArgs a) {
  constexpr int kThreads = PermShape<kExpertMajor>::kThreads;
  constexpr int kSplit = PermShape<kExpertMajor>::kSplit;
  constexpr int kTokensPerBlock = PermShape<kExpertMajor>::kTokensPerBlock;
  constexpr int kMaxVecPerLane = PermShape<kExpertMajor>::kMaxVecPerLane;
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int part = wave % kSplit;  // which share of the row this wave copies
  const int slot = wave / kSplit;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kTokensPerBlock + slot;
  int routed = 0;
  const int nch = kStaged ? static_cast<int>(ceil_div(a.E, kWave)) : 0;
  int64_t *s_dst = reinterpret_cast<int64_t *>(smem + slot * stage_bytes_per_token(nch));
  uint64_t *s_valid = reinterpret_cast<uint64_t *>(smem + slot * stage_bytes_per_token(nch) + nch * kWave * 8);
  if constexpr (kStaged) {
    if (t < a.T) {
      for (int c = part; c < nch; c += kSplit) {
        const int64_t e = static_cast<int64_t>(c) * kWave + lane;
        const int64_t dst = e < a.E ? map_at<kI64, kExpertMajor>(a, t, e) : -1;
        const bool ok = dst >= 0 && dst < a.num_out;
        routed += __popcll(__ballot(dst >= 0));
        if constexpr (kProbs) {
          if (ok && a.pp != nullptr) a.pp[dst] = a.probs[t * a.E + e];
        }
        s_dst[c * kWave + lane] = dst;
        const uint64_t bal = __ballot(ok);
        if (lane == 0) s_valid[c] = bal;
      }
    }
    __syncthreads();
  }
  if (t < a.T) {
    auto chunk_mask = [&](int c, int64_t &dst, bool count) -> uint64_t {
      if constexpr (kStaged) {
        return uniform_u64(s_valid[c]);
      } else {
        const int64_t e = static_cast<int64_t>(c) * kWave + lane;
        dst = e < a.E ? map_at<kI64, kExpertMajor>(a, t, e) : -1;
        const uint64_t mask = __ballot(dst >= 0 && dst < a.num_out);
        if (count) {
          routed += __popcll(__ballot(dst >= 0));
          if constexpr (kProbs) {
            if (dst >= 0 && dst < a.num_out && a.pp != nullptr) a.pp[dst] = a.probs[t * a.E + e];
          }
        }
        return mask;
      }
    };
    auto dest_of = [&](int c, int64_t dst, int b) -> int64_t {
      if constexpr (kStaged) {
        return static_cast<int64_t>(uniform_u64(static_cast<uint64_t>(s_dst[c * kWave + b])));
      } else {
        return readlane64(dst, b);
      }
    };
    const int nchunks = static_cast<int>(ceil_div(a.E, kWave));
    if constexpr (kVec) {
      const int64_t nvec = a.H / 8;  // 16-byte vectors per row
      const u32x4 *src = reinterpret_cast<const u32x4 *>(a.x + t * a.H);
      for (int64_t seg = 0; seg < nvec || seg == 0; seg += kMaxVecPerLane * kWave * kSplit) {
        u32x4 buf[kMaxVecPerLane];
#pragma unroll
        for (int j = 0; j < kMaxVecPerLane; ++j) {
          const int64_t v = seg + (j * kSplit + part) * kWave + lane;
          if constexpr (kNtRow) {
            if (v < nvec) buf[j] = __builtin_nontemporal_load(src + v);
          } else {
            if (v < nvec) buf[j] = src[v];
          }
        }
        for (int c = 0; c < nchunks; ++c) {
          int64_t dst = -1;
          uint64_t mask = chunk_mask(c, dst, seg == 0 && part == 0);
          while (mask) {
            const int b = __builtin_ctzll(mask);
            mask &= mask - 1;
            const int64_t d = dest_of(c, dst, b);
            u32x4 *o = reinterpret_cast<u32x4 *>(a.out + d * a.H);
#pragma unroll
            for (int j = 0; j < kMaxVecPerLane; ++j) {
              const int64_t v = seg + (j * kSplit + part) * kWave + lane;
              if (v < nvec) o[v] = buf[j];  // plain stores: 4-5% faster than non-temporal ones here
            }
          }
        }
        if (nvec == 0) break;
      }
    } else {
      // Scalar path for rows that are not a multiple of 16 bytes or misaligned.
      const uint16_t *src = a.x + t * a.H;
      for (int c = 0; c < nchunks; ++c) {
        int64_t dst = -1;
        uint64_t mask = chunk_mask(c, dst, part == 0);
        while (mask) {
          const int b = __builtin_ctzll(mask);
          mask &= mask - 1;
          const int64_t d = dest_of(c, dst, b);
          uint16_t *o = a.out + d * a.H;
          for (int64_t i = part * kWave + lane; i < a.H; i += kWave * kSplit) o[i] = src[i];
        }
      }
    }
  }
  if (a.block_counts != nullptr) {
    __shared__ int wave_routed[kThreads / kWave];
    if (lane == 0) wave_routed[wave] = routed;
    __syncthreads();
    if (threadIdx.x == 0) {
      int s = 0;
      for (int w = 0; w < kThreads / kWave; ++w) s += wave_routed[w];
      a.block_counts[blockIdx.x] = s;
    }
  }
}

// Map tiles (expert-major maps, and token-major maps with 64 < E; E <= kMaxStagedE; 16-byte rows):
// a workgroup of 8 wavefronts takes kTileTok consecutive tokens. Their map entries are read once,
// coalesced (expert-major: 8 lanes read one expert's entries of the 8 tokens, 64 contiguous bytes
// of an int64 map; token-major: a token's row), and staged in LDS as int32 row ids (-1 for
// entries outside [0, num_out)); the padded LDS row (E rounded up to 64, + 1)
// keeps the transposing writes off a single bank. Then one wavefront per token
// builds the 64-bit ballots of its routed experts, writes the permuted probs,
// loads the token's row into VGPRs (16 vectors per lane per pass)
// and stores it to each destination in ascending expert order.
// 8 tokens, one wavefront each (case21 map, 1 GiB flush: 0.476-0.478 ms; 4 tokens 0.501, 16 tokens 0.486
// (two per wavefront), 32 tokens 0.492; the per-token staged kernel below 0.500).
constexpr int kTileTok = 8;
constexpr int kTileThreads = kTileTok * kWave;
__host__ __device__ inline int tile_row_stride(int nchunks) { return nchunks * kWave + 1; }
__host__ __device__ inline size_t tile_lds_bytes(int nchunks) {
  return static_cast<size_t>(kTileTok) * tile_row_stride(nchunks) * 4 + static_cast<size_t>(kTileTok) * nchunks * 8 + 8;
}

template <bool kI64, bool kProbs, bool kExpertMajor>
__global__ __launch_bounds__(kTileThreads) void permute_tile_kernel(PermuteArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nch = static_cast<int>(ceil_div(a.E, kWave));
  const int stride = tile_row_stride(nch);
  int32_t *s_dst = reinterpret_cast<int32_t *>(smem);
  uint64_t *s_valid = reinterpret_cast<uint64_t *>(smem + ((static_cast<size_t>(kTileTok) * stride * 4 + 7) & ~size_t(7)));
  const int tid = threadIdx.x, lane = lane_id(), wave = threadIdx.x / kWave;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTileTok;
  int routed = 0;
  for (int i = tid; i < kTileTok * nch * kWave; i += kTileThreads) {
    // Expert-major: consecutive threads take consecutive tokens of one expert;
    // token-major: consecutive experts of one token (both coalesced).
    const int e = kExpertMajor ? i / kTileTok : i % (nch * kWave);
    const int tk = kExpertMajor ? i % kTileTok : i / (nch * kWave);
    const int64_t t = t0 + tk;
    int64_t v = -1;
    if (e < a.E && t < a.T) {
      v = load_idx<kI64>(a.map, kExpertMajor ? static_cast<int64_t>(e) * a.T + t : t * a.E + e);
    }
    routed += v >= 0;
    s_dst[tk * stride + e] = (v >= 0 && v < a.num_out) ? static_cast<int32_t>(v) : -1;
  }
  __syncthreads();
  for (int pr = wave; pr < kTileTok * nch; pr += kTileThreads / kWave) {
    const int tk = pr / nch, c = pr % nch;
    const int e = c * kWave + lane;
    const int32_t d = s_dst[tk * stride + e];
    const uint64_t bal = __ballot(d >= 0);
    if (lane == 0) s_valid[tk * nch + c] = bal;
    if constexpr (kProbs) {
      if (d >= 0 && a.pp != nullptr) a.pp[d] = a.probs[(t0 + tk) * a.E + e];
    }
  }
  __syncthreads();
  // One wavefront per token row: measured 2% / 3% faster than two / four (case21 map, 1 GiB flush).
  constexpr int kSplit = 1;
  constexpr int kVecPerLane = 16 / kSplit;
  const int part = wave % kSplit;
  const int64_t nvec = a.H / 8;
  for (int tk = wave / kSplit; tk < kTileTok; tk += kTileThreads / kWave / kSplit) {
    const int64_t t = t0 + tk;
    if (t >= a.T) break;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(a.x + t * a.H);
    for (int64_t seg = 0; seg < nvec; seg += kVecPerLane * kWave * kSplit) {
      u32x4 buf[kVecPerLane];
#pragma unroll
      for (int j = 0; j < kVecPerLane; ++j) {
        const int64_t v = seg + (j * kSplit + part) * kWave + lane;
        if (v < nvec) buf[j] = __builtin_nontemporal_load(src + v);
      }
      for (int c = 0; c < nch; ++c) {
        uint64_t mask = uniform_u64(s_valid[tk * nch + c]);
        while (mask) {
          const int b = __builtin_ctzll(mask);
          mask &= mask - 1;
          const int64_t d = __builtin_amdgcn_readfirstlane(s_dst[tk * stride + c * kWave + b]);
          u32x4 *o = reinterpret_cast<u32x4 *>(a.out + d * a.H);
#pragma unroll
          for (int j = 0; j < kVecPerLane; ++j) {
            const int64_t v = seg + (j * kSplit + part) * kWave + lane;
            if (v < nvec) o[v] = buf[j];
          }
        }
      }
    }
  }
  if (a.block_counts != nullptr) {
    __shared__ int wave_routed[kTileThreads / kWave];
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) routed += __shfl_xor(routed, off);
    if (lane == 0) wave_routed[wave] = routed;
    __syncthreads();
    if (threadIdx.x == 0) {
      int sum = 0;
      for (int w = 0; w < kTileThreads / kWave; ++w) sum += wave_routed[w];
      a.block_counts[blockIdx.x] = sum;
    }
  }
}

// Zero-fills out rows [R, num_out) and pp[R, num_out), R = sum(block_counts).
template <bool kVec>
__global__ __launch_bounds__(kTailThreads) void permute_zero_tail_kernel(const int32_t *block_counts,
                                                                     int64_t nblocks, uint16_t *out,
                                                                     float *pp, int64_t H,
                                                                     int64_t num_out) {
  __shared__ int64_t partial[kTailThreads];
  int64_t s = 0;
  for (int64_t i = threadIdx.x; i < nblocks; i += kTailThreads) s += block_counts[i];
  partial[threadIdx.x] = s;
  __syncthreads();
  for (int w = kTailThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) partial[threadIdx.x] += partial[threadIdx.x + w];
    __syncthreads();
  }
  const int64_t R = partial[0];
  if (R >= num_out) return;
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * kTailThreads + threadIdx.x;
  const int64_t gstride = static_cast<int64_t>(gridDim.x) * kTailThreads;
  if (pp != nullptr) {
    for (int64_t i = R + gtid; i < num_out; i += gstride) pp[i] = 0.0f;
  }
  if constexpr (kVec) {
    u32x4 *o = reinterpret_cast<u32x4 *>(out + R * H);
    const int64_t n = (num_out - R) * H / 8;
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int64_t i = gtid; i < n; i += gstride) __builtin_nontemporal_store(z, o + i);
  } else {
    uint16_t *o = out + R * H;
    const int64_t n = (num_out - R) * H;
    for (int64_t i = gtid; i < n; i += gstride) o[i] = 0;
  }
}

template <bool kI64, bool kExpertMajor, bool kProbs>
void launch_permute_3(const PermuteArgs &a, bool vec, int64_t grid, hipStream_t s) {
  // Row loads: plain when the permuted output is 1 GiB or more, non-temporal below (1 GiB flush between
  // calls; H = 7168 and 8 destinations per token: non-temporal 1.2-2% faster up to 8192 tokens, 0.94 GB
  // written, plain 0.7-2% faster from 12288 tokens, 1.41 GB, to 32768; with 2 or 4 destinations per
  // token, 0.05-0.54 GB written, non-temporal 6-18% faster).
  const bool nt = static_cast<double>(a.num_out) * static_cast<double>(a.H) * 2.0 < 1073741824.0;
  constexpr int kThreads = PermShape<kExpertMajor>::kThreads;
  // Staged for expert-major maps only: 1.5-3% faster there (case21/22/30), 2% slower with a token-major map
  // (case17), whose row of entries is one contiguous read.
  const bool staged = kExpertMajor && a.E > kWave && a.E <= kMaxStagedE;
  const size_t lds = staged ? static_cast<size_t>(PermShape<kExpertMajor>::kTokensPerBlock) *
                                  stage_bytes_per_token(static_cast<int>(ceil_div(a.E, kWave)))
                            : 0;
  if (vec && staged && nt) {
    permute_kernel<kI64, kExpertMajor, kProbs, true, true, true><<<dim3(grid), dim3(kThreads), lds, s>>>(a);
  } else if (vec && staged) {
    permute_kernel<kI64, kExpertMajor, kProbs, true, true, false><<<dim3(grid), dim3(kThreads), lds, s>>>(a);
  } else if (vec && nt) {
    permute_kernel<kI64, kExpertMajor, kProbs, true, false, true><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  } else if (vec) {
    permute_kernel<kI64, kExpertMajor, kProbs, true, false, false><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  } else if (staged) {
    permute_kernel<kI64, kExpertMajor, kProbs, false, true, false><<<dim3(grid), dim3(kThreads), lds, s>>>(a);
  } else {
    permute_kernel<kI64, kExpertMajor, kProbs, false, false, false><<<dim3(grid), dim3(kThreads), 0, s>>>(a);
  }
}

template <bool kI64, bool kExpertMajor>
void launch_permute_2(const PermuteArgs &a, bool vec, int64_t grid, hipStream_t s) {
  if (a.probs != nullptr) {
    launch_permute_3<kI64, kExpertMajor, true>(a, vec, grid, s);
  } else {
    launch_permute_3<kI64, kExpertMajor, false>(a, vec, grid, s);
  }
}

// Source token of each permuted row: the inverse of the row-id map. One thread
// per map entry (coalesced over the map in its own layout); entries outside
// [0, num_out) are skipped.
template <bool kI64>
__global__ __launch_bounds__(256) void permute_index_kernel(const void *map, int64_t T, int64_t E, bool expert_major,
                                                            int32_t *src_token, int64_t num_out) {
  const int64_t n = T * E;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t row = load_idx<kI64>(map, i);
    if (row >= 0 && row < num_out) src_token[row] = static_cast<int32_t>(expert_major ? i % T : i / E);
  }
}

// Extent of a row-id map: max(-1, max entry), the number of entries >= 0 and
// whether those entries are distinct, in one pass. Each block reduces a
// grid-stride share of the entries (16-byte loads when kVec) into partials
// [2 * gridDim.x] and sets byte v of `seen` (zeroed by the caller, n bytes) to
// 1 for every entry v in [0, n) with a plain byte store (an entry named twice
// writes the same value twice: no atomics, whose contention on a bitmap cost
// more than the pass); map_extent_final_kernel adds the partials up in block
// order and counts the set bytes of [0, max]: the map names every row of
// [0, max] exactly once iff count == max + 1 == that byte count.
constexpr int kExtentMaxBlocks = 2048;
constexpr int kExtentUnroll = 4;  // 16-byte vectors each thread loads before using them
template <bool kI64, bool kVec>
__global__ __launch_bounds__(256) void map_extent_partial_kernel(const void *map, int64_t n, int64_t *partials,
                                                                 uint8_t *seen) {
  int64_t mx = -1, cnt = 0;
  auto take = [&](int64_t e) {
    mx = e > mx ? e : mx;
    cnt += e >= 0;
    if (e >= 0 && e < n) seen[e] = 1;
  };
  const int64_t gtid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t gstride = static_cast<int64_t>(gridDim.x) * 256;
  constexpr int kPer = kI64 ? 2 : 4;  // entries per 16-byte vector
  const int64_t nvec = kVec ? n / kPer : 0;
  // kExtentUnroll vectors per thread in flight before any is used
  for (int64_t i0 = gtid; i0 < nvec; i0 += gstride * kExtentUnroll) {
    u32x4 q[kExtentUnroll];
#pragma unroll
    for (int u = 0; u < kExtentUnroll; ++u) {
      const int64_t i = i0 + u * gstride;
      if (i < nvec) q[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(map) + i);
    }
#pragma unroll
    for (int u = 0; u < kExtentUnroll; ++u) {
      if (i0 + u * gstride >= nvec) break;
      if constexpr (kI64) {
        take(static_cast<int64_t>(static_cast<uint64_t>(q[u].x) | (static_cast<uint64_t>(q[u].y) << 32)));
        take(static_cast<int64_t>(static_cast<uint64_t>(q[u].z) | (static_cast<uint64_t>(q[u].w) << 32)));
      } else {
        take(static_cast<int32_t>(q[u].x));
        take(static_cast<int32_t>(q[u].y));
        take(static_cast<int32_t>(q[u].z));
        take(static_cast<int32_t>(q[u].w));
      }
    }
  }
  for (int64_t i = nvec * kPer + gtid; i < n; i += gstride) take(load_idx<kI64>(map, i));
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const int64_t omx = __shfl_xor(mx, off);
    mx = omx > mx ? omx : mx;
    cnt += __shfl_xor(cnt, off);
  }
  __shared__ int64_t s_mx[256 / kWave], s_cnt[256 / kWave];
  const int wave = threadIdx.x / kWave;
  if (lane_id() == 0) {
    s_mx[wave] = mx;
    s_cnt[wave] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 256 / kWave; ++w) {
      mx = s_mx[w] > mx ? s_mx[w] : mx;
      cnt += s_cnt[w];
    }
    partials[2 * blockIdx.x] = mx;
    partials[2 * blockIdx.x + 1] = cnt;
  }
}

constexpr int kExtentFinal = 1024;  // threads of the final kernel (the sum over the row marks)
__global__ __launch_bounds__(kExtentFinal) void map_extent_final_kernel(const int64_t *partials, int nblocks,
                                                               const uint8_t *seen, int64_t *out) {
  __shared__ int64_t s_a[kExtentFinal / kWave], s_b[kExtentFinal / kWave];
  const int wave = threadIdx.x / kWave;
  // at most two (max, count) pairs per thread, both loaded before either is used
  static_assert(kExtentMaxBlocks <= 2 * kExtentFinal, "two partials per thread");
  int64_t m0 = -1, c0 = 0, m1 = -1, c1 = 0;
  const int b0 = threadIdx.x, b1 = threadIdx.x + kExtentFinal;
  if (b0 < nblocks) {
    m0 = partials[2 * b0];
    c0 = partials[2 * b0 + 1];
  }
  if (b1 < nblocks) {
    m1 = partials[2 * b1];
    c1 = partials[2 * b1 + 1];
  }
  int64_t mx = m1 > m0 ? m1 : m0, cnt = c0 + c1;
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const int64_t omx = __shfl_xor(mx, off);
    mx = omx > mx ? omx : mx;
    cnt += __shfl_xor(cnt, off);
  }
  if (lane_id() == 0) {
    s_a[wave] = mx;
    s_b[wave] = cnt;
  }
  __syncthreads();
  mx = s_a[0];
  cnt = s_b[0];
  for (int w = 1; w < kExtentFinal / kWave; ++w) {
    mx = s_a[w] > mx ? s_a[w] : mx;
    cnt += s_b[w];
  }
  __syncthreads();
  // Distinct entries of [0, max]: only needed when the count matches (the bytes are 0 or 1; 16 at a time
  // where the buffer's alignment allows, which the workspace layout gives).
  int64_t pop = 0;
  if (cnt == mx + 1 && mx >= 0) {
    const int64_t rows = mx + 1, nvec = rows / 16;
    constexpr int kU = 8;  // 16-byte vectors per thread in flight before any is counted
    for (int64_t i0 = threadIdx.x; i0 < nvec; i0 += static_cast<int64_t>(kExtentFinal) * kU) {
      u32x4 q[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t i = i0 + static_cast<int64_t>(u) * kExtentFinal;
        q[u] = i < nvec ? reinterpret_cast<const u32x4 *>(seen)[i] : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        pop += __builtin_popcount(q[u].x) + __builtin_popcount(q[u].y) + __builtin_popcount(q[u].z) +
               __builtin_popcount(q[u].w);
      }
    }
    for (int64_t i = nvec * 16 + threadIdx.x; i < rows; i += kExtentFinal) pop += seen[i];
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) pop += __shfl_xor(pop, off);
  if (lane_id() == 0) s_a[wave] = pop;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kExtentFinal / kWave; ++w) pop += s_a[w];
    out[0] = mx;
    out[1] = cnt;
    out[2] = (cnt == mx + 1 && pop == cnt) ? 1 : 0;
  }
}

int64_t map_extent_blocks(int64_t n) { return std::max<int64_t>(1, std::min<int64_t>(kExtentMaxBlocks, ceil_div(n, 256 * 16))); }
// Workspace of moe_map_extent: the partials, then (256-byte aligned) the n bytes of seen rows.
size_t map_extent_seen_offset(int64_t n) {
  return static_cast<size_t>((map_extent_blocks(n) * 2 * sizeof(int64_t) + 255) / 256 * 256);
}

// Zeroes n 16-byte vectors.
__global__ __launch_bounds__(256) void fill_u32x4_kernel(u32x4 *p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    p[i] = u32x4{0u, 0u, 0u, 0u};
  }
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t *p, int64_t n, int32_t v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    p[i] = v;
  }
}

}  // namespace
}  // namespace moe

extern "C" {

size_t moe_permute_workspace_size(int64_t T) {
  if (T < 0) return 0;
  return static_cast<size_t>(moe::ceil_div(T, moe::kMinTokensPerBlock)) * sizeof(int32_t) + 256;
}

int moe_permute(const moe_bf16_t *x, int64_t T, int64_t H, const void *row_id_map, int idx_dtype,
                int map_layout, int64_t E, const float *probs, moe_bf16_t *out,
                float *permuted_probs, int64_t num_out, int zero_tail, void *workspace,
                size_t workspace_bytes, void *stream) {
  using namespace moe;
  if (T < 0 || H < 0 || E < 0 || num_out < 0) {
    return fail(MOE_ERR_SHAPE, "moe_permute: negative size (T=%lld H=%lld E=%lld num_out=%lld)",
                (long long)T, (long long)H, (long long)E, (long long)num_out);
  }
  if (idx_dtype != MOE_IDX_I32 && idx_dtype != MOE_IDX_I64) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute: idx_dtype %d is not MOE_IDX_I32/I64", idx_dtype);
  }
  if (map_layout != MOE_MAP_TOKEN_MAJOR && map_layout != MOE_MAP_EXPERT_MAJOR) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute: map_layout %d is not a moe_map_layout_t", map_layout);
  }
  if ((T * H > 0 && x == nullptr) || (T * E > 0 && row_id_map == nullptr) ||
      (num_out * H > 0 && out == nullptr)) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute: null x, row_id_map or out");
  }
  if (permuted_probs != nullptr && probs == nullptr && T * E > 0) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute: permuted_probs given without probs");
  }
  const bool em = map_layout == MOE_MAP_EXPERT_MAJOR;
  const bool vec = (H % 8 == 0) && is_aligned(x, 16) && is_aligned(out, 16);
  // Map tiles (permute_tile_kernel) for expert-major maps, and for token-major maps with more than 64
  // experts (case17, E = 320, 1 GiB flush: 0.342 ms against 0.378 with 4 wavefronts per token; at c5, E = 64
  // and 8 destinations per token, 4 wavefronts per token stay faster: 0.400 against 0.417 ms).
  const bool map_tile = (em || E > kWave) && vec && E > 0 && E <= kMaxStagedE;
  const int64_t nblocks = ceil_div(T, map_tile ? kTileTok : em ? PermShape<true>::kTokensPerBlock
                                                           : PermShape<false>::kTokensPerBlock);
  if (nblocks > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "moe_permute: T=%lld too large", (long long)T);
  if (zero_tail && (workspace == nullptr || workspace_bytes < moe_permute_workspace_size(T))) {
    return fail(MOE_ERR_WORKSPACE, "moe_permute: zero_tail needs %zu bytes of workspace, got %zu",
                moe_permute_workspace_size(T), workspace_bytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  PermuteArgs a;
  a.x = x;
  a.T = T;
  a.H = H;
  a.E = E;
  a.map = row_id_map;
  a.probs = probs;
  a.out = out;
  a.pp = probs != nullptr ? permuted_probs : nullptr;
  a.num_out = num_out;
  a.block_counts = zero_tail ? static_cast<int32_t *>(workspace) : nullptr;
  if (nblocks > 0 && map_tile) {
    const size_t lds = tile_lds_bytes(static_cast<int>(ceil_div(E, kWave)));
    const bool i64 = idx_dtype == MOE_IDX_I64;
    const dim3 grid(static_cast<uint32_t>(nblocks)), block(kTileThreads);
    if (em) {
      if (i64 && a.probs != nullptr) permute_tile_kernel<true, true, true><<<grid, block, lds, s>>>(a);
      else if (i64) permute_tile_kernel<true, false, true><<<grid, block, lds, s>>>(a);
      else if (a.probs != nullptr) permute_tile_kernel<false, true, true><<<grid, block, lds, s>>>(a);
      else permute_tile_kernel<false, false, true><<<grid, block, lds, s>>>(a);
    } else {
      if (i64 && a.probs != nullptr) permute_tile_kernel<true, true, false><<<grid, block, lds, s>>>(a);
      else if (i64) permute_tile_kernel<true, false, false><<<grid, block, lds, s>>>(a);
      else if (a.probs != nullptr) permute_tile_kernel<false, true, false><<<grid, block, lds, s>>>(a);
      else permute_tile_kernel<false, false, false><<<grid, block, lds, s>>>(a);
    }
    int st = check_launch("moe_permute");
    if (st != MOE_OK) return st;
  } else if (nblocks > 0) {
    const bool i64 = idx_dtype == MOE_IDX_I64;
    if (i64 && em) launch_permute_2<true, true>(a, vec, nblocks, s);
    else if (i64) launch_permute_2<true, false>(a, vec, nblocks, s);
    else if (em) launch_permute_2<false, true>(a, vec, nblocks, s);
    else launch_permute_2<false, false>(a, vec, nblocks, s);
    int st = check_launch("moe_permute");
    if (st != MOE_OK) return st;
  }
  if (zero_tail && num_out > 0) {
    const int64_t tail_elems = num_out * (H > 0 ? H : 1);
    const int64_t grid = std::min<int64_t>(1024, std::max<int64_t>(1, ceil_div(tail_elems, kTailThreads * 8)));
    if (vec) {
      permute_zero_tail_kernel<true><<<dim3(grid), dim3(kTailThreads), 0, s>>>(
          a.block_counts, nblocks, out, a.pp, H, num_out);
    } else {
      permute_zero_tail_kernel<false><<<dim3(grid), dim3(kTailThreads), 0, s>>>(
          a.block_counts, nblocks, out, a.pp, H, num_out);
    }
    return check_launch("moe_permute(zero tail)");
  }
  return MOE_OK;
}

size_t moe_map_extent_workspace_size(int64_t n) {
  if (n < 0) return 0;
  return moe::map_extent_seen_offset(n) + static_cast<size_t>(moe::ceil_div(n, 16)) * 16;
}

int moe_map_extent(const void *row_id_map, int idx_dtype, int64_t n, int64_t *out, void *workspace,
                   size_t workspace_bytes, void *stream) {
  using namespace moe;
  if (n < 0) return fail(MOE_ERR_SHAPE, "moe_map_extent: negative size n=%lld", (long long)n);
  if (idx_dtype != MOE_IDX_I32 && idx_dtype != MOE_IDX_I64) {
    return fail(MOE_ERR_INVALID_ARG, "moe_map_extent: idx_dtype %d is not MOE_IDX_I32/I64", idx_dtype);
  }
  if (out == nullptr || (n > 0 && row_id_map == nullptr)) return fail(MOE_ERR_INVALID_ARG, "moe_map_extent: null map or out");
  const size_t need = moe_map_extent_workspace_size(n);
  if (workspace == nullptr || workspace_bytes < need || !is_aligned(workspace, 16)) {
    return fail(MOE_ERR_WORKSPACE, "moe_map_extent: a 16-byte aligned workspace of %zu bytes is needed (got %zu)", need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nb = map_extent_blocks(n);
  int64_t *partials = static_cast<int64_t *>(workspace);
  uint8_t *seen = reinterpret_cast<uint8_t *>(static_cast<char *>(workspace) + map_extent_seen_offset(n));
  const int64_t vecs = ceil_div(n, 16);
  if (vecs > 0) {
    fill_u32x4_kernel<<<dim3(std::min<int64_t>(2048, ceil_div(vecs, 256))), dim3(256), 0, s>>>(
        reinterpret_cast<u32x4 *>(seen), vecs);
  }
  const bool vec = is_aligned(row_id_map, 16);
  const bool i64 = idx_dtype == MOE_IDX_I64;
  if (i64 && vec) map_extent_partial_kernel<true, true><<<dim3(nb), dim3(256), 0, s>>>(row_id_map, n, partials, seen);
  else if (i64) map_extent_partial_kernel<true, false><<<dim3(nb), dim3(256), 0, s>>>(row_id_map, n, partials, seen);
  else if (vec) map_extent_partial_kernel<false, true><<<dim3(nb), dim3(256), 0, s>>>(row_id_map, n, partials, seen);
  else map_extent_partial_kernel<false, false><<<dim3(nb), dim3(256), 0, s>>>(row_id_map, n, partials, seen);
  map_extent_final_kernel<<<dim3(1), dim3(kExtentFinal), 0, s>>>(partials, static_cast<int>(nb), seen, out);
  return check_launch("moe_map_extent");
}

int moe_permute_index(const void *row_id_map, int idx_dtype, int map_layout, int64_t T, int64_t E,
                      int32_t *src_token, int64_t num_out, int fill, void *stream) {
  using namespace moe;
  if (T < 0 || E < 0 || num_out < 0) {
    return fail(MOE_ERR_SHAPE, "moe_permute_index: negative size (T=%lld E=%lld num_out=%lld)", (long long)T,
                (long long)E, (long long)num_out);
  }
  if (idx_dtype != MOE_IDX_I32 && idx_dtype != MOE_IDX_I64) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute_index: idx_dtype %d is not MOE_IDX_I32/I64", idx_dtype);
  }
  if (map_layout != MOE_MAP_TOKEN_MAJOR && map_layout != MOE_MAP_EXPERT_MAJOR) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute_index: map_layout %d is not a moe_map_layout_t", map_layout);
  }
  if (T > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "moe_permute_index: T=%lld exceeds int32 tokens", (long long)T);
  if ((T * E > 0 && row_id_map == nullptr) || (num_out > 0 && src_token == nullptr)) {
    return fail(MOE_ERR_INVALID_ARG, "moe_permute_index: null row_id_map or src_token");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fill && num_out > 0) {
    const int64_t grid = std::min<int64_t>(1024, ceil_div(num_out, 256));
    moe::fill_i32_kernel<<<dim3(grid), dim3(256), 0, s>>>(src_token, num_out, -1);
    const int st = check_launch("moe_permute_index");
    if (st != MOE_OK) return st;
  }
  if (T * E == 0 || num_out == 0) return MOE_OK;
  const int64_t grid = std::min<int64_t>(4096, ceil_div(T * E, 256));
  const bool em = map_layout == MOE_MAP_EXPERT_MAJOR;
  if (idx_dtype == MOE_IDX_I64) {
    moe::permute_index_kernel<true><<<dim3(grid), dim3(256), 0, s>>>(row_id_map, T, E, em, src_token, num_out);
  } else {
    moe::permute_index_kernel<false><<<dim3(grid), dim3(256), 0, s>>>(row_id_map, T, E, em, src_token, num_out);
  }
  return check_launch("moe_permute_index");
}

}  // extern "C"
