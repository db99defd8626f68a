// Row-id map: routing mask [T, E] -> destination row of every (token, expert).
//
// Math: kernel_cases/case12_moe_row_id_map_pass2.py:43-50
//   row[t, e] = offset[e] + #{t' < t : mask[t', e]}   if mask[t, e], else -1
//   offset[e] = sum_{e' < e} count[e']
// i.e. an expert-major compaction: expert 0's tokens first (ascending t), then
// expert 1's, ...  The same construction appears in case15/17/18/21/22/24/30/32.
//
// Two launches, all integer work on a mask of T*E bytes.  The tokens are cut
// into S <= 64 super-chunks of L tokens (L a multiple of 256), the experts into
// G groups of 32:
//   1. count: block (s, g) counts, for each of its experts, the tokens of
//      super-chunk s that select it -- mask tiles of 256 tokens x 32 experts
//      staged in LDS (16-byte loads, the next tile's issued before the current
//      one is counted), one ballot per 64-token chunk and expert -- and stores
//      counts[s][e] and the group's sum gsum[s][g].
//   2. fill: block (s, g) forms its experts' first rows from those sums alone,
//        offset[e] = sum_{all s', g' < g} gsum[s'][g'] + sum_{all s', e' in g, e' < e} counts[s'][e']
//        first row of expert e in super-chunk s = offset[e] + sum_{s' < s} counts[s'][e],
//      i.e. at most S (G + 32) loads per block for any E, then walks its
//      super-chunk in tiles of 256 tokens: per-chunk counts by ballot, an
//      exclusive scan over the tile's 4 chunks in LDS, and each wave ranks the
//      64 tokens of its chunk for every expert with ballot + mbcnt.  It writes
//      the expert-major rows directly (512 contiguous bytes per wave store), the
//      token-major rows through an LDS transpose, and the source token of every
//      permuted row (src_token[row] = t: the inverse map the grouped GEMM
//      gathers through; a contiguous run per chunk and expert).  Blocks (0, g)
//      store the expert offsets of their group.
// Nothing crosses blocks inside a launch (no counters to clear, no waits on
// other blocks), and the workspace is at most 64 (E + G) int32 values.
#include <mutex>

#include "moe_common.h"

// Scratch memory of moe_row_id_map_noalloc (the counts and group sums of one
// call, at most 64 (E + ceil(E / 32)) int32 values = 1.06 MiB at E = 4096): a
// file-scope device array, one copy per GPU the library runs on, held until
// the process ends.  Host code never passes this name to a kernel: it stands
// for a host-side shadow; the device address comes from hipGetSymbolAddress,
// once per device (noalloc_scratch below).
constexpr size_t kNoAllocScratchBytes = size_t(2) << 20;  // 2 MiB
static __device__ __align__(256) int32_t scratch[kNoAllocScratchBytes / sizeof(int32_t)];

namespace moe {
namespace {

constexpr int kChunk = 64;                       // tokens per chunk = wave width (one ballot)
constexpr int kThreads = 1024;                   // count / fill blocks (16 wavefronts; 512 measured
                                                 // 16% slower at c5, 6% faster at case12)
constexpr int kWaves = kThreads / kWave;
constexpr int kTileChunks = 4;                   // chunks per mask tile
constexpr int kTile = kTileChunks * kChunk;      // 256 tokens per mask tile
constexpr int kEG = 32;                          // experts per block (grid.y)
constexpr int kQ = kWaves / kTileChunks;         // wavefronts per chunk,
constexpr int kEQ = kEG / kQ;                    // each with kEQ of the block's experts
static_assert(kEQ % 4 == 0 && kEQ <= 16, "a wavefront's mask bytes are 1-4 dwords");
constexpr int kMaxE = 4096;
constexpr int kMaxS = 64;                        // super-chunks (grid.x) at most

// Byte tile [kTile][kEG] of the mask, row stride kTileStride bytes (9 dwords: lanes
// reading one column hit distinct banks).
constexpr int kTileStride = kEG + 4;

// Super-chunk length: a multiple of the tile, at most kMaxS super-chunks.
__host__ __device__ inline int64_t super_len(int64_t T) {
  const int64_t per = ceil_div(T, static_cast<int64_t>(kTile) * kMaxS);
  return kTile * (per < 1 ? 1 : per);
}

// Mask tile loader.  Vector form (E % 16 == 0, 16-byte aligned mask): thread i < 256 nv
// holds vector i of the tile (row i / nv, 16-byte part i % nv, nv = eg_n / 16 = 1 or 2),
// fetched into a register one tile ahead.  Rows at or past t_lim read as zeros.
__device__ __forceinline__ u32x4 tile_fetch(const uint8_t *mask, int64_t E, int64_t t0, int64_t t_lim, int64_t eg0,
                                            int nv) {
  const int idx = threadIdx.x;
  const int row = nv == 2 ? idx >> 1 : idx, q = nv == 2 ? idx & 1 : 0;
  u32x4 v = {0u, 0u, 0u, 0u};
  if (row < kTile && t0 + row < t_lim) v = *reinterpret_cast<const u32x4 *>(mask + (t0 + row) * E + eg0 + q * 16);
  return v;
}

__device__ __forceinline__ void tile_store(const u32x4 &v, uint8_t *tile, int nv) {
  const int idx = threadIdx.x;
  const int row = nv == 2 ? idx >> 1 : idx, q = nv == 2 ? idx & 1 : 0;
  if (row < kTile) {
    uint32_t *dst = reinterpret_cast<uint32_t *>(tile + row * kTileStride + q * 16);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
  }
}

// Byte form for other E or alignments (one 0/1 byte per thread and step).
__device__ __forceinline__ void tile_load_bytes(uint8_t *tile, const uint8_t *mask, int64_t E, int64_t t0,
                                                int64_t t_lim, int64_t eg0, int eg_n) {
  for (int i = threadIdx.x; i < kTile * kEG; i += kThreads) {
    const int r = i / kEG, c = i % kEG;
    uint8_t v = 0;
    if (c < eg_n && t0 + r < t_lim) v = mask[(t0 + r) * E + eg0 + c] != 0;
    tile[r * kTileStride + c] = v;
  }
}

// Mask bytes of this lane's token (row `row` of the tile) for the kEQ experts of part jq.
struct LaneBytes {
  uint32_t w[kEQ / 4];
  __device__ __forceinline__ bool operator()(int j) const { return ((w[j >> 2] >> (8 * (j & 3))) & 0xffu) != 0u; }
};
__device__ __forceinline__ LaneBytes lane_bytes(const uint8_t *tile, int row, int jq) {
  const uint32_t *p = reinterpret_cast<const uint32_t *>(tile + row * kTileStride + jq * kEQ);
  LaneBytes b;
#pragma unroll
  for (int q = 0; q < kEQ / 4; ++q) b.w[q] = p[q];
  return b;
}

__global__ __launch_bounds__(256) void rim_zero_kernel(int32_t *p, int64_t n) {
  for (int64_t i = threadIdx.x; i < n; i += 256) p[i] = 0;
}

// counts[s][e] = #{t in super-chunk s : mask[t, e]};  gsum[s][g] = sum over the group's experts.
// Wave w counts chunk w / kQ of each tile for experts (w % kQ) kEQ .. + kEQ - 1 of the group.
__global__ __launch_bounds__(kThreads) void rim_count_kernel(const uint8_t *mask, int64_t T, int64_t E, int64_t L,
                                                             int64_t G, int32_t *counts, int32_t *gsum, bool vec) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kTile * kTileStride];
  __shared__ int32_t s_acc[kTileChunks][kEG];
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int c = wave / kQ, jq = wave % kQ;
  const int64_t s = blockIdx.x, g = blockIdx.y;
  const int64_t eg0 = g * kEG;
  const int eg_n = static_cast<int>(E - eg0 < kEG ? E - eg0 : kEG);
  const int64_t t_begin = s * L, t_end = t_begin + L < T ? t_begin + L : T;
  const int nv = eg_n / 16;
  int32_t acc = 0;  // lane j < kEQ: this wave's count of expert jq * kEQ + j
  u32x4 r = {0u, 0u, 0u, 0u};
  if (vec) r = tile_fetch(mask, E, t_begin, t_end, eg0, nv);
  for (int64_t t0 = t_begin; t0 < t_end; t0 += kTile) {
    if (vec) {
      tile_store(r, tile, nv);
      if (t0 + kTile < t_end) r = tile_fetch(mask, E, t0 + kTile, t_end, eg0, nv);
    } else {
      tile_load_bytes(tile, mask, E, t0, t_end, eg0, eg_n);
    }
    __syncthreads();
    const LaneBytes mb = lane_bytes(tile, c * kChunk + lane, jq);
#pragma unroll
    for (int j = 0; j < kEQ; ++j) {
      if (jq * kEQ + j < eg_n) {
        const int32_t n = __popcll(__ballot(mb(j)));
        if (lane == j) acc += n;
      }
    }
    __syncthreads();  // the tile is rewritten next round
  }
  if (lane < kEQ) s_acc[c][jq * kEQ + lane] = acc;
  __syncthreads();
  if (threadIdx.x < kEG) {  // wave 0, lanes 0..31
    int32_t tot = 0;
#pragma unroll
    for (int cc = 0; cc < kTileChunks; ++cc) tot += s_acc[cc][threadIdx.x];
    if (static_cast<int>(threadIdx.x) >= eg_n) tot = 0;
    else counts[s * E + eg0 + threadIdx.x] = tot;
    int32_t gs = tot;
#pragma unroll
    for (int d = kEG / 2; d > 0; d >>= 1) gs += __shfl_xor(gs, d, kEG);
    if (threadIdx.x == 0) gsum[s * G + g] = gs;
  }
}

// Fill; see the file comment.  S = ceil(T / L).  Wave w handles chunk w / kQ of each tile
// and experts (w % kQ) kEQ .. + kEQ - 1 of the group.
__global__ __launch_bounds__(kThreads) void rim_fill_kernel(const uint8_t *mask, int64_t T, int64_t E, int64_t L,
                                                            int64_t S, int64_t G, const int32_t *counts,
                                                            const int32_t *gsum, int64_t *row_em, int64_t *row_tm,
                                                            int32_t *row_em32, int32_t *expert_offsets,
                                                            int32_t *src_token, int64_t src_capacity, bool vec) {
  constexpr int kParts = kThreads / kEG;  // threads per expert for the sums over super-chunks
  constexpr int kPer = kMaxS / kParts;     // super-chunks per thread
  __shared__ __attribute__((aligned(16))) uint8_t tile[kTile * kTileStride];
  __shared__ int32_t out_tile[kTileChunks][kChunk * (kEG + 1)];
  __shared__ int32_t s_cc[kTileChunks][kEG];  // per-chunk counts of the tile, then the chunks' first rows
  __shared__ int32_t s_run[kEG];              // first row of each expert at the current tile
  __shared__ int32_t s_red[kWaves];
  __shared__ int32_t s_tp[kParts][kEG], s_pp[kParts][kEG];
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int c = wave / kQ, jq = wave % kQ;
  const int64_t s = blockIdx.x, g = blockIdx.y;
  const int64_t eg0 = g * kEG;
  const int eg_n = static_cast<int>(E - eg0 < kEG ? E - eg0 : kEG);
  const int64_t t_begin = s * L, t_end = t_begin + L < T ? t_begin + L : T;
  const int nv = eg_n / 16;
  // The first tile's mask loads go out first; the sums below are loaded behind them.
  u32x4 r = {0u, 0u, 0u, 0u};
  if (vec) r = tile_fetch(mask, E, t_begin, t_end, eg0, nv);

  // Rows before this group: thread (q, k) = (tid / 32, tid % 32) adds the group sums of
  // super-chunks q, q + kParts, ... for the groups k, k + 32, ... below g.
  const int q = threadIdx.x / kEG, k = threadIdx.x % kEG;
  int32_t part = 0;
  for (int64_t g2 = k; g2 < g; g2 += kEG) {
    int32_t v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) v[u] = q + kParts * u < S ? gsum[(q + kParts * u) * G + g2] : 0;
#pragma unroll
    for (int u = 0; u < kPer; ++u) part += v[u];
  }
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) part += __shfl_xor(part, d);
  if (lane == 0) s_red[wave] = part;
  // Expert eg0 + k: its count in super-chunks q, q + kParts, ..., split into before / from s.
  {
    int32_t tp = 0, pp = 0;
    if (k < eg_n) {
      int32_t v[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) v[u] = q + kParts * u < S ? counts[(q + kParts * u) * E + eg0 + k] : 0;
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        tp += v[u];
        if (q + kParts * u < s) pp += v[u];
      }
    }
    s_tp[q][k] = tp;
    s_pp[q][k] = pp;
  }
  __syncthreads();
  if (wave == 0) {
    int32_t tot = 0, pre = 0, before = 0;
    if (lane < kEG) {
#pragma unroll
      for (int qq = 0; qq < kParts; ++qq) {
        tot += s_tp[qq][lane];
        pre += s_pp[qq][lane];
      }
    }
#pragma unroll
    for (int w = 0; w < kWaves; ++w) before += s_red[w];
    int32_t incl = tot;  // lanes >= eg_n hold 0
#pragma unroll
    for (int d = 1; d < kEG; d <<= 1) {
      const int32_t o = __shfl_up(incl, d, kEG);
      if (lane % kEG >= d) incl += o;
    }
    const int32_t offset = before + incl - tot;
    if (lane < eg_n) {
      if (s == 0 && expert_offsets != nullptr) {
        expert_offsets[eg0 + lane] = offset;
        if (eg0 + lane == E - 1) expert_offsets[E] = offset + tot;
      }
      s_run[lane] = offset + pre;
    }
  }
  // (s_run is read after the tile's first barrier)

  for (int64_t t0 = t_begin; t0 < t_end; t0 += kTile) {
    if (vec) {
      tile_store(r, tile, nv);
      if (t0 + kTile < t_end) r = tile_fetch(mask, E, t0 + kTile, t_end, eg0, nv);
    } else {
      tile_load_bytes(tile, mask, E, t0, t_end, eg0, eg_n);
    }
    __syncthreads();
    // This lane's token of chunk c: its 8 mask bytes of quarter jq in a register.
    const LaneBytes selected = lane_bytes(tile, c * kChunk + lane, jq);
    // Counts of chunk c for this wave's experts.
    int32_t my_cc = 0;
#pragma unroll
    for (int j = 0; j < kEQ; ++j) {
      if (jq * kEQ + j < eg_n) {
        const int32_t n = __popcll(__ballot(selected(j)));
        if (lane == j) my_cc = n;
      }
    }
    if (lane < kEQ) s_cc[c][jq * kEQ + lane] = my_cc;
    __syncthreads();
    // First row of each (chunk, expert) of the tile: exclusive scan over the tile's chunks.
    if (threadIdx.x < eg_n) {
      int32_t run = s_run[threadIdx.x];
#pragma unroll
      for (int cc = 0; cc < kTileChunks; ++cc) {
        const int32_t v = s_cc[cc][threadIdx.x];
        s_cc[cc][threadIdx.x] = run;
        run += v;
      }
      s_run[threadIdx.x] = run;
    }
    __syncthreads();
    // Ranks of chunk c's 64 tokens for this wave's experts (lane j < kEQ holds expert
    // jq * kEQ + j's first row in the chunk).
    const int64_t t = t0 + c * kChunk + lane;
    const int32_t first = s_cc[c][jq * kEQ + (lane % kEQ)];
    int32_t *ot = out_tile[c];
#pragma unroll
    for (int j = 0; j < kEQ; ++j) {
      const int jl = jq * kEQ + j;
      if (jl < eg_n) {
        const int64_t e = eg0 + jl;
        const bool sel = selected(j);  // false past t_end (zero rows)
        const uint64_t m = __ballot(sel);
        const int32_t v = sel ? __builtin_amdgcn_readlane(first, j) + lanes_below(m) : -1;
        if (t < t_end) {
          if (row_em != nullptr) row_em[e * T + t] = v;
          if (row_em32 != nullptr) row_em32[e * T + t] = v;
        }
        // The expert's rows of this chunk are consecutive: a contiguous run of source tokens.
        if (sel && src_token != nullptr && v < src_capacity) src_token[v] = static_cast<int32_t>(t);
        ot[lane * (kEG + 1) + jl] = v;
      }
    }
    __syncthreads();
    if (row_tm != nullptr) {
      // Wave (c, jq) stores rows jq * kRows .. of chunk c: element i = lane + 64 n of that
      // [kRows][eg_n] block, its row and column advanced by (64 / eg_n, 64 % eg_n) per step.
      constexpr int kRows = kChunk / kQ;
      const int64_t tw = t0 + c * kChunk + jq * kRows;
      const int step_r = kWave / eg_n, step_c = kWave % eg_n;
      int rr = lane / eg_n, col = lane % eg_n;
      for (int i = lane; i < kRows * eg_n; i += kWave) {
        if (tw + rr < t_end) row_tm[(tw + rr) * E + eg0 + col] = ot[(jq * kRows + rr) * (kEG + 1) + col];
        rr += step_r;
        col += step_c;
        if (col >= eg_n) {
          col -= eg_n;
          ++rr;
        }
      }
    }
    __syncthreads();  // tile, s_cc and out_tile are rewritten next round
  }
}

// Device address of `scratch` on the current device, looked up on the first
// call for that device (with it current) and cached.
int noalloc_scratch(const char *fn, void **out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void *cache[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MOE_ERR_LAUNCH, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(MOE_ERR_CAPACITY, "%s: device %d >= %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return fail(MOE_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev, hipGetErrorString(e));
    }
    cache[dev] = p;
  }
  *out = cache[dev];
  return MOE_OK;
}

}  // namespace
}  // namespace moe

extern "C" {

size_t moe_row_id_map_workspace_size(int64_t T, int64_t E) {
  if (T < 0 || E < 0) return 0;
  // counts [S, E] then group sums [S, G] (int32), S <= 64 super-chunks, G = ceil(E / 32)
  const int64_t S = moe::ceil_div(T, moe::super_len(T)), G = moe::ceil_div(E, moe::kEG);
  return static_cast<size_t>(S * (E + G)) * sizeof(int32_t) + 256;
}

int moe_row_id_map(const uint8_t *routing_map, int64_t T, int64_t E, int64_t *row_expert_major,
                   int64_t *row_token_major, int32_t *row_expert_major_i32,
                   int32_t *expert_offsets, int32_t *src_token, int64_t src_capacity, void *workspace,
                   size_t workspace_bytes, void *stream) {
  using namespace moe;
  if (T < 0 || E < 0 || src_capacity < 0) {
    return fail(MOE_ERR_SHAPE, "moe_row_id_map: negative size (T=%lld E=%lld src_capacity=%lld)", (long long)T,
                (long long)E, (long long)src_capacity);
  }
  if (E > kMaxE) return fail(MOE_ERR_CAPACITY, "moe_row_id_map: E=%lld exceeds %d", (long long)E, kMaxE);
  if (T * E >= (int64_t(1) << 31)) {
    return fail(MOE_ERR_CAPACITY, "moe_row_id_map: T*E=%lld must stay below 2^31 (int32 rows)",
                (long long)(T * E));
  }
  if (T * E > 0 && routing_map == nullptr) return fail(MOE_ERR_INVALID_ARG, "moe_row_id_map: null routing_map");
  if (T * E > 0 && (workspace == nullptr || workspace_bytes < moe_row_id_map_workspace_size(T, E))) {
    return fail(MOE_ERR_WORKSPACE, "moe_row_id_map: needs %zu bytes of workspace, got %zu",
                moe_row_id_map_workspace_size(T, E), workspace_bytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t L = super_len(T), S = ceil_div(T, L), G = ceil_div(E, kEG);
  int32_t *counts = static_cast<int32_t *>(workspace);
  int32_t *gsum = counts + S * E;
  if (T * E == 0) {
    // No (token, expert) pairs: offsets are all zero; nothing else to write.
    // (A fill kernel rather than hipMemsetAsync keeps the call graph-capturable.)
    if (expert_offsets != nullptr) {
      rim_zero_kernel<<<dim3(1), dim3(256), 0, s>>>(expert_offsets, E + 1);
      return check_launch("moe_row_id_map(zero offsets)");
    }
    return MOE_OK;
  }
  const bool vec = (E % 16 == 0) && is_aligned(routing_map, 16);
  const dim3 grid(static_cast<uint32_t>(S), static_cast<uint32_t>(G));
  rim_count_kernel<<<grid, dim3(kThreads), 0, s>>>(routing_map, T, E, L, G, counts, gsum, vec);
  const int st = check_launch("moe_row_id_map(count)");
  if (st != MOE_OK) return st;
  rim_fill_kernel<<<grid, dim3(kThreads), 0, s>>>(routing_map, T, E, L, S, G, counts, gsum, row_expert_major,
                                                 row_token_major, row_expert_major_i32, expert_offsets, src_token,
                                                 src_capacity, vec);
  return check_launch("moe_row_id_map(fill)");
}

int moe_row_id_map_noalloc(const uint8_t *routing_map, int64_t T, int64_t E, int64_t *row_expert_major,
                           int64_t *row_token_major, int32_t *row_expert_major_i32, int32_t *expert_offsets,
                           int32_t *src_token, int64_t src_capacity, void *stream) {
  using namespace moe;
  static const char *fn = "moe_row_id_map_noalloc";
  if (T < 0 || E < 0 || src_capacity < 0) {
    return fail(MOE_ERR_SHAPE, "%s: negative size (T=%lld E=%lld src_capacity=%lld)", fn, (long long)T,
                (long long)E, (long long)src_capacity);
  }
  if (E > kMaxE) return fail(MOE_ERR_CAPACITY, "%s: E=%lld exceeds %d", fn, (long long)E, kMaxE);
  if (T * E >= (int64_t(1) << 31)) {
    return fail(MOE_ERR_CAPACITY, "%s: T*E=%lld must stay below 2^31 (int32 rows)", fn, (long long)(T * E));
  }
  const size_t need = moe_row_id_map_workspace_size(T, E);
  if (need > kNoAllocScratchBytes) {
    return fail(MOE_ERR_CAPACITY,
                "%s: T=%lld E=%lld needs %zu bytes of scratch, the static scratch holds %zu; use moe_row_id_map "
                "with a workspace",
                fn, (long long)T, (long long)E, need, kNoAllocScratchBytes);
  }
  if (T * E == 0) {
    return moe_row_id_map(routing_map, T, E, row_expert_major, row_token_major, row_expert_major_i32,
                          expert_offsets, src_token, src_capacity, nullptr, 0, stream);
  }
  if (routing_map == nullptr) return fail(MOE_ERR_INVALID_ARG, "%s: null routing_map", fn);
  void *ws = nullptr;
  const int st = noalloc_scratch(fn, &ws);
  if (st != MOE_OK) return st;
  return moe_row_id_map(routing_map, T, E, row_expert_major, row_token_major, row_expert_major_i32, expert_offsets,
                        src_token, src_capacity, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"
