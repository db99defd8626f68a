// Row-id map: routing mask [T, E] -> destination row of every (token, expert).
//
// Math: kernel_cases/case12_moe_row_id_map_pass2.py:43-50
//   row[t, e] = offset[e] + #{t' < t : mask[t', e]}   if mask[t, e], else -1
//   offset[e] = sum_{e' < e} count[e']
// i.e. an expert-major compaction: expert 0's tokens first (ascending t), then
// expert 1's, ...  The same construction appears in case15/17/18/21/22/24/30/32.
//
// Three launches, all integer work on a mask of T*E bytes:
//   1. count: block = one 64-token chunk x one group of up to 32 experts
//      (grid.y: 4 groups at E = 64, 10 at E = 320; one block per chunk walking
//      128-expert groups in turn was 1.4-2.3x slower); the chunk's mask tile is loaded into
//      LDS with 16-byte vector loads (one per thread at E = 64), then
//      per-expert popcounts (wave ballots over 64 tokens) -> counts[chunk][e].
//   2. scan: 16 experts per workgroup; per-expert sums over 16 runs of chunks
//      (loads issued in batches of 8), an exclusive scan over the runs in LDS,
//      then counts are rewritten in place as the (chunk, expert) base row
//      relative to the expert's first row, and the expert's total is stored.
//      (A single workgroup scanning every expert took 35 us at E = 320.)
//   3. fill: block = one 64-token chunk x one group of up to 32 experts; the experts' offsets are the
//      exclusive scan of the totals (E <= 4096 values, scanned in LDS by every
//      block; block 0 stores them as expert_offsets[0..E]); mask tile and the
//      chunk's E bases go through LDS, each wave ranks 64 tokens of one expert with ballot +
//      mbcnt and writes the expert-major rows directly (512 contiguous bytes
//      per wave store) and the token-major rows through an LDS transpose.
// Every global load of a thread is independent of its other loads, so a block
// waits for memory about once per phase rather than once per element.
#include <mutex>

#include "moe_common.h"

// Scratch memory of moe_row_id_map_noalloc (the chunk counts and expert totals
// of one call): a file-scope device array, one copy per GPU the library runs
// on, held until the process ends.  Host code never passes this name to a
// kernel: it stands for a host-side shadow; the device address comes from
// hipGetSymbolAddress, once per device (noalloc_scratch below).
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;  // 8 MiB
static __device__ __align__(256) int32_t scratch[kNoAllocScratchBytes / sizeof(int32_t)];

namespace moe {
namespace {

constexpr int kChunk = 64;          // tokens per chunk = wave width (one ballot)
constexpr int kThreads = 256;       // count / fill blocks
constexpr int kWaves = kThreads / kWave;
constexpr int kEG = 32;             // experts per block (grid.y) of the count and fill kernels
constexpr int kMaxE = 4096;

// Byte tile [kChunk][kEG] of the mask, row stride kTileStride bytes (odd word
// count so that lanes reading one column hit distinct banks).
constexpr int kTileStride = kEG + 4;

__device__ __forceinline__ void load_mask_tile(uint8_t *tile, const uint8_t *mask, int64_t T,
                                               int64_t E, int64_t t0, int64_t eg0, int eg_n, bool vec) {
  if (vec) {
    // 16 mask bytes per thread (E % 16 == 0, 16-byte aligned mask), stored as
    // four dwords (the tile row stride is a multiple of 4 bytes).
    const int nv = eg_n / 16;
    for (int i = threadIdx.x; i < kChunk * nv; i += kThreads) {
      const int r = i / nv, q = i % nv;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (t0 + r < T) v = *reinterpret_cast<const u32x4 *>(mask + (t0 + r) * E + eg0 + q * 16);
      uint32_t *dst = reinterpret_cast<uint32_t *>(tile + r * kTileStride + q * 16);
      dst[0] = v.x;
      dst[1] = v.y;
      dst[2] = v.z;
      dst[3] = v.w;
    }
    return;
  }
  for (int i = threadIdx.x; i < kChunk * kEG; i += kThreads) {
    const int r = i / kEG, c = i % kEG;
    uint8_t v = 0;
    if (c < eg_n && t0 + r < T) v = mask[(t0 + r) * E + eg0 + c] != 0;
    tile[r * kTileStride + c] = v;
  }
}

__global__ __launch_bounds__(kThreads) void rim_zero_kernel(int32_t *p, int64_t n) {
  for (int64_t i = threadIdx.x; i < n; i += kThreads) p[i] = 0;
}

__global__ __launch_bounds__(kThreads) void rim_count_kernel(const uint8_t *mask, int64_t T,
                                                             int64_t E, int32_t *counts, bool vec) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kChunk * kTileStride];
  const int64_t chunk = blockIdx.x;
  const int64_t t0 = chunk * kChunk;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int64_t eg0 = static_cast<int64_t>(blockIdx.y) * kEG;  // this block's group of experts
  const int eg_n = static_cast<int>(E - eg0 < kEG ? E - eg0 : kEG);
  load_mask_tile(tile, mask, T, E, t0, eg0, eg_n, vec);
  __syncthreads();
  for (int c = wave; c < eg_n; c += kWaves) {
    const uint64_t m = __ballot(tile[lane * kTileStride + c] != 0);
    if (lane == 0) counts[chunk * E + eg0 + c] = __popcll(m);
  }
}

// Exclusive scan of one int32 per thread over a kThreads-thread block;
// `*total` receives the block's sum.  Ends with a barrier.
__device__ int32_t block_exclusive_scan(int32_t v, int32_t *wave_sums, int32_t *total) {
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  int32_t incl = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == kWave - 1) wave_sums[wave] = incl;
  __syncthreads();
  int32_t before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int32_t ws = wave_sums[w];
    if (w < wave) before += ws;
    all += ws;
  }
  if (threadIdx.x == 0) *total = all;
  __syncthreads();
  return before + incl - v;
}

// Column scan of the chunk counts, kScanExperts experts per workgroup:
//   counts[c][e] -> sum_{c' < c} counts[c'][e]   (in place; relative to the expert's first row)
//   totals[e]    =  sum_c counts[c][e]
// Thread (part, expert) owns a run of ceil(nc / kScanParts) chunks of one
// expert; the runs' sums are scanned in LDS.  The experts' offsets (the scan
// of the totals) are left to the fill kernel, so this pass needs no
// cross-workgroup step.
constexpr int kScanExperts = 16;
constexpr int kScanParts = kThreads / kScanExperts;
__global__ __launch_bounds__(kThreads) void rim_scan_kernel(int32_t *counts, int64_t nc, int64_t E,
                                                            int32_t *totals) {
  __shared__ int32_t part_sums[kThreads];
  constexpr int kBatch = 8;
  const int el = threadIdx.x % kScanExperts, p = threadIdx.x / kScanExperts;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kScanExperts + el;
  const bool active = e < E;
  const int64_t per = ceil_div(nc, kScanParts);
  const int64_t c_begin = p * per, c_end = c_begin + per < nc ? c_begin + per : nc;
  int32_t sum = 0;
  if (active) {
    for (int64_t c = c_begin; c < c_end; c += kBatch) {
      int32_t v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) v[j] = c + j < c_end ? counts[(c + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) sum += v[j];
    }
  }
  part_sums[threadIdx.x] = sum;
  __syncthreads();
  if (active && p == 0) {
    int32_t run = 0;
    for (int q = 0; q < kScanParts; ++q) {
      const int32_t v = part_sums[q * kScanExperts + el];
      part_sums[q * kScanExperts + el] = run;
      run += v;
    }
    totals[e] = run;
  }
  __syncthreads();
  if (active) {
    int32_t run = part_sums[threadIdx.x];
    for (int64_t c = c_begin; c < c_end; c += kBatch) {
      int32_t v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) v[j] = c + j < c_end ? counts[(c + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (c + j < c_end) counts[(c + j) * E + e] = run;
        run += v[j];
      }
    }
  }
}

// base[c][e] holds the chunk's first row relative to expert e's first row;
// each block adds the expert offsets (the exclusive scan of totals, done here
// in LDS: E <= 4096 values) and block 0 stores them as expert_offsets.
__global__ __launch_bounds__(kThreads) void rim_fill_kernel(const uint8_t *mask, int64_t T, int64_t E,
                                                            const int32_t *base, const int32_t *totals,
                                                            int64_t *row_em, int64_t *row_tm, int32_t *row_em32,
                                                            int32_t *expert_offsets, bool vec) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kChunk * kTileStride];
  __shared__ int32_t out_tile[kChunk * (kEG + 1)];
  __shared__ int32_t s_base[kMaxE];
  __shared__ int32_t wave_sums[kWaves];
  __shared__ int32_t grand_total;
  const int64_t chunk = blockIdx.x;
  const int64_t t0 = chunk * kChunk;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int64_t t = t0 + lane;
  // The experts' totals and this chunk's relative bases, read once
  // (independent loads, issued before the first mask tile's loads so the round
  // trips overlap); thread i owns experts [i per, (i + 1) per).
  const int per = static_cast<int>(ceil_div(E, kThreads));
  const int64_t e_first = static_cast<int64_t>(threadIdx.x) * per;
  int32_t tv[kMaxE / kThreads], bv[kMaxE / kThreads];
#pragma unroll
  for (int i = 0; i < kMaxE / kThreads; ++i) {
    tv[i] = 0;
    bv[i] = 0;
    if (i < per && e_first + i < E) {
      tv[i] = totals[e_first + i];
      bv[i] = base[chunk * E + e_first + i];
    }
  }
  const int64_t eg0 = static_cast<int64_t>(blockIdx.y) * kEG;  // this block's group of experts
  const int eg_n = static_cast<int>(E - eg0 < kEG ? E - eg0 : kEG);
  const bool first_block = chunk == 0 && blockIdx.y == 0;
  load_mask_tile(tile, mask, T, E, t0, eg0, eg_n, vec);
  {
    int32_t local = 0;
#pragma unroll
    for (int i = 0; i < kMaxE / kThreads; ++i) local += tv[i];
    int32_t run = block_exclusive_scan(local, wave_sums, &grand_total);
#pragma unroll
    for (int i = 0; i < kMaxE / kThreads; ++i) {
      if (i < per && e_first + i < E) {
        if (first_block && expert_offsets != nullptr) expert_offsets[e_first + i] = run;
        s_base[e_first + i] = run + bv[i];
        run += tv[i];
      }
    }
    if (first_block && expert_offsets != nullptr && threadIdx.x == 0) expert_offsets[E] = grand_total;
  }
  __syncthreads();
  for (int c = wave; c < eg_n; c += kWaves) {
    const int64_t e = eg0 + c;
    const bool sel = tile[lane * kTileStride + c] != 0;
    const uint64_t m = __ballot(sel);
    const int32_t b = s_base[e];
    const int32_t v = sel ? b + lanes_below(m) : -1;
    if (t < T) {
      if (row_em != nullptr) row_em[e * T + t] = v;
      if (row_em32 != nullptr) row_em32[e * T + t] = v;
    }
    out_tile[lane * (kEG + 1) + c] = v;
  }
  __syncthreads();
  if (row_tm != nullptr) {
    for (int i = threadIdx.x; i < kChunk * eg_n; i += kThreads) {
      const int r = i / eg_n, c = i % eg_n;
      if (t0 + r < T) row_tm[(t0 + r) * E + eg0 + c] = out_tile[r * (kEG + 1) + c];
    }
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
  // chunk counts [nc, E] then expert totals [E] (int32)
  return static_cast<size_t>(moe::ceil_div(T, moe::kChunk) * E + E) * sizeof(int32_t) + 256;
}

int moe_row_id_map(const uint8_t *routing_map, int64_t T, int64_t E, int64_t *row_expert_major,
                   int64_t *row_token_major, int32_t *row_expert_major_i32,
                   int32_t *expert_offsets, void *workspace, size_t workspace_bytes,
                   void *stream) {
  using namespace moe;
  if (T < 0 || E < 0) {
    return fail(MOE_ERR_SHAPE, "moe_row_id_map: negative size (T=%lld E=%lld)", (long long)T, (long long)E);
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
  const int64_t nc = ceil_div(T, kChunk);
  int32_t *counts = static_cast<int32_t *>(workspace);
  if (T * E == 0) {
    // No (token, expert) pairs: offsets are all zero; nothing else to write.
    // (A fill kernel rather than hipMemsetAsync keeps the call graph-capturable.)
    if (expert_offsets != nullptr) {
      rim_zero_kernel<<<dim3(1), dim3(kThreads), 0, s>>>(expert_offsets, E + 1);
      return check_launch("moe_row_id_map(zero offsets)");
    }
    return MOE_OK;
  }
  const bool vec = (E % 16 == 0) && is_aligned(routing_map, 16);
  const dim3 chunk_grid(static_cast<uint32_t>(nc), static_cast<uint32_t>(ceil_div(E, kEG)));
  rim_count_kernel<<<chunk_grid, dim3(kThreads), 0, s>>>(routing_map, T, E, counts, vec);
  int st = check_launch("moe_row_id_map(count)");
  if (st != MOE_OK) return st;
  int32_t *totals = counts + nc * E;
  rim_scan_kernel<<<dim3(static_cast<uint32_t>(ceil_div(E, kScanExperts))), dim3(kThreads), 0, s>>>(counts, nc, E,
                                                                                                   totals);
  st = check_launch("moe_row_id_map(scan)");
  if (st != MOE_OK) return st;
  rim_fill_kernel<<<chunk_grid, dim3(kThreads), 0, s>>>(routing_map, T, E, counts, totals, row_expert_major,
                                                       row_token_major, row_expert_major_i32, expert_offsets, vec);
  return check_launch("moe_row_id_map(fill)");
}

int moe_row_id_map_noalloc(const uint8_t *routing_map, int64_t T, int64_t E, int64_t *row_expert_major,
                           int64_t *row_token_major, int32_t *row_expert_major_i32, int32_t *expert_offsets,
                           void *stream) {
  using namespace moe;
  static const char *fn = "moe_row_id_map_noalloc";
  if (T < 0 || E < 0) return fail(MOE_ERR_SHAPE, "%s: negative size (T=%lld E=%lld)", fn, (long long)T, (long long)E);
  if (E > kMaxE) return fail(MOE_ERR_CAPACITY, "%s: E=%lld exceeds %d", fn, (long long)E, kMaxE);
  if (T * E >= (int64_t(1) << 31)) {
    return fail(MOE_ERR_CAPACITY, "%s: T*E=%lld must stay below 2^31 (int32 rows)", fn, (long long)(T * E));
  }
  const size_t need = moe_row_id_map_workspace_size(T, E);
  if (need > kNoAllocScratchBytes) {
    return fail(MOE_ERR_CAPACITY,
                "%s: T=%lld E=%lld needs %zu bytes of scratch (ceil(T/64)*E + E int32 values + 256), the static "
                "scratch holds %zu; use moe_row_id_map with a workspace",
                fn, (long long)T, (long long)E, need, kNoAllocScratchBytes);
  }
  if (T * E == 0) {
    return moe_row_id_map(routing_map, T, E, row_expert_major, row_token_major, row_expert_major_i32,
                          expert_offsets, nullptr, 0, stream);
  }
  if (routing_map == nullptr) return fail(MOE_ERR_INVALID_ARG, "%s: null routing_map", fn);
  void *ws = nullptr;
  const int st = noalloc_scratch(fn, &ws);
  if (st != MOE_OK) return st;
  return moe_row_id_map(routing_map, T, E, row_expert_major, row_token_major, row_expert_major_i32, expert_offsets,
                        ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"
