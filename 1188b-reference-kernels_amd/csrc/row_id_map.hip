// Row-id map: routing mask [T, E] -> destination row of every (token, expert).
//
// Math: kernel_cases/case12_moe_row_id_map_pass2.py:43-50
//   row[t, e] = offset[e] + #{t' < t : mask[t', e]}   if mask[t, e], else -1
//   offset[e] = sum_{e' < e} count[e']
// i.e. an expert-major compaction: expert 0's tokens first (ascending t), then
// expert 1's, ...  The same construction appears in case15/17/18/21/22/24/30/32.
//
// Three launches, all integer work on a mask of T*E bytes:
//   1. count: block = one 64-token chunk; the chunk's mask tile is loaded into
//      LDS with 16-byte vector loads (one per thread at E = 64), then
//      per-expert popcounts (wave ballots over 64 tokens) -> counts[chunk][e].
//   2. scan (one workgroup): per-expert sums over runs of chunks (loads issued
//      in batches of 8), exclusive scans over the runs and over the experts'
//      totals, then counts are rewritten in place as the global base row of
//      (chunk, expert) and expert_offsets[0..E] is emitted.
//   3. fill: block = one 64-token chunk; mask tile and the chunk's E bases go
//      through LDS, each wave ranks 64 tokens of one expert with ballot +
//      mbcnt and writes the expert-major rows directly (512 contiguous bytes
//      per wave store) and the token-major rows through an LDS transpose.
// Every global load of a thread is independent of its other loads, so a block
// waits for memory about once per phase rather than once per element.
#include "moe_common.h"

namespace moe {
namespace {

constexpr int kChunk = 64;          // tokens per chunk = wave width (one ballot)
constexpr int kThreads = 256;       // count / fill blocks
constexpr int kWaves = kThreads / kWave;
constexpr int kEG = 128;            // experts per LDS group in the fill kernel
constexpr int kScanThreads = 1024;  // scan kernel
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
  for (int64_t eg0 = 0; eg0 < E; eg0 += kEG) {
    const int eg_n = static_cast<int>(E - eg0 < kEG ? E - eg0 : kEG);
    __syncthreads();
    load_mask_tile(tile, mask, T, E, t0, eg0, eg_n, vec);
    __syncthreads();
    for (int c = wave; c < eg_n; c += kWaves) {
      const uint64_t m = __ballot(tile[lane * kTileStride + c] != 0);
      if (lane == 0) counts[chunk * E + eg0 + c] = __popcll(m);
    }
  }
}

// Exclusive block-wide scan of one int64 per thread (kScanThreads threads).
__device__ int64_t block_exclusive_scan(int64_t v, int64_t *wave_sums, int64_t *total) {
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  int64_t incl = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int64_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == kWave - 1) wave_sums[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    int64_t ws = lane < kScanThreads / kWave ? wave_sums[lane] : 0;
    int64_t wi = ws;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int64_t o = __shfl_up(wi, d);
      if (lane >= d) wi += o;
    }
    if (lane < kScanThreads / kWave) wave_sums[lane] = wi - ws;
    if (lane == kScanThreads / kWave - 1) *total = wi;
  }
  __syncthreads();
  const int64_t r = wave_sums[wave] + incl - v;
  __syncthreads();
  return r;
}

// counts[c][e] (int32, nc x E) -> base[c][e] = offset[e] + sum_{c' < c} counts[c'][e]
__global__ __launch_bounds__(kScanThreads) void rim_scan_kernel(int32_t *counts, int64_t nc,
                                                                int64_t E, int32_t *expert_offsets) {
  __shared__ int64_t totals[kMaxE];
  __shared__ int64_t wave_sums[kScanThreads / kWave];
  __shared__ int64_t grand_total;
  __shared__ int64_t part_sums[kScanThreads];
  constexpr int kBatch = 8;
  // Threads = parts x experts; each part owns a run of `per` chunks of one expert.
  const int64_t parts = E >= kScanThreads ? 1 : kScanThreads / E;
  const int64_t per = ceil_div(nc, parts);
  // Pass 1: per-part sums, then exclusive scans over parts (per expert) -> totals.
  for (int64_t e0 = 0; e0 < E; e0 += kScanThreads) {
    const int64_t lin = threadIdx.x;
    const int64_t e = e0 + (parts > 1 ? lin % E : lin);
    const int64_t p = parts > 1 ? lin / E : 0;
    const bool active = e < E && p < parts;
    int64_t sum = 0;
    if (active) {
      const int64_t c_begin = p * per, c_end = c_begin + per < nc ? c_begin + per : nc;
      for (int64_t c = c_begin; c < c_end; c += kBatch) {
        int32_t v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) v[j] = c + j < c_end ? counts[(c + j) * E + e] : 0;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) sum += v[j];
      }
    }
    __syncthreads();
    part_sums[threadIdx.x] = sum;
    __syncthreads();
    if (active && p == 0) {
      int64_t run = 0;
      for (int64_t q = 0; q < parts; ++q) {
        const int64_t idx = parts > 1 ? q * E + (e - e0) : threadIdx.x;
        const int64_t v = part_sums[idx];
        part_sums[idx] = run;
        run += v;
      }
      totals[e] = run;
    }
    // With E < kScanThreads there is one sweep and part_sums keeps each part's
    // exclusive prefix for pass 2; with E >= kScanThreads every part starts at
    // chunk 0 (prefix 0).
    __syncthreads();
  }
  // Exclusive scan of totals over experts -> offsets (in totals).
  const int64_t per_e = ceil_div(E, kScanThreads);
  const int64_t eb = threadIdx.x * per_e;
  int64_t local = 0;
  for (int64_t i = 0; i < per_e && eb + i < E; ++i) local += totals[eb + i];
  int64_t run = block_exclusive_scan(local, wave_sums, &grand_total);
  for (int64_t i = 0; i < per_e && eb + i < E; ++i) {
    const int64_t v = totals[eb + i];
    totals[eb + i] = run;
    run += v;
  }
  __syncthreads();
  if (expert_offsets != nullptr) {
    for (int64_t e = threadIdx.x; e < E; e += kScanThreads) expert_offsets[e] = static_cast<int32_t>(totals[e]);
    if (threadIdx.x == 0) expert_offsets[E] = static_cast<int32_t>(grand_total);
  }
  // Pass 2: rewrite counts as base rows = offset[e] + prefix over earlier chunks.
  for (int64_t e0 = 0; e0 < E; e0 += kScanThreads) {
    const int64_t lin = threadIdx.x;
    const int64_t e = e0 + (parts > 1 ? lin % E : lin);
    const int64_t p = parts > 1 ? lin / E : 0;
    const bool active = e < E && p < parts;
    if (active) {
      int64_t run = totals[e] + (parts > 1 ? part_sums[threadIdx.x] : 0);
      const int64_t c_begin = p * per, c_end = c_begin + per < nc ? c_begin + per : nc;
      for (int64_t c = c_begin; c < c_end; c += kBatch) {
        int32_t v[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) v[j] = c + j < c_end ? counts[(c + j) * E + e] : 0;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          if (c + j < c_end) counts[(c + j) * E + e] = static_cast<int32_t>(run);
          run += v[j];
        }
      }
    }
  }
}

// The same scan with every count staged in LDS first (one round of
// independent 16-byte loads), for nc * E <= kLdsScanMax counts and E % 4 == 0:
// thread (part, expert) column-sums a run of chunks, the runs and the experts
// are scanned in LDS, and the bases are written back from LDS with 16-byte
// stores.  One dependent global round trip instead of four.
constexpr int kLdsScanMax = 24576;  // counts (96 KiB of LDS)
__global__ __launch_bounds__(kScanThreads) void rim_scan_lds_kernel(int32_t *counts, int64_t nc, int64_t E,
                                                                    int32_t *expert_offsets) {
  __shared__ __attribute__((aligned(16))) int32_t cnt[kLdsScanMax];
  __shared__ int64_t totals[kMaxE];
  __shared__ int64_t part_sums[kScanThreads];
  __shared__ int64_t wave_sums[kScanThreads / kWave];
  __shared__ int64_t grand_total;
  const int64_t n = nc * E;
  for (int64_t i = threadIdx.x; i < n / 4; i += kScanThreads)
    reinterpret_cast<u32x4 *>(cnt)[i] = reinterpret_cast<const u32x4 *>(counts)[i];
  __syncthreads();
  // Threads = parts x experts (E <= kScanThreads here); part p sums chunks [p per, (p+1) per).
  const int64_t parts = kScanThreads / E;
  const int64_t per = ceil_div(nc, parts);
  const int64_t e = threadIdx.x % E, p = threadIdx.x / E;
  const bool active = p < parts;
  const int64_t c_begin = p * per, c_end = min(c_begin + per, nc);
  int64_t sum = 0;
  if (active)
    for (int64_t c = c_begin; c < c_end; ++c) sum += cnt[c * E + e];
  part_sums[threadIdx.x] = sum;
  __syncthreads();
  if (active && p == 0) {
    int64_t run = 0;
    for (int64_t q = 0; q < parts; ++q) {
      const int64_t v = part_sums[q * E + e];
      part_sums[q * E + e] = run;
      run += v;
    }
    totals[e] = run;
  }
  __syncthreads();
  // Exclusive scan of the totals over experts -> offsets.
  const int64_t local = threadIdx.x < E ? totals[threadIdx.x] : 0;
  const int64_t off = block_exclusive_scan(local, wave_sums, &grand_total);
  if (threadIdx.x < E) totals[threadIdx.x] = off;
  __syncthreads();
  if (expert_offsets != nullptr) {
    for (int64_t i = threadIdx.x; i < E; i += kScanThreads) expert_offsets[i] = static_cast<int32_t>(totals[i]);
    if (threadIdx.x == 0) expert_offsets[E] = static_cast<int32_t>(grand_total);
  }
  // Bases in place in LDS, then stored as 16-byte vectors.
  if (active) {
    int64_t run = totals[e] + part_sums[threadIdx.x];
    for (int64_t c = c_begin; c < c_end; ++c) {
      const int32_t v = cnt[c * E + e];
      cnt[c * E + e] = static_cast<int32_t>(run);
      run += v;
    }
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < n / 4; i += kScanThreads)
    reinterpret_cast<u32x4 *>(counts)[i] = reinterpret_cast<const u32x4 *>(cnt)[i];
}

__global__ __launch_bounds__(kThreads) void rim_fill_kernel(const uint8_t *mask, int64_t T, int64_t E,
                                                            const int32_t *base, int64_t *row_em,
                                                            int64_t *row_tm, int32_t *row_em32, bool vec) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[kChunk * kTileStride];
  __shared__ int32_t out_tile[kChunk * (kEG + 1)];
  __shared__ int32_t s_base[kMaxE];
  const int64_t chunk = blockIdx.x;
  const int64_t t0 = chunk * kChunk;
  const int lane = lane_id(), wave = threadIdx.x / kWave;
  const int64_t t = t0 + lane;
  // This chunk's base row per expert, read once (independent loads). With
  // E <= kThreads the load is issued before the first mask tile's loads and
  // stored after them, so the two round trips overlap.
  int32_t bv = 0;
  if (E <= kThreads) {
    if (threadIdx.x < E) bv = base[chunk * E + threadIdx.x];
  } else {
    for (int64_t e = threadIdx.x; e < E; e += kThreads) s_base[e] = base[chunk * E + e];
  }
  for (int64_t eg0 = 0; eg0 < E; eg0 += kEG) {
    const int eg_n = static_cast<int>(E - eg0 < kEG ? E - eg0 : kEG);
    if (eg0 > 0) __syncthreads();
    load_mask_tile(tile, mask, T, E, t0, eg0, eg_n, vec);
    if (eg0 == 0 && E <= kThreads && threadIdx.x < E) s_base[threadIdx.x] = bv;
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
}

}  // namespace
}  // namespace moe

extern "C" {

size_t moe_row_id_map_workspace_size(int64_t T, int64_t E) {
  if (T < 0 || E < 0) return 0;
  return static_cast<size_t>(moe::ceil_div(T, moe::kChunk) * E) * sizeof(int32_t) + 256;
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
  rim_count_kernel<<<dim3(nc), dim3(kThreads), 0, s>>>(routing_map, T, E, counts, vec);
  int st = check_launch("moe_row_id_map(count)");
  if (st != MOE_OK) return st;
  if (nc * E <= kLdsScanMax && E % 4 == 0 && E <= kScanThreads && is_aligned(counts, 16)) {
    rim_scan_lds_kernel<<<dim3(1), dim3(kScanThreads), 0, s>>>(counts, nc, E, expert_offsets);
  } else {
    rim_scan_kernel<<<dim3(1), dim3(kScanThreads), 0, s>>>(counts, nc, E, expert_offsets);
  }
  st = check_launch("moe_row_id_map(scan)");
  if (st != MOE_OK) return st;
  rim_fill_kernel<<<dim3(nc), dim3(kThreads), 0, s>>>(routing_map, T, E, counts, row_expert_major,
                                                       row_token_major, row_expert_major_i32, vec);
  return check_launch("moe_row_id_map(fill)");
}

}  // extern "C"
