// Per-row router top-k on one wavefront (shared by the stand-alone top-k
// kernel and the router GEMM's fused epilogue).
//
// Math: kernel_cases/case23_ref_aten_topk.py:47-62 -- values/indices are the
// first k entries of a stable descending sort of each row (torch.topk with
// largest=True, sorted=True): larger value first, equal values by smaller
// index, NaN above every number, -0.0 equal to +0.0.  The mask is
// zeros(T,E,bool).scatter_(1, idx, True) (case18...py:86-88) and the merge
// probs are softmax over the k selected values (fp32), scattered to [T, E].
//
// Lane l holds elements l, l+64, ... (kEPL per lane) as 32-bit order keys.
// Each of the k rounds takes the wave-wide maximum of the packed
// (key, ~index) over the lanes' current bests (6 xor-shuffle steps), the
// owning lane retires that element and refreshes its own best.  Lane j keeps
// round j's winner, so lanes < k store values/indices coalesced.
#pragma once

#include "moe_common.h"

namespace moe {

// Order key: a > b as floats (with NaN largest, -0 == +0) iff key(a) > key(b).
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // any NaN
  if ((u & 0x7fffffffu) == 0u) u = 0u;                        // -0 -> +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Top-k of row t (elements load(e), e < E) by the calling wavefront; writes
// values/indices [T, k] and, when non-null, routing_map [T, E] and probs [T, E].
template <int kEPL, typename Load>
__device__ __forceinline__ void topk_row(Load load, int64_t t, int E, int k, float *values, int64_t *indices,
                                         uint8_t *routing_map, float *probs) {
  const int lane = lane_id();
  float val[kEPL];
  uint32_t key[kEPL];
  uint32_t live = 0;  // bit s: element lane + 64 s not yet selected
#pragma unroll
  for (int s = 0; s < kEPL; ++s) {
    const int e = s * kWave + lane;
    val[s] = 0.0f;
    key[s] = 0u;
    if (e < E) {
      val[s] = load(e);
      key[s] = order_key(val[s]);
      live |= 1u << s;
    }
  }
  const uint32_t present = live;

  // Packed best of this lane: (key << 32) | ~index; 0 = nothing left.
  auto lane_best = [&]() -> uint64_t {
    uint64_t best = 0;
#pragma unroll
    for (int s = 0; s < kEPL; ++s) {
      if (live & (1u << s)) {
        const uint64_t p = (static_cast<uint64_t>(key[s]) << 32) | static_cast<uint32_t>(~(s * kWave + lane));
        best = p > best ? p : best;
      }
    }
    return best;
  };

  uint64_t mine = lane_best();
  float my_val = 0.0f;
  int my_idx = 0;
  for (int j = 0; j < k; ++j) {
    uint64_t b = mine;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint64_t o = __shfl_xor(b, d);
      b = o > b ? o : b;
    }
    const int widx = static_cast<int>(~static_cast<uint32_t>(b));
    const int wlane = widx % kWave, wslot = widx / kWave;
    float wval = 0.0f;
    if (lane == wlane) {
#pragma unroll
      for (int s = 0; s < kEPL; ++s)
        if (s == wslot) wval = val[s];
      live &= ~(1u << wslot);
      mine = lane_best();
    }
    wval = readlane_f32(wval, wlane);
    if (lane == j) {
      my_val = wval;
      my_idx = widx;
    }
  }
  if (lane < k) {
    values[t * k + lane] = my_val;
    indices[t * k + lane] = my_idx;
  }

  if (routing_map != nullptr || probs != nullptr) {
    const uint32_t chosen = present & ~live;
    float inv_sum = 0.0f, vmax = 0.0f;
    if (probs != nullptr) {
      vmax = readlane_f32(my_val, 0);
      float ex = lane < k ? expf(my_val - vmax) : 0.0f;
      float sum = ex;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) sum += __shfl_xor(sum, d);
      inv_sum = sum;
    }
#pragma unroll
    for (int s = 0; s < kEPL; ++s) {
      const int e = s * kWave + lane;
      if (e < E) {
        const bool c = (chosen >> s) & 1u;
        if (routing_map != nullptr) routing_map[t * E + e] = c ? 1 : 0;
        if (probs != nullptr) probs[t * E + e] = c ? expf(val[s] - vmax) / inv_sum : 0.0f;
      }
    }
  }
}

}  // namespace moe
