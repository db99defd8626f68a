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
// Each of the k rounds takes the wave-wide maximum key over the lanes' current
// bests (DPP row operations, no LDS crossbar), then the smallest index holding
// it (a ballot when a lane holds one element, else a DPP minimum), so ties go
// to the smaller index; the owning lane retires that element and refreshes its
// own best.  Lane j keeps round j's winner, so lanes < k store values/indices
// coalesced.
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

// Wave-wide maximum / minimum of a 32-bit value, valid in lane 63: quad
// permutes (xor 1, xor 2), half-row and row mirrors (8, 16 lanes), then row
// broadcasts of lanes 15 and 31 (rows 0+1, 2+3, all four). Lanes a step does
// not write keep their value, so each step combines disjoint lane sets.
template <bool kMax>
__device__ __forceinline__ uint32_t wave_reduce_u32(uint32_t v) {
  auto comb = [](uint32_t a, uint32_t b) { return kMax ? (a > b ? a : b) : (a < b ? a : b); };
  const int iv = static_cast<int>(v);
  v = comb(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(iv, iv, 0xB1, 0xF, 0xF, false)));  // quad_perm 1,0,3,2
  int jv = static_cast<int>(v);
  v = comb(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(jv, jv, 0x4E, 0xF, 0xF, false)));  // quad_perm 2,3,0,1
  jv = static_cast<int>(v);
  v = comb(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(jv, jv, 0x141, 0xF, 0xF, false)));  // row_half_mirror
  jv = static_cast<int>(v);
  v = comb(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(jv, jv, 0x140, 0xF, 0xF, false)));  // row_mirror
  jv = static_cast<int>(v);
  v = comb(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(jv, jv, 0x142, 0xA, 0xF, false)));  // row_bcast:15
  jv = static_cast<int>(v);
  v = comb(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(jv, jv, 0x143, 0xC, 0xF, false)));  // row_bcast:31
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// One DPP step of a sum: v + the source lane's v (lanes the step does not
// write add 0: bound_ctrl with old = 0).
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, kRowMask, 0xF, true));
}

// Wave-wide fp32 sum by the same DPP steps (a fixed order), valid in every lane.
__device__ __forceinline__ float wave_sum_f32(float x) {
  float v = dpp_add<0xB1, 0xF>(x);
  v = dpp_add<0x4E, 0xF>(v);
  v = dpp_add<0x141, 0xF>(v);
  v = dpp_add<0x140, 0xF>(v);
  v = dpp_add<0x142, 0xA>(v);
  v = dpp_add<0x143, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
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

  // Best of this lane: largest live key, the smaller slot on equal keys; key
  // 0 = nothing left (every float's order key is above 0).
  uint32_t best_key = 0, best_slot = 0;
  auto lane_best = [&]() {
    best_key = 0;
    best_slot = 0;
#pragma unroll
    for (int s = 0; s < kEPL; ++s) {
      if ((live & (1u << s)) && key[s] > best_key) {
        best_key = key[s];
        best_slot = s;
      }
    }
  };

  lane_best();
  float my_val = 0.0f;
  int my_idx = 0;
  for (int j = 0; j < k; ++j) {
    const uint32_t kmax = wave_reduce_u32<true>(best_key);
    int widx;
    if constexpr (kEPL == 1) {
      widx = __builtin_ctzll(__ballot(best_key == kmax));  // element index = lane
    } else {
      const uint32_t cand = best_key == kmax ? best_slot * kWave + lane : 0xffffffffu;
      widx = static_cast<int>(wave_reduce_u32<false>(cand));
    }
    const int wlane = widx % kWave, wslot = widx / kWave;
    float wval = 0.0f;
    if (lane == wlane) {
#pragma unroll
      for (int s = 0; s < kEPL; ++s)
        if (s == wslot) wval = val[s];
      live &= ~(1u << wslot);
      lane_best();
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
      const float ex = lane < k ? expf(my_val - vmax) : 0.0f;
      inv_sum = wave_sum_f32(ex);
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
