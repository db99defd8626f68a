// Device building blocks shared by the grouped GEMM kernels (gfx950): LDS
// DMA through buffer resources, wait counters, barriers that the scheduler
// does not move, and instruction-group schedules.
#pragma once

#include "moe_common.h"

namespace moe {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

constexpr int kBK = 64;  // reduction depth of one pipeline stage

// Loads of data that nothing writes while the kernel runs (group offsets, the
// lists an earlier kernel made): through the constant address space, so that a
// wave-uniform index becomes a scalar load. A vector load would sit in the
// wavefront's in-order vector-memory counter behind its LDS DMAs, and the wait
// for its value would wait for all of them.
typedef __attribute__((address_space(4))) const int32_t const_i32;
typedef __attribute__((address_space(4))) const int16_t const_i16;
__device__ __forceinline__ int32_t ld_inv(const int32_t *p, int64_t i) { return ((const const_i32 *)p)[i]; }
__device__ __forceinline__ int32_t ld_inv(const int16_t *p, int64_t i) { return ((const const_i16 *)p)[i]; }

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0],[15:14]; expcnt [6:4]; lgkmcnt [11:8]).
constexpr int kWaitVm0 = 0x0f70;    // vmcnt(0)
constexpr int kWaitLgkm0 = 0xc07f;  // lgkmcnt(0)

__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Workgroup barrier that neither the compiler nor the instruction scheduler
// moves any instruction across.
__device__ __forceinline__ void barrier() {
  compiler_fence();
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  compiler_fence();
}

// Waits for this thread's outstanding vector-memory (DMA, stores) or LDS operations.
__device__ __forceinline__ void wait_dma() {
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  compiler_fence();
}
__device__ __forceinline__ void wait_lds() {
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  compiler_fence();
}
// Waits until at most kN of this thread's vector-memory operations are
// outstanding (they complete in issue order).
template <int kN>
__device__ __forceinline__ void wait_vm_n() {
  static_assert(kN >= 0 && kN <= 63, "vmcnt range");
  compiler_fence();
  __builtin_amdgcn_s_waitcnt((kN & 0xf) | ((kN >> 4) << 14) | (0x7 << 4) | (0xf << 8));
  compiler_fence();
}

// Buffer resource over [base, base + bytes): raw buffer loads past `bytes`
// return zeros and stores past it are dropped, without touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// Offset that lies past every resource this code builds (all stay below 2 GiB).
constexpr uint32_t kNoAccess = 0x80000000u;

// 16-byte buffer -> LDS copy: lane i writes bytes [16 i, 16 i + 16) of the 1 KiB
// block at `lds` (wave-uniform); the global address is rsrc base + voff + soff.
// kAux: cache policy bits (2: nt, a streaming load whose lines are not kept for reuse).
template <int kAux = 0>
__device__ __forceinline__ void dma16b(__amdgpu_buffer_rsrc_t rsrc, lds_void *lds, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds, 16, voff, soff, 0, kAux);
#else
  (void)rsrc; (void)lds; (void)voff; (void)soff;
#endif
}

// Instruction-group order spreading kReads LDS reads and kVmem vector-memory
// reads evenly behind kMfma MFMAs.
template <int kMfma, int kReads, int kVmem, int kR = 0>
__device__ __forceinline__ void sched_mix() {
  if constexpr (kR < kMfma) {
    constexpr int nr = kReads * (kR + 1) / kMfma - kReads * kR / kMfma;
    constexpr int nv = kVmem * (kR + 1) / kMfma - kVmem * kR / kMfma;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);
    if constexpr (nv > 0) __builtin_amdgcn_sched_group_barrier(0x020, nv, 0);
    sched_mix<kMfma, kReads, kVmem, kR + 1>();
  }
}

// Compute units of the current device (cached per device).
inline int num_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Tail list of the ping-pong kernels (workspace layout, ints): a group whose
// last 256-row tile would have 1 to 128 rows leaves that tile to the 128-row
// form of the kernel. tails_init_kernel lists those groups in order; after
// their 256-row tiles the persistent workgroups take (group, column tile)
// units u = 0, 1, ... of the list from the counter, unit u = list[u / ntiles],
// column tile u % ntiles.
constexpr int kTailCtr = 0;     // units handed out
constexpr int kTailCount = 32;  // groups in the list (own 128-byte line)
constexpr int kTailList = 64;   // the groups, ascending
#ifndef MOE_GEMM_TAILS_MIN_K
#define MOE_GEMM_TAILS_MIN_K 4096
#endif
constexpr int64_t kTailsMinK = MOE_GEMM_TAILS_MIN_K;  // shortest reduction that uses the 128-row tail tiles
inline size_t tails_bytes(int64_t G) { return sizeof(int) * static_cast<size_t>(kTailList + G); }
constexpr int kTailMaxRows = 128;  // longest tail of the list (the 128-row form's height)

__device__ __forceinline__ bool has_tail(int64_t m) {
  const int64_t r = m % 256;
  return r >= 1 && r <= kTailMaxRows;
}
// 256-row tiles of a group of m rows when its tail (if has_tail) is left to the list.
__device__ __forceinline__ int main_row_tiles(int m) { return (m + 255 - kTailMaxRows) / 256; }

namespace {

// One workgroup of 256 threads: each thread counts the tails of its chunk of
// groups, an exclusive scan over the threads gives the chunk's first list
// position, then each thread lists its chunk's tail groups. Group g is rows
// offsets[g] .. offsets[g + 1] - 1, clamped to [0, M].
__global__ __launch_bounds__(256) void tails_init_kernel(const int32_t *offsets, int64_t G, int64_t M, int *tails) {
  __shared__ int part[256];
  const int t = threadIdx.x;
  const int64_t per = (G + 255) / 256;
  const int64_t g0 = min(G, t * per), g1 = min(G, g0 + per);
  auto tail_at = [&](int64_t g) {
    const int64_t lo = min(max(static_cast<int64_t>(offsets[g]), int64_t(0)), M);
    const int64_t hi = min(max(static_cast<int64_t>(offsets[g + 1]), lo), M);
    return has_tail(hi - lo);
  };
  int n = 0;
  for (int64_t g = g0; g < g1; ++g) n += tail_at(g) ? 1 : 0;
  part[t] = n;
  __syncthreads();
  if (t == 0) {
    int acc = 0;
    for (int i = 0; i < 256; ++i) {
      const int v = part[i];
      part[i] = acc;
      acc += v;
    }
    tails[kTailCount] = acc;
    tails[kTailCtr] = 0;
  }
  __syncthreads();
  int pos = part[t];
  for (int64_t g = g0; g < g1; ++g) {
    if (tail_at(g)) tails[kTailList + pos++] = static_cast<int>(g);
  }
}

}  // namespace

}  // namespace gemm
}  // namespace moe
