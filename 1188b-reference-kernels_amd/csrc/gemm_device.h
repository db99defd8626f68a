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
__device__ __forceinline__ void dma16b(__amdgpu_buffer_rsrc_t rsrc, lds_void *lds, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds, 16, voff, soff, 0, 0);
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

}  // namespace gemm
}  // namespace moe
