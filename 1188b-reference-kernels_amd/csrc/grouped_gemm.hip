// Grouped GEMM forward over ragged expert groups, bf16 MFMA with fp32
// accumulate, optional SwiGLU epilogue.
//
// Math: kernel_cases/case03_moe_grouped_gemm_fc1_fwd.py:57-64 and
// kernel_cases/case04_moe_grouped_gemm_fc2_fwd.py:57-64:
//   out[rows of g] = a[rows of g] @ w[g]^T   ("bf16 in / fp32 accumulate /
//   bf16 out", case03...py:37), rows of g = group_offsets[g] .. [g+1]-1.
// SwiGLU (fused, no reference function): h = silu(y[:, :F]) * y[:, F:] on the
// fp32 accumulators, F = N / 2, rounded once to bf16.
//
// Kernel shape (gfx950):
//   * one persistent workgroup per CU; output tile 256 x 256, K step 64;
//   * A and B tiles stream through a two-stage LDS ring (2 x 2 x 256 x 64
//     bf16 = 128 KiB) filled by global_load_lds_dwordx4 (memory -> LDS without
//     VGPRs), one K step ahead of the MFMAs;
//   * LDS rows are XOR-swizzled in 16-byte chunks (chunk ^ (row / 2) % 8), which
//     makes both the DMA writes (lane-linear 1 KiB blocks) and the MFMA operand
//     reads (16 lanes x 16 B) bank-conflict-free;
//   * kWavesM x kWavesN wavefronts, each owning a 128 x (256 / kWavesN) part of
//     the tile as kMI x kNI blocks of v_mfma_f32_32x32x16_bf16; within a K step
//     the operand fragments of 16-wide sub-step s+1 are read from LDS between
//     the MFMAs of sub-step s (instruction-group scheduling);
//   * SwiGLU tiles load 128 gate rows and the matching 128 up rows of w; each
//     wave's N blocks are gate blocks followed by the up blocks of the same
//     output columns, so the epilogue combines them in registers;
//   * the epilogue rounds to bf16 into an LDS tile and writes 16-byte
//     row-contiguous non-temporal stores;
//   * tiles are numbered expert by expert, and inside an expert in groups of
//     4 row tiles x all column tiles (row tile fastest), so 32 consecutive
//     tile numbers form a 4 x 8 patch that shares A and B panels; workgroup b
//     takes tile round * P + (b % 8) * (P / 8) + b / 8, which hands each XCD
//     (workgroups are dealt round-robin to the 8 XCDs) one such patch per
//     round, so the panels are reused from that XCD's L2.
// Rows past a group's end and columns past N are loaded from a clamped (valid)
// address and their results are discarded; a K tail (K % 64 != 0) is zeroed in
// LDS before use.
#include <algorithm>

#include "moe_common.h"

#ifndef MOE_GEMM_WAVES_N
#define MOE_GEMM_WAVES_N 4
#endif

namespace moe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kWavesM = 2;
constexpr int kGroupM = 4;                        // row tiles per tile-order group
constexpr int kRowBytes = kBK * 2;                // 128: one tile row in LDS
constexpr int kChunks = kBK / 8;                  // 8 chunks of 16 bytes per row
constexpr int kOperandBytes = 256 * kRowBytes;    // 32 KiB: one 256-row operand tile
constexpr int kStageBytes = 2 * kOperandBytes;    // A + B
constexpr int kStages = 2;
constexpr int kRowsPerKiB = 1024 / kRowBytes;     // 8 rows per DMA instruction
constexpr int kSubSteps = kBK / 16;               // MFMA K sub-steps per K step

struct GemmArgs {
  const uint16_t *a;
  const uint16_t *w;
  const int32_t *offsets;
  uint16_t *out;
  int64_t M, K, N, G;
  int64_t ncols;   // output columns: N (NONE) or N / 2 (SWIGLU)
  int64_t ntiles;  // column tiles per expert
  int vec_out;     // output rows are 16-byte aligned (ncols % 8 == 0, aligned base)
};

__device__ __forceinline__ int swz(int row) { return (row >> 1) & (kChunks - 1); }

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

// Waits for this thread's outstanding DMA (vector memory) or LDS operations.
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

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// 16-byte global -> LDS copy (global_load_lds_dwordx4): lane i of the wave
// writes bytes [16 i, 16 i + 16) of the 1 KiB block at `lds` (wave-uniform).
// The builtin exists only for the device pass; the host pass only needs the
// kernel's launch stub.
__device__ __forceinline__ void dma16(const uint16_t *src, lds_void *lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
#else
  (void)src;
  (void)lds;
#endif
}

template <bool kSwiglu>
__device__ __forceinline__ int64_t b_row_clamped(int64_t nt, int r, int64_t ncols, int64_t N) {
  if constexpr (kSwiglu) {
    // rows 0..127: gate columns j0 .. j0+127; rows 128..255: up columns F + j0 ..
    const int64_t j = std::min<int64_t>(nt * (kBN / 2) + (r & 127), ncols - 1);
    return r < 128 ? j : ncols + j;
  } else {
    return std::min<int64_t>(nt * kBN + r, N - 1);
  }
}

template <bool kSwiglu, int kWavesN>
__global__ __launch_bounds__(kWavesM * kWavesN * 64) void grouped_gemm_kernel(GemmArgs p) {
  constexpr int kWaves = kWavesM * kWavesN;
  constexpr int kThreads = kWaves * 64;
  constexpr int kMI = (kBM / kWavesM) / 32;            // 32-row blocks per wave (4)
  constexpr int kNI = (kBN / kWavesN) / 32;            // 32-column blocks per wave (2 or 4)
  constexpr int kDma = kOperandBytes / 1024 / kWaves;  // DMA instructions per operand per stage
  constexpr int kEpiCols = kSwiglu ? kBN / 2 : kBN;    // output columns per tile
  constexpr int kEpiRow = kEpiCols * 2 + 16;           // padded epilogue LDS row (bytes)
  constexpr int kRingBytes = kStages * kStageBytes;
  constexpr int kLdsBytes = kRingBytes > kBM * kEpiRow ? kRingBytes : kBM * kEpiRow;
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
  lds_char *const sbase = (lds_char *)smem;  // address-space cast: LDS pointer arithmetic below

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / kWavesN;
  const int wn = wave % kWavesN;
  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t K = p.K;
  const int ktiles = static_cast<int>(ceil_div(K, kBK));

  // Row ranges are clamped to [0, M] and made non-decreasing, so inconsistent
  // offsets can never send a load or store outside a and out.
  auto group_rows = [&](int64_t g, int64_t &lo, int64_t &hi) {
    lo = min(max(static_cast<int64_t>(p.offsets[g]), int64_t(0)), p.M);
    hi = min(max(static_cast<int64_t>(p.offsets[g + 1]), lo), p.M);
  };
  int64_t g_cur = 0, tiles_before = 0, m_lo, m_hi;
  group_rows(0, m_lo, m_hi);
  int64_t mt_g = ceil_div(m_hi - m_lo, kBM);

  // DMA pattern: lane l fills 16 bytes of a lane-linear 1 KiB LDS block, i.e.
  // row l / 8 of the block's 8 rows, physical chunk l % 8.
  const int dma_row = lane / kChunks;
  const int dma_pchunk = lane % kChunks;

  // Fragment rows of this lane: byte offset of the row | (its swizzle << 4), so
  // that logical chunk c of the row sits at (base ^ (c << 4)).
  int fa_base[kMI], fb_base[kNI];
#pragma unroll
  for (int i = 0; i < kMI; ++i) {
    const int r = wm * (kBM / kWavesM) + i * 32 + (lane & 31);
    fa_base[i] = r * kRowBytes | (swz(r) << 4);
  }
#pragma unroll
  for (int j = 0; j < kNI; ++j) {
    int r;
    if constexpr (kSwiglu) {
      // gate blocks j < kNI/2, then the up blocks of the same output columns
      const int jj = j % (kNI / 2);
      r = (j < kNI / 2 ? 0 : 128) + wn * (128 / kWavesN) + jj * 32 + (lane & 31);
    } else {
      r = wn * (kBN / kWavesN) + j * 32 + (lane & 31);
    }
    fb_base[j] = r * kRowBytes | (swz(r) << 4);
  }
  const int khalf = lane >> 5;

  for (int64_t round = 0;; ++round) {
    const int64_t L = round * P + (b % 8) * (P / 8) + b / 8;
    while (g_cur < p.G && L >= tiles_before + mt_g * p.ntiles) {
      tiles_before += mt_g * p.ntiles;
      ++g_cur;
      if (g_cur < p.G) {
        group_rows(g_cur, m_lo, m_hi);
        mt_g = ceil_div(m_hi - m_lo, kBM);
      }
    }
    if (g_cur >= p.G) break;

    const int64_t q = L - tiles_before;
    const int64_t full = mt_g / kGroupM;
    int64_t mt, nt;
    if (q < full * kGroupM * p.ntiles) {
      const int64_t grp = q / (kGroupM * p.ntiles), r = q % (kGroupM * p.ntiles);
      nt = r / kGroupM;
      mt = grp * kGroupM + r % kGroupM;
    } else {
      const int64_t r = q - full * kGroupM * p.ntiles, gm = mt_g - full * kGroupM;
      nt = r / gm;
      mt = full * kGroupM + r % gm;
    }
    const int64_t row0 = m_lo + mt * kBM;
    const uint16_t *wg = p.w + g_cur * p.N * K;

    // Global source rows of this thread's DMA instructions (clamped, so always
    // valid) and their logical chunk.
    const uint16_t *a_src[kDma];
    const uint16_t *b_src[kDma];
    int dma_chunk[kDma];
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      const int blk = j * kWaves + wave;
      const int r = blk * kRowsPerKiB + dma_row;
      dma_chunk[j] = dma_pchunk ^ swz(r);
      a_src[j] = p.a + std::min<int64_t>(row0 + r, m_hi - 1) * K;
      b_src[j] = wg + b_row_clamped<kSwiglu>(nt, r, p.ncols, p.N) * K;
    }
    auto issue_stage = [&](int kt) {
      lds_char *st = sbase + (kt % kStages) * kStageBytes;
#pragma unroll
      for (int j = 0; j < kDma; ++j) {
        const int blk = j * kWaves + wave;
        // A chunk in the K tail reads the row's last valid chunk instead (zeroed before use).
        const int64_t k = std::min<int64_t>(static_cast<int64_t>(kt) * kBK + dma_chunk[j] * 8, K - 8);
        dma16(a_src[j] + k, reinterpret_cast<lds_void *>(st + blk * 1024));
        dma16(b_src[j] + k, reinterpret_cast<lds_void *>(st + kOperandBytes + blk * 1024));
      }
    };

    f32x16 acc[kMI][kNI];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < kNI; ++j) acc[i][j] = f32x16{};

    barrier();  // the previous tile's epilogue is done with the LDS
    issue_stage(0);

    for (int kt = 0; kt < ktiles; ++kt) {
      wait_dma();  // this thread's DMA of stage kt has landed
      barrier();   // ... and everyone's; stage kt-1's buffer is free
      lds_char *st = sbase + (kt % kStages) * kStageBytes;
      if (K % kBK != 0 && kt == ktiles - 1) {
        // Zero the chunks of the K tail.
        const int kvalid = static_cast<int>(K - static_cast<int64_t>(kt) * kBK);
        for (int idx = tid; idx < 2 * kBM * kChunks; idx += kThreads) {
          const int op = idx / (kBM * kChunks), rem = idx % (kBM * kChunks);
          const int r = rem / kChunks, c = rem % kChunks;
          if (c * 8 >= kvalid) {
            *reinterpret_cast<lds_u32x4 *>(st + op * kOperandBytes + r * kRowBytes + ((c ^ swz(r)) * 16)) =
                u32x4{0u, 0u, 0u, 0u};
          }
        }
        wait_lds();
        barrier();
      }
      if (kt + 1 < ktiles) issue_stage(kt + 1);

      const lds_char *sa = st;
      const lds_char *sb = st + kOperandBytes;
      bf16x8 fa[2][kMI], fb[2][kNI];
      auto load_frags = [&](int ks, int buf) {
        const int c = ks * 2 + khalf;
#pragma unroll
        for (int i = 0; i < kMI; ++i) fa[buf][i] = *reinterpret_cast<const lds_bf16x8 *>(sa + (fa_base[i] ^ (c << 4)));
#pragma unroll
        for (int j = 0; j < kNI; ++j) fb[buf][j] = *reinterpret_cast<const lds_bf16x8 *>(sb + (fb_base[j] ^ (c << 4)));
      };
      load_frags(0, 0);
#pragma unroll
      for (int ks = 0; ks < kSubSteps; ++ks) {
        if (ks + 1 < kSubSteps) load_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
        for (int i = 0; i < kMI; ++i)
#pragma unroll
          for (int j = 0; j < kNI; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ks & 1][i], fb[ks & 1][j], acc[i][j], 0, 0, 0);
      }
      // Instruction groups for the unrolled K step: the reads of sub-step 0,
      // then for each sub-step one MFMA after each read of the next sub-step.
      __builtin_amdgcn_sched_group_barrier(0x100, kMI + kNI, 0);
#pragma unroll
      for (int ks = 0; ks + 1 < kSubSteps; ++ks) {
#pragma unroll
        for (int r = 0; r < kMI + kNI; ++r) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kMI * kNI - (kMI + kNI), 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kMI * kNI, 0);
    }

    // Epilogue: bf16 tile into LDS (accumulator register r of lane l in a 32x32
    // block holds row (r / 4) * 8 + (l / 32) * 4 + (r % 4), column l % 32), then
    // 16-byte row-contiguous stores.
    barrier();  // every wave is done reading the last stage
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm * (kBM / kWavesM) + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if constexpr (kSwiglu) {
#pragma unroll
          for (int j = 0; j < kNI / 2; ++j) {
            const int col = wn * (128 / kWavesN) + j * 32 + (lane & 31);
            const float h = silu(acc[i][j][r]) * acc[i][j + kNI / 2][r];
            *reinterpret_cast<lds_u16 *>(sbase + row * kEpiRow + col * 2) = static_cast<uint16_t>(f32_to_bf16_rne(h));
          }
        } else {
#pragma unroll
          for (int j = 0; j < kNI; ++j) {
            const int col = wn * (kBN / kWavesN) + j * 32 + (lane & 31);
            *reinterpret_cast<lds_u16 *>(sbase + row * kEpiRow + col * 2) =
                static_cast<uint16_t>(f32_to_bf16_rne(acc[i][j][r]));
          }
        }
      }
    }
    wait_lds();  // this wave's LDS writes are done
    barrier();
    const int64_t col0 = nt * kEpiCols;
    constexpr int kChunksPerRow = kEpiCols / 8;
#pragma unroll 4
    for (int idx = tid; idx < kBM * kChunksPerRow; idx += kThreads) {
      const int r = idx / kChunksPerRow, c = idx % kChunksPerRow;
      const int64_t grow = row0 + r;
      const int64_t gcol = col0 + c * 8;
      if (grow >= m_hi || gcol >= p.ncols) continue;
      const lds_char *src = sbase + r * kEpiRow + c * 16;
      uint16_t *dst = p.out + grow * p.ncols + gcol;
      if (p.vec_out && gcol + 8 <= p.ncols) {
        __builtin_nontemporal_store(*reinterpret_cast<const lds_u32x4 *>(src), reinterpret_cast<u32x4 *>(dst));
      } else {
        for (int e = 0; e < 8 && gcol + e < p.ncols; ++e) dst[e] = *reinterpret_cast<const lds_u16 *>(src + 2 * e);
      }
    }
  }
}

int g_num_cus[64] = {0};

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (g_num_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_num_cus[dev] = n;
  }
  return g_num_cus[dev];
}

}  // namespace
}  // namespace moe

extern "C" {

int moe_grouped_gemm(const moe_bf16_t *a, int64_t M_total, int64_t K, const moe_bf16_t *w, int64_t G,
                     int64_t N, const int32_t *group_offsets, int epilogue, moe_bf16_t *out,
                     void *workspace, size_t workspace_bytes, void *stream) {
  using namespace moe;
  (void)workspace;
  (void)workspace_bytes;
  if (M_total < 0 || K < 0 || N < 0 || G < 0) {
    return fail(MOE_ERR_SHAPE, "moe_grouped_gemm: negative size (M=%lld K=%lld N=%lld G=%lld)",
                (long long)M_total, (long long)K, (long long)N, (long long)G);
  }
  if (epilogue != MOE_EPILOGUE_NONE && epilogue != MOE_EPILOGUE_SWIGLU) {
    return fail(MOE_ERR_INVALID_ARG, "moe_grouped_gemm: epilogue %d is not a moe_epilogue_t", epilogue);
  }
  if (G < 1 || G > 4096) return fail(MOE_ERR_CAPACITY, "moe_grouped_gemm: G=%lld outside [1, 4096]", (long long)G);
  if (K % 8 != 0 || K == 0) return fail(MOE_ERR_SHAPE, "moe_grouped_gemm: K=%lld must be a positive multiple of 8", (long long)K);
  const bool swiglu = epilogue == MOE_EPILOGUE_SWIGLU;
  if (swiglu && (N % 2 != 0)) return fail(MOE_ERR_SHAPE, "moe_grouped_gemm: SWIGLU needs an even N (got %lld)", (long long)N);
  if (group_offsets == nullptr) return fail(MOE_ERR_INVALID_ARG, "moe_grouped_gemm: null group_offsets");
  const int64_t ncols = swiglu ? N / 2 : N;
  if (M_total == 0 || ncols == 0) return MOE_OK;
  if (a == nullptr || w == nullptr || out == nullptr) {
    return fail(MOE_ERR_INVALID_ARG, "moe_grouped_gemm: null a, w or out");
  }
  if (!is_aligned(a, 16) || !is_aligned(w, 16)) {
    return fail(MOE_ERR_ALIGN, "moe_grouped_gemm: a and w must be 16-byte aligned");
  }
  GemmArgs p;
  p.a = a;
  p.w = w;
  p.offsets = group_offsets;
  p.out = out;
  p.M = M_total;
  p.K = K;
  p.N = N;
  p.G = G;
  p.ncols = ncols;
  p.ntiles = swiglu ? ceil_div(ncols, kBN / 2) : ceil_div(N, kBN);
  p.vec_out = (ncols % 8 == 0) && is_aligned(out, 16);
  // Persistent grid: one workgroup per CU, a multiple of the 8 XCDs, no more
  // than an upper bound on the tile count.
  const int64_t max_tiles = (ceil_div(M_total, kBM) + G) * p.ntiles;
  int64_t grid = std::min<int64_t>(num_cus(), max_tiles);
  grid = std::max<int64_t>(8, (grid + 7) / 8 * 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr int kWN = MOE_GEMM_WAVES_N;
  constexpr int kThreads = kWavesM * kWN * 64;
  if (swiglu) grouped_gemm_kernel<true, kWN><<<dim3(grid), dim3(kThreads), 0, s>>>(p);
  else grouped_gemm_kernel<false, kWN><<<dim3(grid), dim3(kThreads), 0, s>>>(p);
  return check_launch("moe_grouped_gemm");
}

}  // extern "C"
