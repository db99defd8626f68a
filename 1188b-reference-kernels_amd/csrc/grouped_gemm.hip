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
// Three kernels: grouped_gemm_pp_kernel (last; two wavefronts per SIMD, for
// K % 64 == 0 and K >= 192 with 16-byte output rows, i.e. every MoE shape, with
// an optional 128-row form for group tails), grouped_gemm_pipe_kernel (one
// wavefront per SIMD; the same shapes with a K tail) and grouped_gemm_kernel,
// the drained form for the rest (K <= 128, unaligned outputs). They are
// bit-identical on the shapes they share. Shared shape (gfx950), as the
// drained kernel has it:
//   * one persistent workgroup of 4 wavefronts (one per SIMD) per CU; output
//     tile 256 x 256, K step 64; each wavefront owns 128 x 128 of the tile as
//     4 x 4 blocks of v_mfma_f32_32x32x16_bf16 (256 accumulator registers);
//   * A and B tiles stream through a two-stage LDS ring (2 x 2 x 256 x 64 bf16
//     = 128 KiB) filled by buffer_load_dwordx4 ... lds (memory -> LDS without
//     VGPRs; buffer resources bound each load to the valid rows), one K step
//     ahead of the MFMAs;
//   * LDS rows are XOR-swizzled in 16-byte chunks (chunk ^ (row / 2) % 8), which
//     makes both the DMA writes (lane-linear 1 KiB blocks) and the MFMA operand
//     reads (16 lanes x 16 B) bank-conflict-free;
//   * operand fragments in two register sets of one MFMA sub-step (K 16)
//     each: while the MFMAs of one set run, the other set's next sub-step is
//     read from LDS; one workgroup barrier per K step, after its second
//     sub-step, then the DMA of step kt + 2 goes out under the MFMAs of
//     sub-steps 2 and 3 (instruction-group scheduling);
//   * w is the MFMA's first operand, so the accumulators hold the transposed
//     block and each lane owns 4 consecutive output columns per 4 registers:
//     the epilogue rounds them to bf16 in hardware (RNE) and writes 8-byte
//     words into an LDS tile, then 16-byte row-contiguous non-temporal stores;
//   * SwiGLU tiles load 128 gate rows and the matching 128 up rows of w; each
//     wave's N blocks are gate blocks followed by the up blocks of the same
//     output columns, so the epilogue combines them in registers
//     (silu(g) = g / (1 + 2^(-g log2 e)) with the hardware exp2 and reciprocal);
//   * tiles are numbered expert by expert, and inside an expert in groups of
//     8 row tiles x all column tiles (row tile fastest), so 32 consecutive
//     tile numbers form an 8 x 4 patch that shares A and B panels; workgroup b
//     takes tile round * P + (b % 8) * (P / 8) + b / 8, which hands each XCD
//     (workgroups are dealt round-robin to the 8 XCDs) one such patch per
//     round, so the panels are reused from that XCD's L2.
// Rows past a group's end read as zeros in the pipelined kernel (from a clamped
// valid row in the drained one), columns past N are loaded from a clamped
// (valid) row, and their results are discarded; a K tail (K % 64 != 0) is zeroed in LDS
// before use. Buffer offsets are 32-bit and an out-of-range sentinel sits at
// 2^31: the host requires 512 K, 2 N K (and for the gather 2 x_rows K) bytes to
// stay below 2^31.
//
// Gather variant (moe_grouped_gemm_gather): A row p is x[a_rows[p]]; each
// lane's DMA offset is that source row's, so the permuted A operand of fc1 is
// read straight from the token rows and never materialised.
#include <algorithm>
#include <type_traits>

#include "gemm_device.h"

namespace moe {
namespace {

using namespace gemm;

constexpr int kBM = 256, kBN = 256;
#ifndef MOE_GEMM_GROUP_M
#define MOE_GEMM_GROUP_M 8
#endif
constexpr int kGroupM = MOE_GEMM_GROUP_M;         // row tiles per tile-order group
#ifndef MOE_GEMM_FWD128
#define MOE_GEMM_FWD128 1
#endif
#ifndef MOE_GEMM_FWD128_NB
#define MOE_GEMM_FWD128_NB 0  // column tile width / 32 of the 128-row forward kernel (0: the host picks it)
#endif
#ifndef MOE_GEMM_FWD128_SA
#define MOE_GEMM_FWD128_SA 0  // ring stages of the 128-row forward kernel: A (0: 5, 4 from 192 columns),
#endif
#ifndef MOE_GEMM_FWD128_SB
#define MOE_GEMM_FWD128_SB 0  // B (0: 4, fewer where the LDS holds no more)
#endif
#ifndef MOE_GEMM_FWD128_NT
#define MOE_GEMM_FWD128_NT 1  // the 128-row forward kernel loads the weights non-temporally (each is used by one tile)
#endif
#ifndef MOE_GEMM_PINGPONG
#define MOE_GEMM_PINGPONG 1
#endif
constexpr int kRowBytes = kBK * 2;                // 128: one tile row in LDS
constexpr int kChunks = kBK / 8;                  // 8 chunks of 16 bytes per row
constexpr int kOperandBytes = 256 * kRowBytes;    // 32 KiB: one 256-row operand tile
constexpr int kStageBytes = 2 * kOperandBytes;    // A + B
constexpr int kStages = 2;
constexpr int kRowsPerKiB = 1024 / kRowBytes;     // 8 rows per DMA instruction

struct GemmArgs {
  const uint16_t *a;       // A rows, or the gather source x [a_src_rows, K]
  const int32_t *a_rows;   // gather: A row p = a[a_rows[p]] (nullptr: A row p = a[p])
  int64_t a_src_rows;      // gather: rows of x
  const uint16_t *w;
  const int32_t *offsets;
  uint16_t *out;
  int64_t M, K, N, G;
  int64_t ncols;   // output columns: N (NONE) or N / 2 (SWIGLU)
  int64_t ntiles;  // column tiles per expert
  int vec_out;     // output rows are 16-byte aligned (ncols % 8 == 0, aligned base)
  int *tails;      // ping-pong kernel: tail list (kTail* layout) or nullptr (tails in 256-row tiles)
  // Reduction split of the last tiles (ping-pong kernel, 0: none): the last split_tiles tiles of the
  // static order are left to grouped_gemm_split_kernel, which computes each as split_ways ranges of
  // split_steps K steps (the last range takes the rest) into fp32 planes of 256 x 256 (planes), and
  // split_sum_kernel adds each tile's planes in range order and rounds once.
  int split_tiles, split_ways, split_steps;
  float *planes;
};

constexpr int kPpLdsBytes = 5 * 256 * 128;  // ping-pong kernel LDS: 160 KiB

__device__ __forceinline__ int swz(int row) { return (row >> 1) & (kChunks - 1); }

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


// Four wavefronts (one per SIMD), each 128 x 128 of the 256 x 256 tile as 4 x 4
// blocks of 32 x 32. Fragments of two MFMA sub-steps (K 16 each) live in VGPRs.
// One barrier per step, after its second sub-step, publishes stage kt + 1 (its
// DMA has landed) and frees the LDS slot of stage kt for the DMA of stage kt + 2.
template <bool kSwiglu, bool kGather>
__global__ __launch_bounds__(256) void grouped_gemm_kernel(GemmArgs p) {
  constexpr int kWaves = 4;
  constexpr int kThreads = 256;
  constexpr int kMI = 4, kNI = 4;
  constexpr int kDma = kOperandBytes / 1024 / kWaves;  // 8 DMA instructions per operand per stage
  constexpr int kEpiCols = kSwiglu ? kBN / 2 : kBN;
  constexpr int kEpiRow = kEpiCols * 2 + 16;
  constexpr int kRingBytes = kStages * kStageBytes;
  constexpr int kLdsBytes = kRingBytes > kBM * kEpiRow ? kRingBytes : kBM * kEpiRow;
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t K = p.K;
  const int ktiles = static_cast<int>(ceil_div(K, kBK));
  const bool ktail = (K % kBK) != 0;

  auto group_rows = [&](int64_t g, int64_t &lo, int64_t &hi) {
    lo = min(max(static_cast<int64_t>(ld_inv(p.offsets, g)), int64_t(0)), p.M);
    hi = min(max(static_cast<int64_t>(ld_inv(p.offsets, g + 1)), lo), p.M);
  };
  int64_t g_cur = 0, tiles_before = 0, m_lo, m_hi;
  group_rows(0, m_lo, m_hi);
  int64_t mt_g = ceil_div(m_hi - m_lo, kBM);


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
    // Per-lane values from an opaque copy of the lane index, recomputed per
    // tile rather than hoisted out of the tile loop (where they would stay
    // live across the K loop and spill).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    // Fragment rows 32 apart share the swizzle ((row / 2) % 8 changes by 16), so
    // block i (j) of a wave lies at its first block's address + i (j) x 32 rows
    // (an immediate ds_read offset): one address register per operand. SwiGLU
    // tiles: B blocks 0, 1 are gate rows wn 64 .., blocks 2, 3 the up rows 128 further.
    const int fra = wm * 128 + (ln & 31);
    const int frb = (kSwiglu ? wn * 64 : wn * 128) + (ln & 31);
    const uint32_t fa0 = fra * kRowBytes | (swz(fra) << 4);
    const uint32_t fb0 = frb * kRowBytes | (swz(frb) << 4);
    auto b_blk_rows = [](int j) { return kSwiglu ? (j / (kNI / 2)) * 128 + (j % (kNI / 2)) * 32 : j * 32; };
    const int khalf = ln >> 5;

    // Position inside the group (32-bit: a group's tile count exceeds 2^32 only
    // for outputs of more than 2^48 elements).
    const uint32_t q = static_cast<uint32_t>(L - tiles_before);
    const uint32_t ntl = static_cast<uint32_t>(p.ntiles);
    const uint32_t per_grp = kGroupM * ntl;
    const uint32_t full = static_cast<uint32_t>(mt_g) / kGroupM;
    uint32_t mt, nt;
    if (q < full * per_grp) {
      const uint32_t grp = q / per_grp, r = q - grp * per_grp;
      nt = r / kGroupM;
      mt = grp * kGroupM + r % kGroupM;
    } else {
      const uint32_t r = q - full * per_grp, gm = static_cast<uint32_t>(mt_g) - full * kGroupM;
      nt = r / gm;
      mt = full * kGroupM + (r - nt * gm);
    }
    const int64_t row0 = m_lo + mt * kBM;
    const int rows_valid = static_cast<int>(min(m_hi - row0, int64_t(kBM)));
    const uint16_t *wg = p.w + g_cur * p.N * K;

    // Buffer resources: A over this tile's valid rows (gather: over all of x),
    // B over this expert's matrix.
    const __amdgpu_buffer_rsrc_t ra =
        kGather ? make_rsrc(p.a, static_cast<uint32_t>(p.a_src_rows * K * 2))
                : make_rsrc(p.a + row0 * K, static_cast<uint32_t>(rows_valid * K * 2));
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(wg, static_cast<uint32_t>(p.N * K * 2));
    int a_off[kDma], b_off[kDma];
    const int dma_row = ln / kChunks;
    const int dma_pchunk = ln % kChunks;
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      const int blk = j * kWaves + wave;
      const int r = blk * kRowsPerKiB + dma_row;
      const int lchunk = dma_pchunk ^ swz(r);
      const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;
      if constexpr (kGather) {
        // Source row of x; an index outside x points past the resource (zeros).
        const int32_t src = p.a_rows[row0 + min(r, rows_valid - 1)];
        a_off[j] = (src >= 0 && src < p.a_src_rows)
                       ? static_cast<int>(static_cast<uint32_t>(src) * row_bytes + lchunk * 16)
                       : static_cast<int>(0x80000000u);
      } else {
        a_off[j] = static_cast<int>(static_cast<uint32_t>(min(r, rows_valid - 1)) * row_bytes + lchunk * 16);
      }
      b_off[j] = static_cast<int>(static_cast<uint32_t>(b_row_clamped<kSwiglu>(nt, r, p.ncols, p.N)) * row_bytes +
                                  lchunk * 16);
    }
    // Stage kt into LDS slot kt % 2. Chunks past K read the next row (or zeros
    // past the resource) and are zeroed in LDS before use.
    auto issue_stage = [&](int kt) {
      const uint32_t st = lds_base + (kt % kStages) * kStageBytes;
      const int soff = kt * kBK * 2;
#pragma unroll
      for (int j = 0; j < kDma; ++j) {
        const uint32_t blk = j * kWaves + wave;
        dma16b(ra, (lds_void *)(uintptr_t)(st + blk * 1024), a_off[j], soff);
        dma16b(rb, (lds_void *)(uintptr_t)(st + kOperandBytes + blk * 1024), b_off[j], soff);
      }
    };
    // Half of stage `kt` (operand `op`) into LDS slot `slot`.
    auto issue_half = [&](int kt, int slot, int op) {
      const uint32_t st = lds_base + (slot % kStages) * kStageBytes + op * kOperandBytes;
      const int soff = kt * kBK * 2;
#pragma unroll
      for (int j = 0; j < kDma; ++j) {
        const uint32_t blk = j * kWaves + wave;
        dma16b(op ? rb : ra, (lds_void *)(uintptr_t)(st + blk * 1024), op ? b_off[j] : a_off[j], soff);
      }
    };
    auto zero_ktail = [&](int kt) {
      lds_char *st = sbase + (kt % kStages) * kStageBytes;
      const int kvalid = static_cast<int>(K - static_cast<int64_t>(kt) * kBK);
      for (int idx = tid; idx < 2 * kBM * kChunks; idx += kThreads) {
        const int op = idx / (kBM * kChunks), rem = idx % (kBM * kChunks);
        const int r = rem / kChunks, c = rem % kChunks;
        if (c * 8 >= kvalid) {
          *reinterpret_cast<lds_u32x4 *>(st + op * kOperandBytes + r * kRowBytes + ((c ^ swz(r)) * 16)) =
              u32x4{0u, 0u, 0u, 0u};
        }
      }
    };

    f32x16 acc[kMI][kNI];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < kNI; ++j) acc[i][j] = f32x16{};

    // LDS byte addresses of this lane's fragment rows in the slot read next
    // (logical chunk khalf); sub-step ks reads chunk 2 ks + khalf = addr ^ (ks << 5).
    uint32_t rd_a = 0, rd_b = 0;
    auto set_read_slot = [&](int kt) {
      const uint32_t so = lds_base + (kt % kStages) * kStageBytes;
      rd_a = so + (fa0 ^ (khalf << 4));
      rd_b = so + kOperandBytes + (fb0 ^ (khalf << 4));
    };
    // Two register sets of fragments: sub-steps 0 and 2 of a stage use set 0,
    // 1 and 3 set 1.
    bf16x8 fa[2][kMI], fb[2][kNI];
    auto read_frags = [&](int ks) {
#pragma unroll
      for (int i = 0; i < kMI; ++i)
        fa[ks & 1][i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)((rd_a ^ (ks << 5)) + i * 32 * kRowBytes));
#pragma unroll
      for (int j = 0; j < kNI; ++j)
        fb[ks & 1][j] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)((rd_b ^ (ks << 5)) + b_blk_rows(j) * kRowBytes));
    };
    auto mfma_set = [&](int set) {
#pragma unroll
      for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int j = 0; j < kNI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[set][j], fa[set][i], acc[i][j], 0, 0, 0);
    };
    // Prologue: stages 0 and 1 in flight; sub-steps 0 and 1 of stage 0 read into VGPRs.
    barrier();  // the previous tile's epilogue is done with the LDS
    issue_stage(0);
    if (ktiles > 1) {
      issue_stage(1);
      wait_vm_n<2 * kDma>();
    } else {
      wait_dma();
    }
    barrier();
    if (ktail && ktiles == 1) {
      zero_ktail(0);
      wait_lds();
      barrier();
    }
    set_read_slot(0);
    read_frags(0);
    read_frags(1);

    // Step kt: sub-steps 0 and 1 of stage kt while its sub-steps 2 and 3 are
    // read; one barrier (stage kt + 1 has landed, every wave is done reading
    // stage kt); sub-steps 2 and 3 while the DMA of stage kt + 2 is issued into
    // the slot of stage kt and sub-steps 0 and 1 of stage kt + 1 are read.
    for (int kt = 0; kt + 1 < ktiles; ++kt) {
      mfma_set(0);
      read_frags(2);
      sched_mix<kMI * kNI, kMI + kNI, 0>();
      mfma_set(1);
      read_frags(3);
      sched_mix<kMI * kNI, kMI + kNI, 0>();
      __builtin_amdgcn_sched_barrier(0);
      wait_dma();
      wait_lds();
      barrier();
      if (ktail && kt + 1 == ktiles - 1) {
        zero_ktail(kt + 1);
        wait_lds();
        barrier();
      }
      // Stage kt + 2 into the slot of stage kt (the last step re-reads the
      // final stage into that free slot, so the region below has no branch).
      const int kdma = min(kt + 2, ktiles - 1);
      mfma_set(0);
      issue_half(kdma, kt + 2, 0);
      set_read_slot(kt + 1);
      read_frags(0);
      sched_mix<kMI * kNI, kMI + kNI, kDma>();
      mfma_set(1);
      issue_half(kdma, kt + 2, 1);
      read_frags(1);
      sched_mix<kMI * kNI, kMI + kNI, kDma>();
      __builtin_amdgcn_sched_barrier(0);
    }
    mfma_set(0);
    read_frags(2);
    mfma_set(1);
    read_frags(3);
    mfma_set(0);
    mfma_set(1);
    wait_dma();  // the re-reads of the last steps have landed before the LDS is reused

    barrier();  // every wave is done reading the last stage
    // With w as the MFMA's first operand, register r of lane l in block (i, j)
    // holds output row i * 32 + l % 32 and column j * 32 + (r / 4) * 8 + (l / 32) * 4
    // + r % 4 of this wave's part: 4 consecutive columns per 4 registers, which
    // are rounded (RNE, hardware) and written to the LDS tile as one 8-byte word.
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
      const int row = wm * 128 + i * 32 + (ln & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if constexpr (kSwiglu) {
#pragma unroll
          for (int j = 0; j < kNI / 2; ++j) {
            const int col = wn * 64 + j * 32 + g * 8 + (ln >> 5) * 4;
            float h[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float gt = acc[i][j][4 * g + q];
              h[q] = gt * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gt * -1.4426950408889634f)) *
                     acc[i][j + kNI / 2][4 * g + q];
            }
            const bf16x4 v = {(__bf16)h[0], (__bf16)h[1], (__bf16)h[2], (__bf16)h[3]};
            *reinterpret_cast<lds_bf16x4 *>(sbase + row * kEpiRow + col * 2) = v;
          }
        } else {
#pragma unroll
          for (int j = 0; j < kNI; ++j) {
            const int col = wn * 128 + j * 32 + g * 8 + (ln >> 5) * 4;
            const bf16x4 v = {(__bf16)acc[i][j][4 * g], (__bf16)acc[i][j][4 * g + 1], (__bf16)acc[i][j][4 * g + 2],
                              (__bf16)acc[i][j][4 * g + 3]};
            *reinterpret_cast<lds_bf16x4 *>(sbase + row * kEpiRow + col * 2) = v;
          }
        }
      }
    }
    wait_lds();
    barrier();
    // 32-bit row and column arithmetic (ncols < 2^27: the host bounds N K
    // below 2^30) from an opaque copy of the thread index.
    int tq = tid;
    asm volatile("" : "+v"(tq));
    const int ncols32 = static_cast<int>(p.ncols);
    const int col0 = static_cast<int>(nt) * kEpiCols;
    uint16_t *const obase = p.out + row0 * p.ncols;
    constexpr int kChunksPerRow = kEpiCols / 8;
#pragma unroll 4
    for (int idx = tq; idx < kBM * kChunksPerRow; idx += kThreads) {
      const int r = idx / kChunksPerRow, c = idx % kChunksPerRow;
      const int gcol = col0 + c * 8;
      if (r >= rows_valid || gcol >= ncols32) continue;
      const lds_char *src = sbase + r * kEpiRow + c * 16;
      uint16_t *dst = obase + static_cast<int64_t>(r) * p.ncols + gcol;
      if (p.vec_out && gcol + 8 <= ncols32) {
        __builtin_nontemporal_store(*reinterpret_cast<const lds_u32x4 *>(src), reinterpret_cast<u32x4 *>(dst));
      } else {
        for (int e = 0; e < 8 && gcol + e < ncols32; ++e) dst[e] = *reinterpret_cast<const lds_u16 *>(src + 2 * e);
      }
    }
  }
}

// Pipelined kernel (K > 128, 16-byte output rows): the one the host runs for
// the MoE shapes. Same tile and ring as the kernel above, two differences:
//   * v_mfma_f32_16x16x32_bf16 blocks (8 x 8 of 16 x 16 per wave): half the
//     accumulator traffic per FLOP of the 32 x 32 x 16 form; the board holds
//     a higher shader clock under it (about 1.9 GHz against 1.6 GHz for the
//     32 x 32 form of the same loop at c5), which is what bounds a dense bf16
//     GEMM of this size;
//   * consecutive tiles of a workgroup follow each other without draining the
//     pipeline: the last K step of a tile DMAs the next tile's stage 0 and the
//     step after it (whose MFMAs finish the tile) reads that stage's
//     fragments and DMAs stage 1, like an inner step; the epilogue works on
//     registers only (bf16 RNE in hardware, v_permlane16_swap so a lane holds
//     8 consecutive columns, one 16-byte buffer store; rows past the group end
//     lie past the store resource and are dropped), issued after the next
//     tile's stage DMAs so the next waits leave the stores in flight
//     (vector-memory operations complete in issue order); the first MFMAs of
//     a tile take a zero accumulator operand; the tile after next is found
//     during the epilogue from group offsets staged in LDS, and (gather) its
//     source rows are loaded during the next tile's first step, long before
//     its DMA offsets are formed.
// One K step per wave: 4 units of 32 MFMAs (K half x row-block half); the
// fragments of the next stage are read into the registers each unit frees
// (4, 12 and 12 ds_read_b128 under units 2-4, the last unit running column by
// column so B fragments free up during it; 4 after it), the 16 DMA
// instructions of the stage two ahead are spread over units 2 and 3.
template <bool kSwiglu, bool kGather>
__global__ __launch_bounds__(256) void grouped_gemm_pipe_kernel(GemmArgs p) {
  constexpr int kWaves = 4;
  constexpr int kThreads = 256;
  constexpr int kDma = kOperandBytes / 1024 / kWaves;  // 8 DMA instructions per operand per stage
  constexpr int kEpiCols = kSwiglu ? kBN / 2 : kBN;    // output columns of a tile
  constexpr int kStores = kSwiglu ? 16 : 32;           // 16-byte stores per lane per tile
  constexpr int kMaxG = 4096;
  static_assert(kStores <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[kStages * kStageBytes];
  __shared__ int32_t s_offs[kMaxG + 1];
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t K = p.K;
  const int ktiles = static_cast<int>(ceil_div(K, kBK));  // >= 3 (host)
  const bool ktail = (K % kBK) != 0;

  for (int64_t i = tid; i <= p.G; i += kThreads) s_offs[i] = p.offsets[i];
  __syncthreads();

  // ---- tile walker (group offsets from LDS)
  auto group_rows = [&](int64_t g, int64_t &lo, int64_t &hi) {
    lo = min(max(static_cast<int64_t>(s_offs[g]), int64_t(0)), p.M);
    hi = min(max(static_cast<int64_t>(s_offs[g + 1]), lo), p.M);
  };
  int64_t g_cur = 0, tiles_before = 0, m_lo, m_hi;
  group_rows(0, m_lo, m_hi);
  int64_t mt_g = ceil_div(m_hi - m_lo, kBM);
  struct Tile {
    int64_t g, row0;
    uint32_t nt;
    int rows_valid;
  };
  auto find_tile = [&](int64_t round, Tile &t) -> bool {
    const int64_t L = round * P + (b % 8) * (P / 8) + b / 8;
    while (g_cur < p.G && L >= tiles_before + mt_g * p.ntiles) {
      tiles_before += mt_g * p.ntiles;
      ++g_cur;
      if (g_cur < p.G) {
        group_rows(g_cur, m_lo, m_hi);
        mt_g = ceil_div(m_hi - m_lo, kBM);
      }
    }
    if (g_cur >= p.G) return false;
    const uint32_t q = static_cast<uint32_t>(L - tiles_before);
    const uint32_t ntl = static_cast<uint32_t>(p.ntiles);
    const uint32_t per_grp = kGroupM * ntl;
    const uint32_t full = static_cast<uint32_t>(mt_g) / kGroupM;
    uint32_t mt, nt;
    if (q < full * per_grp) {
      const uint32_t grp = q / per_grp, r = q - grp * per_grp;
      nt = r / kGroupM;
      mt = grp * kGroupM + r % kGroupM;
    } else {
      const uint32_t r = q - full * per_grp, gm = static_cast<uint32_t>(mt_g) - full * kGroupM;
      nt = r / gm;
      mt = full * kGroupM + (r - nt * gm);
    }
    t.g = g_cur;
    t.row0 = m_lo + static_cast<int64_t>(mt) * kBM;
    t.nt = nt;
    t.rows_valid = static_cast<int>(min(m_hi - t.row0, int64_t(kBM)));
    return true;
  };

  // ---- DMA sources of the tile being loaded
  // Gather: source row (in x) of each of this lane's DMA rows of a tile.
  // Without a valid tile the loads still issue (a fixed count of vector-memory
  // operations) over an empty resource and return zeros.
  int32_t src_rows[kDma];
  auto load_rows = [&](const Tile &t, bool valid) {
    if constexpr (kGather) {
      const __amdgpu_buffer_rsrc_t r_rows = make_rsrc(p.a_rows, valid ? static_cast<uint32_t>(p.M * 4) : 0u);
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const uint32_t row0 = static_cast<uint32_t>(t.row0);
#pragma unroll
      for (int j = 0; j < kDma; ++j) {
        const int r = (j * kWaves + wave) * kRowsPerKiB + ln / kChunks;
        const uint32_t off = (row0 + static_cast<uint32_t>(min(r, t.rows_valid - 1))) * 4u;
#if defined(__HIP_DEVICE_COMPILE__)
        src_rows[j] = __builtin_amdgcn_raw_buffer_load_b32(r_rows, static_cast<int>(off), 0, 0);
#else
        (void)off;
        (void)r_rows;
        src_rows[j] = 0;
#endif
      }
    } else {
      (void)t;
      (void)valid;
    }
  };
  __amdgpu_buffer_rsrc_t ra, rb;
  int a_off[kDma], b_off[kDma];
  // DMA offsets in 32-bit arithmetic (the host bounds every panel below 2 GiB).
  const int ncols32 = static_cast<int>(p.ncols), n32 = static_cast<int>(p.N);
  const int src_rows32 = static_cast<int>(min(p.a_src_rows, int64_t(0x7fffffff)));
  auto setup_dma = [&](const Tile &t) {
    const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;
    ra = kGather ? make_rsrc(p.a, static_cast<uint32_t>(p.a_src_rows * K * 2))
                 : make_rsrc(p.a + t.row0 * K, static_cast<uint32_t>(t.rows_valid) * row_bytes);
    rb = make_rsrc(p.w + t.g * p.N * K, static_cast<uint32_t>(p.N * K * 2));
    const int nt = static_cast<int>(t.nt);
    // Recomputed per call (not kept live across the tile loop): the lane's
    // DMA row and chunk from an opaque copy of the lane index.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int drow = ln / kChunks, dchunk = ln % kChunks;
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      const int r = (j * kWaves + wave) * kRowsPerKiB + drow;
      const uint32_t lbytes = static_cast<uint32_t>(dchunk ^ swz(r)) * 16u;
      if constexpr (kGather) {
        // An index outside x points past the resource (zeros).
        const int32_t src = src_rows[j];
        a_off[j] = (r < t.rows_valid && src >= 0 && src < src_rows32)
                       ? static_cast<int>(static_cast<uint32_t>(src) * row_bytes + lbytes)
                       : static_cast<int>(kNoAccess);
      } else {
        // Rows past the group's end read as zeros: their results are dropped,
        // and zero operands cost the (power-bound) MFMAs less energy than a
        // repeated real row (measured 0.7-1.1% faster at c5).
        a_off[j] = r < t.rows_valid ? static_cast<int>(static_cast<uint32_t>(r) * row_bytes + lbytes)
                                    : static_cast<int>(kNoAccess);
      }
      int brow;
      if constexpr (kSwiglu) {
        // rows 0..127: gate columns j0 .. j0+127; rows 128..255: up columns F + j0 ..
        const int c = min(nt * (kBN / 2) + (r & 127), ncols32 - 1);
        brow = r < 128 ? c : ncols32 + c;
      } else {
        brow = min(nt * kBN + r, n32 - 1);
      }
      b_off[j] = static_cast<int>(static_cast<uint32_t>(brow) * row_bytes + lbytes);
    }
  };
  // Operand `op` (0 = A, 1 = B) of K step `kt` of the tile set up last into ring slot `slot`.
  auto issue_half = [&](int kt, int slot, int op) {
    const uint32_t st = lds_base + (slot % kStages) * kStageBytes + op * kOperandBytes;
    const int soff = kt * kBK * 2;
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      const uint32_t blk = j * kWaves + wave;
      dma16b(op ? rb : ra, (lds_void *)(uintptr_t)(st + blk * 1024), op ? b_off[j] : a_off[j], soff);
    }
  };
  auto zero_ktail = [&](int slot) {
    lds_char *st = sbase + (slot % kStages) * kStageBytes;
    const int kvalid = static_cast<int>(K - static_cast<int64_t>(ktiles - 1) * kBK);
    for (int idx = tid; idx < 2 * kBM * kChunks; idx += kThreads) {
      const int op = idx / (kBM * kChunks), rem = idx % (kBM * kChunks);
      const int r = rem / kChunks, c = rem % kChunks;
      if (c * 8 >= kvalid) {
        *reinterpret_cast<lds_u32x4 *>(st + op * kOperandBytes + r * kRowBytes + ((c ^ swz(r)) * 16)) =
            u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  // ---- fragments of v_mfma_f32_16x16x32_bf16: lane l reads row (block +
  // l % 16), the 8 values k = 8 (l / 16) .. + 7 of K half ks (logical chunk
  // 4 ks + l / 16, i.e. address ^ (ks << 6)).
  constexpr int kMI16 = 8, kNI16 = 8;
  const int fq = lane >> 4;
  // Row blocks 16 apart share the swizzle ((row / 2) % 8 changes by 8), so a
  // block's fragment address is the wave's first block's plus a constant
  // (an immediate ds_read offset): one address register per operand.
  const int ra0 = wm * 128 + (lane & 15);
  const int rb0 = (kSwiglu ? wn * 64 : wn * 128) + (lane & 15);
  const uint32_t fa0 = ra0 * kRowBytes + ((fq ^ swz(ra0)) << 4);
  const uint32_t fb0 = kOperandBytes + rb0 * kRowBytes + ((fq ^ swz(rb0)) << 4);
  auto b_blk_off = [](int j) {
    return kSwiglu ? (j / (kNI16 / 2)) * 128 * kRowBytes + (j % (kNI16 / 2)) * 16 * kRowBytes : j * 16 * kRowBytes;
  };
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 acc[kMI16][kNI16];
  uint32_t rd_so = 0;
  auto set_read_slot = [&](int slot) { rd_so = lds_base + (slot % kStages) * kStageBytes; };
  bf16x8 fa[2][kMI16], fb[2][kNI16];
  // A fragments of row blocks 4 ih .. 4 ih + 3 / all B fragments of K half ks.
  auto read_a = [&](int ks, int ih) {
    const uint32_t base = (rd_so + fa0) ^ (ks << 6);
#pragma unroll
    for (int i = 4 * ih; i < 4 * ih + 4; ++i)
      fa[ks][i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(base + i * 16 * kRowBytes));
  };
  auto read_b = [&](int ks) {
    const uint32_t base = (rd_so + fb0) ^ (ks << 6);
#pragma unroll
    for (int j = 0; j < kNI16; ++j)
      fb[ks][j] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(base + b_blk_off(j)));
  };
  auto read_all = [&]() {
    read_a(0, 0);
    read_a(0, 1);
    read_b(0);
    read_a(1, 0);
    read_a(1, 1);
    read_b(1);
  };
  // The step's last unit (K half 1, row blocks 4..7) column by column: after
  // column block j's 4 MFMAs its B fragment is free, and the next stage's is
  // read into it right there (with A blocks 0..3, freed by the unit before);
  // only A blocks 4..7 are read after the unit (reading them under its last
  // MFMAs too measured 0.4% slower).
  auto last_unit_reads = [&]() {
    const uint32_t base_b = (rd_so + fb0) ^ (1 << 6);
    const uint32_t base_a = (rd_so + fa0) ^ (1 << 6);
#pragma unroll
    for (int j = 0; j < kNI16; ++j) {
#pragma unroll
      for (int i = 4; i < 8; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[1][j], fa[1][i], acc[i][j], 0, 0, 0);
      }
      fb[1][j] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(base_b + b_blk_off(j)));
      if (j < 4) fa[1][j] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(base_a + j * 16 * kRowBytes));
    }
  };
  // 32 MFMAs: K half ks, row blocks 4 ih .. 4 ih + 3, all column blocks.
  auto mfma_unit = [&](int ks, int ih, bool zero) {
#pragma unroll
    for (int i = 4 * ih; i < 4 * ih + 4; ++i)
#pragma unroll
      for (int j = 0; j < kNI16; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[ks][j], fa[ks][i], zero ? f32x4{} : acc[i][j], 0, 0, 0);
  };

  // Epilogue of tile t from the accumulators. With w as the MFMA's first
  // operand, register r of lane l in block (i, j) holds output row i * 16 +
  // l % 16 and column j * 16 + 4 (l / 16) + r of this wave's part. After
  // rounding, a block is two packed words per lane; v_permlane16_swap trades
  // rows (16 lanes) 1 and 3 of block j's words with rows 0 and 2 of block j + 1's,
  // so lanes of row q hold the 8 consecutive columns (q / 2) 8 .. + 7 of
  // block j + q % 2.
  auto epilogue = [&](const Tile &t) {
    const uint32_t ld = static_cast<uint32_t>(p.ncols) * 2u;
    const __amdgpu_buffer_rsrc_t ro =
        make_rsrc(p.out + t.row0 * p.ncols, static_cast<uint32_t>(t.rows_valid) * ld);
    // 32-bit column and row arithmetic (the host keeps ncols below 2^22) from
    // an opaque copy of the lane index, so nothing per lane stays live across tiles.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int eq = ln >> 4;
    const int wcol0 = static_cast<int>(t.nt) * kEpiCols + wn * (kEpiCols / 2) + (eq & 1) * 16 + (eq >> 1) * 8;
    constexpr int kOut16 = kSwiglu ? kNI16 / 2 : kNI16;
#pragma unroll
    for (int i = 0; i < kMI16; ++i) {
      const uint32_t orow = static_cast<uint32_t>(wm * 128 + i * 16 + (ln & 15));
#pragma unroll
      for (int jp = 0; jp < kOut16; jp += 2) {
        uint32_t w[2][2];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          float h[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if constexpr (kSwiglu) {
              const float gt = acc[i][jp + d][q];
              h[q] = gt * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gt * -1.4426950408889634f)) *
                     acc[i][jp + d + kNI16 / 2][q];
            } else {
              h[q] = acc[i][jp + d][q];
            }
          }
          const bf16x2 lo = {(__bf16)h[0], (__bf16)h[1]};
          const bf16x2 hi = {(__bf16)h[2], (__bf16)h[3]};
          w[d][0] = __builtin_bit_cast(uint32_t, lo);
          w[d][1] = __builtin_bit_cast(uint32_t, hi);
        }
        u32x4 o;
#if defined(__HIP_DEVICE_COMPILE__)
        const auto s0 = __builtin_amdgcn_permlane16_swap(w[0][0], w[1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(w[0][1], w[1][1], false, false);
        o = u32x4{s0[0], s1[0], s0[1], s1[1]};
#else
        o = u32x4{0u, 0u, 0u, 0u};
#endif
        const int gcol = wcol0 + jp * 16;
        // Columns past the output get an offset past the resource: the store is dropped.
        const uint32_t off = gcol < ncols32 ? orow * ld + static_cast<uint32_t>(gcol) * 2u : kNoAccess;
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_raw_buffer_store_b128(o, ro, static_cast<int>(off), 0, 0);
#else
        (void)off;
        (void)ro;
        (void)o;
#endif
      }
      // One row block at a time: bounds the registers the epilogue holds.
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The part of a K step after its barrier: MFMA units 1-3 of the fragments
  // in VGPRs, the next stage's fragments read from the LDS slot set by
  // set_read_slot into the registers each unit frees, and the DMA of stage
  // `kdma` (of the tile set up last) into ring slot `wr`.
  auto step_body = [&](bool zero, int kdma, int wr) __attribute__((always_inline)) {
    mfma_unit(0, 1, zero);
    read_a(0, 0);
    issue_half(kdma, wr, 0);
    sched_mix<32, 4, 8>();
    mfma_unit(1, 0, false);
    read_a(0, 1);
    read_b(0);
    issue_half(kdma, wr, 1);
    sched_mix<32, 12, 8>();
    last_unit_reads();
    sched_mix<32, 12, 0>();
    read_a(1, 1);
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- first tile: stages 0 and 1 in flight, stage 0 read into VGPRs
  Tile cur{}, nxt{};  // nxt stays zero when no tile follows (its row loads then read nothing)
  if (!find_tile(0, cur)) return;
  load_rows(cur, true);
  setup_dma(cur);
  issue_half(0, 0, 0);
  issue_half(0, 0, 1);
  issue_half(1, 1, 0);
  issue_half(1, 1, 1);
  bool more = find_tile(1, nxt);
  wait_vm_n<2 * kDma>();
  barrier();
  set_read_slot(0);
  read_all();

  int sb = 0;  // ring slot of the current tile's stage 0
  for (int64_t round = 0;; ++round) {
    // One K step: MFMAs of stage kt (fragments in VGPRs), fragments of stage
    // kt + 1 read from LDS, DMA of the stage two ahead (this tile's kt + 2 or,
    // past its end, the next tile's kt + 2 - ktiles) into the slot of stage kt.
    auto step = [&](int kt, bool first, bool last) {
      mfma_unit(0, 0, first);
      __builtin_amdgcn_sched_barrier(0);
      // Stage kt + 1 has landed. In a tile's first step the previous tile's
      // output stores were issued after it and may still be in flight.
      if (first && round > 0) {
        wait_vm_n<kStores>();
      } else {
        wait_dma();
      }
      wait_lds();
      barrier();
      if (first) load_rows(nxt, more);  // read in this tile's last step
      if (ktail && kt + 1 == ktiles - 1) {
        zero_ktail(sb + kt + 1);
        wait_lds();
        barrier();
      }
      // The last step DMAs the next tile's stage 0 (without a next tile it
      // re-reads this tile's last stage into the free slot: no branch below).
      if (last && more) setup_dma(nxt);
      const int kdma = !last ? kt + 2 : (more ? 0 : ktiles - 1);
      set_read_slot(sb + kt + 1);
      step_body(first, kdma, sb + kt + 2);
    };
    // The first and the last step are peeled (with the last step inside the
    // loop as a uniform branch the SwiGLU kernel measured 7% slower at c5).
    step(0, true, false);
    for (int kt = 1; kt + 2 < ktiles; ++kt) step(kt, false, false);
    step(ktiles - 2, false, true);

    // Last step of the tile: it reads the next tile's stage 0 (DMA'd in the
    // step above) and DMAs its stage 1 (without a next tile: reads and DMA of
    // data nobody uses, so the code has no branch).
    mfma_unit(0, 0, false);
    __builtin_amdgcn_sched_barrier(0);
    wait_dma();
    wait_lds();
    barrier();
    set_read_slot(sb + ktiles);
    step_body(false, more ? 1 : ktiles - 1, sb + ktiles + 1);
    epilogue(cur);
    __builtin_amdgcn_sched_barrier(0);
    if (!more) break;
    cur = nxt;
    sb += ktiles;
    more = find_tile(round + 2, nxt);
  }
  wait_dma();  // no LDS DMA outlives the workgroup
}

// ---------------------------------------------------------------------------
// Ping-pong forward kernel (the default for K % 64 == 0, K >= 192, 16-byte
// output rows): 8 wavefronts, two per SIMD, output tile 256 x 256, K step 64.
//
// With one wavefront per SIMD every LDS-DMA instruction (buffer_load ... lds,
// about 40 cycles of issue each under load, 16 per wavefront per K step) and
// every fragment read stalls that SIMD's MFMA stream. Here the two wavefronts
// of a SIMD take turns: in each phase one of them issues its 64 MFMAs (one K
// step of its 64 x 128 part of the tile, fragments in VGPRs) while the other
// reads its fragments of the next stage from LDS and issues its share of the
// stage DMAs; a workgroup barrier ends every phase and the roles swap.
//
// Groups: the two wavefronts of a SIMD (found from the hardware wave id at
// start) form group 0 and group 1; wm = SIMD index selects the tile's rows
// wm * 64 .. + 63, the group its columns grp * 128 .. + 127. Group 0 loads
// stage s in phase 2s and multiplies it in phase 2s + 1; group 1 one phase
// later.
//
// LDS (160 KiB): A ring of 3 slots (256 rows x 64 K), B ring of 2 slots (the
// 128 B rows of group 0, then those of group 1). Stage s of A is read in
// phases 2s and 2s + 1, group 0's B half in phase 2s, group 1's in phase
// 2s + 1. In the load phase of stage s, group 0 DMAs its half of A stage
// s + 2 and group 1's B half of stage s + 1, group 1 its half of A stage s + 2
// and group 0's B half of stage s + 2: each slot is rewritten only after the
// barrier that ends its last reader's phase, and every DMA has two phases to
// land (its issuer waits for it at the end of its next load phase, before the
// barrier that precedes its readers).
//
// The epilogue of a tile (same register layout as the pipelined kernel) runs
// in the wavefront's next load phase; the stores are issued before that
// phase's DMAs and are allowed to stay in flight across its barrier.
struct PpTile {  // rows and groups in 32 bits: the host runs the kernel for M < 2^31
  int g, row0;
  uint32_t nt;
  int rows_valid;
  int unit;  // split kernel: the unit (range * split_tiles + tile); otherwise 0
};

// Tiles of the static order (256-row tiles, no tail list) over all groups.
__device__ __forceinline__ int64_t static_tile_count(const GemmArgs &p) {
  const int M32 = static_cast<int>(p.M);
  int64_t total = 0;
  for (int g = 0; g < static_cast<int>(p.G); ++g) {
    const int lo = min(max(ld_inv(p.offsets, g), 0), M32);
    const int hi = min(max(ld_inv(p.offsets, g + 1), lo), M32);
    total += static_cast<int64_t>((hi - lo + 255) / 256) * p.ntiles;
  }
  return total;
}

// Row tile and column tile of position q inside a group of mt_g row tiles: groups of kGroupM row
// tiles x all column tiles, row tile fastest.
__device__ __forceinline__ void patch_pos(uint32_t q, uint32_t ntl, uint32_t mt_g, uint32_t &mt, uint32_t &nt) {
  const uint32_t per_grp = kGroupM * ntl;
  const uint32_t full = mt_g / kGroupM;
  if (q < full * per_grp) {
    const uint32_t gq = q / per_grp, r = q - gq * per_grp;
    nt = r / kGroupM;
    mt = gq * kGroupM + r % kGroupM;
  } else {
    const uint32_t r = q - full * per_grp, gm = mt_g - full * kGroupM;
    nt = r / gm;
    mt = full * kGroupM + (r - nt * gm);
  }
}

// Tile L of the static order (256-row tiles); false past the last tile.
__device__ __forceinline__ bool static_tile(const GemmArgs &p, int64_t L, PpTile &t) {
  const int M32 = static_cast<int>(p.M);
  int64_t before = 0;
  for (int g = 0; g < static_cast<int>(p.G); ++g) {
    const int lo = min(max(ld_inv(p.offsets, g), 0), M32);
    const int hi = min(max(ld_inv(p.offsets, g + 1), lo), M32);
    const int mt_g = (hi - lo + 255) / 256;
    const int64_t n = static_cast<int64_t>(mt_g) * p.ntiles;
    if (L < before + n) {
      uint32_t mt, nt;
      patch_pos(static_cast<uint32_t>(L - before), static_cast<uint32_t>(p.ntiles), static_cast<uint32_t>(mt_g), mt,
                nt);
      t.g = g;
      t.row0 = lo + static_cast<int>(mt) * 256;
      t.nt = nt;
      t.rows_valid = min(hi - t.row0, 256);
      t.unit = 0;
      return true;
    }
    before += n;
  }
  return false;
}

// kTM = 256: the persistent workgroup b of P (the grid) takes its tiles in
// the static order (those before the split tiles, if any); kTM = 128: the one
// tile *one; kSplit: workgroup b computes split unit b (one K range of one of
// the last split_tiles tiles) into its fp32 plane.
template <bool kSwiglu, bool kGather, int kTM, bool kTails, bool kSplit = false>
__device__ __forceinline__ void pp_body(const GemmArgs &p, char *smem, const PpTile *one) {
  static_assert(kTM == 256 || kTM == 128, "tile rows");
  static_assert(!kSplit || (kTM == 256 && !kTails), "split units are 256-row tiles");
  constexpr int kAS = 3, kBS = 2;                   // ring slots
  constexpr int kASlotBytes = kTM * kRowBytes;      // A stage: kTM rows x 64 K
  constexpr int kSlotBytes = 256 * kRowBytes;       // B stage: 32 KiB, 256 rows x 64 K
  constexpr int kBBase = kAS * kASlotBytes;
  constexpr int kEpiCols = kSwiglu ? kBN / 2 : kBN;  // output columns of a tile
  constexpr int kMI = kTM / 64, kNI = 8;             // 16 x 16 blocks of a wavefront
  constexpr int kWR = kTM / 4;                       // tile rows of a wavefront
  constexpr int kStores = kMI * (kSwiglu ? 2 : 4);   // 16-byte stores per lane per tile
  constexpr int kDmaA = kTM / 64, kDmaB = 4;         // DMA instructions per wavefront per load phase
  constexpr int kABlk = kTM / 16;                    // 8-row A blocks DMA'd by one group per stage
  static_assert(kDmaA + kDmaB + kStores <= 63, "vmcnt range");
  static_assert(kAS * kASlotBytes + kBS * kSlotBytes <= kPpLdsBytes, "LDS");
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));

  // The thread index through an opaque copy: the lane-derived values of the
  // 256-row and the 128-row form are computed separately, not kept live from
  // one form to the other.
  int tid = threadIdx.x;
  if constexpr (kTails) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- roles from the SIMD each wavefront runs on (HW_ID bits 5:4): the two
  // wavefronts of a SIMD must be in different groups. Exchanged through LDS
  // before the ring is used.
  int wm, grp;
  {
    const int simd = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_s_getreg((1 << 11) | (4 << 6) | 4)) & 3;
    volatile int *sid = reinterpret_cast<volatile int *>(smem);
    if (lane == 0) sid[wave] = simd;
    __syncthreads();
    int before = 0, per_simd[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const int s = sid[w] & 3;
      per_simd[s] += 1;
      before += (s == simd) && (w < wave);
    }
    __syncthreads();
    // Two wavefronts per SIMD (the register budget allows no more); if the
    // hardware placed them otherwise, every wavefront falls back to
    // wave-index roles (the test reads the same 8 values in every wavefront).
    const bool ok = per_simd[0] == 2 && per_simd[1] == 2 && per_simd[2] == 2 && per_simd[3] == 2;
    // Wave-uniform (scalar) roles: every DMA resource and offset derived from
    // them stays in scalar registers.
    wm = __builtin_amdgcn_readfirstlane(ok ? simd : (wave & 3));
    grp = __builtin_amdgcn_readfirstlane(ok ? before : (wave >> 2));
  }

  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t K = p.K;
  int S = static_cast<int>(K / kBK);  // K steps per tile (>= 3, K % 64 == 0: host; split units: their range's)

  // ---- tile walker (group offsets read from memory: the ring fills the LDS;
  // rows and groups in 32 bits)
  const int M32 = static_cast<int>(p.M);
  const int G32 = static_cast<int>(p.G);
  auto group_rows = [&](int g, int &lo, int &hi) {
    lo = min(max(ld_inv(p.offsets, g), 0), M32);
    hi = min(max(ld_inv(p.offsets, g + 1), lo), M32);
  };
  // 256-row tiles of a group (kTails: all but a last tile of at most 128
  // rows, which the 128-row form takes).
  auto main_tiles = [&](int m) -> int { return kTails ? main_row_tiles(m) : (m + 255) / 256; };
  int g_cur = 0, m_lo, m_hi;
  int64_t tiles_before = 0;
  group_rows(0, m_lo, m_hi);
  int mt_g = main_tiles(m_hi - m_lo);
  using Tile = PpTile;
  // With a reduction split the static order ends where the split tiles begin.
  int64_t split_base = INT64_MAX;
  if (!kTails && p.split_tiles > 0) split_base = max(static_tile_count(p) - p.split_tiles, int64_t(0));
  auto find_tile = [&](int64_t round, Tile &t) -> bool {
    if constexpr (kTM == 128) {
      if (round > 0) return false;
      t = *one;
      return true;
    }
    int64_t L;
    int unit = 0;
    if constexpr (kSplit) {
      // unit u = range * split_tiles + tile: an XCD's workgroups take neighbouring tiles of one range
      if (round > 0) return false;
      unit = static_cast<int>((b % 8) * (P / 8) + b / 8);
      if (unit >= p.split_tiles * p.split_ways) return false;
      L = split_base + unit % p.split_tiles;
    } else {
      L = round * P + (b % 8) * (P / 8) + b / 8;
      if (L >= split_base) return false;
    }
    while (g_cur < G32 && L >= tiles_before + static_cast<int64_t>(mt_g) * p.ntiles) {
      tiles_before += static_cast<int64_t>(mt_g) * p.ntiles;
      ++g_cur;
      if (g_cur < G32) {
        group_rows(g_cur, m_lo, m_hi);
        mt_g = main_tiles(m_hi - m_lo);
      }
    }
    if (g_cur >= G32) return false;
    uint32_t mt, nt;
    patch_pos(static_cast<uint32_t>(L - tiles_before), static_cast<uint32_t>(p.ntiles), static_cast<uint32_t>(mt_g),
              mt, nt);
    t.g = g_cur;
    t.row0 = m_lo + static_cast<int>(mt) * kTM;
    t.nt = nt;
    t.rows_valid = min(m_hi - t.row0, kTM);
    t.unit = unit;
    return true;
  };
  // Split units: the K range [k0, k0 + 64 S) of the unit's tile (buffer bases move by k0 columns).
  int64_t k0 = 0;
  auto split_range = [&](const Tile &t) {
    if constexpr (kSplit) {
      const int r = t.unit / p.split_tiles;
      k0 = static_cast<int64_t>(r) * p.split_steps * kBK;
      S = r == p.split_ways - 1 ? static_cast<int>(K / kBK) - r * p.split_steps : p.split_steps;
    } else {
      (void)t;
    }
  };

  // ---- DMA sources. This wavefront's A rows: blocks (grp * kTM / 16 + j * 4 +
  // wm), 8 rows each; its B rows: blocks ((1 - grp) * 16 + j * 4 + wm) (the
  // other group's half, see above).
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;
  const int ncols32 = static_cast<int>(p.ncols);
  const int src_rows32 = static_cast<int>(min(p.a_src_rows, int64_t(0x7fffffff)));
  auto a_row = [&](int j, int ln) { return ((grp * kABlk + j * 4 + wm) * kRowsPerKiB) + ln / kChunks; };
  auto b_row = [&](int j, int ln) { return (((1 - grp) * 16 + j * 4 + wm) * kRowsPerKiB) + ln / kChunks; };
  int32_t src_rows[kDmaA];
  auto load_rows = [&](const Tile &t, bool valid) {
    if constexpr (kGather) {
      const __amdgpu_buffer_rsrc_t r_rows = make_rsrc(p.a_rows, valid ? static_cast<uint32_t>(p.M * 4) : 0u);
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const uint32_t row0 = static_cast<uint32_t>(t.row0);
#pragma unroll
      for (int j = 0; j < kDmaA; ++j) {
        const uint32_t off = (row0 + static_cast<uint32_t>(min(a_row(j, ln), max(t.rows_valid - 1, 0)))) * 4u;
#if defined(__HIP_DEVICE_COMPILE__)
        src_rows[j] = __builtin_amdgcn_raw_buffer_load_b32(r_rows, static_cast<int>(off), 0, 0);
#else
        (void)off;
        (void)r_rows;
        src_rows[j] = 0;
#endif
      }
    } else {
      (void)t;
      (void)valid;
    }
  };
  __amdgpu_buffer_rsrc_t ra, rb;
  // A: per-lane offsets (gather: data-dependent rows); B: one per-lane base,
  // the rows of DMA j lie b_step(j) rows further (wave-uniform).
  int a_off[kDmaA];
  int b_base = 0;
  uint32_t b_ncols = 0;  // SwiGLU: rows from a gate row to its up row (ncols), in bytes
  auto setup_a = [&](const Tile &t, bool valid) {
    const uint32_t kb = static_cast<uint32_t>(k0) * 2u;  // split units: columns before the range
    ra = kGather ? make_rsrc(p.a + k0, valid ? static_cast<uint32_t>(p.a_src_rows * K * 2) - kb : 0u)
                 : make_rsrc(p.a + t.row0 * K + k0, valid ? static_cast<uint32_t>(t.rows_valid) * row_bytes - kb : 0u);
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int j = 0; j < kDmaA; ++j) {
      const int r = a_row(j, ln);
      const uint32_t lbytes = static_cast<uint32_t>((ln % kChunks) ^ swz(r)) * 16u;
      if constexpr (kGather) {
        const int32_t src = src_rows[j];
        a_off[j] = (r < t.rows_valid && src >= 0 && src < src_rows32)
                       ? static_cast<int>(static_cast<uint32_t>(src) * row_bytes + lbytes)
                       : static_cast<int>(kNoAccess);
      } else {
        // Rows past the group's end lie past the resource: zeros.
        a_off[j] = static_cast<int>(static_cast<uint32_t>(r) * row_bytes + lbytes);
      }
    }
  };
  // B row of tile row r: plain nt * 256 + r (rows past N lie past the
  // resource: zeros); SwiGLU: half h = r / 128 holds 64 gate rows of output
  // columns c = nt * 128 + h * 64 .., then the 64 up rows (ncols + c) of the
  // same columns. A gate column past ncols reads an up row (in bounds, its
  // output column is dropped); its up row lies past the resource.
  // This wavefront's DMA j covers tile rows b_row(0) + 32 j; j = 0, 1 are gate
  // rows and 2, 3 up rows (SwiGLU), so DMA j reads B row
  // brow(0) + 32 (j % 2) (+ ncols for j >= 2): one base plus a uniform step.
  auto setup_b = [&](const Tile &t, bool valid) {
    rb = make_rsrc(p.w + t.g * p.N * K + k0, valid ? static_cast<uint32_t>(p.N * K * 2) - static_cast<uint32_t>(k0) * 2u : 0u);
    const int nt = static_cast<int>(t.nt);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r = b_row(0, ln);
    const uint32_t lbytes = static_cast<uint32_t>((ln % kChunks) ^ swz(r)) * 16u;
    int brow;
    if constexpr (kSwiglu) {
      brow = nt * (kBN / 2) + (r >> 7) * 64 + (r & 63);
      b_ncols = static_cast<uint32_t>(ncols32) * row_bytes;
    } else {
      brow = nt * kBN + r;
    }
    b_base = static_cast<int>(static_cast<uint32_t>(brow) * row_bytes + lbytes);
  };
  auto b_off = [&](int j) -> int {
    if constexpr (kSwiglu) {
      return b_base + static_cast<int>((j & 1) * 32u * row_bytes + (j >= 2 ? b_ncols : 0u));
    } else {
      return b_base + static_cast<int>(static_cast<uint32_t>(j) * 32u * row_bytes);
    }
  };
  // DMA of this wavefront's share of A stage kt into A slot sa and of its B
  // rows of stage kt_b into B slot sb.
  auto issue = [&](int kt_a, int sa, int kt_b, int sbs) {
    const uint32_t a_dst = lds_base + sa * kASlotBytes;
    const uint32_t b_dst = lds_base + kBBase + sbs * kSlotBytes;
#pragma unroll
    for (int j = 0; j < kDmaA; ++j) {
      const uint32_t blk = grp * kABlk + j * 4 + wm;
      dma16b(ra, (lds_void *)(uintptr_t)(a_dst + blk * 1024), a_off[j], kt_a * kBK * 2);
    }
#pragma unroll
    for (int j = 0; j < kDmaB; ++j) {
      const uint32_t blk = (1 - grp) * 16 + j * 4 + wm;
      dma16b(rb, (lds_void *)(uintptr_t)(b_dst + blk * 1024), b_off(j), kt_b * kBK * 2);
    }
  };

  // ---- fragments (v_mfma_f32_16x16x32_bf16 layout as in the pipelined kernel)
  const int fq = lane >> 4;
  const int ra0 = wm * kWR + (lane & 15);
  const int rb0 = grp * 128 + (lane & 15);
  const uint32_t fa0 = ra0 * kRowBytes + ((fq ^ swz(ra0)) << 4);
  const uint32_t fb0 = rb0 * kRowBytes + ((fq ^ swz(rb0)) << 4);
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 acc[kMI][kNI];
  bf16x8 fa[2][kMI], fb[2][kNI];
  auto read_frags = [&](int sa, int sbs) {
    const uint32_t a_base = lds_base + sa * kASlotBytes + fa0;
    const uint32_t b_base = lds_base + kBBase + sbs * kSlotBytes + fb0;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int i = 0; i < kMI; ++i)
        fa[ks][i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)((a_base ^ (ks << 6)) + i * 16 * kRowBytes));
#pragma unroll
      for (int j = 0; j < kNI; ++j)
        fb[ks][j] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)((b_base ^ (ks << 6)) + j * 16 * kRowBytes));
    }
  };
  auto compute = [&](auto zero_c) {
    constexpr bool zero = decltype(zero_c)::value;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < kMI; ++i)
#pragma unroll
        for (int j = 0; j < kNI; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[ks][j], fa[ks][i],
                                                             (zero && ks == 0) ? f32x4{} : acc[i][j], 0, 0, 0);
  };
  // Split units: the fp32 accumulators to the unit's 256 x 256 plane (row-major). Plane column of a
  // wave's block j: plain j * 16 + its 16 columns of the group's 128; SwiGLU gate blocks 0-3 at
  // columns [0, 128), their up blocks 4-7 at the same columns + 128.
  auto split_store = [&](const Tile &t) {
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.planes + static_cast<int64_t>(t.unit) * 65536, 65536u * 4u);
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
      const uint32_t prow = static_cast<uint32_t>(wm * kWR + i * 16 + (ln & 15));
#pragma unroll
      for (int j = 0; j < kNI; ++j) {
        const int pcol = kSwiglu ? (j >= kNI / 2 ? 128 : 0) + grp * 64 + (j % (kNI / 2)) * 16 + (ln >> 4) * 4
                                 : grp * 128 + j * 16 + (ln >> 4) * 4;
        const uint32_t off = (prow * 256u + static_cast<uint32_t>(pcol)) * 4u;
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), rp, static_cast<int>(off), 0, 0);
#else
        (void)off;
        (void)rp;
#endif
      }
    }
  };
  auto epilogue = [&](const Tile &t) {
    if constexpr (kSplit) {
      split_store(t);
      return;
    }
    const uint32_t ld = static_cast<uint32_t>(p.ncols) * 2u;
    const __amdgpu_buffer_rsrc_t ro =
        make_rsrc(p.out + t.row0 * p.ncols, static_cast<uint32_t>(t.rows_valid) * ld);
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int eq = ln >> 4;
    const int wcol0 = static_cast<int>(t.nt) * kEpiCols + grp * (kEpiCols / 2) + (eq & 1) * 16 + (eq >> 1) * 8;
    constexpr int kOut16 = kSwiglu ? kNI / 2 : kNI;
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
      const uint32_t orow = static_cast<uint32_t>(wm * kWR + i * 16 + (ln & 15));
#pragma unroll
      for (int jp = 0; jp < kOut16; jp += 2) {
        uint32_t w[2][2];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          float h[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if constexpr (kSwiglu) {
              const float gt = acc[i][jp + d][q];
              h[q] = gt * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gt * -1.4426950408889634f)) *
                     acc[i][jp + d + kNI / 2][q];
            } else {
              h[q] = acc[i][jp + d][q];
            }
          }
          const bf16x2 lo = {(__bf16)h[0], (__bf16)h[1]};
          const bf16x2 hi = {(__bf16)h[2], (__bf16)h[3]};
          w[d][0] = __builtin_bit_cast(uint32_t, lo);
          w[d][1] = __builtin_bit_cast(uint32_t, hi);
        }
        u32x4 o;
#if defined(__HIP_DEVICE_COMPILE__)
        const auto s0 = __builtin_amdgcn_permlane16_swap(w[0][0], w[1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(w[0][1], w[1][1], false, false);
        o = u32x4{s0[0], s1[0], s0[1], s1[1]};
#else
        o = u32x4{0u, 0u, 0u, 0u};
#endif
        const int gcol = wcol0 + jp * 16;
        const uint32_t off = gcol < ncols32 ? orow * ld + static_cast<uint32_t>(gcol) * 2u : kNoAccess;
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_raw_buffer_store_b128(o, ro, static_cast<int>(off), 0, 0);
#else
        (void)off;
        (void)ro;
        (void)o;
#endif
      }
    }
  };

  // ---- prologue: A stages 0 and 1, group 0's B rows of stages 0 and 1 (by
  // group 1), group 1's B rows of stage 0 (by group 0).
  Tile cur{}, nxt{};
  if (!find_tile(0, cur)) return;
  split_range(cur);
  load_rows(cur, true);
  setup_a(cur, true);
  setup_b(cur, true);
  {
    const uint32_t b_dst0 = lds_base + kBBase;
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int j = 0; j < kDmaA; ++j) {
        const uint32_t blk = grp * kABlk + j * 4 + wm;
        dma16b(ra, (lds_void *)(uintptr_t)(lds_base + kt * kASlotBytes + blk * 1024), a_off[j], kt * kBK * 2);
      }
    }
    const int nb = grp == 1 ? 2 : 1;
    for (int kt = 0; kt < nb; ++kt) {
#pragma unroll
      for (int j = 0; j < kDmaB; ++j) {
        const uint32_t blk = (1 - grp) * 16 + j * 4 + wm;
        dma16b(rb, (lds_void *)(uintptr_t)(b_dst0 + kt * kSlotBytes + blk * 1024), b_off(j), kt * kBK * 2);
      }
    }
  }
  bool more = find_tile(1, nxt);
  wait_dma();
  barrier();
  if (grp == 1) barrier();  // group 1 runs one phase behind

  int slot_a = 0, slot_b = 0;  // ring slots of the stage being read
  bool have_prev = false;
  Tile prev{};
  for (int64_t round = 0;; ++round) {
    for (int s = 0; s < S; ++s) {
      // ---------------- load phase of stage s
      if (kGather && s == S - 3) load_rows(nxt, more);  // before this phase's other memory operations

      const bool epi = s == 0 && have_prev;
      if (epi) epilogue(prev);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(slot_a, slot_b);
      const int ta = s + 2, tb = s + 1 + grp;  // stages this phase DMAs (of this tile or the next)
      if (ta == S) setup_a(nxt, more);
      if (tb == S) setup_b(nxt, more);
      int sa = slot_a + 2;
      sa = sa >= kAS ? sa - kAS : sa;
      const int sbs = (slot_b + 1 + grp) & 1;
      issue(ta >= S ? ta - S : ta, sa, tb >= S ? tb - S : tb, sbs);
      // The previous load phase's DMAs have landed (only this phase's DMAs,
      // and the epilogue stores issued before them, may still be in flight).
      if (epi) {
        wait_vm_n<kDmaA + kDmaB + kStores>();
      } else {
        wait_vm_n<kDmaA + kDmaB>();
      }
      wait_lds();
      barrier();
      // ---------------- compute phase of stage s
      if (s == 0) {
        compute(std::true_type{});
      } else {
        compute(std::false_type{});
      }
      __builtin_amdgcn_sched_barrier(0);
      barrier();
      slot_a = slot_a + 1 == kAS ? 0 : slot_a + 1;
      slot_b ^= 1;
    }
    prev = cur;
    have_prev = true;
    if (!more) break;
    cur = nxt;
    more = find_tile(round + 2, nxt);
  }
  // Last tile's epilogue in a final load phase; group 0 passes one more
  // barrier so that both groups pass the same number.
  epilogue(prev);
  if (grp == 0) barrier();
  wait_dma();  // no LDS DMA outlives the workgroup
}

// Ping-pong kernel: one persistent workgroup per CU takes its 256-row tiles
// in the static order; with a tail list it then takes tail units from the
// list's counter (wave 0 adds 1, the number reaches the other wavefronts
// through the idle LDS ring) and computes each with the 128-row form of the
// same pipeline, until the units run out. Workgroups whose static tiles end
// early take more units, so the units also even out the last round.
template <bool kSwiglu, bool kGather, bool kTails>
__global__ __launch_bounds__(512) void grouped_gemm_pp_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) char smem[kPpLdsBytes];
  pp_body<kSwiglu, kGather, 256, kTails>(p, smem, nullptr);
  if constexpr (!kTails) return;
  volatile int *bcast = reinterpret_cast<volatile int *>(smem);
  const int ntl = static_cast<int>(p.ntiles);
  for (;;) {
    __syncthreads();  // the ring is idle: every wavefront has left its last tile
    if (threadIdx.x == 0) {
      bcast[0] = __hip_atomic_fetch_add(p.tails + kTailCtr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const int u = __builtin_amdgcn_readfirstlane(bcast[0]);
    __syncthreads();  // every wavefront has read it before the ring is used again
    if (u >= ld_inv(p.tails, kTailCount) * ntl) break;
    const int g = ld_inv(p.tails, kTailList + u / ntl);
    const int M32 = static_cast<int>(p.M);
    const int lo = min(max(ld_inv(p.offsets, g), 0), M32);
    const int hi = min(max(ld_inv(p.offsets, g + 1), lo), M32);
    const int r = (hi - lo) % 256;
    const PpTile t{g, hi - r, static_cast<uint32_t>(u % ntl), r};
    pp_body<kSwiglu, kGather, 128, kTails>(p, smem, &t);
  }
}

// Reduction split of the last tiles (see GemmArgs): workgroup b computes unit
// b into its fp32 plane, then split_sum_kernel adds the planes.
template <bool kSwiglu, bool kGather>
__global__ __launch_bounds__(512) void grouped_gemm_split_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(1024))) char smem[kPpLdsBytes];
  pp_body<kSwiglu, kGather, 256, false, true>(p, smem, nullptr);
}

// Block (tile, 16-row slab): each thread adds the split_ways planes of one row
// and 16 plane columns (SwiGLU: 8 gate and the 8 matching up columns) in
// range order, applies the epilogue (SwiGLU on the fp32 sums as the GEMM
// epilogue does) and stores its 16 (8) bf16 outputs of the valid rows and
// columns.
template <bool kSwiglu>
__global__ __launch_bounds__(256) void split_sum_kernel(GemmArgs p) {
  PpTile t;
  const int64_t base = max(static_tile_count(p) - p.split_tiles, int64_t(0));
  const int tile = blockIdx.x;
  if (!static_tile(p, base + tile, t)) return;
  const int r = blockIdx.y * 16 + threadIdx.x / 16;
  if (r >= t.rows_valid) return;
  constexpr int kCols = kSwiglu ? 8 : 16;  // output columns of a thread
  constexpr int kEpiCols = kSwiglu ? kBN / 2 : kBN;
  const int c = (threadIdx.x % 16) * kCols;
  const int64_t col = static_cast<int64_t>(t.nt) * kEpiCols + c;
  if (col >= p.ncols) return;  // ncols % 8 == 0: a thread's columns are all valid or all past the end
  float v[kCols], up[kCols];
#pragma unroll
  for (int q = 0; q < kCols; ++q) v[q] = up[q] = 0.0f;
  for (int w = 0; w < p.split_ways; ++w) {
    const float *pl = p.planes + (static_cast<int64_t>(w) * p.split_tiles + tile) * 65536 + r * 256;
#pragma unroll
    for (int q = 0; q < kCols; q += 4) {
      const float4 a = *reinterpret_cast<const float4 *>(pl + c + q);
      v[q] += a.x;
      v[q + 1] += a.y;
      v[q + 2] += a.z;
      v[q + 3] += a.w;
      if constexpr (kSwiglu) {
        const float4 u = *reinterpret_cast<const float4 *>(pl + 128 + c + q);
        up[q] += u.x;
        up[q + 1] += u.y;
        up[q + 2] += u.z;
        up[q + 3] += u.w;
      }
    }
  }
  uint32_t o[kCols / 2];
#pragma unroll
  for (int q = 0; q < kCols; q += 2) {
    float h0 = v[q], h1 = v[q + 1];
    if constexpr (kSwiglu) {
      h0 = h0 * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(h0 * -1.4426950408889634f)) * up[q];
      h1 = h1 * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(h1 * -1.4426950408889634f)) * up[q + 1];
    }
    const bf16x2 pr = {(__bf16)h0, (__bf16)h1};
    o[q / 2] = __builtin_bit_cast(uint32_t, pr);
  }
  u32x4 *dst = reinterpret_cast<u32x4 *>(p.out + static_cast<int64_t>(t.row0 + r) * p.ncols + col);
  dst[0] = u32x4{o[0], o[1], o[2], o[3]};
  if constexpr (!kSwiglu) {
    if (col + 8 < p.ncols) dst[1] = u32x4{o[4], o[5], o[6], o[7]};
  }
}

// Forward GEMM for short groups (plain epilogue, A rows in place; e.g.
// kernel_cases/case03_moe_grouped_gemm_fc1_fwd.py: 40 groups of ~102 rows,
// every weight element used by ~102 rows, so the stream of w is the work):
// tiles of 128 rows x 32 kNB columns (a group's rows in ceil(m / 128) row
// tiles, N in column tiles), numbered group by group and dealt round-robin to
// persistent workgroups so an XCD takes neighbouring column tiles of a group
// (its rows come from L2). 8 wavefronts, on each SIMD one computing (64 rows x
// 16 kNB columns as 4 x kNB blocks of v_mfma_f32_16x16x32_bf16, the weight
// fragment first and K ascending: the MFMA sequence of the ping-pong kernel,
// so the output is bit-identical) and one loading: two DMA the tile's rows
// into a ring of kSA stages, two the weight rows into a ring of kSB stages
// (a wavefront's loads complete in issue order, so each operand keeps its own
// lookahead; the weights load non-temporally, each is used by one tile when
// the groups have at most 128 rows). One barrier per step; the stages of a
// workgroup's tiles form one stream, so the next tile's first stages load
// while the last tile's results are stored. The host picks kNB (the column
// tile width) that spreads the tiles most evenly over the workgroups. Output:
// 4 consecutive bf16 columns per lane and block, one 8-byte store; rows past
// the group's end lie past the store resource, columns past N get an offset
// past it.
template <int kNB, bool kNtW = MOE_GEMM_FWD128_NT>
__global__ __launch_bounds__(512) void grouped_gemm_fwd128_kernel(GemmArgs p) {
  constexpr int kTM = 128;
  constexpr int kTN = 32 * kNB;
  constexpr int kABytes = kTM * kRowBytes;       // 16 KiB
  constexpr int kBBytes = kTN * kRowBytes;
  constexpr int kSA = MOE_GEMM_FWD128_SA ? MOE_GEMM_FWD128_SA : (kNB <= 5 ? 5 : 4);
  constexpr int kSBFit = (160 * 1024 - kSA * kABytes) / kBBytes;
  constexpr int kSBCap = MOE_GEMM_FWD128_SB ? MOE_GEMM_FWD128_SB : 4;
  constexpr int kSB = kSBFit > kSBCap ? kSBCap : kSBFit;
  constexpr int kDmaA = kABytes / 1024 / 2, kDmaB = kBBytes / 1024 / 2;  // per loading wavefront
  static_assert(kSA >= 3 && kSB >= 3 && kSA * kABytes + kSB * kBBytes <= 160 * 1024, "LDS budget");
  static_assert((kSA - 1) * kDmaA <= 63 && (kSB - 1) * kDmaB <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[kSA * kABytes + kSB * kBBytes];
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t a_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));
  const uint32_t b_lds = a_lds + kSA * kABytes;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  // ---- roles: the first wavefront of each SIMD computes (index = its SIMD), the second loads (SIMD 0 and
  // 1: the tile's rows, 2 and 3: weight rows), read from HW_ID and exchanged through LDS.
  int role_simd, loader;
  {
    const int simd = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_s_getreg((1 << 11) | (4 << 6) | 4)) & 3;
    volatile int *sid = reinterpret_cast<volatile int *>(smem);
    if (lane == 0) sid[wave] = simd;
    __syncthreads();
    int before = 0, per_simd[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const int sv = sid[w] & 3;
      per_simd[sv] += 1;
      before += (sv == simd) && (w < wave);
    }
    __syncthreads();
    const bool ok = per_simd[0] == 2 && per_simd[1] == 2 && per_simd[2] == 2 && per_simd[3] == 2;
    role_simd = __builtin_amdgcn_readfirstlane(ok ? simd : (wave & 3));
    loader = __builtin_amdgcn_readfirstlane(ok ? before : (wave >> 2));
  }
  const int64_t K = p.K, N = p.N;
  const int ktiles = static_cast<int>(K / kBK);
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;
  const int m32 = static_cast<int>(p.M), g_count = static_cast<int>(p.G);
  const int ntl = static_cast<int>((N + kTN - 1) / kTN);

  // ---- tile walker (every wavefront walks the same tiles): group by group, row tile-major
  struct Tile {
    int g, i0, rows, nt;
  };
  int g_cur = 0, g_lo = 0, g_hi = 0, mt_g = 0;
  int64_t tiles_before = 0;
  auto range = [&](int g) {
    g_lo = min(max(ld_inv(p.offsets, g), 0), m32);
    g_hi = min(max(ld_inv(p.offsets, g + 1), g_lo), m32);
    mt_g = (g_hi - g_lo + kTM - 1) / kTM;
  };
  range(0);
  const int64_t P = gridDim.x, b = blockIdx.x;
  const int64_t r0 = (b % 8) * (P / 8) + b / 8;
  auto find = [&](int64_t round, Tile &t) -> bool {
    const int64_t L = round * P + r0;
    while (g_cur < g_count && L >= tiles_before + static_cast<int64_t>(mt_g) * ntl) {
      tiles_before += static_cast<int64_t>(mt_g) * ntl;
      if (++g_cur < g_count) range(g_cur);
    }
    if (g_cur >= g_count) return false;
    const int q = static_cast<int>(L - tiles_before);
    const int mt = q / ntl;
    t.g = g_cur;
    t.i0 = g_lo + mt * kTM;
    t.rows = min(kTM, g_hi - t.i0);
    t.nt = q - mt * ntl;
    return true;
  };

  Tile t;
  if (!find(0, t)) return;  // no tiles: every wavefront leaves before the first barrier

  if (loader) {
    const bool is_a = role_simd < 2;
    const int li = role_simd & 1;
    int ln = lane;
    asm volatile("" : "+v"(ln));
    auto tile_rsrc = [&](const Tile &u, bool a) {
      // Rows past the tile's rows / past N lie past the resource: zeros.
      return a ? make_rsrc(p.a + static_cast<int64_t>(u.i0) * K, static_cast<uint32_t>(u.rows) * row_bytes)
               : make_rsrc(p.w + static_cast<int64_t>(u.g) * N * K + static_cast<int64_t>(u.nt) * kTN * K,
                           static_cast<uint32_t>(min<int64_t>(kTN, N - static_cast<int64_t>(u.nt) * kTN)) * row_bytes);
    };
    // The stages of this workgroup's tiles form one stream (tile by tile, K ascending), so the rings run on
    // from one tile into the next: the next tile's first stages load while the last one's results are stored.
    auto run = [&](auto is_a_c) {
      constexpr bool kA = decltype(is_a_c)::value;
      constexpr int kS = kA ? kSA : kSB;
      constexpr int kN = kA ? kDmaA : kDmaB;
      constexpr int kSlot = kA ? kABytes : kBBytes;
      const uint32_t ring = (kA ? a_lds : b_lds) + li * kN * 1024;
      const int r_0 = li * kN * 8 + (ln >> 3);  // row of this wavefront's 1 KiB block j (8 rows): r_0 + 8 j
      int off[kN];
#pragma unroll
      for (int j = 0; j < kN; ++j) {
        const int r = r_0 + j * 8;
        off[j] = static_cast<int>(static_cast<uint32_t>(r) * row_bytes + static_cast<uint32_t>(((ln & 7) ^ swz(r)) << 4));
      }
      __amdgpu_buffer_rsrc_t rs = tile_rsrc(t, kA);
      int64_t round = 0;
      int kt = 0;
      bool more = true;
      int64_t issued = 0, end = INT64_MAX;  // stages issued; stages of all tiles (known once the last is issued)
      // The next stage of the stream (its resource and K step); past the last one, the last stage again (the
      // same number of loads in flight in every step; they land in slots nothing reads any more).
      struct Src {
        __amdgpu_buffer_rsrc_t rs;
        int k;
      };
      auto advance = [&]() -> Src {
        const Src v{rs, more ? kt : ktiles - 1};
        ++issued;
        if (more && ++kt == ktiles) {
          kt = 0;
          more = find(++round, t);
          if (more) rs = tile_rsrc(t, kA);
          else end = issued;
        }
        return v;
      };
      constexpr int kAux = (!kA && kNtW) ? 2 : 0;
      auto one = [&](int slot) {
        const Src v = advance();
        const uint32_t dst = ring + slot * kSlot;
#pragma unroll
        for (int j = 0; j < kN; ++j) dma16b<kAux>(v.rs, (lds_void *)(uintptr_t)(dst + j * 1024), off[j], v.k * kBK * 2);
      };
      for (int st = 0; st < kS - 1; ++st) one(st);
      wait_vm_n<(kS - 2) * kN>();  // stage 0 has landed
      barrier();
      int slot = kS - 1;
      // Step s: the computing wavefronts read stage s; its barrier is passed once stage s + 1 has landed.
      // `end` is known here: `issued` runs kS - 1 stages ahead of s.
      for (int64_t s = 0; s < end; ++s) {
        one(slot);  // into the slot of stage s - 1, read before the last barrier
        slot = slot + 1 == kS ? 0 : slot + 1;
        wait_vm_n<(kS - 2) * kN>();
        barrier();
      }
      wait_dma();
    };
    if (is_a) run(std::true_type{});
    else run(std::false_type{});
    return;
  }

  const int wr = role_simd >> 1, wc = role_simd & 1;
  const int frow = lane & 15, fq = lane >> 4;
  auto frag_addr = [&](uint32_t slot_base, int r, int ks) {
    return slot_base + r * kRowBytes + ((((ks << 2) | fq) ^ swz(r)) << 4);
  };
  bf16x8 fa[2][4], fb[2][kNB];
  int sa = 0, sb = 0;  // ring slots of the stage being read
  auto read_half = [&](int ks, int buf) {
    const uint32_t ab = a_lds + sa * kABytes, bb = b_lds + sb * kBBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[buf][i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)frag_addr(ab, wr * 64 + i * 16 + frow, ks));
#pragma unroll
    for (int j = 0; j < kNB; ++j)
      fb[buf][j] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)frag_addr(bb, wc * 16 * kNB + j * 16 + frow, ks));
  };
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 acc[4][kNB];
  auto mfma_half = [&](int buf, bool zero) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[buf][j], fa[buf][i], zero ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j],
                                                           0, 0, 0);
  };
  const uint32_t ld = static_cast<uint32_t>(p.ncols) * 2u;
  barrier();  // stage 0 has landed
  for (int64_t round = 0;;) {
    read_half(0, 0);
    for (int kt = 0; kt < ktiles; ++kt) {
      read_half(1, 1);
      mfma_half(0, kt == 0);
      __builtin_amdgcn_sched_barrier(0);
      wait_lds();  // this wavefront's reads of stage kt are done before its slot can be refilled
      barrier();   // the next stage has landed
      sa = sa + 1 == kSA ? 0 : sa + 1;
      sb = sb + 1 == kSB ? 0 : sb + 1;
      if (kt + 1 < ktiles) read_half(0, 0);
      mfma_half(1, false);
      __builtin_amdgcn_sched_barrier(0);
    }
    // acc[i][j] register r of lane l: row wr 64 + i 16 + l % 16, column wc 16 kNB + j 16 + 4 (l / 16) + r.
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(p.out + static_cast<int64_t>(t.i0) * p.ncols, static_cast<uint32_t>(t.rows) * ld);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t orow = static_cast<uint32_t>(wr * 64 + i * 16 + frow);
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        const int64_t col = static_cast<int64_t>(t.nt) * kTN + wc * 16 * kNB + j * 16 + fq * 4;
        const bf16x2 lo = {(__bf16)acc[i][j][0], (__bf16)acc[i][j][1]};
        const bf16x2 hi = {(__bf16)acc[i][j][2], (__bf16)acc[i][j][3]};
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = {__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
        const uint32_t off = col < N ? orow * ld + static_cast<uint32_t>(col) * 2u : kNoAccess;
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_raw_buffer_store_b64(v, ro, static_cast<int>(off), 0, 0);
#else
        (void)off;
        (void)v;
        (void)ro;
#endif
      }
    }
    if (!find(++round, t)) break;
  }
}

}  // namespace
}  // namespace moe

namespace {

// The tail list applies with long reductions (K >= 4096: c5 fc1 2.4% faster),
// and with short ones where the groups average fewer than 256 rows, i.e. most
// of their rows lie in a tail (case04, 40 groups of 102 rows, K = 2560: 8%
// faster); with short reductions and long groups the 128-row tiles' start and
// drain cost more than the padding they save (c5 fc2: 1.2-2.4% slower).
bool tails_apply(int64_t M_total, int64_t K, int64_t G) {
  return K % moe::gemm::kBK == 0 && (K >= moe::gemm::kTailsMinK || M_total < 256 * G);
}

// Reduction split plan of a one-group GEMM whose 256-row tiles leave the last
// round at most half full (e.g. 320 tiles on 256 CUs): the last `tiles` tiles
// run as `ways` K ranges each, one unit per CU, after the other tiles.
struct SplitPlan {
  int tiles = 0, ways = 0, steps = 0;
  size_t bytes = 0;  // fp32 planes
};

SplitPlan split_plan(int64_t M_total, int64_t K, int64_t N, int64_t G, int64_t cus) {
  using namespace moe;
  SplitPlan sp;
  if (G != 1 || K % kBK != 0 || M_total <= 0 || N <= 0) return sp;
  const int64_t S = K / kBK;
  const int64_t total = ceil_div(M_total, 256) * ceil_div(N, 256);  // SwiGLU: ceil(N/2 / 128), the same
  const int64_t P = std::max<int64_t>(8, cus / 8 * 8);
  const int64_t L = total % P;  // tiles of the last round (all of them when total < P)
  if (L == 0 || 2 * L > P) return sp;
  const int64_t ways = std::min<int64_t>({P / L, S / 3, 8});
  if (ways < 2) return sp;
  sp.tiles = static_cast<int>(L);
  sp.ways = static_cast<int>(ways);
  sp.steps = static_cast<int>(S / ways);
  sp.bytes = static_cast<size_t>(L * ways) * 65536 * sizeof(float);
  return sp;
}

// Column tile width (32 kNB) of the 128-row forward kernel: tiles of groups of the mean row count, the
// rounds over P workgroups priced at their width plus a fixed 32 columns (the tile's A rows and stores).
int fwd128_nb(int64_t M_total, int64_t N, int64_t G, int64_t P) {
  const int64_t mt = moe::ceil_div(moe::ceil_div(M_total, G), 128);
  int best = 4;
  int64_t best_cost = INT64_MAX;
  for (int nb : {4, 5, 6}) {
    const int64_t tn = 32 * nb;
    const int64_t cost = moe::ceil_div(G * mt * moe::ceil_div(N, tn), P) * (tn + 32);
    if (cost < best_cost) best_cost = cost, best = nb;
  }
  return best;
}

int launch_grouped_gemm(const char *fn, const moe_bf16_t *a, int64_t a_src_rows, const int32_t *a_rows,
                        int64_t M_total, int64_t K, const moe_bf16_t *w, int64_t G, int64_t N,
                        const int32_t *group_offsets, int epilogue, moe_bf16_t *out, void *workspace,
                        size_t workspace_bytes, void *stream) {
  using namespace moe;
  const bool gather = a_rows != nullptr;
  if (M_total < 0 || K < 0 || N < 0 || G < 0 || a_src_rows < 0) {
    return fail(MOE_ERR_SHAPE, "%s: negative size (M=%lld K=%lld N=%lld G=%lld)", fn, (long long)M_total,
                (long long)K, (long long)N, (long long)G);
  }
  if (epilogue != MOE_EPILOGUE_NONE && epilogue != MOE_EPILOGUE_SWIGLU) {
    return fail(MOE_ERR_INVALID_ARG, "%s: epilogue %d is not a moe_epilogue_t", fn, epilogue);
  }
  if (G < 1 || G > 4096) return fail(MOE_ERR_CAPACITY, "%s: G=%lld outside [1, 4096]", fn, (long long)G);
  if (K % 8 != 0 || K == 0) return fail(MOE_ERR_SHAPE, "%s: K=%lld must be a positive multiple of 8", fn, (long long)K);
  // 32-bit buffer offsets: a 256-row panel of a (gather: all of x) and one
  // expert's w must each span less than 2 GiB.
  if (K > (int64_t(1) << 22) - 8 || N * K > (int64_t(1) << 30) - 1 || (gather && a_src_rows * K > (int64_t(1) << 30) - 1)) {
    return fail(MOE_ERR_CAPACITY,
                "%s: K=%lld N=%lld (x rows %lld) exceed the 32-bit panel offsets (K < 2^22, N*K and x_rows*K < 2^30)",
                fn, (long long)K, (long long)N, (long long)a_src_rows);
  }
  const bool swiglu = epilogue == MOE_EPILOGUE_SWIGLU;
  if (swiglu && (N % 2 != 0)) return fail(MOE_ERR_SHAPE, "%s: SWIGLU needs an even N (got %lld)", fn, (long long)N);
  if (group_offsets == nullptr) return fail(MOE_ERR_INVALID_ARG, "%s: null group_offsets", fn);
  const int64_t ncols = swiglu ? N / 2 : N;
  if (M_total == 0 || ncols == 0) return MOE_OK;
  if (a == nullptr || w == nullptr || out == nullptr) return fail(MOE_ERR_INVALID_ARG, "%s: null a, w or out", fn);
  if (gather && a_src_rows == 0) return fail(MOE_ERR_SHAPE, "%s: x has no rows", fn);
  if (!is_aligned(a, 16) || !is_aligned(w, 16)) return fail(MOE_ERR_ALIGN, "%s: a and w must be 16-byte aligned", fn);
  GemmArgs p;
  p.a = a;
  p.a_rows = a_rows;
  p.a_src_rows = a_src_rows;
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
  // The pipelined kernel needs three K steps per tile, 16-byte output rows, a
  // 256-row output panel below 2 GiB and (gather) 32-bit offsets into a_rows.
  const bool pipe = K > 2 * kBK && p.vec_out && ncols < (int64_t(1) << 22) && (!gather || M_total < (int64_t(1) << 29));
  // The ping-pong kernel: the same conditions, whole K steps and row numbers in 31 bits.
  const bool pingpong = MOE_GEMM_PINGPONG && pipe && K % kBK == 0 && M_total < (int64_t(1) << 31);
  // Groups of at most 128 rows on average, plain epilogue, A rows in place: 128-row tiles with their own
  // loading wavefronts (no workspace).
  if (MOE_GEMM_FWD128 && pingpong && !swiglu && !gather && M_total <= 128 * G) {
    const int64_t P = std::max<int64_t>(8, num_cus() / 8 * 8);
    switch (MOE_GEMM_FWD128_NB ? MOE_GEMM_FWD128_NB : fwd128_nb(M_total, N, G, P)) {
      case 4: grouped_gemm_fwd128_kernel<4><<<dim3(P), dim3(512), 0, s>>>(p); break;
      case 5: grouped_gemm_fwd128_kernel<5><<<dim3(P), dim3(512), 0, s>>>(p); break;
      default: grouped_gemm_fwd128_kernel<6><<<dim3(P), dim3(512), 0, s>>>(p); break;
    }
    return check_launch(fn);
  }
  // With a workspace and a long reduction, group tails of at most 128 rows
  // are listed first and computed as 128-row tiles after the 256-row ones
  // (with short reductions the 128-row tiles' start and drain measured slower
  // than the padding rows they save).
  p.tails = nullptr;
  p.split_tiles = p.split_ways = p.split_steps = 0;
  p.planes = nullptr;
  // One group whose last round of tiles is sparse: with a large enough workspace, a reduction split of
  // those tiles (the results differ from the unsplit ones only in the order of their fp32 partial sums).
  const SplitPlan sp = pingpong ? split_plan(M_total, K, N, G, num_cus()) : SplitPlan{};
  if (sp.tiles > 0 && workspace != nullptr && workspace_bytes >= sp.bytes && is_aligned(workspace, 256)) {
    p.split_tiles = sp.tiles;
    p.split_ways = sp.ways;
    p.split_steps = sp.steps;
    p.planes = static_cast<float *>(workspace);
    const int64_t units = static_cast<int64_t>(sp.tiles) * sp.ways;
    const int64_t total = ceil_div(M_total, 256) * p.ntiles;
    if (total > sp.tiles) {
      const int64_t g0 = std::max<int64_t>(8, std::min<int64_t>(grid, total - sp.tiles) / 8 * 8);
      if (swiglu) {
        if (gather) grouped_gemm_pp_kernel<true, true, false><<<dim3(g0), dim3(512), 0, s>>>(p);
        else grouped_gemm_pp_kernel<true, false, false><<<dim3(g0), dim3(512), 0, s>>>(p);
      } else {
        if (gather) grouped_gemm_pp_kernel<false, true, false><<<dim3(g0), dim3(512), 0, s>>>(p);
        else grouped_gemm_pp_kernel<false, false, false><<<dim3(g0), dim3(512), 0, s>>>(p);
      }
    }
    const dim3 gu(static_cast<uint32_t>((units + 7) / 8 * 8));
    if (swiglu) {
      if (gather) grouped_gemm_split_kernel<true, true><<<gu, dim3(512), 0, s>>>(p);
      else grouped_gemm_split_kernel<true, false><<<gu, dim3(512), 0, s>>>(p);
      split_sum_kernel<true><<<dim3(sp.tiles, 16), dim3(256), 0, s>>>(p);
    } else {
      if (gather) grouped_gemm_split_kernel<false, true><<<gu, dim3(512), 0, s>>>(p);
      else grouped_gemm_split_kernel<false, false><<<gu, dim3(512), 0, s>>>(p);
      split_sum_kernel<false><<<dim3(sp.tiles, 16), dim3(256), 0, s>>>(p);
    }
    return check_launch(fn);
  }
  if (pingpong && tails_apply(M_total, K, G) && workspace != nullptr && workspace_bytes >= tails_bytes(G) &&
      is_aligned(workspace, 256)) {
    p.tails = static_cast<int *>(workspace);
    tails_init_kernel<<<dim3(1), dim3(256), 0, s>>>(p.offsets, p.G, p.M, p.tails);
  }
  if (pingpong && p.tails != nullptr) {
    if (swiglu) {
      if (gather) grouped_gemm_pp_kernel<true, true, true><<<dim3(grid), dim3(512), 0, s>>>(p);
      else grouped_gemm_pp_kernel<true, false, true><<<dim3(grid), dim3(512), 0, s>>>(p);
    } else {
      if (gather) grouped_gemm_pp_kernel<false, true, true><<<dim3(grid), dim3(512), 0, s>>>(p);
      else grouped_gemm_pp_kernel<false, false, true><<<dim3(grid), dim3(512), 0, s>>>(p);
    }
  } else if (pingpong) {
    if (swiglu) {
      if (gather) grouped_gemm_pp_kernel<true, true, false><<<dim3(grid), dim3(512), 0, s>>>(p);
      else grouped_gemm_pp_kernel<true, false, false><<<dim3(grid), dim3(512), 0, s>>>(p);
    } else {
      if (gather) grouped_gemm_pp_kernel<false, true, false><<<dim3(grid), dim3(512), 0, s>>>(p);
      else grouped_gemm_pp_kernel<false, false, false><<<dim3(grid), dim3(512), 0, s>>>(p);
    }
  } else if (pipe) {
    if (swiglu) {
      if (gather) grouped_gemm_pipe_kernel<true, true><<<dim3(grid), dim3(256), 0, s>>>(p);
      else grouped_gemm_pipe_kernel<true, false><<<dim3(grid), dim3(256), 0, s>>>(p);
    } else {
      if (gather) grouped_gemm_pipe_kernel<false, true><<<dim3(grid), dim3(256), 0, s>>>(p);
      else grouped_gemm_pipe_kernel<false, false><<<dim3(grid), dim3(256), 0, s>>>(p);
    }
  } else if (swiglu) {
    if (gather) grouped_gemm_kernel<true, true><<<dim3(grid), dim3(256), 0, s>>>(p);
    else grouped_gemm_kernel<true, false><<<dim3(grid), dim3(256), 0, s>>>(p);
  } else {
    if (gather) grouped_gemm_kernel<false, true><<<dim3(grid), dim3(256), 0, s>>>(p);
    else grouped_gemm_kernel<false, false><<<dim3(grid), dim3(256), 0, s>>>(p);
  }
  return check_launch(fn);
}

}  // namespace

extern "C" {

size_t moe_grouped_gemm_workspace_size(int64_t M_total, int64_t K, int64_t N, int64_t G) {
  if (G < 1 || G > 4096 || K % moe::gemm::kBK != 0 || K < 0 || N < 0 || M_total < 0) return 0;
  const SplitPlan sp = split_plan(M_total, K, N, G, moe::gemm::num_cus());
  if (sp.tiles > 0) return sp.bytes;
  if (!tails_apply(M_total, K, G)) return 0;
  return (moe::gemm::tails_bytes(G) + 255) / 256 * 256;
}

int moe_grouped_gemm(const moe_bf16_t *a, int64_t M_total, int64_t K, const moe_bf16_t *w, int64_t G,
                     int64_t N, const int32_t *group_offsets, int epilogue, moe_bf16_t *out,
                     void *workspace, size_t workspace_bytes, void *stream) {
  return launch_grouped_gemm("moe_grouped_gemm", a, 0, nullptr, M_total, K, w, G, N, group_offsets, epilogue, out,
                             workspace, workspace_bytes, stream);
}

int moe_grouped_gemm_gather(const moe_bf16_t *x, int64_t x_rows, const int32_t *a_rows, int64_t M_total,
                            int64_t K, const moe_bf16_t *w, int64_t G, int64_t N, const int32_t *group_offsets,
                            int epilogue, moe_bf16_t *out, void *workspace, size_t workspace_bytes, void *stream) {
  if (a_rows == nullptr && M_total > 0) {
    return moe::fail(MOE_ERR_INVALID_ARG, "moe_grouped_gemm_gather: null a_rows");
  }
  return launch_grouped_gemm("moe_grouped_gemm_gather", x, x_rows, a_rows, M_total, K, w, G, N, group_offsets,
                             epilogue, out, workspace, workspace_bytes, stream);
}

}  // extern "C"
