// Grouped GEMM backward over ragged expert groups: input gradient (dgrad, "NN")
// and weight gradient (wgrad, "TN"), bf16 MFMA with fp32 accumulate, bf16 out.
//
// Math (paths relative to the reference repository):
//   dgrad  kernel_cases/case07_moe_grouped_gemm_fc1_dgrad.py:57-64 (= case08,
//          case13, case19 :57-64; case37_ref_musa_asm_bf16_gemm_nn_256x384.py:47-49
//          for one group):  dx[rows of g] = dy[rows of g] @ w[g]
//          dy [M, N], w [G, N, K] -> dx [M, K]
//   wgrad  kernel_cases/case09_moe_grouped_gemm_fc1_wgrad.py:57-64 (= case05
//          :57-64):  dw[g] = dy[rows of g]^T @ x[rows of g]
//          dy [M, N], x [M, K] -> dw [G, N, K]  (a group without rows gets zeros)
// "bf16 in / fp32 accumulate / bf16 out" (case07...py:37).
//
// Both products have an operand whose reduction index is the slow (row)
// index in memory: w[g] is [N][K] with the reduction over N, and in wgrad both
// dy and x are reduced over their rows. Such an operand ("reduction-major",
// RM) is staged in LDS as it lies in memory, 64 reduction rows x 256 columns
// per stage (512-byte rows, 16-byte chunks XOR-swizzled per row), and its MFMA
// fragments are read with ds_read_b64_tr_b16: in each group of 16 lanes,
// lane 4j + q addresses row j, columns 4q .. 4q + 3 of a 4 x 16 block and
// lane i receives column i of rows 0..3, so two such reads (rows 4 apart) give
// a lane 8 consecutive reduction values of one column, the MFMA operand
// layout. dgrad's dy is reduced along its rows' contiguous axis ("KC") and is
// staged like the forward kernel's operands (128-byte rows, ds_read_b128).
//
// Two kernels, both persistent with one workgroup of 4 wavefronts per CU, a
// reduction step of 64 and an LDS ring filled by buffer_load ... lds ahead of
// the MFMAs:
//   * grouped_gemm_bwd_pipe_kernel (every 256 x 256 tile: dgrad with groups
//     above ~160 rows, wgrad, the tf32 router GEMMs): the forward pipelined
//     kernel's shape, v_mfma_f32_16x16x32_bf16 on 2 x 2 waves of 128 x 128,
//     two stages, tiles chained without draining the pipeline, epilogue from
//     registers; described above the kernel;
//   * grouped_gemm_dgrad128_kernel (dgrad with groups of at most ~160 rows, or
//     a reduction that is not whole steps): 128 x 256 tiles (1 x 4 waves of
//     128 x 64, less padding in every group's last row tile),
//     v_mfma_f32_32x32x16_bf16, three stages (its stream of w is HBM-bound and
//     needs two stages in flight); the next step's fragments are read while
//     the current step's MFMAs run; the epilogue rounds to bf16 (RNE,
//     hardware), pairs register groups across the two half-waves with
//     v_permlane32_swap so each lane holds 8 consecutive columns, and stores
//     16 bytes per lane straight from registers through a buffer resource
//     (stores past the tile's valid rows or columns are dropped), after the
//     next tile's first stages have been issued.
// Reduction rows past the end come from past the operand's buffer resource and
// read as zeros (the 128-row kernel zeroes dy's columns past N in LDS).
//
// Tiles are numbered group by group; inside a group in patches of 8 row tiles
// x all column tiles; workgroup b takes tile round * P + (b % 8) * (P / 8) + b / 8
// so each XCD works on one patch per round.
#include <algorithm>
#include <type_traits>

#include "gemm_device.h"

namespace moe {
namespace {

using namespace gemm;

typedef __bf16 v4bf16 __attribute__((__vector_size__(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4bf16 lds_v4bf16;

constexpr int kBN = 256;            // output columns per tile
constexpr int kGroupM = 8;          // row tiles per tile-order patch
constexpr int kSubSteps = kBK / 16;
constexpr int kKCRow = kBK * 2;     // 128-byte rows of a KC operand tile
constexpr int kRMRow = 256 * 2;     // 512-byte rows of an RM operand tile (256 columns)

struct BwdArgs {
  const uint16_t *a;        // dy [M, N]
  const uint16_t *b;        // dgrad: w [G, N, K]; wgrad: x [M, K]
  const int32_t *offsets;   // [G + 1], or nullptr: group g is rows [g chunk, (g + 1) chunk) of M
  void *out;                // dgrad: dx [M, K]; wgrad: dw [G, N, K] (bf16, or fp32 for kOut != 0)
  int64_t M, N, K, G;
  int64_t ntiles;           // column tiles, ceil(K / 256)
  int64_t chunk;            // rows per group when offsets is nullptr
  int64_t kchunk;           // split dgrad: reduction columns of split g = [g kchunk, (g + 1) kchunk), the last to N
  const int16_t *order;     // wgrad (kOrder): the groups in the order the tiles take them
  const int32_t *order_rows;  // wgrad (kOrder): [2 G] the clamped row range (lo, hi) of order[i] at 2 i
  int *tails;               // dgrad ping-pong kernel: tail list (kTail* layout) or nullptr
  int sweep_rows = 0;       // wgrad (kOrder): > 0 leaves the groups of at most this many rows to the sweep kernel
  int sweep_len = 0;        // sweep kernel: tiles per unit (one fixed slab)
  // fp16 dgrad (the tf32 router dgrad, 128-row kernel): the power-of-two scale exponents of dy's rows (int8,
  // permuted within each 128-row block: row 128 b + 32 i + l at byte 128 b + 4 l + i) and of dx's columns
  // (int8 [K]).
  const int8_t *row_exp8 = nullptr;
  const int8_t *col_exp8 = nullptr;
};

// Groups of the largest-first order with more than `limit` rows: the first
// position whose clamped row count is at most `limit` (binary search over the
// ordered row ranges; the counts do not increase along the order).
__device__ __forceinline__ int long_group_count(const int32_t *order_rows, int G, int m32, int limit) {
  int lo = 0, hi = G;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    const int r0 = min(max(ld_inv(order_rows, 2 * mid), 0), m32);
    const int r1 = min(max(ld_inv(order_rows, 2 * mid + 1), r0), m32);
    if (r1 - r0 <= limit) {
      hi = mid;
    } else {
      lo = mid + 1;
    }
  }
  return lo;
}

__device__ __forceinline__ int kc_swz(int row) { return (row >> 1) & 7; }
// RM chunk swizzle of the 128-row kernel's 32 x 32 x 16 fragments (a half-wave
// reads 4 rows x 64 bytes: (row % 4) x 4 chunks spreads them over all banks).
__device__ __forceinline__ int rm_swz(int krow) { return (krow & 3) << 2; }

// One transposing LDS read. The restrict-qualified pointer gives the access
// alias-scope information; without it the compiler assumes the read may
// alias any LDS DMA in flight and waits for all of them (vmcnt(0)) before it.
// The kernel orders its DMA and reads itself (wait + barrier per stage).
__device__ __forceinline__ v4bf16 read_tr(lds_v4bf16 *__restrict__ p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(p);
#else
  (void)p;
  return v4bf16{};
#endif
}

// Fragment of an RM operand whose LDS rows are kRow bytes apart: 8 consecutive
// reduction values of one column per lane, from two transposing reads 4 rows apart.
template <int kRow>
__device__ __forceinline__ bf16x8 read_rm_frag_rows(uint32_t addr) {
#if defined(__HIP_DEVICE_COMPILE__)
  const v4bf16 lo = read_tr((lds_v4bf16 *)(uintptr_t)addr);
  const v4bf16 hi = read_tr((lds_v4bf16 *)(uintptr_t)(addr + 4 * kRow));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#else
  (void)addr;
  return bf16x8{};
#endif
}
// The same with 256-column tiles (kRMRow-byte rows).
__device__ __forceinline__ bf16x8 read_rm_frag(uint32_t addr) { return read_rm_frag_rows<kRMRow>(addr); }

// One 16 x 16 x 32 MFMA on 16-bit operands: bf16, or fp16 (kF16: the tf32 router GEMMs' scaled operands,
// the same bit layout in LDS and registers).
template <bool kF16>
__device__ __forceinline__ f32x4_t mma16(bf16x8 a, bf16x8 b, f32x4_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (kF16) {
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
#else
  (void)a;
  (void)b;
  return c;
#endif
}

// The 128-row dgrad kernel (groups of at most ~160 rows, reductions that are
// not whole steps): 1 x 4 waves of 128 x 64, a three-stage ring (the stream of
// w is HBM-bound here and needs two stages in flight), v_mfma_f32_32x32x16_bf16.
// kOut: 0 = bf16 output, 1 = fp32 output (the next tile's stages are then
// issued after the stores). kNtB: w is streamed once (the groups average at
// most 160 rows, one or two row tiles each): non-temporal loads for it.
// kF16 (the tf32 router dgrad, fp32 output, rows [0, M) as one group): fp16
// operands scaled by powers of two per dy row and per dx column
// (p.row_exp8, p.col_exp8), undone in the epilogue.
// kTN, kStagesT: columns per tile (256, or 128: 256-byte RM rows) and ring
// stages; with 128 columns and 2 stages (64 KiB of LDS, 64 accumulators per
// lane) two workgroups share a CU, so one's stores drain under the other's
// MFMAs.
template <int kOut, bool kNtB = false, bool kF16 = false, int kTN = 256, int kStagesT = 3>
__global__ __launch_bounds__(256, kTN == 128 ? 2 : 1) void grouped_gemm_dgrad128_kernel(BwdArgs p) {
  static_assert(!kF16 || kOut == 1, "fp16 operands: the tf32 router dgrad (fp32 output)");
  static_assert(kTN == 256 || kTN == 128, "256 or 128 columns per tile");
  constexpr int kBM = 128, kWavesM = 1, kStages = kStagesT;
  constexpr int kWaves = 4;
  constexpr int kWavesN = kWaves / kWavesM;
  constexpr int kWaveRows = kBM / kWavesM;
  constexpr int kWaveCols = kTN / kWavesN;
  constexpr int kMI = kWaveRows / 32, kNI = kWaveCols / 32;
  constexpr int kABytes = kBM * kBK * 2;
  constexpr int kBBytes = kTN * kBK * 2;
  constexpr int kRow = kTN * 2;                  // bytes per RM row of the B tile
  constexpr int kRowsPerBlk = 1024 / kRow;       // RM rows per 1 KiB DMA block
  constexpr int kStageBytes = kABytes + kBBytes;
  constexpr int kDmaA = kABytes / 1024 / kWaves, kDmaB = kBBytes / 1024 / kWaves;
  // Next tile's stages issued after the stores (fp32 output; the fp16 form issues them before, as the bf16
  // output does: its tiles have few reduction steps, so the next stages' latency would not be hidden).
  constexpr bool kLate = kOut != 0 && !kF16;
  constexpr int kStores = kLate ? 0 : kMI * kNI * (kOut != 0 ? 4 : 2);  // stores younger than the next stages
  constexpr int kReads = kMI + 2 * kNI;          // LDS reads per sub-step
  constexpr int kMfma = kMI * kNI;              // MFMAs per sub-step
  static_assert(kStages * kStageBytes <= 160 * 1024, "LDS budget");
  static_assert(kStores + (kStages - 1) * (kDmaA + kDmaB) <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[kStages * kStageBytes];
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / kWavesN;
  const int wn = wave % kWavesN;
  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t N = p.N, K = p.K;
  const bool a_ktail = (N % kBK) != 0;  // dy columns past N in the last step

  // ---- tile walker
  auto group_range = [&](int64_t g, int64_t &lo, int64_t &hi) {
    if (p.offsets == nullptr) {
      lo = min(g * p.chunk, p.M);
      hi = min(lo + p.chunk, p.M);
      return;
    }
    lo = min(max(static_cast<int64_t>(ld_inv(p.offsets, g)), int64_t(0)), p.M);
    hi = min(max(static_cast<int64_t>(ld_inv(p.offsets, g + 1)), lo), p.M);
  };
  auto row_tiles = [&](int64_t lo, int64_t hi) -> int64_t { return ceil_div(hi - lo, kBM); };
  int64_t g_cur = 0, tiles_before = 0, g_lo, g_hi;
  group_range(0, g_lo, g_hi);
  int64_t mt_g = row_tiles(g_lo, g_hi);
  struct Tile {
    int64_t g, lo, hi;  // group and its rows
    int64_t i0;         // first output row of the tile
    uint32_t nt;        // column tile
    int ktiles;         // reduction steps (at least 1: an empty reduction reads zeros)
  };
  auto find_tile = [&](int64_t round, Tile &t) -> bool {
    const int64_t L = round * P + (b % 8) * (P / 8) + b / 8;
    while (g_cur < p.G && L >= tiles_before + mt_g * p.ntiles) {
      tiles_before += mt_g * p.ntiles;
      ++g_cur;
      if (g_cur < p.G) {
        group_range(g_cur, g_lo, g_hi);
        mt_g = row_tiles(g_lo, g_hi);
      }
    }
    if (g_cur >= p.G) return false;
    const uint32_t q = static_cast<uint32_t>(L - tiles_before);
    const uint32_t per_grp = kGroupM * static_cast<uint32_t>(p.ntiles);
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
    t.lo = g_lo;
    t.hi = g_hi;
    t.i0 = g_lo + static_cast<int64_t>(mt) * kBM;
    t.nt = nt;
    t.ktiles = static_cast<int>(max(ceil_div(N, kBK), int64_t(1)));
    return true;
  };

  // ---- DMA sources of the tile being loaded
  __amdgpu_buffer_rsrc_t ra, rb;
  int a_off[kDmaA], b_off[kDmaB];
  int a_step = 0, b_step = 0;  // bytes per reduction step
  auto setup_dma = [&](const Tile &t) {
    // RM operand lane map: DMA block blk holds reduction rows 2 blk, 2 blk + 1.
    const int rm_krow = lane / (64 / kRowsPerBlk), rm_pchunk = lane & (kRow / 16 - 1);
    {
      const int rows_valid = static_cast<int>(min(t.hi - t.i0, int64_t(kBM)));
      ra = make_rsrc(p.a + t.i0 * N, static_cast<uint32_t>(rows_valid) * static_cast<uint32_t>(N) * 2u);
      rb = make_rsrc(p.b + t.g * N * K, static_cast<uint32_t>(N * K * 2));
      a_step = kBK * 2;
#pragma unroll
      for (int j = 0; j < kDmaA; ++j) {
        const int r = (j * kWaves + wave) * 8 + (lane >> 3);
        const int lchunk = (lane & 7) ^ kc_swz(r);
        // Rows past the group's end read as zeros (results dropped; zero
        // operands cost the MFMAs less energy than a repeated real row).
        a_off[j] = r < rows_valid ? static_cast<int>(static_cast<uint32_t>(r) * static_cast<uint32_t>(N) * 2u +
                                                     lchunk * 16)
                                  : static_cast<int>(kNoAccess);
      }
    }
    b_step = kBK * static_cast<int>(K) * 2;
    const uint32_t col0 = t.nt * static_cast<uint32_t>(kTN);
#pragma unroll
    for (int j = 0; j < kDmaB; ++j) {
      const int krow = (j * kWaves + wave) * kRowsPerBlk + rm_krow;
      const int lchunk = rm_pchunk ^ rm_swz(krow);
      b_off[j] = static_cast<int>(static_cast<uint32_t>(krow) * static_cast<uint32_t>(K) * 2u + col0 * 2u + lchunk * 16);
    }
  };
  auto issue_a = [&](int kt, int slot) {
    const uint32_t st = lds_base + (slot % kStages) * kStageBytes;
#pragma unroll
    for (int j = 0; j < kDmaA; ++j)
      dma16b(ra, (lds_void *)(uintptr_t)(st + (j * kWaves + wave) * 1024), a_off[j], kt * a_step);
  };
  auto issue_b = [&](int kt, int slot) {
    const uint32_t st = lds_base + (slot % kStages) * kStageBytes + kABytes;
#pragma unroll
    for (int j = 0; j < kDmaB; ++j)
      dma16b<kNtB ? 2 : 0>(rb, (lds_void *)(uintptr_t)(st + (j * kWaves + wave) * 1024), b_off[j], kt * b_step);
  };
  // dgrad: zero dy's chunks past column N in the A tile of stage kt.
  auto zero_ktail_a = [&](int kt) {
    lds_char *st = sbase + (kt % kStages) * kStageBytes;
    const int kvalid = static_cast<int>(N - static_cast<int64_t>(kt) * kBK);
    for (int idx = tid; idx < kBM * 8; idx += kWaves * 64) {
      const int r = idx >> 3, c = idx & 7;
      if (c * 8 >= kvalid) *reinterpret_cast<lds_u32x4 *>(st + r * kKCRow + ((c ^ kc_swz(r)) * 16)) = u32x4{0u, 0u, 0u, 0u};
    }
  };

  // ---- fragment addresses (LDS bytes relative to a stage)
  // RM: lane 16 G + 4 j + q reads row (G / 2) * 8 + j (+ 4 for the second
  // read), bytes ((G & 1) * 16 + 4 q) * 2 of the 32-column block, swizzled.
  const int rm_g = lane >> 4, rm_j = (lane >> 2) & 3, rm_q = lane & 3;
  const int rm_lane = ((rm_g >> 1) * 8 + rm_j) * kRow + (((rm_g & 1) * 2 + (rm_q >> 1)) << 4) + (rm_q & 1) * 8;
  auto rm_base = [&](int c0) { return rm_lane + ((c0 * 2) ^ (rm_j << 6)); };
  const int khalf = lane >> 5;
  int fa_base[kMI], fb_base[kNI];
#pragma unroll
  for (int i = 0; i < kMI; ++i) {
    const int r = wm * kWaveRows + i * 32 + (lane & 31);
    fa_base[i] = (r * kKCRow | (kc_swz(r) << 4)) ^ (khalf << 4);
  }
#pragma unroll
  for (int j = 0; j < kNI; ++j) fb_base[j] = kABytes + rm_base(wn * kWaveCols + j * 32);

  f32x16 acc[kMI][kNI];
  uint32_t rd_a[kMI], rd_b[kNI];
  auto set_read_slot = [&](int kt) {
    const uint32_t so = lds_base + (kt % kStages) * kStageBytes;
#pragma unroll
    for (int i = 0; i < kMI; ++i) rd_a[i] = so + fa_base[i];
#pragma unroll
    for (int j = 0; j < kNI; ++j) rd_b[j] = so + fb_base[j];
  };
  bf16x8 fa[kSubSteps][kMI], fb[kSubSteps][kNI];
  auto read_frags = [&](int ks) {
#pragma unroll
    for (int i = 0; i < kMI; ++i) fa[ks][i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(rd_a[i] ^ (ks << 5)));
#pragma unroll
    for (int j = 0; j < kNI; ++j) fb[ks][j] = read_rm_frag_rows<kRow>(rd_b[j] + ks * 16 * kRow);
  };
  auto mfma_ks = [&](int ks) {
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < kNI; ++j)
        if constexpr (kF16) {
          typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, fb[ks][j]),
                                                            __builtin_bit_cast(f16x8, fa[ks][i]), acc[i][j], 0, 0, 0);
        } else {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ks][j], fa[ks][i], acc[i][j], 0, 0, 0);
        }
  };
  // kF16: the tile's scale exponents, int8 (rows 32 i + l % 32: byte i of ex_row; columns
  // 32 j + 8 g + 4 (l / 32) + r: byte r of ex_col[4 j + g]): the first tile's before its stage DMAs, the
  // next tile's after this tile's stores; the full wait that ends each tile's reduction covers them.
  uint32_t ex_row = 0u, ex_col[kNI * 4] = {};
  auto load_exps = [&](const Tile &t) {
    if constexpr (kF16) {
      const int64_t wrow0 = t.i0 + wm * kWaveRows;
      const bool rows_in = t.hi > wrow0;
      const __amdgpu_buffer_rsrc_t rr = make_rsrc(p.row_exp8 + (rows_in ? wrow0 : 0), rows_in ? 128u : 0u);
      const __amdgpu_buffer_rsrc_t rc = make_rsrc(p.col_exp8, static_cast<uint32_t>(K));
      const int64_t tcol0 = static_cast<int64_t>(t.nt) * kTN + wn * kWaveCols + (lane >> 5) * 4;
#if defined(__HIP_DEVICE_COMPILE__)
      ex_row = __builtin_amdgcn_raw_buffer_load_b32(rr, (lane & 31) * 4, 0, 0);
#pragma unroll
      for (int j = 0; j < kNI; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t gcol = tcol0 + j * 32 + g * 8;
          ex_col[4 * j + g] =
              __builtin_amdgcn_raw_buffer_load_b32(rc, gcol < K ? static_cast<int>(gcol) : static_cast<int>(kNoAccess), 0, 0);
        }
#else
      (void)rr;
      (void)rc;
      (void)tcol0;
#endif
    } else {
      (void)t;
    }
  };

  Tile cur;
  if (!find_tile(0, cur)) return;
  load_exps(cur);
  setup_dma(cur);
  // Every stage slot is filled (stages past the last re-read the last one), so
  // the count of outstanding loads is the same for every tile.
#pragma unroll
  for (int st = 0; st < kStages; ++st) {
    issue_a(min(st, cur.ktiles - 1), st);
    issue_b(min(st, cur.ktiles - 1), st);
  }

  for (int64_t round = 0;; ++round) {
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < kNI; ++j) acc[i][j] = f32x16{};

    // Stage 0 has landed. Younger: the other prefetched stages and, after the
    // first tile, the previous tile's output stores (issued after them).
    if (round == 0) {
      wait_vm_n<(kStages - 1) * (kDmaA + kDmaB)>();
    } else {
      wait_vm_n<kStores + (kStages - 1) * (kDmaA + kDmaB)>();
    }
    barrier();
    const int ktiles = cur.ktiles;
    if (a_ktail && ktiles == 1) {
      zero_ktail_a(0);
      wait_lds();
      barrier();
    }
    set_read_slot(0);
#pragma unroll
    for (int ks = 0; ks < kSubSteps; ++ks) read_frags(ks);

    for (int kt = 0; kt + 1 < ktiles; ++kt) {
      mfma_ks(0);
      __builtin_amdgcn_sched_barrier(0);
      // Stage kt + 1 has landed (and, after the barrier, everyone's; this
      // thread's reads of stage kt are done). Younger and allowed to be in
      // flight: stage kt + 2 and, in the first steps after a tile change, the
      // previous tile's output stores, issued after this tile's first stages.
      if (kt <= kStages - 2 && round > 0) {
        wait_vm_n<(kStages - 2) * (kDmaA + kDmaB) + kStores>();
      } else {
        wait_vm_n<(kStages - 2) * (kDmaA + kDmaB)>();
      }
      wait_lds();
      barrier();
      if (a_ktail && kt + 1 == ktiles - 1) {
        zero_ktail_a(kt + 1);
        wait_lds();
        barrier();
      }
      // Stage kt + 2 into the slot of stage kt (the last step re-reads the
      // final stage into that free slot, so the region below has no branch).
      const int kdma = min(kt + kStages, ktiles - 1);
      set_read_slot(kt + 1);
      read_frags(0);
      mfma_ks(1);
      issue_a(kdma, kt + kStages);
      sched_mix<kMfma, kReads, kDmaA>();
      mfma_ks(2);
      read_frags(1);
      issue_b(kdma, kt + kStages);
      sched_mix<kMfma, kReads, kDmaB>();
      mfma_ks(3);
      read_frags(2);
      sched_mix<kMfma, kReads, 0>();
      read_frags(3);
      __builtin_amdgcn_sched_barrier(0);
    }
    mfma_ks(0);
    mfma_ks(1);
    mfma_ks(2);
    mfma_ks(3);

    // No DMA in flight and every wave done reading the ring: all prefetched
    // stages of the next tile are issued before this tile's output stores, so
    // the next tile's first waits do not wait for the stores.
    wait_dma();
    wait_lds();
    barrier();
    Tile nxt;
    const bool more = find_tile(round + 1, nxt);
    if (more && !kLate) {
      setup_dma(nxt);
#pragma unroll
      for (int st = 0; st < kStages; ++st) {
        issue_a(min(st, nxt.ktiles - 1), st);
        issue_b(min(st, nxt.ktiles - 1), st);
      }
    }

    // Epilogue straight from registers. Register r of lane l in block (i, j)
    // holds output row i * 32 + l % 32 and column j * 32 + (r / 4) * 8 +
    // (l / 32) * 4 + r % 4 of this wave's part. After bf16 rounding each
    // 4-register group is two packed words; v_permlane32_swap trades the upper
    // half-wave's words of group g with the lower half-wave's of group g + 1, so
    // a lower lane holds columns 8g .. 8g + 7 of its row and its upper partner
    // 8g + 8 .. 8g + 15: one 16-byte store each.
    if constexpr (kOut != 0) {
      // fp32: register group g of block (i, j) is 4 consecutive columns of
      // one row, stored as 16 bytes.
      const int64_t wrow0 = cur.i0 + wm * kWaveRows;
      const int rows_out = static_cast<int>(min(max(cur.hi - wrow0, int64_t(0)), int64_t(kWaveRows)));
      float *const obase = static_cast<float *>(p.out);
      const uint32_t ld = static_cast<uint32_t>(K) * 4u;
      const __amdgpu_buffer_rsrc_t ro =
          make_rsrc(obase + (rows_out > 0 ? wrow0 * K : 0), static_cast<uint32_t>(rows_out) * ld);
      const int64_t tcol0 = static_cast<int64_t>(cur.nt) * kTN + wn * kWaveCols;
      const int half = lane >> 5;
#pragma unroll
      for (int i = 0; i < kMI; ++i) {
        const int orow = i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < kNI; ++j) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int64_t gcol = tcol0 + j * 32 + g * 8 + half * 4;
            const uint32_t off = gcol < K ? static_cast<uint32_t>(orow) * ld + static_cast<uint32_t>(gcol) * 4u : kNoAccess;
            float x[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
            if constexpr (kF16) {
              // the scales undone: x 2^-(e_row + e_col), exact unless the result is subnormal
              const int er = static_cast<int8_t>(ex_row >> (8 * i));
#pragma unroll
              for (int r = 0; r < 4; ++r)
                x[r] = __builtin_ldexpf(x[r], -(er + static_cast<int8_t>(ex_col[4 * j + g] >> (8 * r))));
            }
            const u32x4 v = {__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])};
#if defined(__HIP_DEVICE_COMPILE__)
            __builtin_amdgcn_raw_buffer_store_b128(v, ro, static_cast<int>(off), 0, 0);
#else
            (void)off;
            (void)v;
            (void)ro;
#endif
          }
        }
      }
    } else {
      const int64_t wrow0 = cur.i0 + wm * kWaveRows;
      const int rows_out = static_cast<int>(min(max(cur.hi - wrow0, int64_t(0)), int64_t(kWaveRows)));
      const uint16_t *obase = static_cast<const uint16_t *>(p.out);
      const uint32_t ld = static_cast<uint32_t>(K) * 2u;
      const __amdgpu_buffer_rsrc_t ro =
          make_rsrc(obase + (rows_out > 0 ? wrow0 * K : 0), static_cast<uint32_t>(rows_out) * ld);
      const int64_t tcol0 = static_cast<int64_t>(cur.nt) * kTN + wn * kWaveCols;
      const int half = lane >> 5;
#pragma unroll
      for (int i = 0; i < kMI; ++i) {
        const int orow = i * 32 + (lane & 31);
#pragma unroll
        for (int j = 0; j < kNI; ++j) {
          uint32_t w[4][2];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const bf16x2 lo = {(__bf16)acc[i][j][4 * g], (__bf16)acc[i][j][4 * g + 1]};
            const bf16x2 hi = {(__bf16)acc[i][j][4 * g + 2], (__bf16)acc[i][j][4 * g + 3]};
            w[g][0] = __builtin_bit_cast(uint32_t, lo);
            w[g][1] = __builtin_bit_cast(uint32_t, hi);
          }
#pragma unroll
          for (int gp = 0; gp < 4; gp += 2) {
            u32x4 o;
#if defined(__HIP_DEVICE_COMPILE__)
            const auto s0 = __builtin_amdgcn_permlane32_swap(w[gp][0], w[gp + 1][0], false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(w[gp][1], w[gp + 1][1], false, false);
            o = u32x4{s0[0], s1[0], s0[1], s1[1]};
#else
            o = u32x4{0u, 0u, 0u, 0u};
#endif
            const int64_t gcol = tcol0 + j * 32 + (gp + half) * 8;
            // Columns past K get an offset past the resource: the store is dropped.
            const uint32_t off = gcol < K ? static_cast<uint32_t>(orow) * ld + static_cast<uint32_t>(gcol) * 2u : kNoAccess;
#if defined(__HIP_DEVICE_COMPILE__)
            __builtin_amdgcn_raw_buffer_store_b128(o, ro, static_cast<int>(off), 0, 0);
#else
            (void)off;
            (void)ro;
            (void)o;
#endif
          }
        }
      }
    }
    if constexpr (kF16) {
      if (more) load_exps(nxt);
    }
    if (!more) break;
    if constexpr (kLate) {
      setup_dma(nxt);
#pragma unroll
      for (int st = 0; st < kStages; ++st) {
        issue_a(min(st, nxt.ktiles - 1), st);
        issue_b(min(st, nxt.ktiles - 1), st);
      }
    }
    cur = nxt;
  }
}

// ---- pipelined 256 x 256 kernel ---------------------------------------------
// The kernel the host runs for every 256-row tile (dgrad with groups above
// ~160 rows, wgrad, and the tf32 router GEMMs): the forward pipelined kernel's
// shape with reduction-major operands.
//   * v_mfma_f32_16x16x32_bf16, 8 x 8 blocks of 16 x 16 per wave (the board
//     holds a higher clock under it than under the 32 x 32 x 16 form);
//   * consecutive tiles of a workgroup follow each other without draining:
//     a tile's second-to-last step DMAs the next tile's stage 0, its last step
//     reads those fragments and DMAs stage 1, and the epilogue stores straight
//     from registers after that DMA (bf16: v_permlane16_swap pairs two 16-column
//     blocks so a lane holds 8 consecutive columns; fp32: 4 consecutive columns
//     per lane and block as they are);
//   * a tile has at least three reduction steps (the first and the last two
//     are peeled; wgrad tiles of groups with at most 128 rows run steps over
//     zeros: rows past the group's end lie past the operand's buffer resource;
//     the host sends dgrad here only for N a multiple of 64, at least 192);
//   * reduction-major fragments: in 16-lane group G, lane 4 j + q reads rows
//     8 G + j and 8 G + j + 4 of the K half (ds_read_b64_tr_b16), columns
//     c + 4 q .. c + 3q + 3 of a 16-column block, so lane 16 G + i holds the 8
//     reduction values 8 G .. 8 G + 7 of column c + i, the 16 x 16 x 32 operand
//     layout. The 16-byte chunks of a 512-byte LDS row are XOR-swizzled by
//     rm16_swz (row bits 0-1 and 3 into chunk bits 1-3): the 8 rows one
//     half-wave reads at a time fall on 8 distinct 32-byte bank groups.
__device__ __forceinline__ int rm16_swz(int krow) { return ((krow & 3) << 2) | (((krow >> 3) & 1) << 1); }

// kSplit (dgrad, fp32 output): a reduction split of one group. "Group" g is
// split g: the rows of group 0 (group_offsets[0] .. [1] - 1), reduction columns
// [g kchunk, ...) of dy and the same rows of w, written into fp32 plane g
// [M, K] of out (at the same row indices).
// kOrder (wgrad): the tiles take the groups in the order p.order lists them
// (largest first, from group_order_kernel) instead of by index.
template <bool kWgrad, int kOut, bool kSplit = false, bool kOrder = false, bool kF16 = false>
__global__ __launch_bounds__(256) void grouped_gemm_bwd_pipe_kernel(BwdArgs p) {
  static_assert(!kF16 || (kWgrad && kOut == 1), "fp16 operands: the tf32 router wgrad (fp32 planes)");
  static_assert(!kSplit || (!kWgrad && kOut == 1), "the split is a dgrad with fp32 planes");
  static_assert(!kOrder || kWgrad, "the group order is a wgrad schedule");
  constexpr int kBM = 256;
  constexpr int kWaves = 4;
  constexpr int kThreads = 256;
  constexpr int kStages = 2;
  constexpr int kOpBytes = 256 * kBK * 2;            // 32 KiB: one operand of a stage
  constexpr int kStageBytes = 2 * kOpBytes;
  constexpr int kDma = kOpBytes / 1024 / kWaves;     // 8 DMA instructions per operand per stage
  constexpr int kMaxG = 4096;
  constexpr int kStores = kOut == 0 ? 32 : 0;        // bf16 stores per lane and tile (fp32: the next waits take all)
  constexpr int kAR = kWgrad ? 2 : 1;                // LDS reads per A fragment
  constexpr int kMI = 8, kNI = 8;
  static_assert(kStores + 2 * kDma <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[kStages * kStageBytes];
  __shared__ int32_t s_offs[kMaxG + 1];
  __shared__ int16_t s_order[kOrder ? kMaxG : 1];
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t N = p.N, K = p.K;
  const bool chunked = p.offsets == nullptr;

  if (!chunked) {
    const int64_t n_offs = kSplit ? 1 : p.G;  // a split reads group 0's offsets only
    for (int64_t i = tid; i <= n_offs; i += kThreads) s_offs[i] = p.offsets[i];
  }
  if constexpr (kOrder) {
    for (int64_t i = tid; i < p.G; i += kThreads) s_order[i] = p.order[i];
  }
  __syncthreads();

  // ---- tile walker (group offsets from LDS; 32-bit: the host keeps M below
  // 2^31). The values are wave-uniform and read into scalar registers.
  const int m32 = static_cast<int>(p.M);
  auto group_range = [&](int g, int &lo, int &hi) {
    if constexpr (kSplit) g = 0;  // every split covers the rows of group 0
    if (chunked) {
      lo = static_cast<int>(min(static_cast<int64_t>(g) * p.chunk, p.M));
      hi = static_cast<int>(min(static_cast<int64_t>(lo) + p.chunk, p.M));
      return;
    }
    lo = min(max(__builtin_amdgcn_readfirstlane(s_offs[g]), 0), m32);
    hi = min(max(__builtin_amdgcn_readfirstlane(s_offs[g + 1]), lo), m32);
  };
  const int g_count = static_cast<int>(p.G);
  const uint32_t ntl = static_cast<uint32_t>(p.ntiles);
  const uint32_t wg_rows = static_cast<uint32_t>(ceil_div(N, kBM));  // wgrad: row tiles per group
  auto row_tiles = [&](int lo, int hi) -> uint32_t {
    return kWgrad ? wg_rows : static_cast<uint32_t>(hi - lo + kBM - 1) / kBM;
  };
  // Reduction columns of split g (kSplit): [k0, k0 + kred).
  const int kchunk32 = static_cast<int>(p.kchunk);
  auto split_red = [&](int g, int &k0, int &kred) {
    k0 = g * kchunk32;
    kred = g + 1 == g_count ? static_cast<int>(N) - k0 : kchunk32;
  };
  // Group at walk position i.
  auto group_at = [&](int i) -> int {
    if constexpr (kOrder) {
      return min(max(__builtin_amdgcn_readfirstlane(static_cast<int>(s_order[i])), 0), g_count - 1);
    } else {
      return i;
    }
  };
  int g_cur = 0, g_act = group_at(0), g_lo, g_hi;  // walk position, its group, the group's rows
  uint32_t tiles_before = 0;
  group_range(g_act, g_lo, g_hi);
  uint32_t mt_g = row_tiles(g_lo, g_hi);
  struct Tile {
    int g, lo, hi;   // group and its row range (dgrad: output rows; wgrad: reduction rows)
    int i0;          // first output row of the tile (dgrad: in dx; wgrad: in dw[g])
    uint32_t nt;     // column tile
    int rows_valid;  // output rows of the tile
    int ktiles;      // reduction steps (at least 3)
  };
  const uint32_t P32 = static_cast<uint32_t>(P);
  const uint32_t L0 = static_cast<uint32_t>((b % 8) * (P / 8) + b / 8);
  auto find_tile = [&](uint32_t round, Tile &t) -> bool {
    // With the group order (largest first) odd rounds deal the tiles in
    // reverse, so a workgroup that took one of the larger tiles of a round
    // takes one of the smaller ones of the next (the patches stay whole).
    const uint32_t L = round * P32 + ((kOrder && (round & 1u)) ? P32 - 1u - L0 : L0);
    while (g_cur < g_count && L >= tiles_before + mt_g * ntl) {
      tiles_before += mt_g * ntl;
      ++g_cur;
      if (g_cur < g_count) {
        g_act = group_at(g_cur);
        group_range(g_act, g_lo, g_hi);
        mt_g = row_tiles(g_lo, g_hi);
      }
    }
    if (g_cur >= g_count) return false;
    const uint32_t q = L - tiles_before;
    const uint32_t per_grp = kGroupM * ntl;
    const uint32_t full = mt_g / kGroupM;
    uint32_t mt, nt;
    if (q < full * per_grp) {
      const uint32_t grp = q / per_grp, r = q - grp * per_grp;
      nt = r / kGroupM;
      mt = grp * kGroupM + r % kGroupM;
    } else {
      const uint32_t r = q - full * per_grp, gm = mt_g - full * kGroupM;
      nt = r / gm;
      mt = full * kGroupM + (r - nt * gm);
    }
    t.g = g_act;
    t.lo = g_lo;
    t.hi = g_hi;
    t.i0 = (kWgrad ? 0 : g_lo) + static_cast<int>(mt) * kBM;
    t.nt = nt;
    t.rows_valid = min((kWgrad ? static_cast<int>(N) : g_hi) - t.i0, kBM);
    int red = kWgrad ? g_hi - g_lo : static_cast<int>(N);
    if constexpr (kSplit) {
      int k0;
      split_red(g_cur, k0, red);
    }
    t.ktiles = max((red + kBK - 1) / kBK, 3);
    return true;
  };

  // ---- DMA sources of the tile being loaded (32-bit offsets: the host bounds
  // every operand panel below 2 GiB)
  __amdgpu_buffer_rsrc_t ra, rb;
  int a_off[kDma], b_off[kDma];
  int a_step = 0, b_step = 0;  // bytes per reduction step
  const uint32_t n32 = static_cast<uint32_t>(N), k32 = static_cast<uint32_t>(K);
  auto setup_dma = [&](const Tile &t) {
    // Recomputed per tile (not kept live across the tile loop): the lane's
    // DMA row and chunk from an opaque copy of the lane index. A
    // reduction-major DMA block holds reduction rows 2 blk, 2 blk + 1.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int rm_row = ln >> 5, rm_pchunk = ln & 31;
    if constexpr (kWgrad) {
      const uint32_t rows = static_cast<uint32_t>(t.hi - t.lo);
      ra = make_rsrc(p.a + static_cast<int64_t>(t.lo) * N, rows * n32 * 2u);
      rb = make_rsrc(p.b + static_cast<int64_t>(t.lo) * K, rows * k32 * 2u);
      a_step = kBK * static_cast<int>(n32) * 2;
#pragma unroll
      for (int j = 0; j < kDma; ++j) {
        const int krow = (j * kWaves + wave) * 2 + rm_row;
        const uint32_t lchunk = static_cast<uint32_t>(rm_pchunk ^ rm16_swz(krow));
        a_off[j] = static_cast<int>(static_cast<uint32_t>(krow) * n32 * 2u + static_cast<uint32_t>(t.i0) * 2u + lchunk * 16u);
      }
    } else {
      if constexpr (kSplit) {
        // dy columns [k0, k0 + kred) of the tile's rows (the resource ends at the
        // last row's k0 + kred) and w rows [k0, k0 + kred).
        int k0, kred;
        split_red(t.g, k0, kred);
        ra = make_rsrc(p.a + static_cast<int64_t>(t.i0) * N + k0,
                       static_cast<uint32_t>(t.rows_valid - 1) * n32 * 2u + static_cast<uint32_t>(kred) * 2u);
        rb = make_rsrc(p.b + static_cast<int64_t>(k0) * K, static_cast<uint32_t>(kred) * k32 * 2u);
      } else {
        ra = make_rsrc(p.a + static_cast<int64_t>(t.i0) * N, static_cast<uint32_t>(t.rows_valid) * n32 * 2u);
        rb = make_rsrc(p.b + static_cast<int64_t>(t.g) * N * K, static_cast<uint32_t>(N * K * 2));
      }
      a_step = kBK * 2;
#pragma unroll
      for (int j = 0; j < kDma; ++j) {
        const int r = (j * kWaves + wave) * 8 + (ln >> 3);
        const uint32_t lchunk = static_cast<uint32_t>((ln & 7) ^ kc_swz(r));
        // Rows past the group's end read as zeros (results dropped).
        a_off[j] = r < t.rows_valid ? static_cast<int>(static_cast<uint32_t>(r) * n32 * 2u + lchunk * 16u)
                                    : static_cast<int>(kNoAccess);
      }
    }
    b_step = kBK * static_cast<int>(k32) * 2;
    const uint32_t col0 = t.nt * static_cast<uint32_t>(kBN);
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      const int krow = (j * kWaves + wave) * 2 + rm_row;
      const uint32_t lchunk = static_cast<uint32_t>(rm_pchunk ^ rm16_swz(krow));
      b_off[j] = static_cast<int>(static_cast<uint32_t>(krow) * k32 * 2u + col0 * 2u + lchunk * 16u);
    }
  };
  // Operand `op` (0 = A, 1 = B) of reduction step `kt` of the tile set up last into ring slot `slot`.
  auto issue_half = [&](int kt, int slot, int op) {
    const uint32_t st = lds_base + (slot % kStages) * kStageBytes + op * kOpBytes;
    const int soff = kt * (op ? b_step : a_step);
#pragma unroll
    for (int j = 0; j < kDma; ++j) {
      const uint32_t blk = j * kWaves + wave;
      dma16b(op ? rb : ra, (lds_void *)(uintptr_t)(st + blk * 1024), op ? b_off[j] : a_off[j], soff);
    }
  };
  // ---- fragments
  // KC (dgrad's dy): lane l reads row (block + l % 16), the 8 values
  // 8 (l / 16) .. + 7 of K half ks (logical chunk 4 ks + l / 16).
  const int fq = lane >> 4;
  const int ra0 = wm * 128 + (lane & 15);
  const uint32_t fa0 = ra0 * kKCRow + ((fq ^ kc_swz(ra0)) << 4);
  // RM: the lane's row and column bytes within a 16-column block whose 32-byte
  // position is XORed with rmx (the swizzle of the lane's rows).
  const int rg = lane >> 4, rj = (lane >> 2) & 3, rq = lane & 3;
  const uint32_t rm0 = (8 * rg + rj) * kRMRow + ((rq >> 1) << 4) + (rq & 1) * 8;
  const uint32_t rmx = static_cast<uint32_t>((rj << 1) | (rg & 1)) << 5;
  const uint32_t rma0 = rm0 + wm * 256;              // wgrad A: output rows wm 128 ..
  const uint32_t rmb0 = kOpBytes + rm0 + wn * 256;   // B: output columns wn 128 ..
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 acc[kMI][kNI];
  uint32_t rd_so = 0;
  auto set_read_slot = [&](int slot) { rd_so = lds_base + (slot % kStages) * kStageBytes; };
  bf16x8 fa[2][kMI], fb[2][kNI];
  // RM fragment of 16-column block blk, K half ks (base: slot + operand + lane).
  auto rm_frag = [&](uint32_t base, uint32_t x, int blk, int ks) -> bf16x8 {
    const uint32_t a = base + ((static_cast<uint32_t>(blk) * 32u) ^ x) + ks * 32 * kRMRow;
    return read_rm_frag(a);
  };
  // A fragments of row blocks 4 ih .. 4 ih + 3 / all B fragments of K half ks.
  auto read_a = [&](int ks, int ih) {
    if constexpr (kWgrad) {
      uint32_t x = rmx;
      asm volatile("" : "+v"(x));
      const uint32_t base = rd_so + rma0;
#pragma unroll
      for (int i = 4 * ih; i < 4 * ih + 4; ++i) fa[ks][i] = rm_frag(base, x, i, ks);
    } else {
      const uint32_t base = (rd_so + fa0) ^ (ks << 6);
#pragma unroll
      for (int i = 4 * ih; i < 4 * ih + 4; ++i)
        fa[ks][i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(base + i * 16 * kKCRow));
    }
  };
  auto read_b = [&](int ks) {
    uint32_t x = rmx;
    asm volatile("" : "+v"(x));
    const uint32_t base = rd_so + rmb0;
#pragma unroll
    for (int j = 0; j < kNI; ++j) fb[ks][j] = rm_frag(base, x, j, ks);
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
  // column block j's 4 MFMAs its B fragment is free and the next stage's is
  // read into it (with A blocks 0..3, freed by the unit before).
  auto last_unit_reads = [&]() {
    uint32_t x = rmx;
    asm volatile("" : "+v"(x));
    const uint32_t base_b = rd_so + rmb0;
    const uint32_t base_a = kWgrad ? rd_so + rma0 : (rd_so + fa0) ^ (1 << 6);
#pragma unroll
    for (int j = 0; j < kNI; ++j) {
#pragma unroll
      for (int i = 4; i < 8; ++i) {
        acc[i][j] = mma16<kF16>(fb[1][j], fa[1][i], acc[i][j]);
      }
      fb[1][j] = rm_frag(base_b, x, j, 1);
      if (j < 4) {
        if constexpr (kWgrad) {
          fa[1][j] = rm_frag(base_a, x, j, 1);
        } else {
          fa[1][j] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(base_a + j * 16 * kKCRow));
        }
      }
    }
  };
  // 32 MFMAs: K half ks, row blocks 4 ih .. 4 ih + 3, all column blocks.
  auto mfma_unit = [&](int ks, int ih, bool zero) {
#pragma unroll
    for (int i = 4 * ih; i < 4 * ih + 4; ++i)
#pragma unroll
      for (int j = 0; j < kNI; ++j)
        acc[i][j] = mma16<kF16>(fb[ks][j], fa[ks][i], zero ? f32x4{} : acc[i][j]);
  };

  // Epilogue of tile t from the accumulators: register r of lane l in block
  // (i, j) holds output row i * 16 + l % 16 and column j * 16 + 4 (l / 16) + r
  // of this wave's part. Stores go through a resource over the wave's valid
  // rows (rows past it are dropped); columns past K get an offset past it.
  auto epilogue = [&](const Tile &t) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int eq = ln >> 4;
    const int64_t gbase = kWgrad ? static_cast<int64_t>(t.g) * N * K : kSplit ? static_cast<int64_t>(t.g) * p.M * K : 0;
    const int kcols = static_cast<int>(k32);
    if constexpr (kOut == 0) {
      // One resource over the tile's valid rows (below 2^31 bytes: K < 2^22).
      const uint32_t ld = k32 * 2u;
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<const uint16_t *>(p.out) + gbase + static_cast<int64_t>(t.i0) * K,
                                                  static_cast<uint32_t>(t.rows_valid) * ld);
      // After rounding, a block is two packed words per lane; v_permlane16_swap
      // trades rows (16 lanes) 1 and 3 of block j's words with rows 0 and 2 of
      // block j + 1's, so lanes of row q hold the 8 consecutive columns
      // (q / 2) 8 .. + 7 of block j + q % 2.
      const int wcol0 = static_cast<int>(t.nt) * kBN + wn * 128 + (eq & 1) * 16 + (eq >> 1) * 8;
#pragma unroll
      for (int i = 0; i < kMI; ++i) {
        const uint32_t orow = static_cast<uint32_t>(wm * 128 + i * 16 + (ln & 15));
#pragma unroll
        for (int jp = 0; jp < kNI; jp += 2) {
          uint32_t w[2][2];
#pragma unroll
          for (int d = 0; d < 2; ++d) {
            const bf16x2 lo = {(__bf16)acc[i][jp + d][0], (__bf16)acc[i][jp + d][1]};
            const bf16x2 hi = {(__bf16)acc[i][jp + d][2], (__bf16)acc[i][jp + d][3]};
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
          const uint32_t off = gcol < kcols ? orow * ld + static_cast<uint32_t>(gcol) * 2u : kNoAccess;
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
    } else {
      // fp32: 4 consecutive columns per lane and block, stored as 16 bytes
      // through a resource over the wave's valid rows (below 2^31 bytes: K < 2^22).
      const int64_t wrow0 = t.i0 + wm * 128;
      const int rows_out = max(min(t.rows_valid - wm * 128, 128), 0);
      const uint32_t ld = k32 * 4u;
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<float *>(p.out) + gbase + (rows_out > 0 ? wrow0 * K : 0),
                                                  static_cast<uint32_t>(rows_out) * ld);
      const int wcol0 = static_cast<int>(t.nt) * kBN + wn * 128 + eq * 4;
#pragma unroll
      for (int i = 0; i < kMI; ++i) {
        const uint32_t orow = static_cast<uint32_t>(i * 16 + (ln & 15));
#pragma unroll
        for (int j = 0; j < kNI; ++j) {
          const int gcol = wcol0 + j * 16;
          const uint32_t off = gcol < kcols ? orow * ld + static_cast<uint32_t>(gcol) * 4u : kNoAccess;
          const u32x4 v = {__float_as_uint(acc[i][j][0]), __float_as_uint(acc[i][j][1]),
                           __float_as_uint(acc[i][j][2]), __float_as_uint(acc[i][j][3])};
#if defined(__HIP_DEVICE_COMPILE__)
          __builtin_amdgcn_raw_buffer_store_b128(v, ro, static_cast<int>(off), 0, 0);
#else
          (void)off;
          (void)v;
          (void)ro;
#endif
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // The part of a reduction step after its barrier: MFMA units 1-3 of the
  // fragments in VGPRs, the next stage's fragments read from the LDS slot set
  // by set_read_slot into the registers each unit frees, and the DMA of stage
  // `kdma` (of the tile set up last) into ring slot `wr`.
  auto step_body = [&](bool zero, int kdma, int wr) __attribute__((always_inline)) {
    mfma_unit(0, 1, zero);
    read_a(0, 0);
    issue_half(kdma, wr, 0);
    sched_mix<32, 4 * kAR, kDma>();
    mfma_unit(1, 0, false);
    read_a(0, 1);
    read_b(0);
    issue_half(kdma, wr, 1);
    sched_mix<32, 4 * kAR + 2 * kNI, kDma>();
    last_unit_reads();
    sched_mix<32, 2 * kNI + 4 * kAR, 0>();
    read_a(1, 1);
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- first tile: stages 0 and 1 in flight, stage 0 read into VGPRs
  Tile cur{}, nxt{};
  if (!find_tile(0, cur)) return;
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
  for (uint32_t round = 0;; ++round) {
    const int ktiles = cur.ktiles;
    // One reduction step: MFMAs of stage kt (fragments in VGPRs), fragments of
    // stage kt + 1 read from LDS, DMA of the stage two ahead (this tile's
    // kt + 2 or, past its end, the next tile's kt + 2 - ktiles) into the slot of stage kt.
    auto step = [&](int kt, bool first, bool last) __attribute__((always_inline)) {
      mfma_unit(0, 0, first);
      __builtin_amdgcn_sched_barrier(0);
      // Stage kt + 1 has landed. In a tile's first step the previous tile's
      // bf16 output stores were issued after it and may still be in flight.
      if (first && round > 0 && kStores > 0) {
        wait_vm_n<kStores>();
      } else {
        wait_dma();
      }
      wait_lds();
      barrier();
      // The second-to-last step DMAs the next tile's stage 0 (without a next
      // tile it re-reads this tile's last stage into the free slot).
      if (last && more) setup_dma(nxt);
      const int kdma = !last ? kt + 2 : (more ? 0 : ktiles - 1);
      set_read_slot(sb + kt + 1);
      step_body(first, kdma, sb + kt + 2);
    };
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

// Ping-pong backward kernel (bf16 output; dgrad with N % 64 == 0 and N >= 192,
// and wgrad): the forward ping-pong kernel's schedule on the backward operands.
// 8 wavefronts, two per SIMD taking turns: in each phase one issues its 64
// MFMAs (a 64 x 128 part of the 256 x 256 tile: rows wm * 64 .., wm = its
// SIMD; columns grp * 128 .., grp = its group) while the other reads its
// fragments of the next stage and issues its share of the stage DMAs; a
// workgroup barrier ends every phase.
//
// LDS (160 KiB): A in 3 slots of 32 KiB (read by both groups; dgrad's dy as
// 256 rows x 128 bytes, wgrad's dy as 64 reduction rows x 512 bytes), B in 2
// slots, each holding the two groups' column halves as separate 64 x 256-byte
// RM tiles (a DMA block is 4 reduction rows of one half, so each group's half
// is loaded by the other group on its own schedule). The 16-byte chunk swizzle
// of the RM tiles (rm16_swz) stays within 256-byte segments, so the half tiles
// keep the full-row tiles' conflict-free transposing reads.
//
// Stage schedule, waits and slot reuse as in grouped_gemm_pp_kernel: in its
// load phase of stage s a wavefront DMAs its group's half of A stage s + 2 and
// the other group's B half of stage s + 1 (group 0) or s + 2 (group 1); each
// DMA is waited for at the end of its issuer's next load phase (vmcnt <= 8, or
// 8 + 16 after an epilogue's stores). A tile's reduction step count varies
// (wgrad: its group's rows), stages past a tile's end come from the next tile.
//
// dgrad with a tail list: tiles of kTM = 128 rows (a wavefront's 32 rows,
// half the A blocks per stage, the first half of each A slot) for group tails
// of 1 to 128 rows, taken after the 256-row tiles (grouped_gemm_bwd_pp_kernel).
struct BwdTile {
  int g, lo, hi;
  int i0;
  uint32_t nt;
  int rows_valid;
  int ktiles;
};
constexpr int kBwdPpLdsBytes = 5 * 256 * kBK * 2;  // 160 KiB

// kTM = 256: the persistent workgroup b of P (the grid) takes its tiles in
// the static order; kTM = 128: the one tile *one.
template <bool kWgrad, bool kOrder, int kTM, bool kTails>
__device__ __forceinline__ void bwd_pp_body(const BwdArgs &p, char *smem, const BwdTile *one) {
  static_assert(!kOrder || kWgrad, "the group order is a wgrad schedule");
  static_assert(kTM == 256 || (kTM == 128 && !kWgrad), "tile rows");
  static_assert(!kTails || !kWgrad, "tail tiles are a dgrad form");
  constexpr int kBM = kTM;
  constexpr int kAS = 3, kBS = 2;
  constexpr int kSlotBytes = 256 * kBK * 2;  // 32 KiB
  constexpr int kHalfBytes = kSlotBytes / 2;  // one group's B columns
  constexpr int kBBase = kAS * kSlotBytes;
  constexpr int kHalfRow = 256;               // bytes per reduction row of a B half tile
  constexpr int kMI = kTM / 64, kNI = 8;
  constexpr int kWR = kTM / 4;                // dgrad: tile rows of a wavefront
  constexpr int kStores = kMI * 4;            // 16-byte stores per lane per tile
  constexpr int kDmaA = kTM / 64, kDmaB = 4;
  constexpr int kABlk = kTM / 16;             // 1 KiB A blocks DMA'd by one group per stage
  static_assert(kDmaA + kDmaB + kStores <= 63, "vmcnt range");
  static_assert(kAS * kSlotBytes + kBS * kSlotBytes <= kBwdPpLdsBytes, "LDS");
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));

  // The thread index through an opaque copy: the lane-derived values of the
  // 256-row and the 128-row form are computed separately, not kept live from
  // one form to the other.
  int tid = threadIdx.x;
  if constexpr (kTails) asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- roles from the SIMD each wavefront runs on (as in grouped_gemm_pp_kernel)
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
    const bool ok = per_simd[0] == 2 && per_simd[1] == 2 && per_simd[2] == 2 && per_simd[3] == 2;
    wm = __builtin_amdgcn_readfirstlane(ok ? simd : (wave & 3));
    grp = __builtin_amdgcn_readfirstlane(ok ? before : (wave >> 2));
  }

  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t N = p.N, K = p.K;

  // ---- tile walker (group offsets and order read from memory: the ring fills the LDS)
  const int m32 = static_cast<int>(p.M);
  const int g_count = static_cast<int>(p.G);
  auto group_range = [&](int g, int &lo, int &hi) {
    if constexpr (kWgrad) {
      lo = min(max(ld_inv(p.offsets, g), 0), m32);
      hi = min(max(ld_inv(p.offsets, g + 1), lo), m32);
    } else {
      // dgrad: vector loads (measured: the scalar loads' waits, which share the LDS counter, cost c5 fc2
      // dgrad 3% where they fall after the fragment reads; the wgrad walker gains from them)
      lo = min(max(__builtin_amdgcn_readfirstlane(p.offsets[g]), 0), m32);
      hi = min(max(__builtin_amdgcn_readfirstlane(p.offsets[g + 1]), lo), m32);
    }
  };
  const uint32_t ntl = static_cast<uint32_t>(p.ntiles);
  const uint32_t wg_rows = static_cast<uint32_t>(ceil_div(N, kBM));
  // dgrad row tiles of a group (kTails: all but a last tile of at most 128
  // rows, which the 128-row form takes).
  auto row_tiles = [&](int lo, int hi) -> uint32_t {
    return kWgrad ? wg_rows : static_cast<uint32_t>(kTails ? main_row_tiles(hi - lo) : (hi - lo + kBM - 1) / kBM);
  };
  auto group_at = [&](int i) -> int {
    if constexpr (kOrder) {
      return min(max(ld_inv(p.order, i), 0), g_count - 1);
    } else {
      return i;
    }
  };
  // Row range of the i-th group taken: with the order, from the ordered copy the order kernel wrote (one
  // load level per group step instead of the order, then that group's offsets).
  auto range_at = [&](int i, int g, int &lo, int &hi) {
    if constexpr (kOrder) {
      lo = min(max(ld_inv(p.order_rows, 2 * i), 0), m32);
      hi = min(max(ld_inv(p.order_rows, 2 * i + 1), lo), m32);
    } else {
      group_range(g, lo, hi);
    }
  };
  // With a sweep limit the walker ends before the first group the sweep kernel takes.
  int g_end = g_count;
  if constexpr (kOrder) {
    if (p.sweep_rows > 0) g_end = long_group_count(p.order_rows, g_count, m32, p.sweep_rows);
  }
  int g_cur = 0, g_act = group_at(0), g_lo, g_hi;
  uint32_t tiles_before = 0;
  range_at(0, g_act, g_lo, g_hi);
  uint32_t mt_g = row_tiles(g_lo, g_hi);
  using Tile = BwdTile;
  const uint32_t P32 = static_cast<uint32_t>(P);
  const uint32_t L0 = static_cast<uint32_t>((b % 8) * (P / 8) + b / 8);
  auto find_tile = [&](uint32_t round, Tile &t) -> bool {
    if constexpr (kTM == 128) {
      if (round > 0) return false;
      t = *one;
      return true;
    }
    // With the group order (largest first) odd rounds deal the tiles in
    // reverse, so a workgroup that took one of the larger tiles of a round
    // takes one of the smaller ones of the next (the patches stay whole).
    const uint32_t L = round * P32 + ((kOrder && (round & 1u)) ? P32 - 1u - L0 : L0);
    while (g_cur < g_end && L >= tiles_before + mt_g * ntl) {
      tiles_before += mt_g * ntl;
      ++g_cur;
      if (g_cur < g_end) {
        g_act = group_at(g_cur);
        range_at(g_cur, g_act, g_lo, g_hi);
        mt_g = row_tiles(g_lo, g_hi);
      }
    }
    if (g_cur >= g_end) return false;
    const uint32_t q = L - tiles_before;
    const uint32_t per_grp = kGroupM * ntl;
    const uint32_t full = mt_g / kGroupM;
    uint32_t mt, nt;
    if (q < full * per_grp) {
      const uint32_t gq = q / per_grp, r = q - gq * per_grp;
      nt = r / kGroupM;
      mt = gq * kGroupM + r % kGroupM;
    } else {
      const uint32_t r = q - full * per_grp, gm = mt_g - full * kGroupM;
      nt = r / gm;
      mt = full * kGroupM + (r - nt * gm);
    }
    t.g = g_act;
    t.lo = g_lo;
    t.hi = g_hi;
    t.i0 = (kWgrad ? 0 : g_lo) + static_cast<int>(mt) * kBM;
    t.nt = nt;
    t.rows_valid = min((kWgrad ? static_cast<int>(N) : g_hi) - t.i0, kBM);
    const int red = kWgrad ? g_hi - g_lo : static_cast<int>(N);
    // Two stages suffice for the ring (a tile's stages s + 2 and s + 1 + grp cross into the next tile);
    // dgrad reductions have at least three (host).
    t.ktiles = max((red + kBK - 1) / kBK, 2);
    return true;
  };

  // ---- DMA sources: A blocks (grp * kABlk + j * 4 + wm) of a stage; B blocks
  // (j * 4 + wm) of the other group's half.
  const uint32_t n32 = static_cast<uint32_t>(N), k32 = static_cast<uint32_t>(K);
  __amdgpu_buffer_rsrc_t ra, rb;
  int a_off[kDmaA];
  int b_base = 0;
  const int a_step = kWgrad ? kBK * static_cast<int>(n32) * 2 : kBK * 2;  // bytes per reduction step
  const int b_step = kBK * static_cast<int>(k32) * 2;
  auto setup_a = [&](const Tile &t, bool valid) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    if constexpr (kWgrad) {
      const uint32_t rows = valid ? static_cast<uint32_t>(t.hi - t.lo) : 0u;
      ra = make_rsrc(p.a + static_cast<int64_t>(t.lo) * N, rows * n32 * 2u);
#pragma unroll
      for (int j = 0; j < kDmaA; ++j) {
        const int krow = (grp * kABlk + j * 4 + wm) * 2 + (ln >> 5);
        const uint32_t lchunk = static_cast<uint32_t>((ln & 31) ^ rm16_swz(krow));
        a_off[j] = static_cast<int>(static_cast<uint32_t>(krow) * n32 * 2u + static_cast<uint32_t>(t.i0) * 2u + lchunk * 16u);
      }
    } else {
      // Rows past the tile's valid rows lie past the resource: zeros.
      ra = make_rsrc(p.a + static_cast<int64_t>(t.i0) * N, valid ? static_cast<uint32_t>(t.rows_valid) * n32 * 2u : 0u);
#pragma unroll
      for (int j = 0; j < kDmaA; ++j) {
        const int r = (grp * kABlk + j * 4 + wm) * 8 + (ln >> 3);
        const uint32_t lchunk = static_cast<uint32_t>((ln & 7) ^ kc_swz(r));
        a_off[j] = static_cast<int>(static_cast<uint32_t>(r) * n32 * 2u + lchunk * 16u);
      }
    }
  };
  // B half h = 1 - grp: reduction row krow = (j * 4 + wm) * 4 + ln / 16 of DMA j
  // (its swizzle does not depend on j, so DMA j is the base + 16 j rows), 16
  // chunks of columns nt * 256 + h * 128 ...
  auto setup_b = [&](const Tile &t, bool valid) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    if constexpr (kWgrad) {
      const uint32_t rows = valid ? static_cast<uint32_t>(t.hi - t.lo) : 0u;
      rb = make_rsrc(p.b + static_cast<int64_t>(t.lo) * K, rows * k32 * 2u);
    } else {
      rb = make_rsrc(p.b + static_cast<int64_t>(t.g) * N * K, valid ? static_cast<uint32_t>(N * K * 2) : 0u);
    }
    const int krow = wm * 4 + (ln >> 4);
    const uint32_t lchunk = static_cast<uint32_t>((ln & 15) ^ rm16_swz(krow));
    const uint32_t col0 = t.nt * static_cast<uint32_t>(kBN) + static_cast<uint32_t>(1 - grp) * 128u;
    b_base = static_cast<int>(static_cast<uint32_t>(krow) * k32 * 2u + col0 * 2u + lchunk * 16u);
  };
  auto issue = [&](int kt_a, int sa, int kt_b, int sbs) {
    const uint32_t a_dst = lds_base + sa * kSlotBytes;
    const uint32_t b_dst = lds_base + kBBase + sbs * kSlotBytes + (1 - grp) * kHalfBytes;
#pragma unroll
    for (int j = 0; j < kDmaA; ++j) {
      const uint32_t blk = grp * kABlk + j * 4 + wm;
      dma16b(ra, (lds_void *)(uintptr_t)(a_dst + blk * 1024), a_off[j], kt_a * a_step);
    }
#pragma unroll
    for (int j = 0; j < kDmaB; ++j) {
      const uint32_t blk = j * 4 + wm;
      dma16b(rb, (lds_void *)(uintptr_t)(b_dst + blk * 1024), b_base + j * 16 * static_cast<int>(k32) * 2,
             kt_b * b_step);
    }
  };

  // ---- fragments
  const int fq = lane >> 4;
  const int ra0 = wm * kWR + (lane & 15);
  const uint32_t fa0 = ra0 * kKCRow + ((fq ^ kc_swz(ra0)) << 4);  // dgrad A (KC)
  const int rg = lane >> 4, rj = (lane >> 2) & 3, rq = lane & 3;
  const uint32_t rm_in = ((rq >> 1) << 4) + (rq & 1) * 8;
  const uint32_t rma0 = (8 * rg + rj) * kRMRow + rm_in;              // wgrad A: full 512-byte rows
  const uint32_t rmb0 = (8 * rg + rj) * kHalfRow + rm_in;            // B: this group's half tile
  const uint32_t rmx = static_cast<uint32_t>((rj << 1) | (rg & 1)) << 5;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 acc[kMI][kNI];
  bf16x8 fa[2][kMI], fb[2][kNI];
  auto read_frags = [&](int sa, int sbs) {
    uint32_t x = rmx;
    asm volatile("" : "+v"(x));
    const uint32_t b_base_l = lds_base + kBBase + sbs * kSlotBytes + grp * kHalfBytes + rmb0;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if constexpr (kWgrad) {
        const uint32_t a_base_l = lds_base + sa * kSlotBytes + rma0 + ks * 32 * kRMRow;
#pragma unroll
        for (int i = 0; i < kMI; ++i)
          fa[ks][i] = read_rm_frag_rows<kRMRow>(a_base_l + ((static_cast<uint32_t>(wm * kMI + i) * 32u) ^ x));
      } else {
        const uint32_t a_base_l = (lds_base + sa * kSlotBytes + fa0) ^ (ks << 6);
#pragma unroll
        for (int i = 0; i < kMI; ++i)
          fa[ks][i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)(a_base_l + i * 16 * kKCRow));
      }
#pragma unroll
      for (int j = 0; j < kNI; ++j)
        fb[ks][j] = read_rm_frag_rows<kHalfRow>(b_base_l + ks * 32 * kHalfRow + ((static_cast<uint32_t>(j) * 32u) ^ x));
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
  // Epilogue: register r of lane l in block (i, j) holds output row
  // wm * kWR + i * 16 + l % 16 and column grp * 128 + j * 16 + 4 (l / 16) + r of
  // the tile; bf16 RNE, v_permlane16_swap pairs blocks j, j + 1 so each lane
  // stores 8 consecutive columns (16 bytes) through a resource over the tile's
  // valid rows; columns past K get an offset past it.
  auto epilogue = [&](const Tile &t) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int eq = ln >> 4;
    const int64_t gbase = kWgrad ? static_cast<int64_t>(t.g) * N * K : 0;
    const int kcols = static_cast<int>(k32);
    const uint32_t ld = k32 * 2u;
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(static_cast<const uint16_t *>(p.out) + gbase + static_cast<int64_t>(t.i0) * K,
                                                static_cast<uint32_t>(t.rows_valid) * ld);
    const int wcol0 = static_cast<int>(t.nt) * kBN + grp * 128 + (eq & 1) * 16 + (eq >> 1) * 8;
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
      const uint32_t orow = static_cast<uint32_t>(wm * kWR + i * 16 + (ln & 15));
#pragma unroll
      for (int jp = 0; jp < kNI; jp += 2) {
        uint32_t w[2][2];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          const bf16x2 lo = {(__bf16)acc[i][jp + d][0], (__bf16)acc[i][jp + d][1]};
          const bf16x2 hi = {(__bf16)acc[i][jp + d][2], (__bf16)acc[i][jp + d][3]};
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
        const uint32_t off = gcol < kcols ? orow * ld + static_cast<uint32_t>(gcol) * 2u : kNoAccess;
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

  // ---- prologue: A stages 0 and 1, group 0's B half of stages 0 and 1 (by
  // group 1), group 1's B half of stage 0 (by group 0).
  Tile cur{}, nxt{};
  if (!find_tile(0, cur)) return;
  setup_a(cur, true);
  setup_b(cur, true);
  {
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int j = 0; j < kDmaA; ++j) {
        const uint32_t blk = grp * kABlk + j * 4 + wm;
        dma16b(ra, (lds_void *)(uintptr_t)(lds_base + kt * kSlotBytes + blk * 1024), a_off[j], kt * a_step);
      }
    }
    const int nb = grp == 1 ? 2 : 1;
    for (int kt = 0; kt < nb; ++kt) {
      const uint32_t b_dst = lds_base + kBBase + kt * kSlotBytes + (1 - grp) * kHalfBytes;
#pragma unroll
      for (int j = 0; j < kDmaB; ++j) {
        const uint32_t blk = j * 4 + wm;
        dma16b(rb, (lds_void *)(uintptr_t)(b_dst + blk * 1024), b_base + j * 16 * static_cast<int>(k32) * 2,
               kt * b_step);
      }
    }
  }
  bool more = find_tile(1, nxt);
  wait_dma();
  barrier();
  if (grp == 1) barrier();  // group 1 runs one phase behind

  int slot_a = 0, slot_b = 0;
  bool have_prev = false;
  Tile prev{};
  for (uint32_t round = 0;; ++round) {
    const int S = cur.ktiles;
    for (int s = 0; s < S; ++s) {
      // ---------------- load phase of stage s
      const bool epi = s == 0 && have_prev;
      if (epi) epilogue(prev);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(slot_a, slot_b);
      const int ta = s + 2, tb = s + 1 + grp;
      if (ta == S) setup_a(nxt, more);
      if (tb == S) setup_b(nxt, more);
      int sa = slot_a + 2;
      sa = sa >= kAS ? sa - kAS : sa;
      const int sbs = (slot_b + 1 + grp) & 1;
      issue(ta >= S ? ta - S : ta, sa, tb >= S ? tb - S : tb, sbs);
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
  epilogue(prev);
  if (grp == 0) barrier();
  wait_dma();  // no LDS DMA outlives the workgroup
}

// One persistent workgroup per CU takes its 256-row tiles in the static
// order; with a tail list (dgrad) it then takes tail units from the list's
// counter (thread 0 adds 1, the number reaches the other wavefronts through
// the idle LDS ring) and computes each with the 128-row form, until the units
// run out.
template <bool kWgrad, bool kOrder, bool kTails>
__global__ __launch_bounds__(512) void grouped_gemm_bwd_pp_kernel(BwdArgs p) {
  __shared__ __attribute__((aligned(1024))) char smem[kBwdPpLdsBytes];
  bwd_pp_body<kWgrad, kOrder, 256, kTails>(p, smem, nullptr);
  if constexpr (kTails) {
    volatile int *bcast = reinterpret_cast<volatile int *>(smem);
    const int ntl = static_cast<int>(p.ntiles);
    const int ktiles = max((static_cast<int>(p.N) + kBK - 1) / kBK, 3);
    for (;;) {
      __syncthreads();  // the ring is idle: every wavefront has left its last tile
      if (threadIdx.x == 0) {
        bcast[0] = __hip_atomic_fetch_add(p.tails + kTailCtr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      const int u = __builtin_amdgcn_readfirstlane(bcast[0]);
      __syncthreads();  // every wavefront has read it before the ring is used again
      if (u >= p.tails[kTailCount] * ntl) break;
      const int g = p.tails[kTailList + u / ntl];
      const int M32 = static_cast<int>(p.M);
      const int lo = min(max(p.offsets[g], 0), M32);
      const int hi = min(max(p.offsets[g + 1], lo), M32);
      const int r = (hi - lo) % 256;
      const BwdTile t{g, lo, hi, hi - r, static_cast<uint32_t>(u % ntl), r, ktiles};
      bwd_pp_body<kWgrad, kOrder, 128, kTails>(p, smem, &t);
    }
  }
}

// Weight gradient of the short groups (at most kSweepRows rows, e.g.
// kernel_cases/case09_moe_grouped_gemm_fc1_wgrad.py:57-64: 40 groups of ~102
// rows): dw[g] is large and its reduction short, so the work is the stream of
// dw stores. The whole reduction (the group's rows, zeros from past the
// operands' buffer resources up to 128) fits one LDS stage. A unit is (group,
// range of swept tiles, fixed tile): the fixed operand's 256-column slab
// (64 KiB) stays in LDS while the unit's tiles sweep the other operand's
// 128-column slabs (32 KiB, three slots, DMA'd two tiles ahead). Units are
// numbered with the fixed tile fastest and dealt round-robin so that the
// workgroups of an XCD (consecutive numbers) take the same group and range
// with neighbouring fixed tiles: they sweep the same slabs at about the same
// time, and the slabs come from L2. A tile's stores are issued after the DMA
// of the slab two tiles ahead, and the wait before the next tile (for the
// next slab) leaves the stores of this tile and the one before in flight.
// kFixD: dy's slab is fixed (tile 256 dw rows x 128 columns, sweeping x over
// K); else x's (128 x 256, sweeping dy over N). The host picks the
// orientation and the unit length (p.sweep_len) that spread the tiles most
// evenly over the workgroups.
constexpr int kSweepRows = 128;

template <bool kFixD>
__global__ __launch_bounds__(512) void grouped_gemm_wgrad_sweep_kernel(BwdArgs p) {
  constexpr int kDN = kFixD ? 256 : 128;  // dw rows of a tile (dy columns)
  constexpr int kXK = kFixD ? 128 : 256;  // dw columns of a tile (x columns)
  constexpr int kDRow = kDN * 2, kXRow = kXK * 2;  // LDS row bytes of the dy and x slabs
  constexpr int kFixRow = 512, kSwRow = 256;
  constexpr int kFixBytes = kSweepRows * kFixRow, kSwBytes = kSweepRows * kSwRow;
  constexpr int kWN = kDN / 64;                    // wavefronts along the dw rows (64 x 64 each)
  constexpr int kFixDma = kFixBytes / 1024 / 8, kSwDma = kSwBytes / 1024 / 8;  // 1 KiB blocks per wavefront
  constexpr int kStores = 8;                       // 16-byte stores per lane per tile
  static_assert(kWN * (kXK / 64) == 8, "8 wavefronts");
  static_assert(kFixBytes + 3 * kSwBytes <= 160 * 1024, "LDS");
  static_assert(kStores + kSwDma + kStores <= 63 && kFixDma + 2 * kSwDma <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[kFixBytes + 3 * kSwBytes];
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char *)smem));
  const uint32_t fix_lds = lds_base, sw_lds = lds_base + kFixBytes;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wn = wave % kWN, wk = wave / kWN;
  const int m32 = static_cast<int>(p.M), g_count = static_cast<int>(p.G);
  const int N = static_cast<int>(p.N), K = static_cast<int>(p.K);

  const int first = long_group_count(p.order_rows, g_count, m32, kSweepRows);
  const int n_fix = static_cast<int>(kFixD ? ceil_div(N, kDN) : ceil_div(K, kXK));
  const int n_sw = static_cast<int>(kFixD ? ceil_div(K, kXK) : ceil_div(N, kDN));
  const int len = max(1, min(p.sweep_len, n_sw));
  const int n_rng = (n_sw + len - 1) / len;
  const int64_t units = static_cast<int64_t>(g_count - first) * n_rng * n_fix;
  const int64_t P = gridDim.x, b = blockIdx.x;
  const int64_t r = (b % 8) * (P / 8) + b / 8;  // consecutive numbers on one XCD

  int ln = lane;
  asm volatile("" : "+v"(ln));
  // ---- DMA: slab rows of kRow bytes; 1 KiB block B holds rows B * (1024 / kRow) ..; lane l writes row
  // l / (kRow / 16) of the block, chunk position l % (kRow / 16), holding logical chunk position ^
  // rm16_swz(row); wavefront w's blocks are w + 8 j (the swizzle of a lane's row does not depend on j).
  auto lane_off = [&](int row_bytes, int gstride) -> int {
    const int cpr = row_bytes / 16, rpb = 1024 / row_bytes;
    const int row = wave * rpb + ln / cpr;
    const int lchunk = (ln % cpr) ^ rm16_swz(row);
    return row * gstride + lchunk * 16;
  };
  const int fix_stride = (kFixD ? N : K) * 2, sw_stride = (kFixD ? K : N) * 2;
  const int fix_off = lane_off(kFixRow, fix_stride), sw_off = lane_off(kSwRow, sw_stride);
  __amdgpu_buffer_rsrc_t rfix = make_rsrc(p.a, 0u), rsw = make_rsrc(p.b, 0u);
  auto dma_fixed = [&](int fi) {
    int o = fix_off;
    asm volatile("" : "+v"(o));
#pragma unroll
    for (int j = 0; j < kFixDma; ++j)
      dma16b(rfix, (lds_void *)(uintptr_t)(fix_lds + (wave + 8 * j) * 1024), o + j * 8 * (1024 / kFixRow) * fix_stride,
             fi * (kFixD ? kDN : kXK) * 2);
  };
  auto dma_swept = [&](int wi, int slot) {
    int o = sw_off;
    asm volatile("" : "+v"(o));
#pragma unroll
    for (int j = 0; j < kSwDma; ++j)
      dma16b(rsw, (lds_void *)(uintptr_t)(sw_lds + slot * kSwBytes + (wave + 8 * j) * 1024),
             o + j * 8 * (1024 / kSwRow) * sw_stride, wi * (kFixD ? kXK : kDN) * 2);
  };

  // ---- fragments (16-lane group rg reads reduction rows 8 rg .. 8 rg + 7)
  const int rg = lane >> 4, rj = (lane >> 2) & 3, rq = lane & 3;
  const uint32_t rm_in = ((rq >> 1) << 4) + (rq & 1) * 8;
  uint32_t rmx = static_cast<uint32_t>((rj << 1) | (rg & 1)) << 5;
  asm volatile("" : "+v"(rmx));
  const uint32_t fd0 = (8 * rg + rj) * kDRow + rm_in, fx0 = (8 * rg + rj) * kXRow + rm_in;
  f32x4_t acc[4][4];
  // acc[i][j] = dw rows wn * 64 + 16 i .., columns wk * 64 + 16 j .. of the tile, with the MFMA operands of
  // the ping-pong kernel (x fragment first): every dw element is the same MFMA sequence.
  auto compute = [&](int slot) {
    const uint32_t d_lds = (kFixD ? fix_lds : sw_lds + slot * kSwBytes) + fd0;
    const uint32_t x_lds = (kFixD ? sw_lds + slot * kSwBytes : fix_lds) + fx0;
#pragma unroll
    for (int ks = 0; ks < kSweepRows / 32; ++ks) {
      bf16x8 fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[i] = read_rm_frag_rows<kDRow>(d_lds + ks * 32 * kDRow + ((static_cast<uint32_t>(wn * 4 + i) * 32u) ^ rmx));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[j] = read_rm_frag_rows<kXRow>(x_lds + ks * 32 * kXRow + ((static_cast<uint32_t>(wk * 4 + j) * 32u) ^ rmx));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = mma16<false>(fb[j], fa[i], ks == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
    }
  };
  // Epilogue: register r of lane l in block (i, j) holds dw row wn * 64 + i * 16 + l % 16 and column
  // wk * 64 + j * 16 + 4 (l / 16) + r of the tile; bf16 RNE, v_permlane16_swap pairs blocks j, j + 1 so
  // each lane stores 8 consecutive columns (16 bytes). Rows past N lie past the resource, columns past K
  // get an offset past it.
  const uint32_t ld = static_cast<uint32_t>(K) * 2u;
  auto epilogue = [&](int g, int nt, int kt) {
    const __amdgpu_buffer_rsrc_t ro =
        make_rsrc(static_cast<const uint16_t *>(p.out) + static_cast<int64_t>(g) * N * K, static_cast<uint32_t>(N) * ld);
    const int eq = ln >> 4;
    const int col0 = kt * kXK + wk * 64 + (eq & 1) * 16 + (eq >> 1) * 8;
    const uint32_t row0 = static_cast<uint32_t>(nt * kDN + wn * 64 + (ln & 15));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int jp = 0; jp < 4; jp += 2) {
        uint32_t wd[2][2];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          const bf16x2 a0 = {(__bf16)acc[i][jp + d][0], (__bf16)acc[i][jp + d][1]};
          const bf16x2 a1 = {(__bf16)acc[i][jp + d][2], (__bf16)acc[i][jp + d][3]};
          wd[d][0] = __builtin_bit_cast(uint32_t, a0);
          wd[d][1] = __builtin_bit_cast(uint32_t, a1);
        }
        u32x4 o;
#if defined(__HIP_DEVICE_COMPILE__)
        const auto s0 = __builtin_amdgcn_permlane16_swap(wd[0][0], wd[1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(wd[0][1], wd[1][1], false, false);
        o = u32x4{s0[0], s1[0], s0[1], s1[1]};
#else
        o = u32x4{0u, 0u, 0u, 0u};
#endif
        const int gcol = col0 + jp * 16;
        const uint32_t off = gcol < K ? (row0 + i * 16) * ld + static_cast<uint32_t>(gcol) * 2u : kNoAccess;
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

  // ---- units r, r + P, ...: (group position, range, fixed tile), the fixed tile fastest
  for (int64_t u = r; u < units; u += P) {
    const int per_g = n_rng * n_fix;
    const int gi = first + static_cast<int>(u / per_g);
    const int rem = static_cast<int>(u - static_cast<int64_t>(gi - first) * per_g);
    const int rng = rem / n_fix, fi = rem - rng * n_fix;
    const int w0 = rng * len, n = min(len, n_sw - w0);
    const int g = min(max(ld_inv(p.order, gi), 0), g_count - 1);
    const int lo = min(max(ld_inv(p.order_rows, 2 * gi), 0), m32);
    const int hi = min(max(ld_inv(p.order_rows, 2 * gi + 1), lo), m32);
    // Rows past the group's end lie past the resources: zeros.
    const uint32_t rows = static_cast<uint32_t>(hi - lo);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(p.a + static_cast<int64_t>(lo) * N, rows * static_cast<uint32_t>(N) * 2u);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(p.b + static_cast<int64_t>(lo) * K, rows * static_cast<uint32_t>(K) * 2u);
    rfix = kFixD ? rd : rx;
    rsw = kFixD ? rx : rd;
    // The previous unit is done (its stores included) and every wavefront has left its slabs.
    wait_dma();
    barrier();
    dma_fixed(fi);
    dma_swept(w0, 0);
    if (n > 1) dma_swept(w0 + 1, 1);
    wait_dma();
    barrier();
    int slot = 0;
    for (int i = 0; i < n; ++i) {
      const bool ahead = i + 2 < n;
      const int slot2 = slot == 0 ? 2 : slot - 1;  // (i + 2) % 3: the slot tile i - 1 read (barrier since)
      if (ahead) dma_swept(w0 + i + 2, slot2);
      compute(slot);
      const int wi = w0 + i;
      epilogue(g, kFixD ? fi : wi, kFixD ? wi : fi);
      if (i + 1 < n) {
        // Tile i + 1's slab has landed (issued before the stores of tile i - 1); those stores, the slab of
        // tile i + 2 and this tile's stores may be in flight.
        if (ahead) {
          wait_vm_n<kStores + kSwDma + kStores>();
        } else {
          wait_vm_n<kStores + kStores>();
        }
        barrier();
      }
      slot = slot == 2 ? 0 : slot + 1;
    }
  }
}

template <bool kFixD>
void launch_sweep(const BwdArgs &p, hipStream_t s) {
  const int64_t grid = std::max<int64_t>(8, num_cus() / 8 * 8);
  grouped_gemm_wgrad_sweep_kernel<kFixD><<<dim3(static_cast<uint32_t>(grid)), dim3(512), 0, s>>>(p);
}

// Orientation and unit length of the sweep: the fewest tiles on the busiest workgroup (each unit also costs
// about 1.5 tiles of slab loading), counting every group as short.
struct SweepPlan {
  bool fixd;
  int len;
};
SweepPlan sweep_plan(int64_t N, int64_t K, int64_t G, int64_t cus) {
  SweepPlan best{K >= N, 1};
  double best_work = -1.0;
  const int64_t P = std::max<int64_t>(8, cus / 8 * 8);
  for (int f = 0; f < 2; ++f) {
    const bool fixd = f == 0;
    const int64_t n_fix = fixd ? ceil_div(N, 256) : ceil_div(K, 256);
    const int64_t n_sw = fixd ? ceil_div(K, 128) : ceil_div(N, 128);
    const int lens[] = {8, 10, 12, 16, 20, 24, 32, 40, 48, 64};
    for (int li = -1; li < 10; ++li) {
      const int64_t L = li < 0 ? n_sw : lens[li];
      if (L > n_sw || L < 1) continue;
      const int64_t units = G * ceil_div(n_sw, L) * n_fix;
      const int64_t per = ceil_div(units, P);
      const double work = static_cast<double>(per) * (static_cast<double>(L) + 1.5);
      if (best_work < 0 || work < best_work) {
        best_work = work;
        best = {fixd, static_cast<int>(L)};
      }
    }
  }
  return best;
}

template <bool kWgrad, int kOut = 0, bool kSplit = false, bool kOrder = false, bool kF16 = false>
void launch_pipe(const BwdArgs &p, int64_t max_tiles, hipStream_t s) {
  int64_t grid = std::min<int64_t>(num_cus(), max_tiles);
  grid = std::max<int64_t>(8, (grid + 7) / 8 * 8);
  grouped_gemm_bwd_pipe_kernel<kWgrad, kOut, kSplit, kOrder, kF16><<<dim3(grid), dim3(256), 0, s>>>(p);
}

#ifndef MOE_GEMM_BWD_PINGPONG
#define MOE_GEMM_BWD_PINGPONG 1
#endif
// The tf32 router dgrad on the fp16 matrix cores (1) or on the bf16 hi/lo split (0).
#ifndef MOE_ROUTER_DGRAD_F16
#define MOE_ROUTER_DGRAD_F16 1
#endif
// Its GEMM's column tiles: 128 (two workgroups per CU) or 256.
#ifndef MOE_ROUTER_DGRAD_TN
#define MOE_ROUTER_DGRAD_TN 128
#endif
template <bool kWgrad, bool kOrder = false, bool kTails = false>
void launch_pp(const BwdArgs &p, int64_t max_tiles, hipStream_t s) {
  int64_t grid = std::min<int64_t>(num_cus(), max_tiles);
  grid = std::max<int64_t>(8, (grid + 7) / 8 * 8);
  grouped_gemm_bwd_pp_kernel<kWgrad, kOrder, kTails><<<dim3(grid), dim3(512), 0, s>>>(p);
}

// order[rank] = group, rank = the number of groups with more rows (or as many
// and a lower index): the groups largest first, a permutation of 0..G-1 (one
// block; group sizes clamped as the GEMM's tile walker clamps them). A bitonic
// sort in LDS of the keys (~rows << 32 | g), ascending, padded with all-ones
// keys to a power of two: 78 compare-exchange stages of 2 pairs per thread at
// G = 4096 (the rank count of every pair of groups took G^2 / 1024 compares
// per thread).
__global__ __launch_bounds__(1024) void group_order_kernel(const int32_t *offsets, int G, int64_t M, int16_t *order,
                                                           int32_t *order_rows) {
  __shared__ uint64_t s_key[4096];
  int n = 1;
  while (n < G) n <<= 1;
  for (int i = threadIdx.x; i < n; i += 1024) {
    uint64_t key = ~uint64_t(0);
    if (i < G) {
      const int64_t lo = min(max(static_cast<int64_t>(offsets[i]), int64_t(0)), M);
      const int64_t hi = min(max(static_cast<int64_t>(offsets[i + 1]), lo), M);
      key = (static_cast<uint64_t>(~static_cast<uint32_t>(hi - lo)) << 32) | static_cast<uint32_t>(i);
    }
    s_key[i] = key;
  }
  __syncthreads();
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += 1024) {
        const int l = i ^ j;
        if (l > i) {
          const uint64_t a = s_key[i], c = s_key[l];
          const bool up = (i & k) == 0;  // ascending run
          if ((a > c) == up) {
            s_key[i] = c;
            s_key[l] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int r = threadIdx.x; r < G; r += 1024) {
    const int g = static_cast<int>(s_key[r] & 0xffffu);
    const int64_t lo = min(max(static_cast<int64_t>(offsets[g]), int64_t(0)), M);
    const int64_t hi = min(max(static_cast<int64_t>(offsets[g + 1]), lo), M);
    order[r] = static_cast<int16_t>(g);
    order_rows[2 * r] = static_cast<int32_t>(lo);
    order_rows[2 * r + 1] = static_cast<int32_t>(hi);
  }
}

template <int kOut = 0, bool kNtB = false, bool kF16 = false, int kTN = 256, int kStagesT = 3>
void launch_dgrad128(const BwdArgs &p, int64_t max_tiles, hipStream_t s) {
  // one workgroup per CU, two with 128-column tiles
  int64_t grid = std::min<int64_t>((kTN == 128 ? 2 : 1) * num_cus(), max_tiles);
  grid = std::max<int64_t>(8, (grid + 7) / 8 * 8);
  grouped_gemm_dgrad128_kernel<kOut, kNtB, kF16, kTN, kStagesT><<<dim3(grid), dim3(256), 0, s>>>(p);
}

// ---- tf32 GEMMs of the router backward on the bf16 matrix cores ---------
// kernel_cases/case39_ref_musa_asm_tf32_ssgemm_nn_384x256.py:61-68 and
// case31_ref_musa_asm_tf32_ssgemm_tn_128x256.py:61-68 (reference_tf32): both
// operands are fp32 rounded to tf32 (round_tf32_rne, :51-58 / :52-58: add 0x1000 unless the 13
// dropped bits are exactly 0x1000 and the kept LSB is even, then clear them),
// the products are exact and accumulate in fp32.  gfx950 has no tf32 matrix
// instruction, so each tf32 value t is split into bf16 hi = RNE(t) and
// lo = t - hi (at most 4 significant bits: exact in bf16), and
// a b = hi_a hi_b + hi_a lo_b + lo_a hi_b + lo_a lo_b with the last term,
// below 2^-16 |a b|, dropped: three bf16 products per tf32 product, each exact
// in the fp32 accumulator.
__device__ __forceinline__ uint32_t tf32_rne_bits(uint32_t b) {
  const uint32_t low = b & 0x1FFFu, lsb = (b >> 13) & 1u;
  const uint32_t add = (low == 0x1000u && lsb == 0u) ? 0u : 0x1000u;
  return (b + add) & 0xFFFFE000u;
}

// src fp32 [rows, cols] (cols % 4 == 0) -> hi (and a second copy hi2) and lo
// bf16 planes with their own row strides (null planes are skipped).
struct SplitArgs {
  const float *src;
  int64_t rows, cols;
  uint16_t *hi, *hi2, *lo;
  int64_t ld_hi, ld_hi2, ld_lo;
};

__global__ __launch_bounds__(256) void tf32_split_kernel(SplitArgs p) {
  const int64_t q = p.cols / 4;
  const int64_t total = p.rows * q;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / q, c = (i - r * q) * 4;
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p.src + r * p.cols + c));
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t = __uint_as_float(tf32_rne_bits(in[e]));
      h[e] = f32_to_bf16_rne(t);
      l[e] = f32_to_bf16_rne(t - bf16_to_f32(h[e]));
    }
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 hv = {h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    const u32x2 lv = {l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
    if (p.hi != nullptr) *reinterpret_cast<u32x2 *>(p.hi + r * p.ld_hi + c) = hv;
    if (p.hi2 != nullptr) *reinterpret_cast<u32x2 *>(p.hi2 + r * p.ld_hi2 + c) = hv;
    if (p.lo != nullptr) *reinterpret_cast<u32x2 *>(p.lo + r * p.ld_lo + c) = lv;
  }
}

void launch_split(const SplitArgs &a, hipStream_t s) {
  const int64_t n = a.rows * (a.cols / 4);
  if (n <= 0) return;
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), 8192));
  tf32_split_kernel<<<dim3(grid), dim3(256), 0, s>>>(a);
}

// ---- tf32 wgrad on the fp16 matrix cores --------------------------------
// A tf32 value has 11 significant bits, as many as fp16. Scaled by the power of
// two 2^e that brings the largest magnitude of its column into [2^14, 2^15),
// every tf32-rounded value of the column is an fp16 value, exactly unless it
// lies 2^29 or more below that largest one (it then rounds to an fp16
// subnormal: an error below 2^-38 of the column's largest magnitude). The
// product of two fp16 values is exact in fp32, so one fp16 MFMA replaces the
// three bf16 products of the hi/lo split, and the fp32 sums are scaled back by
// 2^-(e_row + e_col) (exact) when the reduction planes are added. The scale
// comes from the largest finite magnitude (Inf and NaN entries stay Inf and
// NaN when scaled, so every finite value still converts exactly); a column
// with no finite nonzero value keeps scale 1.
__device__ __forceinline__ float finite_abs(float x) {
  const float a = fabsf(x);
  return a < __builtin_huge_valf() ? a : 0.f;  // Inf and NaN -> 0
}
__device__ __forceinline__ int scale_exp(float mx) {
  if (!(mx > 0.f) || !(mx < __builtin_huge_valf())) return 0;
  int e = 0;
  (void)__builtin_frexpf(mx, &e);  // mx = f 2^e, f in [0.5, 1)
  return 15 - e;                   // mx 2^(15 - e) in [2^14, 2^15)
}

// Largest finite magnitude per column over a slab of rows: block (x, y) covers cg
// groups of 4 columns from x 4 cg and rows y rps .. + rps - 1, its threads
// split over the groups (t % cg) and 256 / cg interleaved row phases (t / cg,
// combined in LDS), 8 independent rows per round; part[y][c].
__global__ __launch_bounds__(256) void colmax_partial_kernel(const float *src, int64_t R, int64_t C, int64_t rps, int cg,
                                                             float *part) {
  __shared__ u32x4 red[256];
  const int t = threadIdx.x;
  const int ph = 256 / cg, g = t % cg, f = t / cg;
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * cg + g) * 4;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rps, r1 = min(R, r0 + rps);
  float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
  if (f < ph && c < C) {
    for (int64_t r = r0 + f; r < r1; r += 8 * ph) {
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t ru = r + u * ph;
        v[u] = ru < r1 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + ru * C + c)) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        m0 = fmaxf(m0, finite_abs(__uint_as_float(v[u].x)));
        m1 = fmaxf(m1, finite_abs(__uint_as_float(v[u].y)));
        m2 = fmaxf(m2, finite_abs(__uint_as_float(v[u].z)));
        m3 = fmaxf(m3, finite_abs(__uint_as_float(v[u].w)));
      }
    }
  }
  red[t] = u32x4{__float_as_uint(m0), __float_as_uint(m1), __float_as_uint(m2), __float_as_uint(m3)};
  __syncthreads();
  if (f == 0 && c < C) {
    for (int k = 1; k < ph; ++k) {
      const u32x4 o = red[t + k * cg];
      m0 = fmaxf(m0, __uint_as_float(o.x));
      m1 = fmaxf(m1, __uint_as_float(o.y));
      m2 = fmaxf(m2, __uint_as_float(o.z));
      m3 = fmaxf(m3, __uint_as_float(o.w));
    }
    *reinterpret_cast<u32x4 *>(part + static_cast<int64_t>(blockIdx.y) * C + c) =
        u32x4{__float_as_uint(m0), __float_as_uint(m1), __float_as_uint(m2), __float_as_uint(m3)};
  }
}

// exp[c] = scale_exp(largest of part[0..S)[c]) (S <= 64: eight independent loads per round); kI8: clamped to
// at most 127 (columns whose largest magnitude lies below 2^-112) and also written as int8 to exp8.
template <bool kI8 = false>
__global__ __launch_bounds__(256) void colmax_final_kernel(const float *part, int S, int64_t C, int32_t *exp,
                                                           int8_t *exp8) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= C) return;
  float m = 0.f;
  for (int y0 = 0; y0 < S; y0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = y0 + u < S ? part[static_cast<int64_t>(y0 + u) * C + c] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) m = fmaxf(m, v[u]);
  }
  if constexpr (kI8) {
    const int e = min(scale_exp(m), 127);
    exp[c] = e;
    exp8[c] = static_cast<int8_t>(e);
  } else {
    (void)exp8;
    exp[c] = scale_exp(m);
  }
}

// Row-scaled fp16 copy for the tf32 router dgrad: one wavefront per row r of src [R, C] (C % 4 == 0), the row's
// first 1024 values read once and kept in registers for the conversion:
// e = scale_exp(largest finite magnitude of the row), at most 127; dst[r][c] = fp16(tf32(src[r][c]) 2^e) (RNE) and
// exp8 at the row's permuted position (128 b + 4 (r % 32) + (r % 128) / 32 for r = 128 b + (r % 128)).
// Rows R .. R8 - 1 (R8 = R rounded up to 128) only get exponent 0.
__global__ __launch_bounds__(256) void tf32_to_f16_rows_kernel(const float *src, int64_t R, int64_t R8, int64_t C,
                                                               uint16_t *dst, int8_t *exp8) {
  constexpr int kKeep = 4;  // 16-byte vectors per lane kept in registers between the two passes (rows of <= 1024)
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (r >= R8) return;
  const int64_t q = C / 4;
  const u32x4 *row = reinterpret_cast<const u32x4 *>(src + r * C);
  auto vmax = [](float m, const u32x4 &v) {
    return fmaxf(m, fmaxf(fmaxf(finite_abs(__uint_as_float(v.x)), finite_abs(__uint_as_float(v.y))),
                          fmaxf(finite_abs(__uint_as_float(v.z)), finite_abs(__uint_as_float(v.w)))));
  };
  float m = 0.f;
  u32x4 keep[kKeep];
#pragma unroll
  for (int u = 0; u < kKeep; ++u) {
    const int64_t i = lane + u * kWave;
    keep[u] = (r < R && i < q) ? __builtin_nontemporal_load(row + i) : u32x4{0u, 0u, 0u, 0u};
    m = vmax(m, keep[u]);
  }
  if (r < R) {
    for (int64_t i = lane + kKeep * kWave; i < q; i += kWave) m = vmax(m, row[i]);
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  const int e = r < R ? min(scale_exp(m), 127) : 0;
  if (lane == 0) {
    const int64_t w = r % 128;
    exp8[r - w + (w % 32) * 4 + w / 32] = static_cast<int8_t>(e);
  }
  if (r >= R) return;
  auto convert = [&](int64_t i, const u32x4 &v) {
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float t = __builtin_ldexpf(__uint_as_float(tf32_rne_bits(in[k])), e);
      h[k] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(t));
    }
    *reinterpret_cast<u32x2 *>(dst + r * C + i * 4) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  };
#pragma unroll
  for (int u = 0; u < kKeep; ++u) {
    const int64_t i = lane + u * kWave;
    if (i < q) convert(i, keep[u]);
  }
  for (int64_t i = lane + kKeep * kWave; i < q; i += kWave) convert(i, row[i]);
}

// dst[r][c] = fp16(tf32(src[r][c]) 2^exp[c]) (RNE; C % 4 == 0).
__global__ __launch_bounds__(256) void tf32_to_f16_cols_kernel(const float *src, int64_t R, int64_t C, const int32_t *exp,
                                                               uint16_t *dst) {
  const int64_t q = C / 4;
  const int64_t total = R * q;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / q, c = (i - r * q) * 4;
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + r * C + c));
    const int4 e = *reinterpret_cast<const int4 *>(exp + c);
    const uint32_t in[4] = {v.x, v.y, v.z, v.w};
    const int ex[4] = {e.x, e.y, e.z, e.w};
    uint32_t h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float t = __builtin_ldexpf(__uint_as_float(tf32_rne_bits(in[k])), ex[k]);
      h[k] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(t));
    }
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2 *>(dst + r * C + c) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  }
}

// out[n][k] = 2^-(row_exp[n] + col_exp[k]) sum over s of part[s][n][k], s ascending (K % 4 == 0).
__global__ __launch_bounds__(256) void sum_planes_scaled_kernel(const float *part, int planes, int64_t N, int64_t K,
                                                                const int32_t *row_exp, const int32_t *col_exp, float *out) {
  const int64_t n = N * K;
  const int64_t q = n / 4, qk = K / 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < q; i += stride) {
    u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(part) + i);
    float x = __uint_as_float(a.x), y = __uint_as_float(a.y), z = __uint_as_float(a.z), w = __uint_as_float(a.w);
    for (int s = 1; s < planes; ++s) {
      const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(part + s * n) + i);
      x += __uint_as_float(b.x);
      y += __uint_as_float(b.y);
      z += __uint_as_float(b.z);
      w += __uint_as_float(b.w);
    }
    const int64_t row = i / qk, col = (i - row * qk) * 4;
    const int er = row_exp[row];
    const int4 ec = *reinterpret_cast<const int4 *>(col_exp + col);
    x = __builtin_ldexpf(x, -(er + ec.x));
    y = __builtin_ldexpf(y, -(er + ec.y));
    z = __builtin_ldexpf(z, -(er + ec.z));
    w = __builtin_ldexpf(w, -(er + ec.w));
    *(reinterpret_cast<u32x4 *>(out) + i) = u32x4{__float_as_uint(x), __float_as_uint(y), __float_as_uint(z), __float_as_uint(w)};
  }
}

// Column-max slabs of an [R, C] operand: at most 64 slabs of at least 64 rows (C is not used: the slab
// count only bounds the final pass's loads per column).
struct ColmaxPlan {
  int64_t S, rps;
  int cg;      // groups of 4 columns per block (the rest of the 256 threads split the rows)
  int64_t xb;  // blocks across the columns
};
ColmaxPlan colmax_plan(int64_t R, int64_t C) {
  const int64_t S = std::max<int64_t>(1, std::min<int64_t>(64, ceil_div(R, 64)));
  const int64_t rps = std::max<int64_t>(1, ceil_div(R, S));
  int cg = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(256, ceil_div(C, 4))));
  const int64_t slabs = ceil_div(std::max<int64_t>(R, 1), rps);
  // At least 512 workgroups where the shape allows: fewer column groups per block, more row phases
  // (case39's weight, 320 rows: 40 -> 640 workgroups).
  while (cg > 1 && ceil_div(ceil_div(C, 4), cg) * slabs < 512) cg >>= 1;
  return {slabs, rps, cg, std::max<int64_t>(1, ceil_div(ceil_div(C, 4), cg))};
}


// dx rows r of group 0 (offsets[0] <= r < offsets[1], clamped to [0, M)):
// dx[r][c] = bf16 RNE of the sum over s of part[s][r][c], s ascending; other
// rows are not written (K % 4 == 0, 16-byte aligned part, 8-byte aligned dx).
__global__ __launch_bounds__(256) void sum_planes_rows_bf16_kernel(const float *part, int planes, int64_t M, int64_t K,
                                                                   const int32_t *offsets, uint16_t *dx) {
  const int64_t lo = min(max(static_cast<int64_t>(offsets[0]), int64_t(0)), M);
  const int64_t hi = min(max(static_cast<int64_t>(offsets[1]), lo), M);
  const int64_t n = M * K;
  const int64_t q_lo = lo * K / 4, q_hi = hi * K / 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = q_lo + static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < q_hi; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(part) + i);
    float x = __uint_as_float(a.x), y = __uint_as_float(a.y), z = __uint_as_float(a.z), w = __uint_as_float(a.w);
    for (int s = 1; s < planes; ++s) {
      const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(part + s * n) + i);
      x += __uint_as_float(b.x);
      y += __uint_as_float(b.y);
      z += __uint_as_float(b.z);
      w += __uint_as_float(b.w);
    }
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 o = {f32_to_bf16_rne(x) | (f32_to_bf16_rne(y) << 16), f32_to_bf16_rne(z) | (f32_to_bf16_rne(w) << 16)};
    *reinterpret_cast<u32x2 *>(dx + 4 * i) = o;
  }
}

constexpr size_t kWsAlign = 256;
size_t align_up(size_t x) { return (x + kWsAlign - 1) / kWsAlign * kWsAlign; }

}  // namespace
}  // namespace moe

namespace {

int check_common(const char *fn, int64_t M_total, int64_t N, int64_t K, int64_t G, const int32_t *group_offsets) {
  using namespace moe;
  if (M_total < 0 || N < 0 || K < 0 || G < 0) {
    return fail(MOE_ERR_SHAPE, "%s: negative size (M=%lld N=%lld K=%lld G=%lld)", fn, (long long)M_total,
                (long long)N, (long long)K, (long long)G);
  }
  if (G < 1 || G > 4096) return fail(MOE_ERR_CAPACITY, "%s: G=%lld outside [1, 4096]", fn, (long long)G);
  if (M_total > (int64_t(1) << 31) - 1) return fail(MOE_ERR_CAPACITY, "%s: M=%lld rows exceed 2^31 - 1", fn, (long long)M_total);
  if (N % 8 != 0 || K % 8 != 0) {
    return fail(MOE_ERR_SHAPE, "%s: N=%lld and K=%lld must be multiples of 8", fn, (long long)N, (long long)K);
  }
  if (group_offsets == nullptr) return fail(MOE_ERR_INVALID_ARG, "%s: null group_offsets", fn);
  return MOE_OK;
}

// Reduction split of a one-group dgrad whose output has fewer tiles than half
// the CUs (case37: 2 x 32 tiles): s splits of whole 64-column steps (at least
// three each; the last split takes the remainder), at most one split per
// otherwise idle CU and 16 in all. s = 1: no split.
struct DgradSplit {
  int64_t s, kchunk;
};

DgradSplit dgrad_split_plan(int64_t M, int64_t N, int64_t K, int64_t G) {
  using namespace moe;
  DgradSplit pl{1, 0};
  if (G != 1 || M <= 160 || M > (int64_t(1) << 31) - 1 || N % kBK != 0 || N < 6 * kBK || K == 0) return pl;
  const int64_t tiles = ceil_div(M, 256) * ceil_div(K, kBN);
  const int64_t cus = gemm::num_cus();
  if (2 * tiles > cus) return pl;
  const int64_t ksteps = N / kBK;
  const int64_t s = std::min<int64_t>(std::min<int64_t>(cus / tiles, ksteps / 3), 16);
  if (s < 2) return pl;
  const int64_t kc = ksteps / s;  // >= 3
  pl.s = ksteps / kc;
  pl.kchunk = kc * kBK;
  return pl;
}

// dgrad runs the 256-row ping-pong kernel (no split; groups of more than 160
// rows on average; whole reduction steps) with a reduction long enough for the
// 128-row tail tiles: group tails of 1 to 128 rows then take 128-row tiles
// after the 256-row ones, listed in a workspace of tails_bytes(G).
bool dgrad_pp_tails(int64_t M, int64_t N, int64_t G) {
  using namespace moe;
  return MOE_GEMM_BWD_PINGPONG && G >= 1 && G <= 4096 && M > 160 * G && M < (int64_t(1) << 31) && N % kBK == 0 &&
         N >= std::max<int64_t>(3 * kBK, gemm::kTailsMinK);
}

// tf32 router dgrad, grad_input [M, N] = grad_output [M, K] weight [K, N]. With more than 160 rows and a
// reduction of whole steps (K % 64 == 0, K >= 192) it runs on the fp16 matrix cores: grad_output's rows and
// weight's columns are scaled by powers of two into the fp16 range (one exact fp16 product per tf32
// product) and the GEMM's epilogue undoes both scales; otherwise it runs on the bf16 hi/lo split (three
// products, a 3K reduction). Workspace (byte offsets, each 256-byte aligned): fp16 path: the fp16 copies
// a16 [M, K] and b16 [K, N], the int8 row exponents (M rounded up to 128), the column exponents (int32 and
// int8) and the column-max slabs; split path: the stacked bf16 operands [M, 3K] and [3K, N].
struct DgradTf32Layout {
  bool f16;
  moe::ColmaxPlan cb;
  int64_t m8;  // M rounded up to 128
  size_t a16, b16, row_e8, col_e32, col_e8, part_b, total;
};
DgradTf32Layout dgrad_tf32_layout(int64_t M, int64_t K, int64_t N) {
  using moe::align_up;
  DgradTf32Layout l{};
  l.f16 = MOE_ROUTER_DGRAD_F16 != 0;
  if (!l.f16) {
    l.total = align_up(static_cast<size_t>(M) * 3 * K * 2) + align_up(static_cast<size_t>(3 * K) * N * 2);
    return l;
  }
  l.cb = moe::colmax_plan(K, N);
  l.m8 = moe::ceil_div(M, 128) * 128;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  l.a16 = take(static_cast<size_t>(M) * K * 2);
  l.b16 = take(static_cast<size_t>(K) * N * 2);
  l.row_e8 = take(static_cast<size_t>(l.m8));
  l.col_e32 = take(static_cast<size_t>(N) * 4);
  l.col_e8 = take(static_cast<size_t>(N));
  l.part_b = take(static_cast<size_t>(l.cb.S) * N * 4);
  l.total = off;
  return l;
}

}  // namespace

extern "C" {

size_t moe_grouped_gemm_dgrad_workspace_size(int64_t M_total, int64_t N, int64_t K, int64_t G) {
  if (M_total < 0 || N < 0 || K < 0 || G < 1) return 0;
  const DgradSplit sp = dgrad_split_plan(M_total, N, K, G);
  if (sp.s > 1) return moe::align_up(static_cast<size_t>(sp.s) * M_total * K * 4);
  return dgrad_pp_tails(M_total, N, G) ? moe::align_up(moe::gemm::tails_bytes(G)) : 0;
}

int moe_grouped_gemm_dgrad(const moe_bf16_t *dy, int64_t M_total, int64_t N, const moe_bf16_t *w, int64_t G,
                           int64_t K, const int32_t *group_offsets, moe_bf16_t *dx, void *workspace,
                           size_t workspace_bytes, void *stream) {
  using namespace moe;
  const char *fn = "moe_grouped_gemm_dgrad";
  if (int rc = check_common(fn, M_total, N, K, G, group_offsets)) return rc;
  // 32-bit buffer offsets: a 256-row panel of dy and one expert's w stay below 2 GiB.
  if (N > (int64_t(1) << 22) - 8 || K > (int64_t(1) << 22) - 8 || N * K > (int64_t(1) << 30) - 1) {
    return fail(MOE_ERR_CAPACITY, "%s: N=%lld K=%lld exceed the 32-bit panel offsets (N, K < 2^22, N*K < 2^30)", fn,
                (long long)N, (long long)K);
  }
  if (M_total == 0 || K == 0) return MOE_OK;
  if (dx == nullptr || (N > 0 && (dy == nullptr || w == nullptr))) {
    return fail(MOE_ERR_INVALID_ARG, "%s: null dy, w or dx", fn);
  }
  if (!is_aligned(dy, 16) || !is_aligned(w, 16) || !is_aligned(dx, 16)) {
    return fail(MOE_ERR_ALIGN, "%s: dy, w and dx must be 16-byte aligned", fn);
  }
  BwdArgs p;
  p.a = dy;
  p.b = w;
  p.offsets = group_offsets;
  p.out = dx;
  p.M = M_total;
  p.N = N;
  p.K = K;
  p.G = G;
  p.ntiles = ceil_div(K, kBN);
  p.chunk = 0;
  p.kchunk = 0;
  p.order = nullptr;
  p.order_rows = nullptr;
  p.tails = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // One group with few output tiles (fewer than half the CUs) and a workspace
  // for the fp32 partials: the reduction is split over the idle CUs.
  const DgradSplit sp = dgrad_split_plan(M_total, N, K, G);
  const size_t need = sp.s > 1 ? align_up(static_cast<size_t>(sp.s) * M_total * K * 4) : 0;
  if (sp.s > 1 && workspace != nullptr && workspace_bytes >= need && is_aligned(workspace, kWsAlign)) {
    float *planes = static_cast<float *>(workspace);
    p.out = planes;
    p.G = sp.s;
    p.kchunk = sp.kchunk;
    launch_pipe<false, 1, true>(p, ceil_div(M_total, 256) * p.ntiles * sp.s, s);
    const int64_t q = M_total * K / 4;
    const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(ceil_div(q, 256), 4096));
    sum_planes_rows_bf16_kernel<<<dim3(grid), dim3(256), 0, s>>>(planes, static_cast<int>(sp.s), M_total, K,
                                                                group_offsets, reinterpret_cast<uint16_t *>(dx));
    return check_launch(fn);
  }
  // 128-row tiles when the groups average at most 160 rows (less padding in
  // every group's last row tile) and for reductions that are not whole steps
  // of at least three (N % 64 != 0 or N < 192); the pipelined 256-row kernel otherwise.
  // With short groups w is streamed once: non-temporal loads (case08 0.387 -> 0.365 ms, case07 unchanged).
  if (M_total <= 160 * G) {
    launch_dgrad128<0, true>(p, (ceil_div(M_total, 128) + G) * p.ntiles, s);
  } else if (N % kBK != 0 || N < 3 * kBK) {
    launch_dgrad128(p, (ceil_div(M_total, 128) + G) * p.ntiles, s);
  } else if (MOE_GEMM_BWD_PINGPONG) {
    // With a workspace and a long reduction, group tails of at most 128 rows
    // are listed first and computed as 128-row tiles after the 256-row ones.
    if (dgrad_pp_tails(M_total, N, G) && workspace != nullptr && workspace_bytes >= gemm::tails_bytes(G) &&
        is_aligned(workspace, kWsAlign)) {
      p.tails = static_cast<int *>(workspace);
      gemm::tails_init_kernel<<<dim3(1), dim3(256), 0, s>>>(group_offsets, G, M_total, p.tails);
      launch_pp<false, false, true>(p, (ceil_div(M_total, 256) + G) * p.ntiles, s);
    } else {
      launch_pp<false>(p, (ceil_div(M_total, 256) + G) * p.ntiles, s);
    }
  } else {
    launch_pipe<false>(p, (ceil_div(M_total, 256) + G) * p.ntiles, s);
  }
  return check_launch(fn);
}

// The group order (largest first, dealt in reverse on odd rounds) evens out
// the steps per workgroup when the group sizes are skewed: c5 fc2 wgrad (224
// tiles per expert) 3.64 -> 3.51 ms and fc1 wgrad (448) 7.18 -> 6.94 ms on one
// box against the index order (the order alone, dealt the same way every
// round: fc2 6-7% faster, fc1 1% slower).
size_t moe_grouped_gemm_wgrad_workspace_size(int64_t M_total, int64_t N, int64_t K, int64_t G) {
  (void)M_total;
  if (G < 2 || G > 4096 || N <= 0 || K <= 0) return 0;
  return moe::align_up(static_cast<size_t>(G) * sizeof(int16_t)) + static_cast<size_t>(G) * 2 * sizeof(int32_t);
}

int moe_grouped_gemm_wgrad(const moe_bf16_t *dy, const moe_bf16_t *x, int64_t M_total, int64_t N, int64_t K,
                           int64_t G, const int32_t *group_offsets, moe_bf16_t *dw, void *workspace,
                           size_t workspace_bytes, void *stream) {
  using namespace moe;
  const char *fn = "moe_grouped_gemm_wgrad";
  if (int rc = check_common(fn, M_total, N, K, G, group_offsets)) return rc;
  // 32-bit buffer offsets: all of dy, all of x and one group's dw stay below 2 GiB.
  if (M_total * N > (int64_t(1) << 30) - 1 || M_total * K > (int64_t(1) << 30) - 1 ||
      N * K > (int64_t(1) << 30) - 1) {
    return fail(MOE_ERR_CAPACITY, "%s: M=%lld N=%lld K=%lld exceed the 32-bit offsets (M*N, M*K, N*K < 2^30)", fn,
                (long long)M_total, (long long)N, (long long)K);
  }
  if (N == 0 || K == 0) return MOE_OK;
  if (dw == nullptr || (M_total > 0 && (dy == nullptr || x == nullptr))) {
    return fail(MOE_ERR_INVALID_ARG, "%s: null dy, x or dw", fn);
  }
  if (!is_aligned(dy, 16) || !is_aligned(x, 16) || !is_aligned(dw, 16)) {
    return fail(MOE_ERR_ALIGN, "%s: dy, x and dw must be 16-byte aligned", fn);
  }
  BwdArgs p;
  p.a = dy;
  p.b = x;
  p.offsets = group_offsets;
  p.out = dw;
  p.M = M_total;
  p.N = N;
  p.K = K;
  p.G = G;
  p.ntiles = ceil_div(K, kBN);
  p.chunk = 0;
  p.kchunk = 0;
  p.order = nullptr;
  p.order_rows = nullptr;
  p.tails = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t tiles = G * ceil_div(N, 256) * p.ntiles;
  // Every group has the same tile count and a tile costs in proportion to its
  // group's rows: with a workspace the tiles take the groups largest first,
  // which spreads the work over the workgroups more evenly (skewed routing).
  const size_t need = moe_grouped_gemm_wgrad_workspace_size(M_total, N, K, G);
  if (need > 0 && workspace != nullptr && workspace_bytes >= need && is_aligned(workspace, 4)) {
    int16_t *order = static_cast<int16_t *>(workspace);
    int32_t *order_rows = reinterpret_cast<int32_t *>(static_cast<char *>(workspace) +
                                                      align_up(static_cast<size_t>(G) * sizeof(int16_t)));
    group_order_kernel<<<dim3(1), dim3(1024), 0, s>>>(group_offsets, static_cast<int>(G), M_total, order,
                                                      order_rows);
    p.order = order;
    p.order_rows = order_rows;
    // Groups averaging under 256 rows: the groups of at most 128 rows go to the sweep kernel (the dw store
    // stream), the rest to the ping-pong kernel, whose walker ends where the sweep's groups begin.
    if (MOE_GEMM_BWD_PINGPONG && M_total < 256 * G && N < (int64_t(1) << 22) && K < (int64_t(1) << 22)) {
      const SweepPlan sp = sweep_plan(N, K, G, num_cus());
      p.sweep_rows = kSweepRows;
      p.sweep_len = sp.len;
      if (sp.fixd) {
        launch_sweep<true>(p, s);
      } else {
        launch_sweep<false>(p, s);
      }
    }
    if (MOE_GEMM_BWD_PINGPONG) {
      launch_pp<true, true>(p, tiles, s);
    } else {
      launch_pipe<true, 0, false, true>(p, tiles, s);
    }
  } else if (MOE_GEMM_BWD_PINGPONG) {
    launch_pp<true>(p, tiles, s);
  } else {
    launch_pipe<true>(p, tiles, s);
  }
  return check_launch(fn);
}

size_t moe_router_dgrad_tf32_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M < 0 || K < 0 || N < 0) return 0;
  return dgrad_tf32_layout(M, K, N).total;
}

int moe_router_dgrad_tf32(const float *grad_output, int64_t M, int64_t K, const float *weight, int64_t N,
                          float *grad_input, void *workspace, size_t workspace_bytes, void *stream) {
  using namespace moe;
  const char *fn = "moe_router_dgrad_tf32";
  if (M < 0 || K < 0 || N < 0) {
    return fail(MOE_ERR_SHAPE, "%s: negative size (M=%lld K=%lld N=%lld)", fn, (long long)M, (long long)K, (long long)N);
  }
  if (K % 8 != 0 || N % 8 != 0) return fail(MOE_ERR_SHAPE, "%s: K=%lld and N=%lld must be multiples of 8", fn, (long long)K, (long long)N);
  if (3 * K > (int64_t(1) << 22) - 8 || N > (int64_t(1) << 22) - 8 || 3 * K * N > (int64_t(1) << 30) - 1) {
    return fail(MOE_ERR_CAPACITY, "%s: K=%lld N=%lld exceed the 32-bit offsets (3K, N < 2^22, 3K*N < 2^30)", fn,
                (long long)K, (long long)N);
  }
  if (M == 0 || N == 0) return MOE_OK;
  if (grad_input == nullptr || (K > 0 && (grad_output == nullptr || weight == nullptr))) {
    return fail(MOE_ERR_INVALID_ARG, "%s: null grad_output, weight or grad_input", fn);
  }
  if (!is_aligned(grad_output, 16) || !is_aligned(weight, 16) || !is_aligned(grad_input, 16)) {
    return fail(MOE_ERR_ALIGN, "%s: grad_output, weight and grad_input must be 16-byte aligned", fn);
  }
  const DgradTf32Layout l = dgrad_tf32_layout(M, K, N);
  const size_t need = l.total;
  if (workspace == nullptr || workspace_bytes < need || !is_aligned(workspace, kWsAlign)) {
    return fail(MOE_ERR_WORKSPACE, "%s: a 256-byte aligned workspace of %zu bytes is needed (got %zu)", fn, need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (l.f16) {
    char *w = static_cast<char *>(workspace);
    uint16_t *a16 = reinterpret_cast<uint16_t *>(w + l.a16);
    uint16_t *b16 = reinterpret_cast<uint16_t *>(w + l.b16);
    int8_t *row_e8 = reinterpret_cast<int8_t *>(w + l.row_e8);
    int32_t *col_e32 = reinterpret_cast<int32_t *>(w + l.col_e32);
    int8_t *col_e8 = reinterpret_cast<int8_t *>(w + l.col_e8);
    float *part_b = reinterpret_cast<float *>(w + l.part_b);
    // Scale exponents of weight's columns and its fp16 copy, then grad_output's rows with their fp16 copy.
    colmax_partial_kernel<<<dim3(static_cast<uint32_t>(l.cb.xb), static_cast<uint32_t>(l.cb.S)), dim3(256), 0, s>>>(
        weight, K, N, l.cb.rps, l.cb.cg, part_b);
    colmax_final_kernel<true><<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0, s>>>(
        part_b, static_cast<int>(l.cb.S), N, col_e32, col_e8);
    const int64_t gb = std::max<int64_t>(1, std::min<int64_t>(ceil_div(K * N / 4, 256), 8192));
    tf32_to_f16_cols_kernel<<<dim3(static_cast<uint32_t>(gb)), dim3(256), 0, s>>>(weight, K, N, col_e32, b16);
    tf32_to_f16_rows_kernel<<<dim3(static_cast<uint32_t>(ceil_div(l.m8, 4))), dim3(256), 0, s>>>(grad_output, M, l.m8,
                                                                                                 K, a16, row_e8);
    if (int rc = check_launch(fn)) return rc;
    BwdArgs p;
    p.a = a16;
    p.b = b16;
    p.offsets = nullptr;
    p.out = grad_input;
    p.M = M;
    p.N = K;
    p.K = N;
    p.G = 1;
    constexpr int kTN = MOE_ROUTER_DGRAD_TN;
    p.ntiles = ceil_div(N, kTN);
    p.chunk = M;
    p.kchunk = 0;
    p.order = nullptr;
    p.order_rows = nullptr;
    p.tails = nullptr;
    p.row_exp8 = row_e8;
    p.col_exp8 = col_e8;
    launch_dgrad128<1, false, true, kTN, kTN == 128 ? 2 : 3>(p, (ceil_div(M, 128) + 1) * p.ntiles, s);
    return check_launch(fn);
  }
  // A' = [A_hi | A_hi | A_lo] [M, 3K] and B' = [B_hi; B_lo; B_hi] [3K, N]:
  // A' B' = A_hi B_hi + A_hi B_lo + A_lo B_hi, one GEMM with a 3K reduction.
  uint16_t *a3 = static_cast<uint16_t *>(workspace);
  uint16_t *b3 = reinterpret_cast<uint16_t *>(static_cast<char *>(workspace) + align_up(static_cast<size_t>(M) * 3 * K * 2));
  SplitArgs sa{grad_output, M, K, a3, a3 + K, a3 + 2 * K, 3 * K, 3 * K, 3 * K};
  SplitArgs sb{weight, K, N, b3, b3 + 2 * K * N, b3 + K * N, N, N, N};
  launch_split(sa, s);
  launch_split(sb, s);
  if (int rc = check_launch(fn)) return rc;
  BwdArgs p;
  p.a = a3;
  p.b = b3;
  p.offsets = nullptr;
  p.out = grad_input;
  p.M = M;
  p.N = 3 * K;
  p.K = N;
  p.G = 1;
  p.ntiles = ceil_div(N, kBN);
  p.chunk = M;
  p.kchunk = 0;
  p.order = nullptr;
  p.order_rows = nullptr;
  p.tails = nullptr;
  if (M <= 160 || (3 * K) % kBK != 0 || 3 * K < 3 * kBK) launch_dgrad128<1>(p, (ceil_div(M, 128) + 1) * p.ntiles, s);
  else launch_pipe<false, 1>(p, (ceil_div(M, 256) + 1) * p.ntiles, s);
  return check_launch(fn);
}

}  // extern "C"

namespace {

// Reduction split of the tf32 router wgrad: the output has few tiles
// (case31: 2 x 32 for 256 CUs), so the M rows are cut into uniform chunks run
// as groups of one launch, every chunk writing its own fp32 partial
// [N, K]; a last pass adds the partials in chunk order.
struct WgradPlan {
  int64_t s;  // chunks (1 = no split)
  int64_t c;  // rows per chunk
};

WgradPlan wgrad_plan(int64_t rows, int64_t N, int64_t K) {
  WgradPlan pl{1, rows};
  const int64_t tiles = moe::ceil_div(N, 256) * moe::ceil_div(K, 256);
  if (rows == 0 || tiles >= 256) return pl;
  // one round of work items on 256 CUs (case31: 4 chunks of 4096 rows, 0.403-0.406 -> 0.391-0.392 ms against 8
  // chunks in two rounds: one tile epilogue per CU and half the planes; 16 chunks: 0.446-0.450)
  int64_t s = std::min<int64_t>(moe::ceil_div(256, tiles), std::max<int64_t>(1, rows / 512));
  s = std::max<int64_t>(1, std::min<int64_t>(s, 64));
  if (s == 1) return pl;
  // Chunks are multiples of 64 rows (whole reduction steps).
  pl.c = moe::ceil_div(moe::ceil_div(rows, s), 64) * 64;
  pl.s = moe::ceil_div(rows, pl.c);
  return pl;
}

// Workspace of the tf32 wgrad (byte offsets, each 256-byte aligned): the fp16
// copies of grad_output [M, N] and inp [M, K], the scale exponents of their
// columns, the column-max slabs, and the fp32 planes of the reduction chunks
// (one plane at least: the scale is undone where the planes are added).
struct WgradTf32Layout {
  WgradPlan pl;
  moe::ColmaxPlan ca, cb;
  size_t a16, b16, row_exp, col_exp, part_a, part_b, planes, total;
};
WgradTf32Layout wgrad_tf32_layout(int64_t M, int64_t N, int64_t K) {
  using moe::align_up;
  WgradTf32Layout l;
  l.pl = wgrad_plan(M, N, K);
  l.ca = moe::colmax_plan(M, N);
  l.cb = moe::colmax_plan(M, K);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  l.a16 = take(static_cast<size_t>(M) * N * 2);
  l.b16 = take(static_cast<size_t>(M) * K * 2);
  l.row_exp = take(static_cast<size_t>(N) * 4);
  l.col_exp = take(static_cast<size_t>(K) * 4);
  l.part_a = take(static_cast<size_t>(l.ca.S) * N * 4);
  l.part_b = take(static_cast<size_t>(l.cb.S) * K * 4);
  l.planes = take(static_cast<size_t>(l.pl.s) * N * K * 4);
  l.total = off;
  return l;
}


}  // namespace

extern "C" {

size_t moe_router_wgrad_tf32_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0) return 0;
  return wgrad_tf32_layout(M, N, K).total;
}

int moe_router_wgrad_tf32(const float *grad_output, int64_t M, int64_t N, const float *inp, int64_t K,
                          float *grad_weight, void *workspace, size_t workspace_bytes, void *stream) {
  using namespace moe;
  const char *fn = "moe_router_wgrad_tf32";
  if (M < 0 || K < 0 || N < 0) {
    return fail(MOE_ERR_SHAPE, "%s: negative size (M=%lld N=%lld K=%lld)", fn, (long long)M, (long long)N, (long long)K);
  }
  if (K % 8 != 0 || N % 8 != 0) return fail(MOE_ERR_SHAPE, "%s: N=%lld and K=%lld must be multiples of 8", fn, (long long)N, (long long)K);
  if (M * N > (int64_t(1) << 30) - 1 || M * K > (int64_t(1) << 30) - 1 || N * K > (int64_t(1) << 30) - 1) {
    return fail(MOE_ERR_CAPACITY, "%s: M=%lld N=%lld K=%lld exceed the 32-bit offsets (M*N, M*K, N*K < 2^30)", fn,
                (long long)M, (long long)N, (long long)K);
  }
  if (N == 0 || K == 0) return MOE_OK;
  if (grad_weight == nullptr || (M > 0 && (grad_output == nullptr || inp == nullptr))) {
    return fail(MOE_ERR_INVALID_ARG, "%s: null grad_output, inp or grad_weight", fn);
  }
  if (!is_aligned(grad_output, 16) || !is_aligned(inp, 16) || !is_aligned(grad_weight, 16)) {
    return fail(MOE_ERR_ALIGN, "%s: grad_output, inp and grad_weight must be 16-byte aligned", fn);
  }
  const WgradTf32Layout l = wgrad_tf32_layout(M, N, K);
  if (workspace == nullptr || workspace_bytes < l.total || !is_aligned(workspace, kWsAlign)) {
    return fail(MOE_ERR_WORKSPACE, "%s: a 256-byte aligned workspace of %zu bytes is needed (got %zu)", fn, l.total,
                workspace == nullptr ? size_t(0) : workspace_bytes);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  char *w = static_cast<char *>(workspace);
  uint16_t *a16 = reinterpret_cast<uint16_t *>(w + l.a16);
  uint16_t *b16 = reinterpret_cast<uint16_t *>(w + l.b16);
  int32_t *row_exp = reinterpret_cast<int32_t *>(w + l.row_exp);
  int32_t *col_exp = reinterpret_cast<int32_t *>(w + l.col_exp);
  float *part_a = reinterpret_cast<float *>(w + l.part_a);
  float *part_b = reinterpret_cast<float *>(w + l.part_b);
  float *planes = reinterpret_cast<float *>(w + l.planes);
  // Scale exponents of grad_output's columns (dw rows) and inp's columns (dw columns), then the fp16 copies.
  colmax_partial_kernel<<<dim3(static_cast<uint32_t>(l.ca.xb), static_cast<uint32_t>(l.ca.S)), dim3(256), 0, s>>>(
      grad_output, M, N, l.ca.rps, l.ca.cg, part_a);
  colmax_partial_kernel<<<dim3(static_cast<uint32_t>(l.cb.xb), static_cast<uint32_t>(l.cb.S)), dim3(256), 0, s>>>(
      inp, M, K, l.cb.rps, l.cb.cg, part_b);
  colmax_final_kernel<<<dim3(static_cast<uint32_t>(ceil_div(N, 256))), dim3(256), 0, s>>>(part_a, static_cast<int>(l.ca.S), N,
                                                                                          row_exp, nullptr);
  colmax_final_kernel<<<dim3(static_cast<uint32_t>(ceil_div(K, 256))), dim3(256), 0, s>>>(part_b, static_cast<int>(l.cb.S), K,
                                                                                          col_exp, nullptr);
  if (M > 0) {
    const int64_t ga = std::max<int64_t>(1, std::min<int64_t>(ceil_div(M * N / 4, 256), 8192));
    const int64_t gb = std::max<int64_t>(1, std::min<int64_t>(ceil_div(M * K / 4, 256), 8192));
    tf32_to_f16_cols_kernel<<<dim3(static_cast<uint32_t>(ga)), dim3(256), 0, s>>>(grad_output, M, N, row_exp, a16);
    tf32_to_f16_cols_kernel<<<dim3(static_cast<uint32_t>(gb)), dim3(256), 0, s>>>(inp, M, K, col_exp, b16);
  }
  if (int rc = check_launch(fn)) return rc;
  // dw planes over the reduction chunks (fp16 MFMA, exact products, fp32 sums), then their sum scaled back.
  BwdArgs p;
  p.a = a16;
  p.b = b16;
  p.offsets = nullptr;
  p.out = planes;
  p.M = M;
  p.N = N;
  p.K = K;
  p.G = l.pl.s;
  p.ntiles = ceil_div(K, kBN);
  p.chunk = l.pl.c;
  p.kchunk = 0;
  p.order = nullptr;
  p.order_rows = nullptr;
  p.tails = nullptr;
  launch_pipe<true, 1, false, false, true>(p, ceil_div(N, 256) * p.ntiles * p.G, s);
  const int64_t q = N * K / 4;
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(ceil_div(q, 256), 4096));
  sum_planes_scaled_kernel<<<dim3(static_cast<uint32_t>(grid)), dim3(256), 0, s>>>(planes, static_cast<int>(l.pl.s), N, K,
                                                                                   row_exp, col_exp, grad_weight);
  return check_launch(fn);
}

}  // extern "C"
