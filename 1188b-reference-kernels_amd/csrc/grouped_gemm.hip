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
//   * one persistent workgroup per CU, 512 threads = 8 wavefronts;
//   * output tile 256 x 256, K step 64, A and B tiles double-buffered in LDS
//     (2 stages x 2 operands x 256 rows x 144 bytes = 144 KiB of the 160 KiB);
//     the 16-byte row padding makes the MFMA operand reads conflict-free;
//   * waves form a 2 (M) x 4 (N) grid, each owns 128 x 64 of the tile as
//     4 x 2 blocks of v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators/lane);
//   * SwiGLU tiles load 128 gate rows and the matching 128 up rows of w, and
//     each wave's two N blocks are the gate and up halves of the same 32
//     output columns, so the epilogue combines them in registers;
//   * tiles are numbered expert by expert, and inside an expert in groups of
//     4 row tiles x all column tiles (row tile fastest), so 32 consecutive
//     tile numbers form a 4 x 8 patch that shares A and B panels; workgroup b
//     takes tile round * P + (b % 8) * (P / 8) + b / 8, which hands each XCD
//     (workgroups are dealt round-robin to the 8 XCDs) one such patch per
//     round, so the panels are reused from that XCD's L2.
#include <algorithm>

#include "moe_common.h"

namespace moe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 512;
constexpr int kLdsRow = kBK + 8;  // bf16 per LDS row (144 bytes)
constexpr int kMI = 4, kNI = 2;   // 32x32 blocks per wave (M, N)
constexpr int kGroupM = 4;        // row tiles per tile-order group
constexpr int kVecPerThread = (kBM * kBK / 8) / kThreads;  // 16-byte vectors per operand per thread (4)

struct GemmArgs {
  const uint16_t *a;
  const uint16_t *w;
  const int32_t *offsets;
  uint16_t *out;
  int64_t M, K, N, G;
  int64_t ncols;   // output columns: N (NONE) or N / 2 (SWIGLU)
  int64_t ntiles;  // column tiles per expert
};

// Row of w[g] (in [0, N)) that B-tile row r of column tile nt reads.
template <bool kSwiglu>
__device__ __forceinline__ int64_t b_row(int64_t nt, int r, int64_t ncols) {
  if constexpr (kSwiglu) {
    // rows 0..127: gate columns j0 .. j0+127; rows 128..255: up columns F + j0 ..
    const int64_t j = nt * (kBN / 2) + (r & 127);
    return r < 128 ? j : ncols + j;
  } else {
    return nt * kBN + r;
  }
}

template <bool kSwiglu>
__device__ __forceinline__ bool b_row_ok(int64_t nt, int r, int64_t ncols, int64_t N) {
  if constexpr (kSwiglu) {
    return nt * (kBN / 2) + (r & 127) < ncols;
  } else {
    return nt * kBN + r < N;
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <bool kSwiglu>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][kBN * kLdsRow];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2;  // 0..1
  const int wn = wave & 3;   // 0..3
  const int64_t P = gridDim.x;
  const int64_t b = blockIdx.x;
  const int64_t ktiles = ceil_div(p.K, kBK);

  // Group cursor: tiles before group g_cur, and group g_cur's row range.
  int64_t g_cur = 0, tiles_before = 0;
  // Row ranges are clamped to [0, M] and made non-decreasing, so inconsistent
  // offsets can never send a load or store outside a and out.
  auto group_rows = [&](int64_t g, int64_t &lo, int64_t &hi) {
    lo = min(max(static_cast<int64_t>(p.offsets[g]), int64_t(0)), p.M);
    hi = min(max(static_cast<int64_t>(p.offsets[g + 1]), lo), p.M);
  };
  int64_t m_lo, m_hi;
  group_rows(0, m_lo, m_hi);
  int64_t mt_g = ceil_div(m_hi - m_lo, kBM);

  for (int64_t round = 0;; ++round) {
    const int64_t L = round * P + (b % 8) * (P / 8) + b / 8;
    // Advance the cursor to the group holding logical tile L.
    while (g_cur < p.G && L >= tiles_before + mt_g * p.ntiles) {
      tiles_before += mt_g * p.ntiles;
      ++g_cur;
      if (g_cur < p.G) {
        group_rows(g_cur, m_lo, m_hi);
        mt_g = ceil_div(m_hi - m_lo, kBM);
      }
    }
    if (g_cur >= p.G) break;

    // Tile (row tile mt, column tile nt) inside group g_cur.
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
    const int64_t row0 = m_lo + mt * kBM;  // first A row of the tile
    const uint16_t *wg = p.w + g_cur * p.N * p.K;

    // Global -> register staging for one K step.
    u32x4 ra[kVecPerThread], rb[kVecPerThread];
    auto load_tile = [&](int64_t kt) {
      const int64_t k0 = kt * kBK;
#pragma unroll
      for (int i = 0; i < kVecPerThread; ++i) {
        const int v = tid + i * kThreads;
        const int r = v >> 3, c = v & 7;
        const int64_t kk = k0 + c * 8;
        const int64_t arow = row0 + r;
        ra[i] = u32x4{0u, 0u, 0u, 0u};
        rb[i] = u32x4{0u, 0u, 0u, 0u};
        if (arow < m_hi && kk < p.K) ra[i] = *reinterpret_cast<const u32x4 *>(p.a + arow * p.K + kk);
        if (b_row_ok<kSwiglu>(nt, r, p.ncols, p.N) && kk < p.K)
          rb[i] = *reinterpret_cast<const u32x4 *>(wg + b_row<kSwiglu>(nt, r, p.ncols) * p.K + kk);
      }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
      for (int i = 0; i < kVecPerThread; ++i) {
        const int v = tid + i * kThreads;
        const int r = v >> 3, c = v & 7;
        *reinterpret_cast<u32x4 *>(&lds_a[buf][r * kLdsRow + c * 8]) = ra[i];
        *reinterpret_cast<u32x4 *>(&lds_b[buf][r * kLdsRow + c * 8]) = rb[i];
      }
    };

    f32x16 acc[kMI][kNI];
#pragma unroll
    for (int i = 0; i < kMI; ++i)
#pragma unroll
      for (int j = 0; j < kNI; ++j) acc[i][j] = f32x16{};

    // B-tile row of this wave's N block j.
    int bro[kNI];
#pragma unroll
    for (int j = 0; j < kNI; ++j) bro[j] = kSwiglu ? j * 128 + wn * 32 : wn * 64 + j * 32;

    __syncthreads();  // previous tile's readers are done with both buffers
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int64_t kt = 0; kt < ktiles; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < ktiles) load_tile(kt + 1);
#pragma unroll
      for (int ks = 0; ks < kBK / 16; ++ks) {
        const int kcol = ks * 16 + (lane >> 5) * 8;
        bf16x8 fa[kMI], fb[kNI];
#pragma unroll
        for (int i = 0; i < kMI; ++i)
          fa[i] = *reinterpret_cast<const bf16x8 *>(&lds_a[cur][(wm * 128 + i * 32 + (lane & 31)) * kLdsRow + kcol]);
#pragma unroll
        for (int j = 0; j < kNI; ++j)
          fb[j] = *reinterpret_cast<const bf16x8 *>(&lds_b[cur][(bro[j] + (lane & 31)) * kLdsRow + kcol]);
#pragma unroll
        for (int i = 0; i < kMI; ++i)
#pragma unroll
          for (int j = 0; j < kNI; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
      if (kt + 1 < ktiles) store_tile(cur ^ 1);
      __syncthreads();
    }

    // Epilogue.  Accumulator register r of lane l in a 32x32 block holds
    // row (r / 4) * 8 + (l / 32) * 4 + (r % 4), column l % 32.
#pragma unroll
    for (int i = 0; i < kMI; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + wm * 128 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (row >= m_hi) continue;
        if constexpr (kSwiglu) {
          const int64_t col = nt * (kBN / 2) + wn * 32 + (lane & 31);
          if (col < p.ncols) {
            const float h = silu(acc[i][0][r]) * acc[i][1][r];
            p.out[row * p.ncols + col] = static_cast<uint16_t>(f32_to_bf16_rne(h));
          }
        } else {
#pragma unroll
          for (int j = 0; j < kNI; ++j) {
            const int64_t col = nt * kBN + wn * 64 + j * 32 + (lane & 31);
            if (col < p.N) p.out[row * p.N + col] = static_cast<uint16_t>(f32_to_bf16_rne(acc[i][j][r]));
          }
        }
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
  if (K % 8 != 0) return fail(MOE_ERR_SHAPE, "moe_grouped_gemm: K=%lld must be a multiple of 8", (long long)K);
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
  // Persistent grid: one workgroup per CU, a multiple of the 8 XCDs, no more
  // than an upper bound on the tile count.
  const int64_t max_tiles = (ceil_div(M_total, kBM) + G) * p.ntiles;
  int64_t grid = std::min<int64_t>(num_cus(), max_tiles);
  grid = std::max<int64_t>(8, (grid + 7) / 8 * 8);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (swiglu) grouped_gemm_kernel<true><<<dim3(grid), dim3(kThreads), 0, s>>>(p);
  else grouped_gemm_kernel<false><<<dim3(grid), dim3(kThreads), 0, s>>>(p);
  return check_launch("moe_grouped_gemm");
}

}  // extern "C"
