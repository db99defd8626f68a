// Router gate GEMM (logits in fp32 from bf16 inputs), optionally followed by
// the router top-k, routing mask and merge probs.
//
// Math: kernel_cases/case38_ref_musa_asm_bf16_ssgemm_nt_320x256.py:46-53
// (reference_fp32): logits[M, N] = inp[M, K] @ weight[N, K]^T, bf16 in, fp32
// accumulate, fp32 out (moe_router_dtype=fp32, :8-13).  The top-k is the
// routine of topk_device.h (case23_ref_aten_topk.py:47-62; mask and probs as
// moe_topk) applied to each logits row.
//
// Kernel shape (gfx950): one workgroup of 4 wavefronts per 64-row tile
// holding all N (<= 512) columns; each wavefront computes 64 rows x 16 kNB
// columns as 4 x kNB blocks of v_mfma_f32_16x16x32_bf16 (the weight fragment
// is the first operand, so a lane holds 4 consecutive columns of one row).  A
// and weight tiles stream through a 3-stage LDS ring (2 stages when N > 320)
// filled by buffer_load ... lds two steps ahead; rows are 128 bytes with
// 16-byte chunks XOR-swizzled by (row / 2) % 8; the fp32 tile is staged in LDS
// (row stride 16 bytes past a multiple of 256) and stored as rows.  The top-k
// runs as a second pass over the logits rows, one wavefront per row, so it
// keeps the whole chip busy (run in the GEMM's epilogue it serialised 16 rows
// per wavefront and was slower than the GEMM plus the pass).
#include <algorithm>
#include <type_traits>

#include "gemm_device.h"
#include "topk_device.h"

namespace moe {
namespace {

using namespace gemm;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) float lds_f32;

constexpr int kBM = 64;
constexpr int kRow = kBK * 2;  // 128-byte LDS rows

struct RouterArgs {
  const uint16_t *inp;  // [M, K]
  const uint16_t *w;    // [N, K]
  float *out;           // [M, N] fp32 logits (the output, or workspace for the top-k pass)
  int64_t M, K;
  int N;
  int vec_out;          // rows of out are 16-byte aligned (N % 4 == 0, aligned base)
};

__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

template <int kNB>
__global__ __launch_bounds__(256) void router_gemm_kernel(RouterArgs p) {
  constexpr int kWaves = 4;
  constexpr int kNT = 64 * kNB;                 // weight rows (logits columns) per tile
  constexpr int kABytes = kBM * kRow;           // 8 KiB
  constexpr int kBBytes = kNT * kRow;
  constexpr int kStageBytes = kABytes + kBBytes;
  constexpr int kStages = 3 * kStageBytes <= 150 * 1024 ? 3 : 2;
  constexpr int kDmaA = kABytes / 1024 / kWaves;  // 2
  constexpr int kDmaB = kBBytes / 1024 / kWaves;  // 2 kNB
  constexpr int kDma = kDmaA + kDmaB;
  constexpr int kEpiStride = kNT * 4 + 16;      // fp32 logits row in LDS
  constexpr int kRingBytes = kStages * kStageBytes;
  constexpr int kLdsBytes = kRingBytes > kBM * kEpiStride ? kRingBytes : kBM * kEpiStride;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
  static_assert((kStages - 1) * kDma <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t K = p.K;
  const int N = p.N;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kBM;
  const int rows_valid = static_cast<int>(min(p.M - row0, int64_t(kBM)));
  const int ktiles = static_cast<int>(ceil_div(K, kBK));
  const bool ktail = (K % kBK) != 0;

  // DMA: 1 KiB blocks of 8 rows; lane -> (row, logical chunk) of its 16 bytes.
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(p.inp + row0 * K, static_cast<uint32_t>(rows_valid) * static_cast<uint32_t>(K) * 2u);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.w, static_cast<uint32_t>(N) * static_cast<uint32_t>(K) * 2u);
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;
  int a_off[kDmaA], b_off[kDmaB];
#pragma unroll
  for (int j = 0; j < kDmaA; ++j) {
    const int r = (j * kWaves + wave) * 8 + (lane >> 3);
    a_off[j] = static_cast<int>(static_cast<uint32_t>(min(r, rows_valid - 1)) * row_bytes + (((lane & 7) ^ swz(r)) << 4));
  }
#pragma unroll
  for (int j = 0; j < kDmaB; ++j) {
    const int r = (j * kWaves + wave) * 8 + (lane >> 3);
    b_off[j] = static_cast<int>(static_cast<uint32_t>(min(r, N - 1)) * row_bytes + (((lane & 7) ^ swz(r)) << 4));
  }
  auto issue = [&](int kt, int slot) {
    const uint32_t st = lds_base + (slot % kStages) * kStageBytes;
    const int soff = kt * kBK * 2;
#pragma unroll
    for (int j = 0; j < kDmaA; ++j)
      dma16b(ra, (lds_void *)(uintptr_t)(st + (j * kWaves + wave) * 1024), a_off[j], soff);
#pragma unroll
    for (int j = 0; j < kDmaB; ++j)
      dma16b(rb, (lds_void *)(uintptr_t)(st + kABytes + (j * kWaves + wave) * 1024), b_off[j], soff);
  };
  // Chunks past K in the last stage read the next row (or zeros): zero them.
  auto zero_ktail = [&](int kt) {
    lds_char *st = sbase + (kt % kStages) * kStageBytes;
    const int kvalid = static_cast<int>(K - static_cast<int64_t>(kt) * kBK);
    for (int idx = tid; idx < (kBM + kNT) * 8; idx += kWaves * 64) {
      const int r = idx >> 3, c = idx & 7;
      if (c * 8 >= kvalid) *reinterpret_cast<lds_u32x4 *>(st + r * kRow + ((c ^ swz(r)) << 4)) = u32x4{0u, 0u, 0u, 0u};
    }
  };

  // Fragments of v_mfma_f32_16x16x32_bf16: lane l reads row (block + l % 16),
  // the 8 values k = 8 (l / 16) .. + 7 of the sub-step (logical chunk 4 ks + l / 16).
  const int frow = lane & 15, fq = lane >> 4;
  auto frag_addr = [&](uint32_t slot_base, int r, int ks) {
    return slot_base + r * kRow + ((((ks << 2) | fq) ^ swz(r)) << 4);
  };

  f32x4 acc[4][kNB];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: stages 0 .. kStages - 2 (re-reads past the last stage keep the
  // count of outstanding loads fixed).
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue(min(s, ktiles - 1), s);

  for (int kt = 0; kt < ktiles; ++kt) {
    // Stage kt has landed (younger: kStages - 2 stages); after the barrier,
    // every wave's, and every wave is done with stage kt - 1's slot.
    wait_vm_n<(kStages - 2) * kDma>();
    wait_lds();
    barrier();
    if (ktail && kt == ktiles - 1) {
      zero_ktail(kt);
      wait_lds();
      barrier();
    }
    issue(min(kt + kStages - 1, ktiles - 1), kt + kStages - 1);
    const uint32_t sb = lds_base + (kt % kStages) * kStageBytes;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 fa[4], fb[kNB];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[i] = *reinterpret_cast<const lds_bf16x8 *>((uintptr_t)frag_addr(sb, i * 16 + frow, ks));
#pragma unroll
      for (int j = 0; j < kNB; ++j)
        fb[j] = *reinterpret_cast<const lds_bf16x8 *>(
            (uintptr_t)frag_addr(sb + kABytes, wave * 16 * kNB + j * 16 + frow, ks));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kNB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
  }
  wait_dma();  // the re-reads of the last steps
  wait_lds();
  barrier();

  // Epilogue. acc[i][j] register r of lane l: row i * 16 + l % 16, column
  // wave * 16 kNB + j * 16 + 4 (l / 16) + r; staged in LDS, stored as rows.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = i * 16 + frow;
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
      const int c = wave * 16 * kNB + j * 16 + fq * 4;
      *reinterpret_cast<lds_f32x4 *>(sbase + r * kEpiStride + c * 4) = acc[i][j];
    }
  }
  wait_lds();
  barrier();
  float *out = p.out + row0 * N;
  if (p.vec_out) {
    const int cpr = N / 4;  // 16-byte chunks per row
    for (int idx = tid; idx < rows_valid * cpr; idx += kWaves * 64) {
      const int r = idx / cpr, c = idx - r * cpr;
      *reinterpret_cast<f32x4 *>(out + static_cast<int64_t>(r) * N + c * 4) =
          *reinterpret_cast<const lds_f32x4 *>(sbase + r * kEpiStride + c * 16);
    }
  } else {
    for (int idx = tid; idx < rows_valid * N; idx += kWaves * 64) {
      const int r = idx / N, c = idx - r * N;
      out[static_cast<int64_t>(r) * N + c] = *reinterpret_cast<const lds_f32 *>(sbase + r * kEpiStride + c * 4);
    }
  }
}

// Router GEMM for 128 < N <= 512 with K % 64 == 0 (case38: N = 320): one
// workgroup per 128-row x 32 kNB-column tile (kNB = ceil(N / 64), so two
// column tiles cover N: each CU streams half the weight, where the 64-row
// tiles above stream all of it for half the rows). Consecutive tiles are the
// two column halves of one row tile, and an XCD takes a contiguous run of
// tiles, so the input rows are fetched once into that XCD's L2 for both
// halves. 8 wavefronts, on each SIMD one computing and one loading: the
// computing wavefront of SIMD w computes rows (w / 2) 64 .. + 63, columns
// (w % 2) 16 kNB .. as 4 x kNB blocks of v_mfma_f32_16x16x32_bf16 (the same
// MFMA sequence over K as the 64-row kernel, so the logits are bit-identical),
// with the fragments of the two 32-deep halves of a step double-buffered in
// registers (each half's reads go out under the other half's MFMAs). Two
// loading wavefronts DMA the input rows into a ring of kSA stages, two the
// weight rows into a ring of kSB stages. A wavefront's loads complete in issue
// order, so with the loads split by operand each ring runs its own lookahead:
// the input (HBM) kSA - 1 steps ahead, the weight (Infinity Cache / L2)
// kSB - 1, the LDS split between the rings (one ring holding both operands
// at one depth, loaded by the computing wavefronts, ran case38 in 125 us
// against 97). One workgroup barrier per step: the loaders have waited for
// stage kt + 1, the computing wavefronts have read all of stage kt. fp32
// results are stored from the accumulators (a lane holds 4 consecutive
// columns of one row).
template <int kNB>
__global__ __launch_bounds__(512) void router_ws_kernel(RouterArgs p, int tiles) {
  constexpr int kTM = 128;
  constexpr int kTN = 32 * kNB;
  constexpr int kABytes = kTM * kRow;            // 16 KiB
  constexpr int kBBytes = kTN * kRow;
  constexpr int kSA = kNB <= 5 ? 5 : 4;
  constexpr int kSBFit = (160 * 1024 - kSA * kABytes) / kBBytes;
  constexpr int kSB = kSBFit > 4 ? 4 : kSBFit;
  constexpr int kDmaA = kABytes / 1024 / 2, kDmaB = kBBytes / 1024 / 2;  // per loading wavefront
  constexpr int kReads = 4 + kNB;
  static_assert(kSB >= 3 && kSA * kABytes + kSB * kBBytes <= 160 * 1024, "LDS budget");
  static_assert((kSA - 1) * kDmaA <= 63 && (kSB - 1) * kDmaB <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[kSA * kABytes + kSB * kBBytes];
  lds_char *const sbase = (lds_char *)smem;
  const uint32_t a_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sbase));
  const uint32_t b_lds = a_lds + kSA * kABytes;

  const int64_t P = gridDim.x, b = blockIdx.x;
  const int tile = static_cast<int>((b % 8) * (P / 8) + b / 8);
  if (tile >= tiles) return;
  const int rt = tile >> 1, ct = tile & 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  // ---- roles: the first wavefront of each SIMD computes (index = its SIMD), the second loads
  // (SIMD 0 and 1: input rows, 2 and 3: weight rows), read from HW_ID and exchanged through LDS.
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
  const int64_t K = p.K;
  const int N = p.N;
  const int64_t row0 = static_cast<int64_t>(rt) * kTM;
  const int col0 = ct * kTN;
  const int rows_valid = static_cast<int>(min(p.M - row0, int64_t(kTM)));
  const int cols_valid = min(N - col0, kTN);
  const int ktiles = static_cast<int>(K / kBK);
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;

  if (loader) {
    // Rows past the tile's valid rows / columns lie past the resources: zeros.
    const bool is_a = role_simd < 2;
    const int li = role_simd & 1;
    const __amdgpu_buffer_rsrc_t rsrc =
        is_a ? make_rsrc(p.inp + row0 * K, static_cast<uint32_t>(rows_valid) * row_bytes)
             : make_rsrc(p.w + static_cast<int64_t>(col0) * K, static_cast<uint32_t>(cols_valid) * row_bytes);
    const int ndma = is_a ? kDmaA : kDmaB;
    const int blk0 = li * ndma;  // this wavefront's 1 KiB blocks (8 rows each) of a stage: blk0 ..
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int r0 = blk0 * 8 + (ln >> 3);  // row of block blk0 + j: r0 + 8 j
    auto issue = [&](auto is_a_c, int kt, int slot) {
      constexpr bool kA = decltype(is_a_c)::value;
      constexpr int n = kA ? kDmaA : kDmaB;
      const uint32_t st = (kA ? a_lds + slot * kABytes : b_lds + slot * kBBytes) + blk0 * 1024;
      const int soff = kt * kBK * 2;
#pragma unroll
      for (int j = 0; j < n; ++j) {
        const int r = r0 + j * 8;
        const int off = static_cast<int>(static_cast<uint32_t>(r) * row_bytes + (((ln & 7) ^ swz(r)) << 4));
        dma16b(rsrc, (lds_void *)(uintptr_t)(st + j * 1024), off, soff);
      }
    };
    // Stages past the last re-read it (the count of outstanding loads stays the same in every step);
    // they land in slots nothing reads any more.
    if (is_a) {
      for (int st = 0; st < kSA - 1; ++st) issue(std::true_type{}, min(st, ktiles - 1), st);
      wait_vm_n<(kSA - 2) * kDmaA>();
      barrier();
      int slot = kSA - 1;  // slot of stage kt + kSA - 1 = slot of stage kt - 1
      for (int kt = 0; kt < ktiles; ++kt) {
        issue(std::true_type{}, min(kt + kSA - 1, ktiles - 1), slot);
        slot = slot + 1 == kSA ? 0 : slot + 1;
        wait_vm_n<(kSA - 2) * kDmaA>();  // stage kt + 1 has landed
        barrier();
      }
    } else {
      for (int st = 0; st < kSB - 1; ++st) issue(std::false_type{}, min(st, ktiles - 1), st);
      wait_vm_n<(kSB - 2) * kDmaB>();
      barrier();
      int slot = kSB - 1;
      for (int kt = 0; kt < ktiles; ++kt) {
        issue(std::false_type{}, min(kt + kSB - 1, ktiles - 1), slot);
        slot = slot + 1 == kSB ? 0 : slot + 1;
        wait_vm_n<(kSB - 2) * kDmaB>();
        barrier();
      }
    }
    (void)ndma;
    wait_dma();  // the re-reads of the last steps
    return;
  }

  const int wr = role_simd >> 1, wc = role_simd & 1;
  const int frow = lane & 15, fq = lane >> 4;
  auto frag_addr = [&](uint32_t slot_base, int r, int ks) {
    return slot_base + r * kRow + ((((ks << 2) | fq) ^ swz(r)) << 4);
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
  f32x4 acc[4][kNB];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < kNB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mfma_half = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[buf][j], fa[buf][i], acc[i][j], 0, 0, 0);
  };
  barrier();  // stage 0 has landed
  read_half(0, 0);
  for (int kt = 0; kt < ktiles; ++kt) {
    read_half(1, 1);
    mfma_half(0);
    sched_mix<4 * kNB, kReads, 0>();
    __builtin_amdgcn_sched_barrier(0);
    wait_lds();  // this wavefront's reads of stage kt are done before the slot can be refilled
    barrier();   // stage kt + 1 has landed
    sa = sa + 1 == kSA ? 0 : sa + 1;
    sb = sb + 1 == kSB ? 0 : sb + 1;
    if (kt + 1 < ktiles) read_half(0, 0);
    mfma_half(1);
    sched_mix<4 * kNB, kReads, 0>();
    __builtin_amdgcn_sched_barrier(0);
  }

  // acc[i][j] register r of lane l: row wr 64 + i 16 + l % 16, column wc 16 kNB + j 16 + 4 (l / 16) + r.
  float *out = p.out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = wr * 64 + i * 16 + frow;
    if (r >= rows_valid) continue;
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
      const int c = wc * 16 * kNB + j * 16 + fq * 4;
      if (c < cols_valid) *reinterpret_cast<f32x4 *>(out + (row0 + r) * N + col0 + c) = acc[i][j];
    }
  }
}

// Top-k pass, one wavefront per row of the logits (topk_device.h).
struct TopkArgs {
  const float *logits;
  int64_t M;
  int N, k;
  float *values;
  int64_t *indices;
  uint8_t *routing_map;
  float *probs;
};

template <int kEPL>
__global__ __launch_bounds__(256) void router_topk_kernel(TopkArgs p) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  if (t >= p.M) return;
  const float *row = p.logits + t * p.N;
  topk_row<kEPL>([&](int e) { return row[e]; }, t, p.N, p.k, p.values, p.indices, p.routing_map, p.probs);
}

int launch(const char *fn, const moe_bf16_t *inp, int64_t M, int64_t K, const moe_bf16_t *weight, int64_t N,
           int64_t k, float *logits, float *values, int64_t *indices, uint8_t *routing_map, float *probs,
           bool topk, void *workspace, size_t workspace_bytes, void *stream) {
  if (M < 0 || K < 0 || N < 0) {
    return fail(MOE_ERR_SHAPE, "%s: negative size (M=%lld K=%lld N=%lld)", fn, (long long)M, (long long)K,
                (long long)N);
  }
  if (N < 1 || N > 512) return fail(MOE_ERR_CAPACITY, "%s: N=%lld outside [1, 512]", fn, (long long)N);
  if (K % 8 != 0 || K == 0) return fail(MOE_ERR_SHAPE, "%s: K=%lld must be a positive multiple of 8", fn, (long long)K);
  if (K > (int64_t(1) << 22) - 8 || N * K > (int64_t(1) << 30) - 1) {
    return fail(MOE_ERR_CAPACITY, "%s: K=%lld N=%lld exceed the 32-bit offsets (K < 2^22, N*K < 2^30)", fn,
                (long long)K, (long long)N);
  }
  if (topk) {
    if (k < 1 || k > N) return fail(MOE_ERR_SHAPE, "%s: k=%lld out of range for N=%lld", fn, (long long)k, (long long)N);
    if (k > 64) return fail(MOE_ERR_CAPACITY, "%s: k=%lld exceeds the 64 supported", fn, (long long)k);
  }
  if (M == 0) return MOE_OK;
  if (inp == nullptr || weight == nullptr) return fail(MOE_ERR_INVALID_ARG, "%s: null inp or weight", fn);
  if (!topk && logits == nullptr) return fail(MOE_ERR_INVALID_ARG, "%s: null logits", fn);
  if (topk && (values == nullptr || indices == nullptr)) return fail(MOE_ERR_INVALID_ARG, "%s: null values or indices", fn);
  if (!is_aligned(inp, 16) || !is_aligned(weight, 16)) return fail(MOE_ERR_ALIGN, "%s: inp and weight must be 16-byte aligned", fn);
  if (ceil_div(M, kBM) > 0x7fffffff) return fail(MOE_ERR_CAPACITY, "%s: M=%lld too large", fn, (long long)M);
  // Without a logits output the top-k pass reads them from the workspace.
  const size_t plane = static_cast<size_t>(M) * static_cast<size_t>(N) * sizeof(float);
  const size_t need = logits == nullptr ? plane : 0;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    return fail(MOE_ERR_WORKSPACE, "%s: workspace of %zu bytes needed (got %zu)", fn, need,
                workspace == nullptr ? size_t(0) : workspace_bytes);
  }
  if (need > 0 && !is_aligned(workspace, 16)) return fail(MOE_ERR_ALIGN, "%s: workspace must be 16-byte aligned", fn);
  RouterArgs p;
  p.inp = inp;
  p.w = weight;
  p.out = logits != nullptr ? logits : static_cast<float *>(workspace);
  p.M = M;
  p.K = K;
  p.N = static_cast<int>(N);
  p.vec_out = (N % 4 == 0) && is_aligned(p.out, 16);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t grid = ceil_div(M, kBM);
  const int nb = static_cast<int>(ceil_div(N, 64));
  // 128 < N with whole 64-column steps and 16-byte output rows: 128-row tiles over half of N each.
  const bool tiled = N > 128 && K % kBK == 0 && p.vec_out && ceil_div(M, 128) * 2 <= 0x7fffffff;
  if (tiled) {
    const int row_tiles = static_cast<int>(ceil_div(M, 128));
    const int tiles = row_tiles * 2;
    const dim3 g(static_cast<uint32_t>((tiles + 7) / 8 * 8));
    switch (nb) {
      case 3: router_ws_kernel<3><<<g, dim3(512), 0, s>>>(p, tiles); break;
      case 4: router_ws_kernel<4><<<g, dim3(512), 0, s>>>(p, tiles); break;
      case 5: router_ws_kernel<5><<<g, dim3(512), 0, s>>>(p, tiles); break;
      case 6: router_ws_kernel<6><<<g, dim3(512), 0, s>>>(p, tiles); break;
      case 7: router_ws_kernel<7><<<g, dim3(512), 0, s>>>(p, tiles); break;
      default: router_ws_kernel<8><<<g, dim3(512), 0, s>>>(p, tiles); break;
    }
  } else switch (nb) {
    case 1: router_gemm_kernel<1><<<dim3(grid), dim3(256), 0, s>>>(p); break;
    case 2: router_gemm_kernel<2><<<dim3(grid), dim3(256), 0, s>>>(p); break;
    case 3: router_gemm_kernel<3><<<dim3(grid), dim3(256), 0, s>>>(p); break;
    case 4: router_gemm_kernel<4><<<dim3(grid), dim3(256), 0, s>>>(p); break;
    case 5: router_gemm_kernel<5><<<dim3(grid), dim3(256), 0, s>>>(p); break;
    case 6: router_gemm_kernel<6><<<dim3(grid), dim3(256), 0, s>>>(p); break;
    case 7: router_gemm_kernel<7><<<dim3(grid), dim3(256), 0, s>>>(p); break;
    default: router_gemm_kernel<8><<<dim3(grid), dim3(256), 0, s>>>(p); break;
  }
  if (int rc = check_launch(fn)) return rc;
  if (!topk) return MOE_OK;
  TopkArgs t;
  t.logits = p.out;
  t.M = M;
  t.N = p.N;
  t.k = static_cast<int>(k);
  t.values = values;
  t.indices = indices;
  t.routing_map = routing_map;
  t.probs = probs;
  const int64_t tgrid = ceil_div(M, 4);
  switch (nb) {
    case 1: router_topk_kernel<1><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
    case 2: router_topk_kernel<2><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
    case 3: router_topk_kernel<3><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
    case 4: router_topk_kernel<4><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
    case 5: router_topk_kernel<5><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
    case 6: router_topk_kernel<6><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
    case 7: router_topk_kernel<7><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
    default: router_topk_kernel<8><<<dim3(tgrid), dim3(256), 0, s>>>(t); break;
  }
  return check_launch(fn);
}

}  // namespace
}  // namespace moe

extern "C" {

size_t moe_router_workspace_size(int64_t M, int64_t K, int64_t N) {
  (void)K;
  if (M <= 0 || N <= 0) return 0;
  return static_cast<size_t>(M) * static_cast<size_t>(N) * sizeof(float);
}

int moe_router_logits(const moe_bf16_t *inp, int64_t M, int64_t K, const moe_bf16_t *weight, int64_t N,
                      float *logits, void *workspace, size_t workspace_bytes, void *stream) {
  return moe::launch("moe_router_logits", inp, M, K, weight, N, 0, logits, nullptr, nullptr, nullptr, nullptr,
                     false, workspace, workspace_bytes, stream);
}

int moe_router_topk(const moe_bf16_t *inp, int64_t M, int64_t K, const moe_bf16_t *weight, int64_t N, int64_t k,
                    float *logits, float *values, int64_t *indices, uint8_t *routing_map, float *probs,
                    void *workspace, size_t workspace_bytes, void *stream) {
  return moe::launch("moe_router_topk", inp, M, K, weight, N, k, logits, values, indices, routing_map, probs, true,
                     workspace, workspace_bytes, stream);
}

}  // extern "C"
