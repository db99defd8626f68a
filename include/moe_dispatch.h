/*
 * moe_dispatch.h -- C ABI of the MI355X (gfx950) MoE expert-dispatch library
 * (libmoe_dispatch.so).
 *
 * Every entry point:
 *   - takes device pointers, int64_t sizes and enum selectors, plus a
 *     hipStream_t passed as `void *stream` (NULL = the null stream);
 *   - validates its arguments on the host before any HIP call and returns a
 *     non-zero moe_status_t on failure (the message is available from
 *     moe_last_error(), thread-local);
 *   - never allocates device memory and never synchronises the host: scratch
 *     memory comes from the caller through (workspace, workspace_bytes), sized
 *     by the matching *_workspace_size() query;
 *   - enqueues its kernels on `stream` and returns MOE_ERR_LAUNCH if the launch
 *     itself fails.
 *
 * Device-side index safety: a map entry or index that points outside the
 * destination/source buffer is skipped (never dereferenced); kernels do not
 * fault on bad indices.  Callers that need the reference's IndexError /
 * ValueError on such inputs validate them first (the Python layer does).
 *
 * Types: bf16 tensors are raw bit patterns (moe_bf16_t); routing masks are one
 * byte per element (torch.bool / uint8, non-zero = selected); fp32 is float.
 * All tensors are dense row-major (C-contiguous).
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   case12 kernel_results/case12_moe_row_id_map_pass2/binding.cpp:11-34
 *   case17 kernel_results/case17_moe_permute_with_mask_map/binding.cpp:8-32
 *   case15 kernel_results/case15_moe_unpermute_mask_fwd/binding.cpp:10-20
 *   case23 kernel_results/case23_aten_topk/binding.cpp:6-24
 *   case06 kernel_results/case06_cp_seq_chunk_index_select/binding.cpp:13-49
 *   case18 kernel_cases/case18_moe_permute_bwd_unpermute_mask.py:68-78 (no bundle)
 *   case03/case04 kernel_cases/case03_moe_grouped_gemm_fc1_fwd.py:57-64,
 *                 kernel_cases/case04_moe_grouped_gemm_fc2_fwd.py:57-64 (no bundle)
 *   case07/08/13/19 (and case37) kernel_cases/case07_moe_grouped_gemm_fc1_dgrad.py:57-64
 *                 (dgrad, no bundle)
 *   case05/case09 kernel_cases/case09_moe_grouped_gemm_fc1_wgrad.py:57-64 (wgrad, no bundle)
 *   case38        kernel_cases/case38_ref_musa_asm_bf16_ssgemm_nt_320x256.py:46-53 (router logits)
 *   case39/case31 kernel_cases/case39_ref_musa_asm_tf32_ssgemm_nn_384x256.py:61-68,
 *                 kernel_cases/case31_ref_musa_asm_tf32_ssgemm_tn_128x256.py:61-68 (tf32 router GEMMs)
 *   case11/case25 kernel_cases/case11_router_bwd_cast_bf16_to_fp32.py:43-44,
 *                 kernel_cases/case25_ref_unary_cast_fp32_to_bf16.py:56-72 (casts)
 */
#ifndef MOE_DISPATCH_H_
#define MOE_DISPATCH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_DISPATCH_ABI_VERSION 13

typedef uint16_t moe_bf16_t;

typedef enum {
  MOE_OK = 0,
  MOE_ERR_INVALID_ARG = 1, /* null pointer where one is required, bad enum  */
  MOE_ERR_SHAPE = 2,       /* negative or inconsistent sizes                */
  MOE_ERR_ALIGN = 3,       /* pointer alignment the kernel requires         */
  MOE_ERR_CAPACITY = 4,    /* size beyond what this build supports (e.g. k) */
  MOE_ERR_WORKSPACE = 5,   /* workspace missing or too small                */
  MOE_ERR_LAUNCH = 6,      /* hipGetLastError() after the launch            */
} moe_status_t;

/* Index dtype of a row-id map or index vector. */
typedef enum { MOE_IDX_I32 = 0, MOE_IDX_I64 = 1 } moe_idx_dtype_t;

/* Layout of a row-id map.
 *   MOE_MAP_TOKEN_MAJOR  : map[t * E + e]  ([T, E], "non-trans", case12/case17)
 *   MOE_MAP_EXPERT_MAJOR : map[e * T + t]  ([E, T], "trans", case15/18/21/22/24/30/32) */
typedef enum { MOE_MAP_TOKEN_MAJOR = 0, MOE_MAP_EXPERT_MAJOR = 1 } moe_map_layout_t;

/* Epilogue of the grouped GEMM. */
typedef enum {
  MOE_EPILOGUE_NONE = 0,   /* out[m, n] = bf16(acc[m, n]), out is [M, N]                     */
  MOE_EPILOGUE_SWIGLU = 1, /* out[m, j] = bf16(silu(acc[m, j]) * acc[m, F + j]), F = N / 2    */
} moe_epilogue_t;

/* ---- library ---------------------------------------------------------- */
int moe_abi_version(void);
const char *moe_status_string(int status);
/* Message of the last non-zero status returned on the calling thread. */
const char *moe_last_error(void);

/* ---- a1/a2: router top-k + mask map + merge probs ----------------------
 * Replaces case23 kernel_function(input, k, dim=1, largest=True, sorted=True)
 * (kernel_results/case23_aten_topk/kernel.py:14-25, binding.cpp:6-24), whose
 * contract is torch.topk == first k of a stable descending sort
 * (kernel_cases/case23_ref_aten_topk.py:47-62).
 *   logits  fp32 [T, E]
 *   values  fp32 [T, k]   descending; ties -> smaller index first; NaN largest
 *   indices int64 [T, k]
 *   routing_map (nullable) uint8 [T, E]: 1 at the k selected experts, else 0
 *               (zeros(T,E,bool).scatter_(1, idx, True), case18...py:86-88)
 *   probs (nullable) fp32 [T, E]: softmax over the k selected values, scattered
 *               to the selected experts, 0 elsewhere (merge probs; no reference
 *               function -- closed form torch.softmax(values, -1)).
 * Limits: 1 <= k <= min(E, 64), E <= 1024. */
int moe_topk(const float *logits, int64_t T, int64_t E, int64_t k, float *values,
             int64_t *indices, uint8_t *routing_map, float *probs, void *stream);

/* ---- a3: row-id map ---------------------------------------------------
 * Replaces case12 kernel_function(routing_map) -> (row_id_map [E,T] int64,
 * row_id_map_non_trans [T,E] int64)
 * (kernel_results/case12_moe_row_id_map_pass2/kernel.py:4-6, binding.cpp:11-34;
 *  math kernel_cases/case12_moe_row_id_map_pass2.py:43-61):
 *   row[t, e] = offset[e] + #{t' < t : mask[t', e]}  if mask[t, e] else -1,
 *   offset[e] = sum_{e' < e} count[e'].
 * Every output is optional (nullable):
 *   row_expert_major     int64 [E, T]
 *   row_token_major      int64 [T, E]
 *   row_expert_major_i32 int32 [E, T]   (deep_ep dtype, case24...py:71-84)
 *   expert_offsets       int32 [E + 1]  offset[e]; [E] = R = total routed rows
 *   src_token            int32 [src_capacity]: the source token of every
 *                        permuted row, src_token[row[t, e]] = t for row < src_capacity
 *                        (the inverse map; no reference function -- the token
 *                        case17's permute copies into that row).  With
 *                        src_capacity >= R every row 0..R-1 is written (the map
 *                        is a bijection onto them); rows >= R are left as they are.
 * Two kernel launches (a column scan of the mask, then the fill).
 * Workspace: moe_row_id_map_workspace_size(T, E) bytes.  E <= 4096. */
size_t moe_row_id_map_workspace_size(int64_t T, int64_t E);
int moe_row_id_map(const uint8_t *routing_map, int64_t T, int64_t E, int64_t *row_expert_major,
                   int64_t *row_token_major, int32_t *row_expert_major_i32,
                   int32_t *expert_offsets, int32_t *src_token, int64_t src_capacity,
                   void *workspace, size_t workspace_bytes, void *stream);

/* ---- a3': row-id map without a workspace (allocates nothing) -------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): moe_row_id_map with the same arguments and results, whose
 * scratch (the per-super-chunk counts, at most 64 (E + ceil(E/32)) int32
 * values) lives in a 2 MiB device array the library holds per GPU until the
 * process ends.
 * Limits: as moe_row_id_map (E <= 4096, T*E < 2^31), within which the 2 MiB
 *   always suffice; a larger need would fail with MOE_ERR_CAPACITY.
 * Every call on a GPU shares that GPU's scratch: calls that overlap on one GPU
 * (on different streams or host threads) race; calls ordered on one stream do
 * not.  Nothing in the scratch needs to start at zero. */
int moe_row_id_map_noalloc(const uint8_t *routing_map, int64_t T, int64_t E,
                           int64_t *row_expert_major, int64_t *row_token_major,
                           int32_t *row_expert_major_i32, int32_t *expert_offsets,
                           int32_t *src_token, int64_t src_capacity, void *stream);

/* ---- a4/a5: permute -----------------------------------------------------
 * Replaces case17 kernel_function(x, row_id_map, probs) -> (out, permuted_probs)
 * (kernel_results/case17_moe_permute_with_mask_map/binding.cpp:8-32; math
 * kernel_cases/case17_moe_permute_with_mask_map.py:58-71) and the expert-major
 * variants case21 (:52-68), case22 (:47-69), case30 (:44-58):
 *   out[map(t, e)] = x[t]; permuted_probs[map(t, e)] = probs[t, e]  for map >= 0.
 *   x     bf16 [T, H];  map [T, E] or [E, T] (layout), int32 or int64
 *   probs fp32 [T, E] (nullable; then permuted_probs must be NULL too)
 *   out   bf16 [num_out, H]; permuted_probs fp32 [num_out] (nullable)
 * zero_tail != 0: rows of out / permuted_probs at index >= R (R = number of
 *   map entries >= 0) are zero-filled, matching the reference's new_zeros
 *   when num_out exceeds R.  This assumes the entries >= 0 name exactly the
 *   rows 0..R-1 (a map built by moe_row_id_map does); for any other map the
 *   caller zeroes out / permuted_probs first and passes zero_tail == 0 (the
 *   case21/22/30 drop-ins do, after reading max and count of the map).  Needs
 *   moe_permute_workspace_size(T) bytes of workspace; with zero_tail == 0 the
 *   workspace may be NULL and rows no entry names are left untouched.
 * Map entries >= num_out are skipped. */
size_t moe_permute_workspace_size(int64_t T);
int moe_permute(const moe_bf16_t *x, int64_t T, int64_t H, const void *row_id_map, int idx_dtype,
                int map_layout, int64_t E, const float *probs, moe_bf16_t *out,
                float *permuted_probs, int64_t num_out, int zero_tail, void *workspace,
                size_t workspace_bytes, void *stream);

/* ---- a4': source token of each permuted row (inverse row-id map) -------
 * No function of its own in the reference: the token index that the permute
 * (case17 kernel_function, kernel_results/case17_moe_permute_with_mask_map/
 * binding.cpp; math kernel_cases/case17_moe_permute_with_mask_map.py) copies
 * into each permuted row, i.e. the inverse of the row-id map built by
 * kernel_cases/case12_moe_row_id_map_pass2.py:
 *   src_token[map(t, e)] = t  for every map(t, e) in [0, num_out);
 *   fill != 0: every row is first set to -1, so rows no map entry names stay -1.
 * Feeds moe_grouped_gemm_gather, which then reads permuted rows straight from x. */
int moe_permute_index(const void *row_id_map, int idx_dtype, int map_layout, int64_t T, int64_t E,
                      int32_t *src_token, int64_t num_out, int fill, void *stream);

/* ---- a4'': extent of a row-id map --------------------------------------
 * No kernel of its own in the reference: its scatter functions size their
 * output as max(row_id_map) + 1, read back with torch
 * (kernel_cases/case21_ref_permute_with_mask_map_trans.py:64, case22...:62,
 * case30...:54; kernel_results/case17_moe_permute_with_mask_map/binding.cpp:24).
 * One pass over the n entries of a map (any layout) computes the values the
 * scatter drop-ins need:
 *   out[0] = max(-1, largest entry)  (the output row count is out[0] + 1)
 *   out[1] = number of entries >= 0
 *   out[2] = 1 if the entries >= 0 name every row of [0, out[0]] exactly once
 *            (out[1] == out[0] + 1 and no entry repeats), else 0: only then
 *            does a scatter write every output row, so that the reference's
 *            zero-initialised output (new_zeros) needs no clearing.
 * out: int64 [3] on the device, written by the last of three kernels (a
 * clear of n bytes; per-block partials that also mark each entry's row with
 * a byte; their sum in block order with the count of marked rows).
 * Workspace: moe_map_extent_workspace_size(n) bytes (the partials and n
 * bytes of row marks), 16-byte aligned. */
size_t moe_map_extent_workspace_size(int64_t n);
int moe_map_extent(const void *row_id_map, int idx_dtype, int64_t n, int64_t *out, void *workspace,
                   size_t workspace_bytes, void *stream);

/* ---- a8: unpermute (combine), optional probability-weighted merge ------
 * Replaces case15 kernel_function(pin, row_id_map) -> out
 * (kernel_results/case15_moe_unpermute_mask_fwd/binding.cpp:10-20; math
 * kernel_cases/case15_moe_unpermute_mask_fwd.py:58-64, int32 variant
 * kernel_cases/case24_ref_moe_unpermute_mask_kernel_false.py:45-68):
 *   out[t] = bf16_rne( sum over e ascending, map(t,e) >= 0, of
 *                      [merge_probs[t, e] *] float(pin[map(t, e)]) )
 * fp32 accumulation starts at 0.0f, adds in ascending expert order, and the
 * weighted form multiplies then adds (no fused multiply-add).
 *   pin bf16 [R, H]; merge_probs fp32 [T, E] (nullable); out bf16 [T, H];
 *   out_acc (nullable) fp32 [T, H]: the fp32 sums before rounding (the int32
 *   reference reference_unpermute_mask returns them, case24...py:66-68).
 * Map entries >= R are skipped.  Limits: E <= 4096 (as moe_row_id_map). */
int moe_unpermute(const moe_bf16_t *pin, int64_t R, int64_t H, const void *row_id_map,
                  int idx_dtype, int map_layout, int64_t E, int64_t T, const float *merge_probs,
                  moe_bf16_t *out, float *out_acc, void *stream);

/* ---- a9: permute backward ----------------------------------------------
 * Replaces case18 Model.forward(dperm_act, dpp, row_id_map) -> (dact, dprobs)
 * (kernel_cases/case18_moe_permute_bwd_unpermute_mask.py:68-78; int32 variant
 * kernel_cases/case32_ref_moe_unpermute_mask_kernel.py:46-76):
 *   dact[t]      = bf16_rne( sum_e ascending float(dperm_act[map(t, e)]) )
 *   dprobs[t, e] = dpp[map(t, e)] if map(t, e) >= 0 else 0
 *   dperm_act bf16 [R, H]; dpp fp32 [R]; dact bf16 [T, H]; dprobs fp32 [T, E];
 *   out_acc (nullable) fp32 [T, H]: the fp32 sums (case32...py:74-76 returns them).
 * Limits: E <= 4096 (as moe_row_id_map). */
int moe_permute_bwd(const moe_bf16_t *dperm_act, int64_t R, int64_t H, const float *dpp,
                    const void *row_id_map, int idx_dtype, int map_layout, int64_t E, int64_t T,
                    moe_bf16_t *dact, float *dprobs, float *out_acc, void *stream);

/* ---- a10: row gather ------------------------------------------------------
 * Replaces case06 index_select_bf16(x, index)
 * (kernel_results/case06_cp_seq_chunk_index_select/binding.cpp:13-49; math
 * kernel_cases/case06_cp_seq_chunk_index_select.py:38-40):
 *   out[i, :] = src[index[i], :]  for i < n_index; row = row_elems bf16.
 * An index outside [0, src_rows) zero-fills its output row. */
int moe_index_select(const moe_bf16_t *src, int64_t src_rows, int64_t row_elems,
                     const void *index, int idx_dtype, int64_t n_index, moe_bf16_t *out,
                     void *stream);

/* ---- a6/a7: grouped GEMM forward -----------------------------------------
 * Replaces case03/case04 Model.forward(x, w) = cat_g( x[seg_g] @ w[g].T )
 * (kernel_cases/case03_moe_grouped_gemm_fc1_fwd.py:57-64,
 *  kernel_cases/case04_moe_grouped_gemm_fc2_fwd.py:57-64), "bf16 in / fp32
 * accumulate / bf16 out" (case03...py:37), plus the fused SwiGLU epilogue.
 *   a   bf16 [M_total, K] (rows of group g are group_offsets[g] .. [g+1]-1)
 *   w   bf16 [G, N, K]     (out x in, "NT": out = a @ w[g]^T)
 *   group_offsets int32 [G + 1] on the device, non-decreasing, [0] = 0,
 *                 [G] <= M_total (rows beyond [G] are not written)
 *   out bf16 [M_total, N] (MOE_EPILOGUE_NONE) or [M_total, N / 2] (SWIGLU:
 *       gate = columns [0, N/2), up = [N/2, N); silu(g) = g / (1 + exp(-g)),
 *       computed in fp32 on the fp32 accumulators, then one bf16 rounding).
 * Limits: K % 8 == 0, N % 2 == 0 (SWIGLU), 1 <= G <= 4096, K < 2^22, N * K < 2^30.
 * Workspace: optional; moe_grouped_gemm_workspace_size bytes, 256-byte
 *   aligned. What it holds depends on the shape:
 *   - G == 1 whose 256 x 256 output tiles leave the last round on the GPU's
 *     CUs at most half full (e.g. case10: 320 tiles on 256 CUs), K % 64 == 0,
 *     K >= 384: fp32 planes for a reduction split of that round's tiles. The
 *     other tiles run as usual; each of the last ones is computed as 2 to 8
 *     K ranges (one per CU) into its own fp32 plane, and a last kernel adds
 *     a tile's planes in range order and rounds once. The result is
 *     deterministic; it differs from the unsplit one only in the order of
 *     the fp32 partial sums (both are within the fp32-accumulation bound).
 *   - otherwise, K % 64 == 0 and either K >= 4096 or M_total < 256 G (the
 *     groups average fewer than 256 rows): a group whose last 256-row tile
 *     would hold 1 to 128 rows has that tile computed as a 128-row tile: a
 *     small kernel first lists those groups, and the GEMM's workgroups take
 *     the 128-row tiles from the list after their 256-row tiles (so the tiles
 *     also even out the last round). Every output element is summed in the
 *     same order either way: the result is the same bit for bit. With shorter
 *     reductions and longer groups a 128-row tile's start and drain cost more
 *     than the padding rows it saves, and the size is 0.
 *   Either is used only where the two-wavefronts-per-SIMD kernel runs (output
 *   rows of a multiple of 16 bytes on a 16-byte aligned out, fewer than 2^22
 *   output columns, M_total < 2^31, and M_total < 2^29 for the gather form);
 *   a workspace is ignored elsewhere, and NULL, 0 or a smaller size runs every
 *   tile whole with 256 rows. Calls that share a workspace must not overlap.
 *   moe_grouped_gemm (A rows in place) with MOE_EPILOGUE_NONE and groups of
 *   at most 128 rows on average (M_total <= 128 G, e.g. case03/04) under the
 *   same conditions runs 128-row tiles of 128-192 columns with no workspace
 *   (a given one is not used), with the same summation order: the same
 *   result bit for bit. */
size_t moe_grouped_gemm_workspace_size(int64_t M_total, int64_t K, int64_t N, int64_t G);
int moe_grouped_gemm(const moe_bf16_t *a, int64_t M_total, int64_t K, const moe_bf16_t *w,
                     int64_t G, int64_t N, const int32_t *group_offsets, int epilogue,
                     moe_bf16_t *out, void *workspace, size_t workspace_bytes, void *stream);

/* ---- a4+a6: permute fused into the grouped GEMM's A operand --------------
 * Replaces the composition permute (case17 kernel_function, see moe_permute)
 * followed by the fc1 grouped GEMM (case03 Model.forward, see
 * moe_grouped_gemm) when the permuted activations are only the GEMM's input:
 *   out = moe_grouped_gemm(a = x[a_rows], ...)
 *   x bf16 [x_rows, K]; a_rows int32 [M_total] (moe_permute_index output):
 *   row p of the GEMM is x[a_rows[p]]; an index outside [0, x_rows) reads zeros.
 * Other arguments, results and limits as moe_grouped_gemm. */
int moe_grouped_gemm_gather(const moe_bf16_t *x, int64_t x_rows, const int32_t *a_rows,
                            int64_t M_total, int64_t K, const moe_bf16_t *w, int64_t G, int64_t N,
                            const int32_t *group_offsets, int epilogue, moe_bf16_t *out,
                            void *workspace, size_t workspace_bytes, void *stream);

/* ---- grouped GEMM backward: input gradient ("NN") ------------------------
 * Replaces case07/case08/case13/case19 Model.forward(dy, w) =
 * cat_g( dy[seg_g] @ w[g] ) (kernel_cases/case07_moe_grouped_gemm_fc1_dgrad.py:57-64,
 * case08_moe_grouped_gemm_fc2_dgrad.py:57-64, case13...:57-64, case19...:57-64)
 * and, for one group, case37's NN GEMM (kernel_cases/
 * case37_ref_musa_asm_bf16_gemm_nn_256x384.py:47-49); bf16 in / fp32
 * accumulate / bf16 out (case07...py:37).
 *   dy  bf16 [M_total, N] (rows of group g are group_offsets[g] .. [g+1]-1)
 *   w   bf16 [G, N, K]    (the forward's [out, in] weights; dx = dy @ w[g])
 *   group_offsets int32 [G + 1] on the device, as moe_grouped_gemm
 *   dx  bf16 [M_total, K] (rows beyond group_offsets[G] are not written)
 * Limits: N % 8 == 0, K % 8 == 0, 1 <= G <= 4096, M_total < 2^31, N, K < 2^22,
 *   N * K < 2^30; dy, w, dx 16-byte aligned. N == 0 gives zeros.
 * Workspace: optional. With at least moe_grouped_gemm_dgrad_workspace_size
 *   bytes (256-byte aligned), a single group whose output has fewer tiles
 *   than half the CUs (case37) splits its reduction over the idle CUs into
 *   fp32 partial planes in the workspace, summed in split order (deterministic)
 *   and rounded once; otherwise (NULL, 0, or a smaller size) one pass as above.
 *   Without a split, groups of more than 160 rows on average and a reduction
 *   N >= 4096 (N % 64 == 0), the workspace (4 * (64 + G) bytes, rounded up to
 *   256) lists the groups whose last 256-row tile would hold 1 to 128 rows;
 *   those tiles then run as 128-row tiles after the 256-row ones (the same
 *   results bit for bit, less padding). The list is rebuilt on the stream by
 *   every call: calls that share one workspace must not overlap.
 *   The size is 0 where neither applies; it depends on the current device's
 *   CU count. */
size_t moe_grouped_gemm_dgrad_workspace_size(int64_t M_total, int64_t N, int64_t K, int64_t G);
int moe_grouped_gemm_dgrad(const moe_bf16_t *dy, int64_t M_total, int64_t N, const moe_bf16_t *w,
                           int64_t G, int64_t K, const int32_t *group_offsets, moe_bf16_t *dx,
                           void *workspace, size_t workspace_bytes, void *stream);

/* ---- grouped GEMM backward: weight gradient ("TN") -----------------------
 * Replaces case05/case09 Model.forward(dy, x) = stack_g( dy[seg_g]^T @ x[seg_g] )
 * (kernel_cases/case09_moe_grouped_gemm_fc1_wgrad.py:57-64,
 *  kernel_cases/case05_moe_grouped_gemm_fc2_wgrad.py:57-64); bf16 in / fp32
 * accumulate / bf16 out.
 *   dy  bf16 [M_total, N]; x bf16 [M_total, K] (rows of group g as above)
 *   dw  bf16 [G, N, K]: dw[g] = sum over the rows of g of dy[r]^T x[r]
 *       (a group without rows gets zeros, like torch.mm over an empty K)
 * Limits: N % 8 == 0, K % 8 == 0, 1 <= G <= 4096, M_total * N, M_total * K and
 *   N * K < 2^30; dy, x, dw 16-byte aligned.
 * Workspace: optional. With moe_grouped_gemm_wgrad_workspace_size bytes
 *   (4-byte aligned; 2 G bytes rounded up to 256, then 8 G bytes), a first
 *   kernel lists the groups largest first (int16 group ids, then each one's
 *   int32 row range) and the GEMM's tiles take them in that order, dealt to
 *   the workgroups in reverse on every other round, which evens out the work
 *   per workgroup when the group sizes are skewed; each tile's result is the
 *   same bit for bit either way. When the groups average under 256 rows, the
 *   groups of at most 128 rows (the end of that order) are computed by a
 *   kernel that keeps their whole reduction in LDS and sweeps the output
 *   tiles (the dw store stream), again the same bits. The size is 0 (no
 *   order) for one group. */
size_t moe_grouped_gemm_wgrad_workspace_size(int64_t M_total, int64_t N, int64_t K, int64_t G);
int moe_grouped_gemm_wgrad(const moe_bf16_t *dy, const moe_bf16_t *x, int64_t M_total, int64_t N,
                           int64_t K, int64_t G, const int32_t *group_offsets, moe_bf16_t *dw,
                           void *workspace, size_t workspace_bytes, void *stream);

/* ---- router gate GEMM (logits) -------------------------------------------
 * Replaces case38's router GEMM te_general_gemm(weight, inp, out_dtype=fp32,
 * layout="TN") (kernel_cases/case38_ref_musa_asm_bf16_ssgemm_nt_320x256.py:1-35;
 * golden reference_fp32 :46-53): logits = inp @ weight^T, bf16 in, fp32
 * accumulate, fp32 out.
 *   inp    bf16 [M, K];  weight bf16 [N, K] (num_experts x hidden)
 *   logits fp32 [M, N]
 * Limits: 1 <= N <= 512, K % 8 == 0, K < 2^22, N * K < 2^30; inp and weight
 *   16-byte aligned.
 * Workspace: none (pass NULL, 0). */
size_t moe_router_workspace_size(int64_t M, int64_t K, int64_t N);
int moe_router_logits(const moe_bf16_t *inp, int64_t M, int64_t K, const moe_bf16_t *weight, int64_t N,
                      float *logits, void *workspace, size_t workspace_bytes, void *stream);

/* ---- router gate GEMM fused with top-k, routing mask and merge probs -----
 * moe_router_logits followed by moe_topk on its rows (case23 ordering, mask
 * and softmax probs as moe_topk), enqueued together; `logits` may be NULL,
 * then the fp32 logits are kept in the workspace only.
 * Limits: as moe_router_logits, and 1 <= k <= min(N, 64).
 * Workspace: moe_router_workspace_size(M, K, N) bytes when logits is NULL,
 *   none otherwise. */
int moe_router_topk(const moe_bf16_t *inp, int64_t M, int64_t K, const moe_bf16_t *weight, int64_t N,
                    int64_t k, float *logits, float *values, int64_t *indices, uint8_t *routing_map,
                    float *probs, void *workspace, size_t workspace_bytes, void *stream);

/* ---- element casts (router backward) ------------------------------------
 * Replace case11 Model.forward(x) = x.to(torch.float32)
 * (kernel_cases/case11_router_bwd_cast_bf16_to_fp32.py:43-44) and case25's
 * timed inp.to(torch.bfloat16) (kernel_cases/case25_ref_unary_cast_fp32_to_bf16.py:107,
 * golden round_bf16_rne :56-66: round to nearest even).  Any NaN -> 0x7FC0.
 * n elements, contiguous; any alignment (16/32-byte aligned pointers take the
 * vector path).  Workspace: none. */
int moe_cast_bf16_to_f32(const moe_bf16_t *src, int64_t n, float *dst, void *stream);
int moe_cast_f32_to_bf16(const float *src, int64_t n, moe_bf16_t *dst, void *stream);

/* ---- router backward GEMMs in tf32 -------------------------------------
 * Replace case39's router dgrad te_general_gemm(weight.to(fp32), grad_output,
 * layout="NN") and case31's router wgrad te_general_gemm(inp.to(fp32),
 * grad_output, layout="NT"): golden reference_tf32
 * (kernel_cases/case39_ref_musa_asm_tf32_ssgemm_nn_384x256.py:61-68,
 *  kernel_cases/case31_ref_musa_asm_tf32_ssgemm_tn_128x256.py:61-68): both fp32
 * operands rounded to tf32 (round_tf32_rne, :51-58), products accumulated in
 * fp32, fp32 out.
 *   Both run on the fp16 matrix cores: a tf32 value has fp16's 11 significant
 *     bits; each operand row or column along which the sum runs is scaled by
 *     the power of two that brings its largest magnitude into [2^14, 2^15),
 *     so its values are fp16 values (exactly, unless 2^29 or more below that
 *     largest one: then within 2^-38 of it), the products are exact in fp32,
 *     and the sums are scaled back exactly (unless the result is an fp32
 *     subnormal); the scale comes from the largest finite magnitude (Inf and
 *     NaN entries stay Inf and NaN), a row or column with no finite nonzero
 *     value keeps scale 1, one whose largest is below 2^-112 takes 2^127.
 *   dgrad: grad_input [M, N] = tf32(grad_output [M, K]) @ tf32(weight [K, N]):
 *     grad_output scaled per row, weight per column, the scales undone in the
 *     GEMM's epilogue.
 *   wgrad: grad_weight [N, K] = tf32(grad_output [M, N])^T @ tf32(inp [M, K]):
 *     both scaled per column, undone where the reduction planes are added.
 * Limits: the column counts (K and N) % 8 == 0; dgrad 3K, N < 2^22 and
 *   3K*N < 2^30; wgrad M*N, M*K, N*K < 2^30; 16-byte aligned tensors.
 * Workspace: the *_workspace_size bytes, 256-byte aligned (dgrad: the fp16
 *   copies, M K + K N values, the row and column exponents and the
 *   column-max slabs; wgrad: the fp16 copies, M N + M K values, the column
 *   exponents, column-max slabs and the fp32 planes of the reduction chunks,
 *   at least one). */
size_t moe_router_dgrad_tf32_workspace_size(int64_t M, int64_t K, int64_t N);
int moe_router_dgrad_tf32(const float *grad_output, int64_t M, int64_t K, const float *weight, int64_t N,
                          float *grad_input, void *workspace, size_t workspace_bytes, void *stream);
size_t moe_router_wgrad_tf32_workspace_size(int64_t M, int64_t N, int64_t K);
int moe_router_wgrad_tf32(const float *grad_output, int64_t M, int64_t N, const float *inp, int64_t K,
                          float *grad_weight, void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MOE_DISPATCH_H_ */
