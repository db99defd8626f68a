"""GPU parity of the grouped GEMM (fc1 + SwiGLU, fc2) against the fp32 oracle.

Tolerance: rtol 1.6e-2 / atol 1e-2 against the fp32-accumulated golden
(x.float() @ w.float().T per group, kernel_cases/case35...py:41-48) -- the
bf16 bound of the task statement.  Small shapes are checked in full on the
CPU; the benchmark shapes (configs c3 / c4) are checked in full on their three
smallest non-empty groups and on sampled rows of every other group, all
against the CPU oracle (ref_torch.grouped_gemm_fp32 on the host).
"""
from __future__ import annotations

import pytest
import torch

from oracle import ref_torch

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1.6e-2, 1e-2


def _check(got, ref, what):
    torch.testing.assert_close(got.float().cpu(), ref.float().cpu(), rtol=RTOL, atol=ATOL, msg=lambda m: f"{what}: {m}")


@pytest.mark.parametrize("sizes,K,N", [
    ([256], 64, 256),                    # one full tile
    ([1], 8, 1),                         # degenerate
    ([300, 0, 17, 513], 200, 264),       # ragged, an empty group, K and N tails
    ([5, 7, 0, 0, 1000], 7168, 320),     # K of the benchmark
    ([130] * 3, 2048, 7168),             # fc2 shape class
])
def test_grouped_gemm_plain(pkg, dev, sizes, K, N):
    g = torch.Generator().manual_seed(sum(sizes) + K + N)
    x = torch.randn(sum(sizes), K, generator=g).to(torch.bfloat16)
    w = (torch.randn(len(sizes), N, K, generator=g) * 0.05).to(torch.bfloat16)
    out = pkg.cases.case04_moe_grouped_gemm_fc2_fwd.kernel_function(x.to(dev), w.to(dev), sizes)
    _check(out, ref_torch.grouped_gemm_fp32(x, w, sizes), f"plain sizes={sizes} K={K} N={N}")


@pytest.mark.parametrize("sizes,K,N", [([256], 64, 512), ([100, 0, 333], 136, 272), ([64, 700], 7168, 4096)])
def test_grouped_gemm_swiglu(pkg, dev, sizes, K, N):
    g = torch.Generator().manual_seed(sum(sizes) * 3 + K)
    x = torch.randn(sum(sizes), K, generator=g).to(torch.bfloat16)
    w = (torch.randn(len(sizes), N, K, generator=g) * 0.05).to(torch.bfloat16)
    out = pkg.cases.case03_moe_grouped_gemm_fc1_fwd.kernel_function(x.to(dev), w.to(dev), sizes, swiglu=True)
    ref = ref_torch.swiglu(ref_torch.grouped_gemm_fp32(x, w, sizes))
    assert out.shape == (sum(sizes), N // 2)
    _check(out, ref, f"swiglu sizes={sizes} K={K} N={N}")


def test_grouped_gemm_identity_exact(pkg, dev):
    # x @ (c I)^T with c a power of two is exact in bf16: the result must be bit-identical.
    x = torch.randn(600, 256).to(torch.bfloat16)
    w = torch.stack([torch.eye(256), 4 * torch.eye(256), 0.5 * torch.eye(256)]).to(torch.bfloat16)
    out = pkg.cases.case04_moe_grouped_gemm_fc2_fwd.kernel_function(x.to(dev), w.to(dev), [100, 300, 200]).cpu()
    assert torch.equal(out[:100], x[:100])
    assert torch.equal(out[100:400], (4 * x[100:400].float()).to(torch.bfloat16))
    assert torch.equal(out[400:], (0.5 * x[400:].float()).to(torch.bfloat16))


def test_grouped_gemm_uniform_model(pkg, dev):
    # case03/04 Model(num_groups, tokens) with the uniform group_sizes (reduced sizes).
    case = pkg.cases.case04_moe_grouped_gemm_fc2_fwd
    x, w = case.get_inputs(dev, tokens=1000, groups=8, n=384, k=256)
    out = case.Model(8, 1000)(x, w)
    _check(out, ref_torch.grouped_gemm_fp32(x.cpu(), w.cpu(), case.group_sizes(1000, 8)), "uniform model")


@pytest.mark.parametrize("case_name", ["case10_grouped_gemm_single_group_fc1_fwd",
                                       "case14_grouped_gemm_single_group_fc2_fwd"])
def test_single_group_reference_cases_full(pkg, dev, case_name):
    # The reference's one-group forward cases at their own shapes (4096 x 8192 -> 5120 and 4096 x 2560 -> 8192,
    # kernel_cases/case10_grouped_gemm_single_group_fc1_fwd.py:25-28, case14...:25-28), every output element
    # against the CPU oracle, through the Model with the case's uniform sizes and through kernel_function.
    case = getattr(pkg.cases, case_name)
    x, w = case.get_inputs(dev)
    assert x.shape == (case.TOKENS, case.K) and w.shape == (1, case.N, case.K)
    out = case.Model()(x, w)
    assert out.shape == (case.TOKENS, case.N)
    _check(out, ref_torch.grouped_gemm_fp32(x.cpu(), w.cpu(), case.group_sizes(case.TOKENS, 1)), case_name)
    again = case.kernel_function(x, w)
    assert torch.equal(again.cpu(), out.cpu()), "two calls differ"


@pytest.mark.parametrize("M,K,N,swiglu,gather,rows", [
    (1000, 1024, 1000, False, False, 1000),   # 16 tiles: every tile split (5 ranges of 3 K steps)
    (1000, 1024, 1040, True, False, 1000),    # SwiGLU: the sums of gate and up, then silu(g) * u
    (1000, 1024, 1040, True, True, 1000),     # gathered A rows (fc1 of a one-expert layer)
    (1000, 1024, 1000, False, False, 700),    # the group ends before M: rows past it untouched
    (4100, 8192, 5120, False, False, 4100),   # 340 tiles: 256 unsplit, the last 84 in 3 ranges (a 4-row tail)
    (300, 640, 264, False, False, 300),       # output columns not a multiple of 16
])
def test_single_group_reduction_split(pkg, dev, M, K, N, swiglu, gather, rows):
    # One group whose last round of 256 x 256 tiles is at most half full: with the workspace those tiles run
    # as K ranges into fp32 planes, added in range order. Against the CPU oracle at the task tolerance, and
    # against the same GEMM without a workspace (no split) at the same tolerance.
    ops = pkg.ops
    assert pkg._lib.lib().moe_grouped_gemm_workspace_size(M, K, N, 1) >= 65536 * 4 * 2, "no split planned"
    g = torch.Generator().manual_seed(M + K + N + rows)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(1, N, K, generator=g) * 0.05).to(torch.bfloat16)
    offs = torch.tensor([0, rows], dtype=torch.int32, device=dev)
    ncols = N // 2 if swiglu else N
    out = torch.full((M + 2, ncols), 3.0, dtype=torch.bfloat16, device=dev)  # guard rows around the output
    if gather:
        src = torch.randperm(M, generator=g)[:M].to(torch.int32)
        ops.grouped_gemm_gather(x.to(dev), src.to(dev), w.to(dev), offs, swiglu=swiglu, out=out[1:M + 1])
        a = x[src.long()]
    else:
        ops.grouped_gemm(x.to(dev), w.to(dev), offs, swiglu=swiglu, out=out[1:M + 1])
        a = x
    got = out.cpu()
    assert torch.all(got[0] == 3.0) and torch.all(got[M + 1] == 3.0), "stored outside out"
    assert torch.all(got[1 + rows:M + 1] == 3.0), "rows past the group were written"
    ref = ref_torch.grouped_gemm_fp32(a[:rows], w, [rows])
    if swiglu:
        ref = ref_torch.swiglu(ref)
    _check(got[1:rows + 1], ref, f"split M={M} K={K} N={N} swiglu={swiglu} gather={gather} rows={rows}")
    empty = torch.empty(0, dtype=torch.uint8, device=dev)
    if gather:
        plain = ops.grouped_gemm_gather(x.to(dev), src.to(dev), w.to(dev), offs, swiglu=swiglu, workspace=empty)
    else:
        plain = ops.grouped_gemm(x.to(dev), w.to(dev), offs, swiglu=swiglu, workspace=empty)
    _check(got[1:rows + 1], plain[:rows], "split against unsplit")


def _sampled_check(x, w, offs, out, swiglu, rows_per_group=48, seed=0, full_groups=()):
    """Rows of every group (all rows of the groups in full_groups, else a sample plus both
    ends) against the CPU oracle, one group at a time (x, w and out may live on the GPU)."""
    g = torch.Generator().manual_seed(seed)
    for gi in range(w.shape[0]):
        lo, hi = int(offs[gi]), int(offs[gi + 1])
        if hi == lo:
            continue
        if gi in full_groups:
            rows = torch.arange(lo, hi)
        else:
            rows = torch.randint(lo, hi, (min(rows_per_group, hi - lo),), generator=g)
            rows = torch.cat([rows, torch.tensor([lo, hi - 1])])
        ref = ref_torch.grouped_gemm_fp32(x[rows.to(x.device)].cpu(), w[gi:gi + 1].cpu(), [rows.numel()])
        if swiglu:
            ref = ref_torch.swiglu(ref)
        _check(out[rows.to(out.device)], ref, f"group {gi} ({'all' if gi in full_groups else 'sampled'} rows)")


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_grouped_gemm_benchmark_configs(pkg, dev, name):
    cfg = pkg.inputs.GEMM_CONFIGS[name]
    sizes = pkg.inputs.zipf_group_sizes(cfg["total"], cfg["groups"])
    assert sizes[-1] == 0 and sum(sizes) == cfg["total"]
    x = pkg.inputs.randn_bf16((cfg["total"], cfg["K"]), seed=1, device=dev)
    w = pkg.inputs.randn_bf16((cfg["groups"], cfg["N"], cfg["K"]), std=0.02, seed=2, device=dev)
    offs = pkg.ops.group_offsets_from_splits(sizes, dev)
    out = pkg.ops.grouped_gemm(x, w, offs, swiglu=cfg["swiglu"])
    smallest = sorted((m, gi) for gi, m in enumerate(sizes) if m > 0)[:3]
    _sampled_check(x, w, offs.cpu(), out, cfg["swiglu"], full_groups={gi for _, gi in smallest})


def test_grouped_gemm_uniform_8192_per_expert(pkg, dev):
    # The uniform M_e = 8192 point of config c4 (peak-MFMA reference shape).
    x = pkg.inputs.randn_bf16((16 * 8192, 2048), seed=3, device=dev)
    w = pkg.inputs.randn_bf16((16, 7168, 2048), std=0.02, seed=4, device=dev)
    offs = pkg.ops.group_offsets_from_splits([8192] * 16, dev)
    out = pkg.ops.grouped_gemm(x, w, offs)
    _sampled_check(x, w, offs.cpu(), out, False, rows_per_group=16)


def test_grouped_gemm_errors(pkg, dev):
    x = torch.zeros(4, 12, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(1, 8, 12, dtype=torch.bfloat16, device=dev)
    offs = torch.tensor([0, 4], dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        pkg.ops.grouped_gemm(x, w, offs)
    with pytest.raises(ValueError):
        pkg.ops.grouped_gemm(x, w[:, :, :8], offs)


@pytest.mark.parametrize("sizes,K,N,swiglu,gather", [
    ([300, 0, 17, 513], 200, 264, False, False),      # ragged, empty group, K and N tails
    # K % 64 == 0 runs the two-wavefronts-per-SIMD kernel:
    ([300, 0, 17, 513], 192, 264, False, False),      # three K steps, N tail, ragged, empty group
    ([1, 0, 2], 192, 8, False, False),                # tiny groups, one partial column tile
    ([40] * 600, 256, 512, False, False),             # 600 groups: many tile changes per workgroup
    ([100, 0, 333], 192, 272, True, True),            # SwiGLU with 136 output columns, gather
    ([257, 255, 0, 513], 320, 1024, True, False),     # row tails of 1 and 255, SwiGLU
    ([40] * 300, 384, 512, False, True),              # gather, many groups
    ([40] * 600, 200, 512, False, False),             # 600 groups: many tile changes per workgroup
    ([2000, 3, 1500], 2048, 7168, False, False),      # fc2 class, several tiles per workgroup
    ([64, 700, 0, 1500], 7168, 4096, True, False),    # fc1 class
    ([40] * 300, 136, 272, True, True),               # K tail, three K steps, gather
    ([900, 0, 2100], 7168, 4096, True, True),         # fc1 gather class
])
def test_pipelined_kernel_matches_drained_kernel(pkg, dev, sizes, K, N, swiglu, gather):
    """K > 128 with 16-byte output rows runs the pipelined kernel (16x16x32 MFMAs,
    tiles back to back, register epilogue); an output 2 bytes off 16-byte alignment
    runs the drained kernel (32x32x16 MFMAs, LDS-staged epilogue). Both accumulate
    K in the same ascending order in fp32 and round once: equal bit for bit."""
    g = torch.Generator().manual_seed(sum(sizes) + K + N)
    M = sum(sizes)
    w = (torch.randn(len(sizes), N, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    offs = pkg.ops.group_offsets_from_splits(sizes, dev)
    ncols = N // 2 if swiglu else N
    buf = torch.full((M * ncols + 16,), float("nan"), dtype=torch.bfloat16, device=dev)
    drained = buf[1:1 + M * ncols].view(M, ncols)
    assert drained.data_ptr() % 16 != 0
    if gather:
        X = 777
        x = torch.randn(X, K, generator=g).to(torch.bfloat16).to(dev)
        rows = torch.randint(0, X, (M,), generator=g, dtype=torch.int32).to(dev)
        piped = pkg.ops.grouped_gemm_gather(x, rows, w, offs, swiglu=swiglu)
        pkg.ops.grouped_gemm_gather(x, rows, w, offs, swiglu=swiglu, out=drained)
    else:
        x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
        piped = pkg.ops.grouped_gemm(x, w, offs, swiglu=swiglu)
        pkg.ops.grouped_gemm(x, w, offs, swiglu=swiglu, out=drained)
    torch.cuda.synchronize()
    assert torch.equal(piped.view(torch.int16), drained.view(torch.int16)), f"sizes={sizes[:4]} K={K} N={N}"
    # and both against the fp32 golden on sampled rows of every group
    a = x[rows.long()] if gather else x
    _sampled_check(a, w, offs.cpu(), piped, swiglu, rows_per_group=8)


@pytest.mark.parametrize("sizes,K,N,swiglu,gather", [
    # tails of 1, 127, 128 (128-row tiles), 129, 255 (256-row tiles), whole tiles, empty groups
    ([1, 127, 128, 129, 255, 256, 512, 0, 385, 640], 4096, 512, False, False),
    ([1, 127, 128, 129, 255, 256, 512, 0, 385, 640], 4096, 1024, True, True),
    ([3, 0, 70, 2000, 128, 4097], 7168, 4096, True, False),       # fc1 class, K of the benchmark
    ([40] * 200 + [300] * 20, 4096, 256, False, True),            # many 128-row tiles: several per workgroup
    ([1] * 64, 4096, 8, False, False),                            # tails only, one partial column tile
    ([102] * 39 + [118], 2560, 1024, False, False),               # short reduction, groups under 256 rows (case04)
    ([90, 0, 300, 17] * 5, 448, 512, True, True),                 # short reduction, 101 rows per group on average
])
def test_tail_tiles_match_full_tiles(pkg, dev, sizes, K, N, swiglu, gather):
    """With its workspace the forward GEMM computes a group's last row tile of 1 to 128 rows as a
    128-row tile, taken from a list after the 256-row tiles; without it every row tile has 256
    rows. The per-element K order and rounding are the same: equal bit for bit."""
    g = torch.Generator().manual_seed(sum(sizes) + K + N + 7)
    M = sum(sizes)
    w = (torch.randn(len(sizes), N, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    offs = pkg.ops.group_offsets_from_splits(sizes, dev)
    assert pkg.ops._lib.lib().moe_grouped_gemm_workspace_size(M, K, N, len(sizes)) > 0
    none = torch.empty(0, dtype=torch.uint8, device=dev)
    if gather:
        X = 501
        x = torch.randn(X, K, generator=g).to(torch.bfloat16).to(dev)
        rows = torch.randint(0, X, (M,), generator=g, dtype=torch.int32).to(dev)
        tails = pkg.ops.grouped_gemm_gather(x, rows, w, offs, swiglu=swiglu)
        full = pkg.ops.grouped_gemm_gather(x, rows, w, offs, swiglu=swiglu, workspace=none)
    else:
        x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
        ws = torch.full((4096,), 0xAB, dtype=torch.uint8, device=dev)  # stale contents: the list kernel rewrites it
        tails = pkg.ops.grouped_gemm(x, w, offs, swiglu=swiglu, workspace=ws)
        tails2 = pkg.ops.grouped_gemm(x, w, offs, swiglu=swiglu, workspace=ws)  # the same workspace again
        full = pkg.ops.grouped_gemm(x, w, offs, swiglu=swiglu, workspace=none)
        assert torch.equal(tails.view(torch.int16), tails2.view(torch.int16))
    torch.cuda.synchronize()
    assert torch.equal(tails.view(torch.int16), full.view(torch.int16)), f"sizes={sizes[:6]} K={K} N={N}"
    a = x[rows.long()] if gather else x
    _sampled_check(a, w, offs.cpu(), tails, swiglu, rows_per_group=8)


@pytest.mark.parametrize("sizes,K,N", [
    ([102] * 39 + [118], 8192, 5120),                             # case03 shape (160-column tiles)
    ([102] * 39 + [118], 2560, 8192),                             # case04 shape
    ([3, 0, 700, 41, 128, 129, 1, 64, 100, 5] * 4, 448, 520),     # ragged: groups of 6 row tiles, empty groups
    ([1] * 300, 192, 200),                                        # 3 K steps: the rings run across tiles
    ([0, 0, 5], 192, 136),                                        # a single tile
    ([128] * 8, 1024, 8),                                         # one partial column tile per group
])
def test_short_group_kernel_bit_identical(pkg, dev, sizes, K, N):
    """Groups of at most 128 rows on average (plain epilogue, rows in place) run 128-row tiles with
    loading wavefronts; the gathered form with identity rows runs the ping-pong kernel. Both take the
    same v_mfma_f32_16x16x32_bf16 sequence per output element: equal bit for bit, nothing written past
    the output, and both against the CPU oracle."""
    g = torch.Generator().manual_seed(sum(sizes) + 3 * K + N)
    M, G = sum(sizes), len(sizes)
    assert M <= 128 * G
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(G, N, K, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    offs = pkg.ops.group_offsets_from_splits(sizes, dev)
    buf = torch.full((M * N + 256,), float("nan"), dtype=torch.bfloat16, device=dev)
    out = buf[:M * N].view(M, N)
    pkg.ops.grouped_gemm(x, w, offs, out=out)
    rows = torch.arange(M, dtype=torch.int32, device=dev)
    pp = pkg.ops.grouped_gemm_gather(x, rows, w, offs)
    again = pkg.ops.grouped_gemm(x, w, offs)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), pp.view(torch.int16)), f"sizes={sizes[:6]} K={K} N={N}"
    assert torch.equal(again.view(torch.int16), pp.view(torch.int16))
    assert torch.isnan(buf[M * N:].float()).all()
    _sampled_check(x, w, offs.cpu(), out, False, rows_per_group=8)
