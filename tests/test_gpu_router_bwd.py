"""GPU parity of the tf32 router backward GEMMs (case39 dgrad, case31 wgrad).

The golden (reference_tf32, case39...:61-68 / case31...:61-68) multiplies tf32-rounded operands
exactly and accumulates in fp32.  Here every tf32 product is one exact product of fp16 values scaled
by powers of two (dgrad: per grad_output row and per weight column; wgrad: per operand column),
accumulated in fp32 in another order, so the bound is
|ours - golden| <= 1e-4 * sum_k |a_k b_k| + 1e-5.  The cases' own checks against an explicit sum
(case39: 1e-3, case31: 1e-2 absolute) are applied as written at full size; the full-size goldens
are computed on the CPU.
"""
from __future__ import annotations

import pytest
import torch

from oracle import ref_torch

pytestmark = pytest.mark.gpu


def _bound_check(got, ref, absprod, what):
    err = (got.cpu().double() - ref.double()).abs()
    bound = 1e-4 * absprod.double() + 1e-5
    assert bool((err <= bound).all()), f"{what}: worst err/bound {(err / bound).max().item():.3f}"


# Reductions of whole and partial 64-wide steps (K = 40, 1000, 1200), output columns past a column tile, row
# tiles with 1-127 valid rows, grad_output rows longer than the 1024 values the row conversion keeps in registers.
@pytest.mark.parametrize("M,K,N", [(64, 64, 256), (5, 8, 8), (300, 320, 520), (1000, 64, 8192), (130, 1000, 264),
                                   (700, 192, 1000), (129, 40, 72), (300, 1200, 136)])
def test_router_dgrad_tf32_shapes(pkg, dev, M, K, N):
    g = torch.Generator().manual_seed(M + K + N)
    go = torch.randn(M, K, generator=g)
    w = torch.randn(K, N, generator=g).to(torch.bfloat16).float()
    got = pkg.ops.router_dgrad_tf32(go.to(dev), w.to(dev))
    ref = ref_torch.router_dgrad_tf32(go, w)
    absprod = ref_torch.round_tf32_rne(go).abs() @ ref_torch.round_tf32_rne(w).abs()
    _bound_check(got, ref, absprod, f"dgrad M={M} K={K} N={N}")


@pytest.mark.parametrize("M,N,K", [(64, 64, 256), (5, 8, 8), (1000, 320, 520), (4096, 64, 1000), (0, 16, 24)])
def test_router_wgrad_tf32_shapes(pkg, dev, M, N, K):
    g = torch.Generator().manual_seed(3 * M + N + K)
    go = torch.randn(M, N, generator=g)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).float()
    got = pkg.ops.router_wgrad_tf32(go.to(dev), x.to(dev))
    assert got.shape == (N, K)
    ref = ref_torch.router_wgrad_tf32(go, x)
    absprod = ref_torch.round_tf32_rne(go).abs().t() @ ref_torch.round_tf32_rne(x).abs()
    _bound_check(got, ref, absprod, f"wgrad M={M} N={N} K={K}")


def test_case39_full_size(pkg, dev):
    case = pkg.cases.case39_ref_musa_asm_tf32_ssgemm_nn_384x256
    go, w = case.make_inputs(seed=0, device=dev)
    got = case.kernel_function(go, w)
    assert got.shape == (case.M, case.N) and got.dtype == torch.float32
    a, b = ref_torch.round_tf32_rne(go.cpu()), ref_torch.round_tf32_rne(w.cpu())
    ref = ref_torch.router_dgrad_tf32(go.cpu(), w.cpu())
    bound = 1e-4 * (a.abs() @ b.abs()) + 1e-5
    assert bool(((got.cpu() - ref).abs() <= bound).all())
    a, b = a.to(dev), b.to(dev)
    rows = torch.tensor([0, case.M // 2, case.M - 1], device=dev)
    manual = (a[rows].double().unsqueeze(-1) * b.double().unsqueeze(0)).sum(dim=1)
    assert (got[rows].double() - manual).abs().max().item() <= 1e-3


def test_case31_full_size(pkg, dev):
    case = pkg.cases.case31_ref_musa_asm_tf32_ssgemm_tn_128x256
    go, x = case.make_inputs(seed=0, device=dev)
    got = case.kernel_function(go, x)
    assert got.shape == (case.N, case.K) and got.dtype == torch.float32
    a, b = ref_torch.round_tf32_rne(go.cpu()), ref_torch.round_tf32_rne(x.cpu())
    ref = ref_torch.router_wgrad_tf32(go.cpu(), x.cpu())
    bound = 1e-4 * (a.abs().t() @ b.abs()) + 1e-5
    assert bool(((got.cpu() - ref).abs() <= bound).all())
    a, b = a.to(dev), b.to(dev)
    cols = torch.tensor([0, case.N // 2, case.N - 1], device=dev)
    manual = torch.stack([(a[:, c].double().unsqueeze(1) * b.double()).sum(dim=0) for c in cols.tolist()])
    assert (got[cols].double() - manual).abs().max().item() <= 1e-2


def test_router_wgrad_tf32_columns_of_any_scale(pkg, dev):
    # Each operand column is scaled by its own power of two into the fp16 range: columns of grad_output
    # near 1e-30 and 1e18, and of inp near 1e-20 and 1e15, keep the relative accuracy of the others
    # (the bound without its absolute term on the scaled rows and columns of dw).
    M, N, K = 1000, 64, 520
    g = torch.Generator().manual_seed(77)
    go = torch.randn(M, N, generator=g)
    x = torch.randn(M, K, generator=g)
    go[:, 3] *= 1e-30
    go[:, 5] *= 1e18
    x[:, 7] *= 1e-20
    x[:, 9] *= 1e15
    got = pkg.ops.router_wgrad_tf32(go.to(dev), x.to(dev)).cpu().double()
    ref = ref_torch.router_wgrad_tf32(go.double(), x.double())
    absprod = ref_torch.round_tf32_rne(go).abs().t().double() @ ref_torch.round_tf32_rne(x).abs().double()
    rel = (got - ref).abs() / absprod.clamp(min=1e-300)
    assert bool(torch.isfinite(got).all())
    for what, sel in (("row 3", rel[3]), ("row 5", rel[5]), ("column 7", rel[:, 7]), ("column 9", rel[:, 9]),
                      ("all", rel)):
        assert rel.numel() and bool((sel <= 1e-4).all()), f"{what}: worst relative error {sel.max().item():.3e}"


def test_router_dgrad_tf32_rows_and_columns_of_any_scale(pkg, dev):
    # grad_output's rows and weight's columns are each scaled by their own power of two into the fp16 range:
    # rows near 1e-30, 1e-25 and 1e18, columns near 1e-20 and 1e15 keep the relative accuracy of the others.
    # Reference: the float64 sum of the tf32-rounded operands' products; outputs in fp32's subnormal range
    # (row 600 x column 7, ~1e-44) are held to an absolute 2^-126, fp32's smallest normal.
    M, K, N = 700, 320, 520
    g = torch.Generator().manual_seed(78)
    go = torch.randn(M, K, generator=g)
    w = torch.randn(K, N, generator=g)
    go[3] *= 1e-30
    go[5] *= 1e18
    go[600] *= 1e-25
    w[:, 7] *= 1e-20
    w[:, 9] *= 1e15
    got = pkg.ops.router_dgrad_tf32(go.to(dev), w.to(dev)).cpu().double()
    a, b = ref_torch.round_tf32_rne(go).double(), ref_torch.round_tf32_rne(w).double()
    ref = a @ b
    excess = (got - ref).abs() - (1e-4 * (a.abs() @ b.abs()) + 2.0 ** -126)
    assert bool(torch.isfinite(got).all())
    for what, sel in (("row 3", excess[3]), ("row 5", excess[5]), ("row 600", excess[600]),
                      ("column 7", excess[:, 7]), ("column 9", excess[:, 9]), ("all", excess)):
        assert bool((sel <= 0).all()), f"{what}: error above the bound by {sel.max().item():.3e}"


@pytest.mark.parametrize("which", ["dgrad", "wgrad"])
def test_router_tf32_inf_and_nan_entries(pkg, dev, which):
    # A row / column holding Inf (or NaN) and finite values above fp16's range: the scale comes from the largest
    # finite magnitude, so the finite values convert exactly and the Inf / NaN entries stay Inf / NaN; the
    # outputs match torch's fp32 product of the tf32-rounded operands in their Inf (with sign) and NaN
    # positions, and the finite ones within the bound.
    g = torch.Generator().manual_seed(91)
    if which == "dgrad":
        M, K, N = 300, 320, 264
        a = torch.randn(M, K, generator=g)
        b = torch.randn(K, N, generator=g)
        a[10, 0], a[10, 1], a[10, 2] = float("inf"), 1e6, -3e5  # one grad_output row: Inf and large finite values
        a[11, 5] = float("nan")
        b[3, 20], b[4, 20] = float("-inf"), 2e5                 # one weight column
        got = pkg.ops.router_dgrad_tf32(a.to(dev), b.to(dev)).cpu()
        ra, rb = ref_torch.round_tf32_rne(a), ref_torch.round_tf32_rne(b)
        ref = ref_torch.router_dgrad_tf32(a, b)
        absprod = ra.abs() @ rb.abs()
    else:
        M, N, K = 1000, 64, 520
        a = torch.randn(M, N, generator=g)
        b = torch.randn(M, K, generator=g)
        a[0, 6], a[1, 6], a[2, 6] = float("inf"), 1e6, -3e5     # one grad_output column
        a[7, 8] = float("nan")
        b[3, 30], b[4, 30] = float("-inf"), 2e5                 # one inp column
        got = pkg.ops.router_wgrad_tf32(a.to(dev), b.to(dev)).cpu()
        ra, rb = ref_torch.round_tf32_rne(a), ref_torch.round_tf32_rne(b)
        ref = ref_torch.router_wgrad_tf32(a, b)
        absprod = ra.abs().t() @ rb.abs()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    assert torch.equal(torch.isposinf(got), torch.isposinf(ref)) and torch.equal(torch.isneginf(got), torch.isneginf(ref))
    fin = torch.isfinite(ref)
    assert int((~fin).sum()) > 0 and int(fin.sum()) > 0
    err = (got[fin].double() - ref[fin].double()).abs()
    assert bool((err <= 1e-4 * absprod[fin].double() + 1e-5).all())
