"""GPU parity of the router gate GEMM (fp32 logits) and of its fused top-k.

Logits: fp32 accumulation of bf16 products in another order than the golden
(inp.float() @ weight.float().T, kernel_cases/case38...:46-53), so the bound is
absolute: |ours - golden| <= 2e-3 + 1e-5 |golden| (the case's own check allows
1e-3 against an explicit sum, :64-79, which is applied as written on its rows).
The fused top-k must be bit-identical to moe_topk run on the logits the same
kernel writes, and the logits of both entry points bit-identical.
"""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bits_equal
from oracle import ref_torch

pytestmark = pytest.mark.gpu


def _check_logits(got, inp, w, what):
    ref = ref_torch.router_logits_fp32(inp.cpu(), w.cpu())
    err = (got.cpu() - ref).abs()
    bound = 2e-3 + 1e-5 * ref.abs()
    assert bool((err <= bound).all()), f"{what}: max err {err.max().item():.3e}"


@pytest.mark.parametrize("M,K,N", [
    (64, 64, 64),        # one tile, one step
    (1, 8, 1),           # degenerate
    (100, 200, 8),       # row tail, K tail, narrow N
    (300, 1000, 100),    # N not a multiple of 16
    (257, 4096, 320),    # the case's N, row tail
    (130, 512, 512),     # widest N (two-stage ring)
    (64, 7168, 64),      # c5 router shape class (E = 64, H = 7168)
])
def test_router_logits_shapes(pkg, dev, M, K, N):
    g = torch.Generator().manual_seed(M + K + N)
    inp = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16)
    got = pkg.ops.router_logits(inp.to(dev), w.to(dev))
    assert got.shape == (M, N) and got.dtype == torch.float32
    _check_logits(got, inp, w, f"M={M} K={K} N={N}")


@pytest.mark.parametrize("M,K,N", [
    (257, 4096, 320),    # the case's N: 128-row tiles over half of N (kNB = 5)
    (300, 1024, 136),    # kNB = 3
    (129, 640, 250),     # kNB = 4, column tail
    (200, 2048, 384),    # kNB = 6
    (64, 512, 448),      # kNB = 7
    (130, 512, 512),     # kNB = 8
])
def test_router_tiles_bit_identical_to_row_kernel(pkg, dev, M, K, N):
    # 128 < N with whole 64-column steps and 16-byte output rows runs as 128-row tiles over half of N, with
    # the loads in wavefronts of their own; an output 4 bytes off 16-byte alignment runs the 64-row kernel.
    # Each logit is the same MFMA sequence over K in both: bit-identical, and within the bound of the oracle.
    g = torch.Generator().manual_seed(5 * M + K + N)
    inp = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16)
    tiled = pkg.ops.router_logits(inp.to(dev), w.to(dev))
    buf = torch.empty(M * N + 4, dtype=torch.float32, device=dev)
    rows = pkg.ops.router_logits(inp.to(dev), w.to(dev), out=buf[1:1 + M * N].view(M, N))
    assert rows.data_ptr() % 16 == 4
    assert_bits_equal(tiled, rows, f"tiles vs 64-row kernel M={M} K={K} N={N}")
    _check_logits(tiled, inp, w, f"M={M} K={K} N={N}")


def test_case38_full_shape(pkg, dev):
    # The case's seeded inputs at full size: every logit against the CPU oracle, and the case's
    # own explicit-sum rule on its three rows.
    case = pkg.cases.case38_ref_musa_asm_bf16_ssgemm_nt_320x256
    inp, w = case.make_inputs(seed=0, device=dev)
    got = case.kernel_function(inp, w)
    assert got.shape == (case.M, case.N)
    ref = ref_torch.router_logits_fp32(inp.cpu(), w.cpu()).to(dev)
    err = (got - ref).abs()
    assert bool((err <= 2e-3 + 1e-5 * ref.abs()).all()), f"max err {err.max().item():.3e}"
    rows = torch.tensor([0, case.M // 2, case.M - 1], device=dev)
    manual = (inp[rows].double().unsqueeze(-1) * w.double().t().unsqueeze(0)).sum(dim=1)
    assert (got[rows].double() - manual).abs().max().item() <= 1e-3


@pytest.mark.parametrize("M,K,N,k", [(64, 64, 64, 8), (300, 1000, 100, 3), (1000, 2048, 320, 8),
                                     (77, 512, 512, 64), (5, 8, 1, 1), (16384, 8192, 320, 8)])
def test_router_topk_fused_matches_topk(pkg, dev, M, K, N, k):
    g = torch.Generator().manual_seed(3 * M + K + N + k)
    inp = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(dev)
    vals, idx, logits, mask, probs = pkg.ops.router_topk(inp, w, k, with_logits=True, with_mask=True,
                                                         with_probs=True)
    assert_bits_equal(logits, pkg.ops.router_logits(inp, w), "logits of the two entry points")
    rv, ri, rm, rp = pkg.ops.topk(logits, k, with_mask=True, with_probs=True)
    assert_bits_equal(vals, rv, "values")
    assert torch.equal(idx.cpu(), ri.cpu()), "indices"
    assert torch.equal(mask.cpu(), rm.cpu()), "mask"
    assert_bits_equal(probs, rp, "probs")
    # and the oracle's top-k of those logits (stable descending order)
    ov, oi = ref_torch.topk(logits.cpu(), k)
    assert torch.equal(oi, idx.cpu())
    assert_bits_equal(vals, ov, "values vs oracle")


def test_router_topk_without_optional_outputs(pkg, dev):
    inp = torch.randn(200, 256, device=dev).to(torch.bfloat16)
    w = torch.randn(64, 256, device=dev).to(torch.bfloat16)
    vals, idx = pkg.ops.router_topk(inp, w, 6)
    rv, ri = pkg.ops.topk(pkg.ops.router_logits(inp, w), 6)
    assert_bits_equal(vals, rv, "values")
    assert torch.equal(idx.cpu(), ri.cpu())
