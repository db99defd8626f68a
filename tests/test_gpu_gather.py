"""GPU: source-token index of permuted rows and the grouped GEMM that gathers its
A rows through it (the permute fused into fc1).

The gather GEMM must equal the plain grouped GEMM on the materialised rows bit
for bit (same tiles, same accumulation order), and within the bf16 tolerance of
the fp32 oracle; the index must be the exact inverse of the row-id map.
"""
from __future__ import annotations

import pytest
import torch

from oracle import ref_torch

pytestmark = pytest.mark.gpu


def _inverse(row_map_tm: torch.Tensor, num_out: int) -> torch.Tensor:
    """Brute-force inverse of a token-major map on the CPU (-1 where unnamed)."""
    inv = torch.full((num_out,), -1, dtype=torch.int32)
    T, E = row_map_tm.shape
    for t in range(T):
        for e in range(E):
            r = int(row_map_tm[t, e])
            if 0 <= r < num_out:
                inv[r] = t
    return inv


@pytest.mark.parametrize("layout", ["token_major", "expert_major"])
@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_permute_index_inverts_map(pkg, dev, layout, dtype):
    g = torch.Generator().manual_seed(7)
    T, E, k = 300, 12, 3
    sel = torch.rand(T, E, generator=g).argsort(dim=1)[:, :k]
    mask = torch.zeros(T, E, dtype=torch.bool).scatter_(1, sel, True)
    mask[5] = False                                   # a token routed nowhere
    em, tm = ref_torch.row_id_map(mask)
    R = int(mask.sum())
    m = (tm if layout == "token_major" else em).to(dtype)
    got = pkg.ops.permute_index(m.to(dev), R, layout=layout).cpu()
    assert torch.equal(got, _inverse(tm, R))
    # num_out larger than the routed rows: the tail stays -1 with fill, the map rows are set
    got2 = pkg.ops.permute_index(m.to(dev), R + 37, layout=layout, fill=True).cpu()
    assert torch.equal(got2, _inverse(tm, R + 37))
    assert torch.equal(got2[R:], torch.full((37,), -1, dtype=torch.int32))


def test_permute_index_c5_size(pkg, dev):
    c = pkg.inputs.CONFIGS["c5"]
    T, E, k = c["tokens"], c["experts"], c["topk"]
    logits = pkg.inputs.router_logits(T, E, skew=c["skew"], seed=20261205, device=dev)
    _, _, mask = pkg.ops.topk(logits, k, with_mask=True)
    tm = pkg.ops.row_id_map(mask, expert_major=False, token_major=True)["token_major"]
    src = pkg.ops.permute_index(tm, T * k)
    # inverse property at full size: map[src[p], e] == p for the expert owning row p
    rows = torch.arange(T * k, device=dev)
    assert bool((src >= 0).all())
    assert bool((tm[src.long()] == rows[:, None]).any(dim=1).all())
    # and every token appears exactly k times
    assert bool((torch.bincount(src.long(), minlength=T) == k).all())


@pytest.mark.parametrize("sizes,K,N,swiglu", [
    ([300, 0, 17, 513], 200, 264, False),   # ragged, empty group, K and N tails
    ([64, 700], 7168, 4096, True),          # fc1 shape class
    ([256, 256], 2048, 512, False),
])
def test_grouped_gemm_gather_matches_materialised(pkg, dev, sizes, K, N, swiglu):
    g = torch.Generator().manual_seed(sum(sizes) + K + N + swiglu)
    X = 523
    M = sum(sizes)
    x = torch.randn(X, K, generator=g).to(torch.bfloat16)
    rows = torch.randint(0, X, (M,), generator=g, dtype=torch.int32)
    rows[3] = -1                                      # out of range: a zero row
    rows[7] = X + 5
    w = (torch.randn(len(sizes), N, K, generator=g) * 0.05).to(torch.bfloat16)
    offs = pkg.ops.group_offsets_from_splits(sizes, dev)
    xd, rd, wd = x.to(dev), rows.to(dev), w.to(dev)
    got = pkg.ops.grouped_gemm_gather(xd, rd, wd, offs, swiglu=swiglu)
    a = torch.zeros(M, K, dtype=torch.bfloat16)
    ok = (rows >= 0) & (rows < X)
    a[ok] = x[rows[ok].long()]
    plain = pkg.ops.grouped_gemm(a.to(dev), wd, offs, swiglu=swiglu)
    assert torch.equal(got.view(torch.int16), plain.view(torch.int16))
    ref = ref_torch.grouped_gemm_fp32(a, w, sizes)
    if swiglu:
        ref = ref_torch.swiglu(ref)
    torch.testing.assert_close(got.float().cpu(), ref.float(), rtol=1.6e-2, atol=1e-2)


def test_moe_ffn_fused_permute_equals_unfused(pkg, dev):
    g = torch.Generator().manual_seed(13)
    T, H, F, E, k = 700, 512, 256, 16, 4
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    logits = (torch.randn(T, E, generator=g) + torch.randn(E, generator=g) * 1.5).to(dev)
    w1 = (torch.randn(E, 2 * F, H, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    w2 = (torch.randn(E, H, F, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    fused = pkg.moe_ffn.MoEFFN(w1, w2, k)(x, logits).clone()
    unfused = pkg.moe_ffn.MoEFFN(w1, w2, k, fused_permute=False)(x, logits)
    assert torch.equal(fused.view(torch.int16), unfused.view(torch.int16))
