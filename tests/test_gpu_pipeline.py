"""GPU: the composed MoE FFN forward, and size-independent properties at the
benchmark sizes (configs c1 / c2 / c5)."""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bits_equal
from oracle import ref_torch

pytestmark = pytest.mark.gpu


def test_moe_ffn_small_matches_oracle(pkg, dev):
    g = torch.Generator().manual_seed(11)
    T, H, F, E, k = 300, 512, 256, 16, 4
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g) + torch.randn(E, generator=g) * 1.5
    w1 = (torch.randn(E, 2 * F, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, F, generator=g) * 0.02).to(torch.bfloat16)
    layer = pkg.moe_ffn.MoEFFN(w1.to(dev), w2.to(dev), k)
    out = layer(x.to(dev), logits.to(dev)).cpu()
    ref = ref_torch.moe_ffn_forward(x, logits, w1, w2, k)
    torch.testing.assert_close(out.float(), ref.float(), rtol=1.6e-2, atol=1e-2)


def test_config_c1_row_id_map_and_permute(pkg, dev):
    # c1: T=4096, H=2048, E=8, top-2; int32 [8, 4096] map and the [8192, 2048] permuted x, bit-exact.
    c = pkg.inputs.CONFIGS["c1"]
    logits = pkg.inputs.router_logits(c["tokens"], c["experts"], skew=c["skew"], seed=20261201)
    x = pkg.inputs.randn_bf16((c["tokens"], c["hidden"]), seed=20261201)
    _, _, mask, probs = pkg.ops.topk(logits.to(dev), c["topk"], with_mask=True, with_probs=True)
    maps = pkg.ops.row_id_map(mask, expert_major_i32=True, expert_offsets=True)
    v, i = ref_torch.topk(logits, c["topk"])
    rm, rp = ref_torch.mask_and_probs(v, i, c["experts"])
    em, tm = ref_torch.row_id_map(rm)
    assert maps["expert_major_i32"].shape == (8, 4096)
    assert_bits_equal(maps["expert_major_i32"], em.to(torch.int32), "c1 int32 map")
    out, pp = pkg.cases.case17_moe_permute_with_mask_map.kernel_function(x.to(dev), maps["token_major"], probs)
    ref_out, ref_pp = ref_torch.permute_token_major(x, tm, probs.cpu(), 8192)
    assert out.shape == (8192, 2048)
    assert_bits_equal(out, ref_out, "c1 permuted x")
    assert_bits_equal(pp, ref_pp, "c1 permuted probs")


def test_config_c2_round_trip_and_merge(pkg, dev):
    # c2: T=8192, H=7168, E=64, top-8 with skewed routing.
    c = pkg.inputs.CONFIGS["c2"]
    T, H, E, k = c["tokens"], c["hidden"], c["experts"], c["topk"]
    logits = pkg.inputs.router_logits(T, E, skew=c["skew"], seed=20261202, device=dev)
    x = pkg.inputs.randn_bf16((T, H), seed=20261202, device=dev)
    _, _, mask, probs = pkg.ops.topk(logits, k, with_mask=True, with_probs=True)
    maps = pkg.ops.row_id_map(mask, expert_offsets=True)
    xp, _ = pkg.ops.permute(x, maps["token_major"], num_out=T * k, layout="token_major", zero_tail=False)
    # Round trip: unweighted combine of the k copies is exactly k * x (k = 8, a power of two).
    back = pkg.ops.unpermute(xp, maps["expert_major"], layout="expert_major")
    assert torch.equal(back, (x.float() * k).to(torch.bfloat16))
    # Expert blocks: rows offsets[e]..offsets[e+1] of xp are the tokens of expert e in order.
    offs = maps["expert_offsets"].cpu()
    assert int(offs[-1]) == T * k
    for e in (0, E // 2, E - 1):
        toks = mask[:, e].nonzero().squeeze(1)
        assert torch.equal(xp[int(offs[e]):int(offs[e + 1])], x[toks])
    # Merge with probs summing to 1: within bf16 rounding of x; bit-exact vs the oracle on a slice.
    merged = pkg.ops.unpermute(xp, maps["token_major"], probs, layout="token_major")
    torch.testing.assert_close(merged.float(), x.float(), rtol=1.6e-2, atol=1e-2)
    sl = slice(0, 512)
    em_slice = maps["expert_major"][:, sl].cpu()
    rows = em_slice[em_slice >= 0]
    ref = ref_torch.unpermute_merge(xp.cpu(), maps["expert_major"][:, sl].cpu(), probs[sl].cpu())
    assert rows.numel() == 512 * k
    assert_bits_equal(merged[sl], ref, "c2 merge slice")
    # Permute backward with the seeded grad: dact equals the oracle on the same slice.
    grad = pkg.inputs.randn_bf16((T * k, H), seed=20261212, device=dev)
    dpp = torch.randn(T * k, generator=torch.Generator(device=dev).manual_seed(5), device=dev)
    dact, dprobs = pkg.ops.permute_bwd(grad, dpp, maps["expert_major"], layout="expert_major")
    ref_dact, ref_dprobs = ref_torch.permute_bwd(grad.cpu(), dpp.cpu(), maps["expert_major"][:, sl].cpu())
    assert_bits_equal(dact[sl], ref_dact, "c2 dact slice")
    assert_bits_equal(dprobs[sl], ref_dprobs, "c2 dprobs slice")


def test_config_c5_layer_properties(pkg, dev):
    # c5 full layer: run once; routing is checked exactly against the oracle, the output
    # on a token sample against an fp32 recomputation of those tokens.
    c = pkg.inputs.CONFIGS["c5"]
    T, H, E, k, F = c["tokens"], c["hidden"], c["experts"], c["topk"], c["ffn"]
    x = pkg.inputs.randn_bf16((T, H), seed=20261205, device=dev)
    logits = pkg.inputs.router_logits(T, E, skew=c["skew"], seed=20261205, device=dev)
    w1 = pkg.inputs.randn_bf16((E, 2 * F, H), std=0.02, seed=20261215, device=dev)
    w2 = pkg.inputs.randn_bf16((E, H, F), std=0.02, seed=20261225, device=dev)
    layer = pkg.moe_ffn.MoEFFN(w1, w2, k)
    out = layer(x, logits)
    v, i = ref_torch.topk(logits.cpu(), k)
    rm, _ = ref_torch.mask_and_probs(v, i, E)
    assert torch.equal(layer.last["mask"].cpu(), rm)
    _, tm = ref_torch.row_id_map(rm)
    assert torch.equal(layer.last["row_map"].cpu(), tm)
    probs = layer.last["probs"]
    for t in (0, 1, T // 2, T - 1):
        acc = torch.zeros(H, device=dev)
        for e in sorted(i[t].tolist()):
            y = x[t:t + 1].float() @ w1[e].float().t()
            hh = ref_torch.swiglu(y).to(torch.bfloat16).float()
            acc += probs[t, e] * (hh @ w2[e].float().t())[0]
        torch.testing.assert_close(out[t].float(), acc, rtol=2e-2, atol=2e-2)
