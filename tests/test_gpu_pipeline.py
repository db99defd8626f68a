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
    # Merge with probs summing to 1: within bf16 rounding of x; bit-exact vs the oracle on every token
    # (the oracle runs on the host in chunks of 1024 tokens; each token's sum depends on its own map column).
    merged = pkg.ops.unpermute(xp, maps["token_major"], probs, layout="token_major")
    torch.testing.assert_close(merged.float(), x.float(), rtol=1.6e-2, atol=1e-2)
    xp_c, em_c, probs_c, merged_c = xp.cpu(), maps["expert_major"].cpu(), probs.cpu(), merged.cpu()
    # Permute backward with the seeded grad: dact and dprobs equal the oracle on every token.
    grad = pkg.inputs.randn_bf16((T * k, H), seed=20261212, device=dev)
    dpp = torch.randn(T * k, generator=torch.Generator(device=dev).manual_seed(5), device=dev)
    dact, dprobs = pkg.ops.permute_bwd(grad, dpp, maps["expert_major"], layout="expert_major")
    grad_c, dpp_c, dact_c, dprobs_c = grad.cpu(), dpp.cpu(), dact.cpu(), dprobs.cpu()
    for t0 in range(0, T, 1024):
        sl = slice(t0, t0 + 1024)
        ref = ref_torch.unpermute_merge(xp_c, em_c[:, sl], probs_c[sl])
        assert_bits_equal(merged_c[sl], ref, f"c2 merge tokens {t0}..")
        ref_dact, ref_dprobs = ref_torch.permute_bwd(grad_c, dpp_c, em_c[:, sl])
        assert_bits_equal(dact_c[sl], ref_dact, f"c2 dact tokens {t0}..")
        assert_bits_equal(dprobs_c[sl], ref_dprobs, f"c2 dprobs tokens {t0}..")


def _c5_sample(mask: torch.Tensor, n: int, seed: int) -> torch.Tensor:
    """n token ids: the first and the last token of every expert's group (its rows in the
    permuted order start and end there), the rest drawn at random."""
    picks = set()
    for e in range(mask.shape[1]):
        toks = mask[:, e].nonzero().squeeze(1)
        if toks.numel():
            picks.update((int(toks[0]), int(toks[-1])))
    g = torch.Generator().manual_seed(seed)
    for t in torch.randperm(mask.shape[0], generator=g).tolist():
        if len(picks) >= n:
            break
        picks.add(t)
    return torch.tensor(sorted(picks))


def test_config_c5_layer_matches_oracle(pkg, dev):
    # c5 full layer: routing exact against the oracle; the output of 1024 tokens (covering
    # both group ends of every expert the skewed router gives tokens) against the oracle's fp32-GEMM layer
    # recomputed on the host for those tokens, at the task's bf16 tolerance.
    c = pkg.inputs.CONFIGS["c5"]
    T, H, E, k, F = c["tokens"], c["hidden"], c["experts"], c["topk"], c["ffn"]
    x = pkg.inputs.randn_bf16((T, H), seed=20261205, device=dev)
    logits = pkg.inputs.router_logits(T, E, skew=c["skew"], seed=20261205, device=dev)
    w1 = pkg.inputs.randn_bf16((E, 2 * F, H), std=0.02, seed=20261215, device=dev)
    w2 = pkg.inputs.randn_bf16((E, H, F), std=0.02, seed=20261225, device=dev)
    layer = pkg.moe_ffn.MoEFFN(w1, w2, k)
    out = layer(x, logits)
    logits_c = logits.cpu()
    v, i = ref_torch.topk(logits_c, k)
    rm, _ = ref_torch.mask_and_probs(v, i, E)
    assert torch.equal(layer.last["mask"].cpu(), rm)
    _, tm = ref_torch.row_id_map(rm)
    assert torch.equal(layer.last["row_map"].cpu(), tm)
    sample = _c5_sample(rm, 1024, seed=5)
    used = rm.any(0)
    assert sample.numel() == 1024 and torch.equal(rm[sample].any(0), used), "every expert with tokens is covered"
    assert int(used.sum()) >= E // 2
    ref = ref_torch.moe_ffn_forward_fp32(x.cpu()[sample], logits_c[sample], w1.cpu(), w2.cpu(), k)
    torch.testing.assert_close(out.cpu()[sample].float(), ref.float(), rtol=1.6e-2, atol=1e-2)


def test_moe_ffn_output_survives_a_second_call(pkg, dev):
    # Each forward returns a new tensor (or the caller's out=): a second call with other
    # inputs leaves the first result untouched.
    g = torch.Generator().manual_seed(13)
    T, H, F, E, k = 256, 256, 128, 8, 2
    w1 = (torch.randn(E, 2 * F, H, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    w2 = (torch.randn(E, H, F, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    layer = pkg.moe_ffn.MoEFFN(w1, w2, k)
    x1, x2 = (torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(2))
    l1, l2 = (torch.randn(T, E, generator=g).to(dev) for _ in range(2))
    y1 = layer(x1, l1)
    y1_copy = y1.clone()
    y2 = layer(x2, l2)
    torch.cuda.synchronize()
    assert y1.data_ptr() != y2.data_ptr()
    assert torch.equal(y1, y1_copy)
    out = torch.empty_like(y1)
    assert layer(x1, l1, out=out) is out
    assert torch.equal(out, y1_copy)
