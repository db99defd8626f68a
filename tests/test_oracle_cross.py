"""Pins the oracle where the reference's golden vectors stop (CPU).

Each check is chosen so that a plausible slip -- a dropped offset, a wrong
index or layout, a different summation order, a mishandled tie -- fails it:
  * brute force: explicit Python loops on tiny random inputs (with float32
    arithmetic step by step where rounding matters);
  * invariants of the construction (bijection onto [0, R), contiguous
    ascending blocks per expert);
  * agreement of the two independent restatements (eager torch, plain C);
  * closed forms (identity weights, power-of-two scaling, numpy float64 GEMM).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle_c, ref_torch


def _rand_mask(T, E, p, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(T, E, generator=g) < p


# ------------------------------------------------------------- row-id map
@pytest.mark.parametrize("T,E,p,seed", [(1, 1, 1.0, 0), (7, 3, 0.5, 1), (33, 8, 0.3, 2), (50, 9, 0.0, 3),
                                        (64, 5, 1.0, 4), (17, 64, 0.2, 5)])
def test_row_id_map_brute_force(T, E, p, seed):
    rm = _rand_mask(T, E, p, seed)
    expect = [[-1] * E for _ in range(T)]
    nxt = 0
    for e in range(E):
        for t in range(T):
            if rm[t, e]:
                expect[t][e] = nxt
                nxt += 1
    expect = torch.tensor(expect, dtype=torch.int64).reshape(T, E)
    em, tm = ref_torch.row_id_map(rm)
    assert torch.equal(tm, expect) and torch.equal(em, expect.t())
    row_c, offs_c = oracle_c.row_id_map(rm.numpy())
    assert np.array_equal(row_c, expect.numpy())
    assert np.array_equal(offs_c, ref_torch.expert_offsets(rm).numpy())


def test_row_id_map_invariants():
    rm = _rand_mask(2000, 37, 0.15, 11)
    em, tm = ref_torch.row_id_map(rm)
    R = int(rm.sum())
    assert torch.equal(tm[tm >= 0].sort().values, torch.arange(R))  # bijection onto [0, R)
    offs = ref_torch.expert_offsets(rm)
    for e in range(37):
        rows = em[e][em[e] >= 0]
        assert torch.equal(rows, torch.arange(int(offs[e]), int(offs[e + 1])))  # contiguous, ascending t
    assert torch.equal((tm >= 0), rm)


# ------------------------------------------------------------------ permute
@pytest.mark.parametrize("expert_major", [False, True])
def test_permute_brute_force(expert_major):
    T, E, H = 23, 6, 5
    rm = _rand_mask(T, E, 0.4, 21)
    em, tm = ref_torch.row_id_map(rm)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    probs = torch.rand(T, E, generator=g) * rm
    R = int(rm.sum())
    num_out = R + 3  # tail rows stay zero
    out = torch.zeros(num_out, H, dtype=torch.bfloat16)
    pp = torch.zeros(num_out)
    for t in range(T):
        for e in range(E):
            d = int(tm[t, e])
            if d >= 0:
                out[d] = x[t]
                pp[d] = probs[t, e]
    got, gpp = ref_torch.permute_token_major(x, tm, probs, num_out)
    assert torch.equal(got, out) and torch.equal(gpp, pp)
    m = em if expert_major else tm
    oc, ppc = oracle_c.permute(x.view(torch.int16).numpy(), m.numpy(), num_out, probs.numpy(),
                               expert_major=expert_major)
    assert np.array_equal(oc, out.view(torch.int16).numpy()) and np.array_equal(ppc, pp.numpy())
    if expert_major:
        o2, p2 = ref_torch.permute_expert_major(x, em, probs)
        assert torch.equal(o2, out[:R]) and torch.equal(p2, pp[:R])


# ---------------------------------------------------------------- unpermute
def _wide(R, H, g):
    """bf16 values spread over 2^-14 .. 2^14, so fp32 sums of a few of them round."""
    scale = torch.exp2(torch.randint(-14, 15, (R, H), generator=g).float())
    return (torch.randn(R, H, generator=g) * scale).to(torch.bfloat16)


def _brute_unpermute(pin, em, probs=None):
    """Ascending-expert fp32 sum, one numpy.float32 operation at a time."""
    E, T = em.shape
    H = pin.shape[1]
    pf = pin.float().numpy()
    acc = np.zeros((T, H), np.float32)
    for t in range(T):
        for h in range(H):
            a = np.float32(0.0)
            for e in range(E):
                s = int(em[e, t])
                if s < 0:
                    continue
                v = np.float32(pf[s, h])
                if probs is not None:
                    v = np.float32(np.float32(probs[t, e]) * v)
                a = np.float32(a + v)
            acc[t, h] = a
    return acc


@pytest.mark.parametrize("merge", [False, True])
def test_unpermute_brute_force(merge):
    T, E, H = 19, 7, 6
    rm = _rand_mask(T, E, 0.5, 31)
    em, tm = ref_torch.row_id_map(rm)
    g = torch.Generator().manual_seed(32)
    R = int(rm.sum())
    # wide per-element dynamic range so that a different summation order changes the rounding
    pin = _wide(R, H, g)
    probs = torch.rand(T, E, generator=g) * rm if merge else None
    acc = _brute_unpermute(pin, em, probs.numpy() if merge else None)
    out_bits = oracle_c.bf16_rne(acc)
    if merge:
        acc_t, out_t = ref_torch.unpermute_merge(pin, em, probs, with_acc=True)
        assert np.array_equal(acc_t.numpy(), acc)
        # token-major map gives the same order
        assert torch.equal(ref_torch.unpermute_merge(pin, tm, probs, expert_major=False), out_t)
    else:
        out_t = ref_torch.unpermute(pin, em)
        acc_l, out_l = ref_torch.unpermute_mask(pin, em.to(torch.int32))
        assert np.array_equal(acc_l.numpy(), acc) and torch.equal(out_l, out_t)
    assert np.array_equal(out_t.view(torch.int16).numpy().view(np.uint16), out_bits)
    out_c, acc_c = oracle_c.unpermute(pin.view(torch.int16).numpy().view(np.uint16), em.numpy(),
                                      probs.numpy() if merge else None)
    assert np.array_equal(acc_c, acc) and np.array_equal(out_c, out_bits)
    out_c2, _ = oracle_c.unpermute(pin.view(torch.int16).numpy().view(np.uint16), tm.numpy(),
                                   probs.numpy() if merge else None, expert_major=False)
    assert np.array_equal(out_c2, out_bits)


def test_unpermute_order_matters():
    # A reversed (descending-expert) sum must differ somewhere on these inputs, so the
    # brute-force comparison above does pin the order.
    T, E, H = 64, 8, 32
    rm = torch.ones(T, E, dtype=torch.bool)
    em, _ = ref_torch.row_id_map(rm)
    g = torch.Generator().manual_seed(5)
    pin = _wide(T * E, H, g)
    fwd = _brute_unpermute(pin, em)
    rev = _brute_unpermute(pin, em.flip(0))
    assert not np.array_equal(fwd, rev)


def test_permute_then_unpermute_is_k_times_x():
    # Closed form: every token goes to exactly k = 4 experts, so the unweighted sum of its
    # copies is 4 * x exactly (power-of-two scaling, no rounding).
    T, E, H = 40, 8, 16
    g = torch.Generator().manual_seed(9)
    idx = torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :4]
    rm = torch.zeros(T, E, dtype=torch.bool).scatter_(1, idx, True)
    em, tm = ref_torch.row_id_map(rm)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    xp, _ = ref_torch.permute_token_major(x, tm, torch.zeros(T, E), T * 4)
    assert torch.equal(ref_torch.unpermute(xp, em), (x.float() * 4).to(torch.bfloat16))


def test_permute_bwd_brute_force():
    T, E, H = 15, 5, 4
    rm = _rand_mask(T, E, 0.6, 41)
    em, _ = ref_torch.row_id_map(rm)
    g = torch.Generator().manual_seed(42)
    R = int(rm.sum())
    dperm = torch.randn(R, H, generator=g).to(torch.bfloat16)
    dpp = torch.randn(R, generator=g)
    dact, dprobs = ref_torch.permute_bwd(dperm, dpp, em)
    expect_p = torch.zeros(T, E)
    for t in range(T):
        for e in range(E):
            if em[e, t] >= 0:
                expect_p[t, e] = dpp[em[e, t]]
    assert torch.equal(dprobs, expect_p)
    acc = _brute_unpermute(dperm, em)
    assert np.array_equal(dact.view(torch.int16).numpy().view(np.uint16), oracle_c.bf16_rne(acc))
    acc2, _, gathered = ref_torch.unpermute_mask_probgrad(dperm, em.to(torch.int32), dpp)
    assert np.array_equal(acc2.numpy(), acc) and torch.equal(gathered, expect_p)


# -------------------------------------------------------------------- top-k
def _brute_topk(row, k):
    def key(i):
        v = float(row[i])
        if np.isnan(v):
            return (0, 0.0, i)  # NaN first
        return (1, -v, i)  # larger value first, then smaller index (-0 == +0)
    order = sorted(range(len(row)), key=key)[:k]
    return [row[i] for i in order], order


@pytest.mark.parametrize("kind", ["randn", "ties", "zeros", "neg", "ninf", "nan", "signed_zero"])
def test_topk_brute_force(kind):
    g = torch.Generator().manual_seed(len(kind) * 101)
    T, E, k = 12, 20, 6
    if kind == "randn":
        x = torch.randn(T, E, generator=g)
    elif kind == "ties":
        x = torch.randint(0, 3, (T, E), generator=g).float()
    elif kind == "zeros":
        x = torch.zeros(T, E)
    elif kind == "neg":
        x = -torch.rand(T, E, generator=g)
    elif kind == "ninf":
        x = torch.randn(T, E, generator=g)
        x[:, :15] = float("-inf")
    elif kind == "nan":
        x = torch.randn(T, E, generator=g)
        x[::2, 3] = float("nan")
        x[::3, 11] = float("nan")
    else:
        x = torch.zeros(T, E)
        x[:, ::2] = -0.0
        x[:, 5] = 1.0
    v, i = ref_torch.topk(x, k)
    vc, ic = oracle_c.topk(x.numpy(), k)
    for t in range(T):
        bv, bi = _brute_topk(x[t].tolist(), k)
        assert i[t].tolist() == bi, (kind, t)
        assert ic[t].tolist() == bi, (kind, t)
        assert np.array_equal(v[t].numpy().view(np.int32), np.array(bv, np.float32).view(np.int32))
        assert np.array_equal(vc[t].view(np.int32), np.array(bv, np.float32).view(np.int32))


def test_mask_and_probs_closed_form():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(10, 8, generator=g)
    v, i = ref_torch.topk(logits, 3)
    rm, probs = ref_torch.mask_and_probs(v, i, 8)
    assert torch.equal(rm.sum(1), torch.full((10,), 3))
    ex = np.exp(v.double().numpy() - v.double().numpy()[:, :1])
    p64 = ex / ex.sum(1, keepdims=True)
    for t in range(10):
        for j in range(3):
            assert abs(float(probs[t, i[t, j]]) - p64[t, j]) < 1e-6
        assert abs(float(probs[t].sum()) - 1.0) < 1e-6


# ------------------------------------------------------------- grouped GEMM
def test_grouped_gemm_fp32_against_float64():
    g = torch.Generator().manual_seed(51)
    sizes = [5, 0, 17, 1]
    K, N = 24, 10
    x = torch.randn(sum(sizes), K, generator=g).to(torch.bfloat16)
    w = torch.randn(len(sizes), N, K, generator=g).to(torch.bfloat16)
    got = ref_torch.grouped_gemm_fp32(x, w, sizes)
    xs, ws = x.double().numpy(), w.double().numpy()
    off = 0
    for gi, m in enumerate(sizes):
        ref = xs[off:off + m] @ ws[gi].T
        assert np.allclose(got[off:off + m].numpy(), ref, rtol=1e-5, atol=1e-5)
        off += m
    # bf16 per-group torch.mm form stays within the bf16 tolerance of the fp32 golden
    bf = ref_torch.grouped_gemm(x, w, sizes)
    torch.testing.assert_close(bf.float(), got, rtol=1.6e-2, atol=1e-2)


def test_grouped_gemm_identity_weights_exact():
    sizes = [3, 4]
    x = torch.randn(7, 16).to(torch.bfloat16)
    w = torch.stack([torch.eye(16), 2 * torch.eye(16)]).to(torch.bfloat16)
    got = ref_torch.grouped_gemm_fp32(x, w, sizes)
    assert torch.equal(got[:3], x[:3].float()) and torch.equal(got[3:], 2 * x[3:].float())


def test_grouped_gemm_dgrad_fp32_against_float64():
    # Brute force in float64 per group; a transposed w or a dropped group fails it.
    g = torch.Generator().manual_seed(52)
    sizes = [5, 0, 17, 1]
    N, K = 24, 10
    dy = torch.randn(sum(sizes), N, generator=g).to(torch.bfloat16)
    w = torch.randn(len(sizes), N, K, generator=g).to(torch.bfloat16)
    got = ref_torch.grouped_gemm_dgrad_fp32(dy, w, sizes)
    assert got.shape == (sum(sizes), K)
    d, ws = dy.double().numpy(), w.double().numpy()
    off = 0
    for gi, m in enumerate(sizes):
        for r in range(m):
            for c in range(K):
                ref = sum(d[off + r, n] * ws[gi, n, c] for n in range(N))
                assert abs(float(got[off + r, c]) - ref) <= 1e-5 * (1 + abs(ref))
        off += m
    bf = ref_torch.grouped_gemm_dgrad(dy, w, sizes)
    torch.testing.assert_close(bf.float(), got, rtol=1.6e-2, atol=1e-2)


def test_grouped_gemm_dgrad_is_forward_with_transposed_weights():
    # dgrad(dy, w) = forward(dy, w^T): ties the dgrad oracle to the pinned forward one.
    g = torch.Generator().manual_seed(53)
    sizes = [3, 9, 0, 4]
    N, K = 16, 24
    dy = torch.randn(sum(sizes), N, generator=g).to(torch.bfloat16)
    w = torch.randn(len(sizes), N, K, generator=g).to(torch.bfloat16)
    a = ref_torch.grouped_gemm_dgrad_fp32(dy, w, sizes)
    b = ref_torch.grouped_gemm_fp32(dy, w.transpose(1, 2).contiguous(), sizes)
    torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


def test_grouped_gemm_wgrad_fp32_against_float64():
    # Sum of per-row outer products in float64; an empty group must come out zero.
    g = torch.Generator().manual_seed(54)
    sizes = [5, 0, 11, 1]
    N, K = 12, 8
    dy = torch.randn(sum(sizes), N, generator=g).to(torch.bfloat16)
    x = torch.randn(sum(sizes), K, generator=g).to(torch.bfloat16)
    got = ref_torch.grouped_gemm_wgrad_fp32(dy, x, sizes)
    assert got.shape == (len(sizes), N, K)
    d, xs = dy.double().numpy(), x.double().numpy()
    off = 0
    for gi, m in enumerate(sizes):
        ref = np.zeros((N, K))
        for r in range(off, off + m):
            ref += np.outer(d[r], xs[r])
        assert np.allclose(got[gi].numpy(), ref, rtol=1e-5, atol=1e-5)
        off += m
    assert torch.count_nonzero(got[1]) == 0
    bf = ref_torch.grouped_gemm_wgrad(dy, x, sizes)
    torch.testing.assert_close(bf.float(), got, rtol=1.6e-2, atol=1e-2)


def test_grouped_gemm_wgrad_closed_forms():
    # One row per group: dw[g] is the outer product of that row (exact in fp32 for bf16 inputs);
    # one group over all rows: dw[0] = dy^T x.
    g = torch.Generator().manual_seed(55)
    dy = torch.randn(3, 8, generator=g).to(torch.bfloat16)
    x = torch.randn(3, 16, generator=g).to(torch.bfloat16)
    got = ref_torch.grouped_gemm_wgrad_fp32(dy, x, [1, 1, 1])
    for r in range(3):
        assert torch.equal(got[r], torch.outer(dy[r].float(), x[r].float()))
    whole = ref_torch.grouped_gemm_wgrad_fp32(dy, x, [3])
    torch.testing.assert_close(whole[0], got.sum(0), rtol=1e-6, atol=1e-6)


def test_router_logits_fp32_against_explicit_sum():
    # The case's own check (explicit broadcast sum, case38...:64-79) and float64, on small shapes.
    g = torch.Generator().manual_seed(56)
    inp = torch.randn(5, 40, generator=g).to(torch.bfloat16)
    w = torch.randn(7, 40, generator=g).to(torch.bfloat16)
    got = ref_torch.router_logits_fp32(inp, w)
    manual = (inp.float().unsqueeze(-1) * w.float().t().unsqueeze(0)).sum(dim=1)
    assert (got - manual).abs().max().item() <= 1e-4
    ref = inp.double().numpy() @ w.double().numpy().T
    assert np.allclose(got.numpy(), ref, rtol=1e-6, atol=1e-5)
    assert got.shape == (5, 7) and got.dtype == torch.float32


def test_round_tf32_known_answers_and_bound():
    # The case's own tie checks (case39...:70-79): 1.0 + half ulp stays, 1.0 + 1.5 ulp rounds up.
    ties = torch.tensor([0x3F801000, 0x3F803000], dtype=torch.int32).view(torch.float32)
    got = ref_torch.round_tf32_rne(ties).view(torch.int32).tolist()
    assert got == [0x3F800000, 0x3F804000]
    # Independent restatement: nearest multiple of 2^(e-10) (ties to even) via float64.
    g = torch.Generator().manual_seed(57)
    x = torch.randn(20000, generator=g) * torch.exp(torch.randn(20000, generator=g) * 5)
    r = ref_torch.round_tf32_rne(x)
    assert bool(((r.view(torch.int32) & 0x1FFF) == 0).all())
    xd = x.double().numpy()
    e = np.floor(np.log2(np.abs(xd)))
    q = 2.0 ** (e - 10)
    ref = np.round(xd / q) * q   # numpy rounds half to even
    assert np.array_equal(r.double().numpy(), ref)


def test_router_tf32_gemms_against_float64():
    g = torch.Generator().manual_seed(58)
    a = torch.randn(9, 24, generator=g)
    b = torch.randn(24, 16, generator=g)
    got = ref_torch.router_dgrad_tf32(a, b)
    ref = ref_torch.round_tf32_rne(a).double().numpy() @ ref_torch.round_tf32_rne(b).double().numpy()
    assert np.allclose(got.numpy(), ref, rtol=1e-6, atol=1e-5)
    x = torch.randn(9, 16, generator=g)
    got = ref_torch.router_wgrad_tf32(a, x)
    ref = ref_torch.round_tf32_rne(a).double().numpy().T @ ref_torch.round_tf32_rne(x).double().numpy()
    assert got.shape == (24, 16) and np.allclose(got.numpy(), ref, rtol=1e-6, atol=1e-5)


def test_swiglu_closed_form():
    y = torch.tensor([[0.0, 1.0, 2.0, -3.0], [-1.0, 4.0, 0.5, 0.25]])
    h = ref_torch.swiglu(y).double().numpy()
    g, u = y[:, :2].double().numpy(), y[:, 2:].double().numpy()
    assert np.allclose(h, g / (1 + np.exp(-g)) * u, rtol=1e-6, atol=1e-7)


def test_index_select_against_numpy():
    g = torch.Generator().manual_seed(61)
    src = torch.randn(6, 3, 5, generator=g).to(torch.bfloat16)
    idx = torch.tensor([5, 0, 0, 2], dtype=torch.int32)
    got = ref_torch.index_select(src, idx)
    assert torch.equal(got.view(torch.int16), torch.from_numpy(np.take(src.view(torch.int16).numpy(), idx.numpy(), 0)))
    assert np.array_equal(oracle_c.index_select(src.view(torch.int16).numpy(), idx.numpy()),
                          got.view(torch.int16).numpy())


def test_moe_ffn_composition_tiny():
    # The composed oracle equals the stage-by-stage brute force on a tiny layer.
    g = torch.Generator().manual_seed(71)
    T, H, F, E, k = 9, 8, 4, 4, 2
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    w1 = (torch.randn(E, 2 * F, H, generator=g) * 0.5).to(torch.bfloat16)
    w2 = (torch.randn(E, H, F, generator=g) * 0.5).to(torch.bfloat16)
    out = ref_torch.moe_ffn_forward(x, logits, w1, w2, k)
    v, i = ref_torch.topk(logits, k)
    _, probs = ref_torch.mask_and_probs(v, i, E)
    expect = torch.zeros(T, H)
    for t in range(T):
        acc = torch.zeros(H)
        for e in sorted(i[t].tolist()):
            y = (x[t:t + 1] @ w1[e].t()).float()  # per-row bf16 mm as the grouped form computes it
            hh = ref_torch.swiglu(y).to(torch.bfloat16)
            z = (hh @ w2[e].t()).float()[0]
            acc = acc + probs[t, e] * z
        expect[t] = acc
    torch.testing.assert_close(out.float(), expect, rtol=2e-2, atol=2e-2)


def test_moe_ffn_fp32_composition_against_float64_brute_force():
    # The fp32-GEMM layer oracle equals a per-token float64 loop (bf16 roundings of h and z at the
    # same points), and a subset of tokens gives those tokens' rows of the full layer.
    g = torch.Generator().manual_seed(73)
    T, H, F, E, k = 23, 16, 8, 6, 3
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g) + torch.randn(E, generator=g) * 1.5
    w1 = (torch.randn(E, 2 * F, H, generator=g) * 0.5).to(torch.bfloat16)
    w2 = (torch.randn(E, H, F, generator=g) * 0.5).to(torch.bfloat16)
    out = ref_torch.moe_ffn_forward_fp32(x, logits, w1, w2, k)
    v, i = ref_torch.topk(logits, k)
    _, probs = ref_torch.mask_and_probs(v, i, E)
    expect = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        for e in sorted(i[t].tolist()):
            y = x[t].double() @ w1[e].double().t()
            gate, up = y[:F], y[F:]
            hh = (gate * torch.sigmoid(gate) * up).to(torch.bfloat16)
            z = (hh.double() @ w2[e].double().t()).to(torch.bfloat16)
            expect[t] += probs[t, e].double() * z.double()
    torch.testing.assert_close(out.double(), expect, rtol=1e-2, atol=1e-2)
    sub = torch.tensor([0, 5, 17, 22])
    assert torch.equal(ref_torch.moe_ffn_forward_fp32(x[sub], logits[sub], w1, w2, k), out[sub])


def test_source_tokens_inverts_the_map_and_feeds_the_permute():
    # Brute-force double loop, and the permute relation x[src] == permuted rows.
    g = torch.Generator().manual_seed(79)
    T, E, k, H = 40, 7, 3, 5
    sel = torch.rand(T, E, generator=g).argsort(dim=1)[:, :k]
    mask = torch.zeros(T, E, dtype=torch.bool).scatter_(1, sel, True)
    mask[3] = False
    _, tm = ref_torch.row_id_map(mask)
    R = int(mask.sum())
    src = ref_torch.source_tokens(tm, R + 4)
    brute = torch.full((R + 4,), -1, dtype=torch.int32)
    for t in range(T):
        for e in range(E):
            if tm[t, e] >= 0:
                brute[tm[t, e]] = t
    assert torch.equal(src, brute) and bool((src[:R] >= 0).all()) and bool((src[R:] == -1).all())
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    xp, _ = ref_torch.permute_token_major(x, tm, torch.zeros(T, E), R)
    assert torch.equal(x[src[:R].long()], xp)
