"""GPU parity of the dispatch kernels against the oracle (bit-exact).

Row-id map, permute, unpermute (plain and merge), permute backward, top-k and
index_select, through the C ABI, on seeded inputs, including the edge cases the
reference tests (empty / ragged inputs, experts with no tokens, expert-major
and token-major maps, int32 and int64 maps, rows that are not a multiple of
16 bytes, ties / -inf / NaN in top-k).
"""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bits_equal
from oracle import ref_torch

pytestmark = pytest.mark.gpu


def _mask(T, E, k=None, p=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    if k is not None:
        idx = torch.argsort(torch.rand(T, E, generator=g), dim=1)[:, :k]
        return torch.zeros(T, E, dtype=torch.bool).scatter_(1, idx, True)
    return torch.rand(T, E, generator=g) < p


# ------------------------------------------------------------- row-id map
@pytest.mark.parametrize("T,E,k,p", [
    (1, 1, 1, None), (63, 3, None, 0.5), (64, 8, 2, None), (65, 7, None, 0.3), (1000, 130, None, 0.04),
    (4096, 8, 2, None), (16384, 64, 8, None), (300, 5, None, 0.0), (257, 1024, None, 0.01),
    (200, 48, 4, None), (70, 2000, None, 0.01), (33, 4096, None, 0.002), (5000, 160, 8, None),
    # more than 4096 chunks of 64 tokens: the column scan carries its sums across rounds
    (270000, 4, 1, None), (300001, 6, None, 0.3),
])
def test_row_id_map_matches_oracle(pkg, dev, T, E, k, p):
    rm = _mask(T, E, k, p, seed=T + E)
    R = int(rm.sum())
    src = torch.full((R + 5,), -7, dtype=torch.int32, device=dev)
    r = pkg.ops.row_id_map(rm.to(dev), expert_major=True, token_major=True, expert_major_i32=True,
                           expert_offsets=True, src_out=src)
    em, tm = ref_torch.row_id_map(rm)
    assert_bits_equal(r["expert_major"], em, "expert-major map")
    assert_bits_equal(r["token_major"], tm, "token-major map")
    assert_bits_equal(r["expert_major_i32"], em.to(torch.int32), "int32 map")
    assert_bits_equal(r["expert_offsets"], ref_torch.expert_offsets(rm), "expert offsets")
    # source token of every permuted row; rows past R are left as they were
    assert_bits_equal(r["src_token"][:R], ref_torch.source_tokens(tm, R), "source tokens")
    assert bool((r["src_token"][R:] == -7).all())
    # only the source index (no map output): same rows, and a capacity below R writes the rows below it
    r2 = pkg.ops.row_id_map(rm.to(dev), expert_major=False, token_major=False, src_rows=max(R // 2, 0))
    assert_bits_equal(r2["src_token"], ref_torch.source_tokens(tm, max(R // 2, 0)), "source tokens, half")


def test_row_id_map_reference_case12_full(pkg, dev):
    case = pkg.cases.case12_moe_row_id_map_pass2
    rm = case.make_routing_map()
    em, tm = case.kernel_function(rm.to(dev))
    ref_em, ref_tm = ref_torch.row_id_map(rm)
    assert_bits_equal(em, ref_em, "case12 [E,T]")
    assert_bits_equal(tm, ref_tm, "case12 [T,E]")
    R = int(rm.sum())
    r = pkg.ops.row_id_map(rm.to(dev), expert_major=False, token_major=False, expert_offsets=True, src_rows=R)
    assert_bits_equal(r["src_token"], ref_torch.source_tokens(ref_tm, R), "case12 source tokens")
    assert_bits_equal(r["expert_offsets"], ref_torch.expert_offsets(rm), "case12 offsets")


def test_row_id_map_empty(pkg, dev):
    r = pkg.ops.row_id_map(torch.zeros(0, 5, dtype=torch.bool, device=dev), expert_offsets=True)
    assert r["expert_major"].shape == (5, 0) and r["token_major"].shape == (0, 5)
    assert torch.equal(r["expert_offsets"].cpu(), torch.zeros(6, dtype=torch.int32))


# ------------------------------------------------------------------ permute
@pytest.mark.parametrize("layout", ["token_major", "expert_major"])
@pytest.mark.parametrize("idx", [torch.int64, torch.int32])
# E <= 64: map read per wavefront; 64 < E <= 1024: staged in LDS once per workgroup (vector and scalar rows,
# partial last workgroup); E > 1024: per-wavefront reads again.
@pytest.mark.parametrize("T,E,k,H", [(300, 8, 2, 2048), (129, 64, 8, 7168), (70, 320, 6, 136), (33, 5, 3, 13),
                                     (23, 200, 5, 13), (41, 1100, 4, 64)])
def test_permute_matches_oracle(pkg, dev, layout, idx, T, E, k, H):
    rm = _mask(T, E, k, seed=3 * T + E)
    em, tm = ref_torch.row_id_map(rm)
    g = torch.Generator().manual_seed(T * H)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    probs = torch.rand(T, E, generator=g) * rm
    R = T * k
    for num_out, zero_tail in ((R, False), (R + 5, True)):
        m = (tm if layout == "token_major" else em).to(idx)
        out, pp = pkg.ops.permute(x.to(dev), m.to(dev), probs.to(dev), num_out=num_out, layout=layout,
                                  zero_tail=zero_tail)
        ref_out, ref_pp = ref_torch.permute_token_major(x, tm, probs, num_out)
        assert_bits_equal(out, ref_out, f"permute out num_out={num_out}")
        assert_bits_equal(pp, ref_pp, f"permuted probs num_out={num_out}")


# The per-token kernel loads the x row with non-temporal loads below 1 GiB of permuted output and with plain
# loads from 1 GiB on: 9300 tokens write 1.067e9 bytes, 9400 tokens 1.078e9 (H = 7168, 8 rows per token).
@pytest.mark.parametrize("T", [9300, 9400], ids=["nt_row_loads", "plain_row_loads"])
def test_permute_row_load_policies_large(pkg, dev, T):
    E, k, H = 64, 8, 7168
    assert (T * k * H * 2 >= 1 << 30) == (T == 9400)
    rm = _mask(T, E, k, seed=T)
    _, tm = ref_torch.row_id_map(rm)
    x = pkg.inputs.randn_bf16((T, H), seed=T, device=dev)
    probs = torch.rand(T, E, generator=torch.Generator().manual_seed(T)) * rm
    out, pp = pkg.ops.permute(x, tm.to(dev), probs.to(dev), num_out=T * k, layout="token_major",
                              zero_tail=False)
    t, e = rm.nonzero(as_tuple=True)
    rows = tm[t, e]
    assert torch.equal(torch.sort(rows).values, torch.arange(T * k, dtype=rows.dtype)), "every row is named once"
    rows_d, t_d = rows.to(dev), t.to(dev)
    assert torch.equal(out[rows_d].view(torch.int16), x[t_d].view(torch.int16))
    assert torch.equal(pp.cpu()[rows], probs[t, e])


@pytest.mark.parametrize("layout", ["token_major", "expert_major"])
@pytest.mark.parametrize("E", [96, 320])
def test_permute_stores_stay_inside_out(pkg, dev, layout, E):
    """Regression: a 64-bit ballot rebuilt from two 32-bit scalar halves must not sign-extend the low half.

    With expert c*64+31 routed (bit 31 of the chunk's ballot), a sign-extended low half set bits 32..63 too,
    and the kernel stored rows to the map entries of unrouted experts (-1: one row before `out`). Here `out` is
    a view inside a sentinel-filled buffer whose guard rows must stay untouched.
    """
    T, k, H = 64, 4, 64
    rm = torch.zeros(T, E, dtype=torch.bool)
    for t in range(T):
        rm[t, [31, 64 + 31 if E > 95 else 1, (t * 7) % E, (t * 13 + 5) % E]] = True  # lane 31 of chunks 0 and 1
    em, tm = ref_torch.row_id_map(rm)
    R = int(rm.sum())
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(E)).to(torch.bfloat16)
    probs = torch.rand(T, E, generator=torch.Generator().manual_seed(E + 1)) * rm
    sentinel = torch.full((R + 2, H), 7.0, dtype=torch.bfloat16, device=dev)
    pp = torch.full((R + 2,), 7.0, dtype=torch.float32, device=dev)
    m = (tm if layout == "token_major" else em).to(dev)
    pkg.ops.permute(x.to(dev), m, probs.to(dev), num_out=R, layout=layout, zero_tail=False,
                    out=sentinel[1:R + 1], permuted_probs=pp[1:R + 1])
    assert torch.all(sentinel[0] == 7.0) and torch.all(sentinel[R + 1] == 7.0), "row stored outside out"
    assert pp[0].item() == 7.0 and pp[R + 1].item() == 7.0, "prob stored outside permuted_probs"
    ref_out, ref_pp = ref_torch.permute_token_major(x, tm, probs, R)
    assert_bits_equal(sentinel[1:R + 1], ref_out, "permute out")
    assert_bits_equal(pp[1:R + 1], ref_pp, "permuted probs")


def test_permute_case17_reference_inputs(pkg, dev):
    # The case17 generator at the reference shape class (T reduced to 4096 to keep
    # the CPU oracle quick; the routing stream is the reference's own).
    case = pkg.cases.case17_moe_permute_with_mask_map
    x, m, probs = case.get_inputs(dev, tokens=4096, hidden=1024)
    R = int((m >= 0).sum())
    out, pp = case.kernel_function(x, m, probs)
    ref_out, ref_pp = ref_torch.permute_token_major(x.cpu(), m.cpu(), probs.cpu(), R)
    assert_bits_equal(out, ref_out, "case17 out")
    assert_bits_equal(pp, ref_pp, "case17 pp")
    # Model interface with num_out > R zero-fills the tail (new_zeros)
    out2, pp2 = case.Model(320, R + 7)(x, m, probs)
    ref2, refpp2 = ref_torch.permute_token_major(x.cpu(), m.cpu(), probs.cpu(), R + 7)
    assert_bits_equal(out2, ref2, "case17 Model out")
    assert_bits_equal(pp2, refpp2, "case17 Model pp")


@pytest.mark.parametrize("mod,fn", [("case21_permute_with_mask_map_trans", "permute_with_mask_map_trans"),
                                    ("case30_moe_permute_mask_kernel", "permute_mask")])
def test_permute_expert_major_cases(pkg, dev, mod, fn):
    case = getattr(pkg.cases, mod)
    m = case.make_row_id_map(2048, 64, 8, device=dev)
    assert_bits_equal(m, ref_torch.modular_row_id_map(2048, 64, 8), "modular map")
    g = torch.Generator().manual_seed(0)
    inp = torch.randn(2048, 512, generator=g).to(torch.bfloat16)
    out = getattr(case, fn)(inp.to(dev), m)
    assert_bits_equal(out, ref_torch.permute_expert_major(inp, m.cpu()), f"{mod} out")
    assert m[8, 0].item() == -1 and out.shape == (2048 * 8, 512)


def test_permute_with_probs_case22(pkg, dev):
    case = pkg.cases.case22_moe_permute_mask_kernel_true
    m = case.make_row_id_map(1024, 320, 8, device=dev)
    probs = case.make_probs(m, seed=1, device=dev)
    g = torch.Generator().manual_seed(0)
    inp = torch.randn(1024, 256, generator=g).to(torch.bfloat16)
    out, pp = case.permute_mask_with_probs(inp.to(dev), m, probs)
    ref_out, ref_pp = ref_torch.permute_expert_major(inp, m.cpu(), probs.cpu())
    assert_bits_equal(out, ref_out, "case22 out")
    assert_bits_equal(pp, ref_pp, "case22 pp")


def _padded_expert_major_map(T, E, k, pad, seed):
    """Expert-major map whose experts start at multiples of `pad` rows (a capacity-padded layout):
    the rows between one expert's last token and the next expert's first are named by no entry."""
    g = torch.Generator().manual_seed(seed)
    mask = torch.zeros(T, E, dtype=torch.bool).scatter_(1, torch.rand(T, E, generator=g).topk(k, 1).indices, True)
    m = torch.full((E, T), -1, dtype=torch.int64)
    base = 0
    for e in range(E):
        toks = mask[:, e].nonzero().squeeze(1)
        m[e, toks] = base + torch.arange(toks.numel())
        base += (toks.numel() + pad - 1) // pad * pad if toks.numel() else pad
    return m


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_map_extent_matches_torch(pkg, dev, dtype):
    # max(-1, largest entry) and the count of entries >= 0, in one pass: vector body and scalar tail,
    # a misaligned view (scalar path), an all -1 map, an empty map, and the case21 map at full size.
    g = torch.Generator().manual_seed(12)
    maps = [torch.randint(-1, 1000, (37, 101), generator=g), torch.full((8, 8), -1), torch.empty(0, 5),
            torch.randint(-1, 3, (1,), generator=g), torch.randint(-5, 70000, (300001,), generator=g)]
    for m in maps:
        m = m.to(dtype).to(dev)
        assert pkg.ops.map_extent(m) == _extent_ref(m), tuple(m.shape)
    base = torch.randint(-1, 50, (4097,), generator=g).to(dtype).to(dev)
    view = base[1:]  # 4 or 8 bytes past a 16-byte boundary
    assert pkg.ops.map_extent(view) == _extent_ref(view)
    em = pkg.cases.case21_permute_with_mask_map_trans.make_row_id_map(device=dev).to(dtype)
    assert pkg.ops.map_extent(em) == _extent_ref(em)
    assert pkg.ops.map_extent(em)[2], "a row-id map names every row once"
    # Large maps: several rounds of the partial pass's four loads per thread over 2048 blocks (a partial last
    # round and a scalar tail), and a permutation whose 2^23 + 5 row marks the final pass counts in many rounds.
    big = torch.randint(-1, 1 << 20, (2 ** 24 + 3,), generator=g).to(dtype).to(dev)
    assert pkg.ops.map_extent(big) == _extent_ref(big)
    perm = torch.randperm(2 ** 23 + 5, generator=g).to(dtype).to(dev)
    assert pkg.ops.map_extent(perm) == (2 ** 23 + 4, 2 ** 23 + 5, True)
    perm[77] = perm[78]  # one row named twice, one never
    got = pkg.ops.map_extent(perm)
    assert got == _extent_ref(perm) and not got[2]


def _extent_ref(m: torch.Tensor) -> tuple[int, int, bool]:
    """(max(-1, largest entry), count of entries >= 0, whether those entries are exactly 0 .. max)."""
    v = m[m >= 0].cpu().long()
    mx = int(v.max()) if v.numel() else -1
    return mx, int(v.numel()), bool(v.numel() == mx + 1 and torch.unique(v).numel() == v.numel())


@pytest.mark.parametrize("dtype", [torch.int64, torch.int32])
def test_map_extent_bijective_flag(pkg, dev, dtype):
    # The third value is set only for maps whose entries >= 0 are 0 .. max, each once: a permutation of
    # a row-id map (any layout), but not a map whose count matches max + 1 through a repeat and a hole
    # ({0, 0, 2}), nor one with a hole alone or a repeat alone; bits past the first 32 and in the last
    # partial word of the bitmap are exercised by the larger maps.
    g = torch.Generator().manual_seed(13)
    perm = torch.randperm(5000, generator=g)
    holed = perm.clone()
    holed[holed == 4099] = 17  # 17 twice, 4099 missing: count still == max + 1
    cases = [(torch.tensor([0, 0, 2, -1]), False), (torch.tensor([[0, -1], [-1, 2]]), False),
             (torch.tensor([1, 0, 1]), False), (torch.tensor([2, -1, 0, 1]), True), (torch.full((3, 3), -1), True),
             (perm.reshape(50, 100), True), (holed.reshape(100, 50), False), (perm[:4097], False)]
    for m, want in cases:
        m = m.to(dtype).to(dev)
        got = pkg.ops.map_extent(m)
        assert got == _extent_ref(m), (tuple(m.shape), got)
        assert got[2] is want, (tuple(m.shape), got)


@pytest.mark.parametrize("mod,fn,probs", [("case21_permute_with_mask_map_trans", "permute_with_mask_map_trans", False),
                                          ("case30_moe_permute_mask_kernel", "permute_mask", False),
                                          ("case22_moe_permute_mask_kernel_true", "permute_mask_with_probs", True)])
def test_permute_sparse_maps_zero_the_unnamed_rows(pkg, dev, mod, fn, probs):
    # Maps that do not name every row below their max: a capacity-padded expert-major layout
    # and a hand-made one with holes. The unnamed rows are zero, as the reference's new_zeros
    # leaves them (kernel_cases/case22_ref_moe_permute_mask_kernel_true.py:63-67).
    case = getattr(pkg.cases, mod)
    g = torch.Generator().manual_seed(9)
    for m in (_padded_expert_major_map(300, 12, 3, pad=64, seed=4),
              torch.tensor([[0, -1, 5], [-1, 2, -1]], dtype=torch.int64)):
        E, T = m.shape
        inp = torch.randn(T, 136, generator=g).to(torch.bfloat16)
        pr = torch.rand(T, E, generator=g) * (m >= 0).t()
        # the destination buffers first hold garbage, so stale rows would show
        torch.empty(4 << 20, dtype=torch.uint8, device=dev).fill_(0x7F)
        if probs:
            out, pp = getattr(case, fn)(inp.to(dev), m.to(dev), pr.to(dev))
            ref_out, ref_pp = ref_torch.permute_expert_major(inp, m, pr)
            assert_bits_equal(pp, ref_pp, f"{mod} permuted probs")
        else:
            out = getattr(case, fn)(inp.to(dev), m.to(dev))
            ref_out = ref_torch.permute_expert_major(inp, m)
        assert_bits_equal(out, ref_out, f"{mod} out")
        assert int(m.max()) + 1 > int((m >= 0).sum()), "the map has unnamed rows"
    # case17 without num_out derives R = max + 1 the same way (token-major map)
    m = _padded_expert_major_map(200, 8, 2, pad=32, seed=5)
    x = torch.randn(200, 64, generator=g).to(torch.bfloat16)
    pr = torch.rand(200, 8, generator=g)
    tm = m.t().contiguous()
    out, pp = pkg.cases.case17_moe_permute_with_mask_map.kernel_function(x.to(dev), tm.to(dev), pr.to(dev))
    ref_out, ref_pp = ref_torch.permute_token_major(x, tm, pr * (tm >= 0), int(m.max()) + 1)
    assert_bits_equal(out, ref_out, "case17 sparse out")
    assert_bits_equal(pp, ref_pp, "case17 sparse pp")


@pytest.mark.parametrize("mod,fn", [("case21_permute_with_mask_map_trans", "permute_with_mask_map_trans"),
                                    ("case30_moe_permute_mask_kernel", "permute_mask")])
def test_scatter_map_with_repeat_and_hole_zeroes_the_hole(pkg, dev, mod, fn):
    # Entries {0, 0, 2}: as many as max + 1, yet row 1 is named by no entry and row 0 twice. The hole
    # is zero, as the reference's new_zeros leaves it; row 2 is its token's row; row 0 is one of its two
    # tokens' rows (the reference writes them in turn, kernel_cases/case21_ref_permute_with_mask_map_trans.py:60-68).
    case = getattr(pkg.cases, mod)
    g = torch.Generator().manual_seed(10)
    m = torch.tensor([[0, -1, -1], [-1, 0, 2]], dtype=torch.int64)
    inp = torch.randn(3, 72, generator=g).to(torch.bfloat16)
    torch.empty(4 << 20, dtype=torch.uint8, device=dev).fill_(0x7F)  # stale memory would show in row 1
    out = getattr(case, fn)(inp.to(dev), m.to(dev)).cpu()
    assert out.shape == (3, 72)
    assert torch.equal(out[1], torch.zeros(72, dtype=torch.bfloat16)), "the unnamed row is not zero"
    assert torch.equal(out[2], inp[2])
    assert torch.equal(out[0], inp[0]) or torch.equal(out[0], inp[1])


def test_permute_known_answer_on_gpu(pkg, dev):
    inp = (torch.arange(8, dtype=torch.bfloat16).reshape(2, 4) + 1).to(dev)
    m = torch.tensor([[0, -1], [-1, 2], [1, -1], [-1, -1]], dtype=torch.int64, device=dev)
    probs = torch.tensor([[10.0, 0.0, 20.0, 0.0], [0.0, 30.0, 0.0, 0.0]], device=dev)
    out, pp = pkg.cases.case22_moe_permute_mask_kernel_true.permute_mask_with_probs(inp, m, probs)
    assert torch.equal(out.cpu(), torch.stack([inp[0], inp[0], inp[1]]).cpu())
    assert torch.equal(pp.cpu(), torch.tensor([10.0, 20.0, 30.0]))


# ---------------------------------------------------------------- unpermute
def _wide(R, H, seed):
    g = torch.Generator().manual_seed(seed)
    scale = torch.exp2(torch.randint(-14, 15, (R, H), generator=g).float())
    return (torch.randn(R, H, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("layout", ["token_major", "expert_major"])
@pytest.mark.parametrize("idx", [torch.int64, torch.int32])
@pytest.mark.parametrize("merge", [False, True])
# Shapes cover both launch forms: one wavefront per 1 KiB slice of the row (up to
# 16 per token) and 4 tokens per workgroup for short rows (with a partial last
# workgroup), each with the map read per wavefront (E <= 64) or staged in LDS
# (E > 64, including a partial last 64-expert chunk, E = 1024, and E up to the
# row-id map's 4096, where short rows put fewer tokens in a workgroup so the staged
# entries fit the LDS), plus the scalar path for rows that are not a multiple of 8.
@pytest.mark.parametrize("T,E,k,H", [(257, 8, 2, 2048), (96, 64, 8, 7168), (40, 320, 6, 72), (21, 9, 4, 11),
                                     (43, 130, 3, 24), (29, 200, 5, 13), (33, 1024, 8, 4096),
                                     (19, 2000, 7, 40), (13, 4096, 9, 16), (11, 4096, 3, 1000)])
def test_unpermute_matches_oracle(pkg, dev, layout, idx, merge, T, E, k, H):
    rm = _mask(T, E, k, seed=T + 7 * E)
    em, tm = ref_torch.row_id_map(rm)
    pin = _wide(T * k, H, seed=T * H + E)
    g = torch.Generator().manual_seed(E)
    probs = torch.rand(T, E, generator=g) * rm if merge else None
    m = (tm if layout == "token_major" else em).to(idx)
    acc, out = pkg.ops.unpermute(pin.to(dev), m.to(dev), probs.to(dev) if merge else None, layout=layout,
                                 with_acc=True)
    if merge:
        ref_acc, ref_out = ref_torch.unpermute_merge(pin, em, probs, with_acc=True)
    else:
        ref_acc, ref_out = ref_torch.unpermute_mask(pin, em)
    assert_bits_equal(acc, ref_acc, "fp32 accumulator")
    assert_bits_equal(out, ref_out, "bf16 output")


def test_unpermute_case15_reference_inputs(pkg, dev):
    case = pkg.cases.case15_moe_unpermute_mask_fwd
    pin, m = case.get_inputs(dev, tokens=2048, hidden=2048)
    out = case.kernel_function(pin, m)
    assert_bits_equal(out, ref_torch.unpermute(pin.cpu(), m.cpu()), "case15 out")


def test_unpermute_known_answers_case24_case32(pkg, dev):
    grad_in = torch.tensor([[4, 1], [4, 1], [7, 0]], dtype=torch.bfloat16, device=dev)
    m = torch.tensor([[0, -1], [-1, 2], [1, -1], [-1, -1]], dtype=torch.int32, device=dev)
    acc, stored = pkg.cases.case24_moe_unpermute_mask_kernel_false.unpermute_mask(grad_in, m)
    expect = torch.tensor([[8.0, 2.0], [7.0, 0.0]])
    assert torch.equal(acc.cpu(), expect) and torch.equal(stored.cpu(), expect.to(torch.bfloat16))
    pg = torch.tensor([10.0, 20.0, 30.0], device=dev)
    acc, stored, gathered = pkg.cases.case32_moe_unpermute_mask_kernel.unpermute_mask(grad_in, m, pg)
    assert torch.equal(gathered.cpu(), torch.tensor([[10.0, 0.0, 20.0, 0.0], [0.0, 30.0, 0.0, 0.0]]))
    with pytest.raises(ValueError):
        pkg.cases.case24_moe_unpermute_mask_kernel_false.unpermute_mask(grad_in[:2], m)


def test_unpermute_cases_24_32_modular(pkg, dev):
    m = pkg.cases.case24_moe_unpermute_mask_kernel_false.make_row_id_map(512, 64, 8, device=dev)
    assert m.dtype == torch.int32
    grad_in = _wide(512 * 8, 256, seed=5)
    pg = torch.randn(512 * 8)
    acc, stored = pkg.cases.case24_moe_unpermute_mask_kernel_false.unpermute_mask(grad_in.to(dev), m)
    ref_acc, ref_stored = ref_torch.unpermute_mask(grad_in, m.cpu())
    assert_bits_equal(acc, ref_acc, "case24 acc")
    assert_bits_equal(stored, ref_stored, "case24 bf16")
    acc, stored, gathered = pkg.cases.case32_moe_unpermute_mask_kernel.unpermute_mask(grad_in.to(dev), m, pg.to(dev))
    ref = ref_torch.unpermute_mask_probgrad(grad_in, m.cpu(), pg)
    assert_bits_equal(acc, ref[0], "case32 acc")
    assert_bits_equal(stored, ref[1], "case32 bf16")
    assert_bits_equal(gathered, ref[2], "case32 prob grad")


# -------------------------------------------------------------- permute bwd
@pytest.mark.parametrize("T,E,k,H", [(512, 320, 8, 1024), (200, 64, 8, 7168), (37, 6, 2, 20), (19, 130, 4, 40),
                                     (23, 100, 3, 9), (17, 4096, 5, 24)])
def test_permute_bwd_matches_oracle(pkg, dev, T, E, k, H):
    rm = _mask(T, E, k, seed=11 * T)
    em, _ = ref_torch.row_id_map(rm)
    dperm = _wide(T * k, H, seed=H)
    dpp = torch.randn(T * k)
    dact, dprobs = pkg.cases.case18_moe_permute_bwd_unpermute_mask.kernel_function(
        dperm.to(dev), dpp.to(dev), em.to(dev))
    ref_dact, ref_dprobs = ref_torch.permute_bwd(dperm, dpp, em)
    assert_bits_equal(dact, ref_dact, "dact")
    assert_bits_equal(dprobs, ref_dprobs, "dprobs")


def test_permute_bwd_case18_generator(pkg, dev):
    case = pkg.cases.case18_moe_permute_bwd_unpermute_mask
    dperm, dpp, m = case.get_inputs(dev, tokens=512, hidden=1024)
    dact, dprobs = case.kernel_function(dperm, dpp, m)
    ref_dact, ref_dprobs = ref_torch.permute_bwd(dperm.cpu(), dpp.cpu(), m.cpu())
    assert_bits_equal(dact, ref_dact, "case18 dact")
    assert_bits_equal(dprobs, ref_dprobs, "case18 dprobs")


# -------------------------------------------------------------------- top-k
def _topk_inputs():
    g = torch.Generator().manual_seed(3)
    cases = []
    for s in (0, 1, 7):
        cases.append((f"traced seed {s}", torch.randn(2048, 320, generator=torch.Generator().manual_seed(s)), 8))
    cases.append(("small", torch.tensor([[0.1, 0.5, 0.3, 0.2], [4.0, 1.0, 3.0, 2.0]]), 2))
    for m, n, k in [(1, 320, 8), (17, 320, 8), (1000, 320, 8), (2048, 320, 1), (2048, 320, 4), (256, 64, 8),
                    (128, 33, 8), (64, 16, 3), (300, 1024, 64), (77, 8, 2), (100, 64, 64)]:
        cases.append((f"shape {m}x{n} k{k}", torch.randn(m, n, generator=torch.Generator().manual_seed(m + n)), k))
    cases.append(("ties randint(0,5)", torch.randint(0, 5, (4096, 320), generator=g).float(), 8))
    cases.append(("all zeros", torch.zeros(64, 320), 8))
    cases.append(("all negative", -torch.rand(512, 320, generator=g), 8))
    inf = torch.randn(64, 320, generator=g)
    inf[:, :40] = float("-inf")
    cases.append(("-inf columns", inf, 8))
    nan = torch.randn(64, 64, generator=g)
    nan[::2, 5] = float("nan")
    nan[::3, 60] = float("nan")
    cases.append(("nan", nan, 8))
    sz = torch.zeros(32, 64)
    sz[:, ::3] = -0.0
    cases.append(("signed zeros", sz, 8))
    return cases


@pytest.mark.parametrize("tag,x,k", _topk_inputs(), ids=lambda v: v if isinstance(v, str) else "")
def test_topk_matches_oracle(pkg, dev, tag, x, k):
    v, i = pkg.cases.case23_aten_topk.kernel_function(x.to(dev), k)
    rv, ri = ref_torch.topk(x, k)
    assert_bits_equal(i, ri, f"{tag} indices")
    assert_bits_equal(v, rv, f"{tag} values")


def test_topk_mask_probs(pkg, dev):
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(4096, 64, generator=g) + torch.randn(64, generator=g) * 1.5
    v, i, mask, probs = pkg.ops.topk(logits.to(dev), 8, with_mask=True, with_probs=True)
    rv, ri = ref_torch.topk(logits, 8)
    rm, rp = ref_torch.mask_and_probs(rv, ri, 64)
    assert_bits_equal(i, ri, "indices")
    assert torch.equal(mask.cpu(), rm)
    # softmax in fp32: GPU expf vs CPU exp differ by an ulp or two
    torch.testing.assert_close(probs.cpu(), rp, rtol=2e-6, atol=1e-7)
    assert torch.all((probs.cpu() > 0) == rm)


def test_topk_errors(pkg, dev):
    kf = pkg.cases.case23_aten_topk.kernel_function
    x = torch.randn(4, 16, device=dev)
    with pytest.raises(ValueError):
        kf(x, 8, largest=False)
    with pytest.raises(ValueError):
        kf(x, 8, dim=0)
    with pytest.raises(ValueError):
        kf(x[0], 8)
    v, i = kf(x, 100)  # k is clamped to N like the bundle
    assert v.shape == (4, 16)


# ------------------------------------------------------------- index_select
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_index_select_case06_shape_class(pkg, dev, idx_dtype):
    case = pkg.cases.case06_cp_seq_chunk_index_select
    k_ag, v_ag, index = case.get_inputs(dev, tok=1024)
    index = torch.tensor([1, 0, 1], dtype=idx_dtype, device=dev)
    ko, vo = case.kernel_function(k_ag, v_ag, index)
    assert_bits_equal(ko, ref_torch.index_select(k_ag.cpu(), index.cpu()), "k")
    assert_bits_equal(vo, ref_torch.index_select(v_ag.cpu(), index.cpu()), "v")


def test_index_select_odd_rows_and_out_of_range(pkg, dev):
    g = torch.Generator().manual_seed(2)
    src = torch.randn(50, 7, 3, generator=g).to(torch.bfloat16)
    idx = torch.tensor([3, 49, 0, 0, 17], dtype=torch.int64)
    out = pkg.ops.index_select(src.to(dev), idx.to(dev))
    assert_bits_equal(out, ref_torch.index_select(src, idx), "odd row gather")
    bad = pkg.ops.index_select(src.to(dev), torch.tensor([2, 50, -1], device=dev))
    assert torch.equal(bad[0].cpu(), src[2]) and not bad[1:].cpu().float().abs().sum()
