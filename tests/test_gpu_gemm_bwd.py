"""GPU parity of the grouped GEMM backward (dgrad "NN", wgrad "TN") against the fp32 oracle.

Tolerance: rtol 1.6e-2 / atol 1e-2 against the fp32-accumulated golden
(per group dy.float() @ w.float() / dy.float().T @ x.float();
kernel_cases/case37_ref_musa_asm_bf16_gemm_nn_256x384.py:47-49 is the same
rule for one group) -- one bf16 rounding of an fp32 sum.  Small shapes and
the reference cases' own shapes (case05/07/08/09/13/19/37) are checked in
full against the CPU oracle.
Exact cases (scaled identities, one-row outer products) must be bit-identical.
"""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bits_equal
from oracle import ref_torch

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1.6e-2, 1e-2


def _check(got, ref, what):
    torch.testing.assert_close(got.float(), ref.float().to(got.device), rtol=RTOL, atol=ATOL,
                               msg=lambda m: f"{what}: {m}")


def _offsets(sizes, dev):
    o = [0]
    for s in sizes:
        o.append(o[-1] + s)
    return torch.tensor(o, dtype=torch.int32, device=dev)


# ------------------------------------------------------------------ dgrad
@pytest.mark.parametrize("sizes,N,K", [
    ([128], 64, 256),                      # one 128-row tile
    ([1], 8, 8),                           # degenerate
    ([256, 256], 128, 256),                # 256-row tiles
    ([300, 0, 17, 513], 200, 264),         # ragged, empty group, N % 64 and K % 256 tails (256-row tiles)
    ([5, 7, 0, 100, 1], 136, 72),          # small groups (128-row tiles), tails
    ([90] * 6, 512, 1032),                 # 128-row tiles, several column tiles
    ([700, 3, 1200], 2048, 520),           # long reduction, 256-row tiles
    ([400, 0, 333, 512], 192, 264),        # pipelined kernel at its shortest reduction (3 steps), column tail
    ([600, 1], 6144, 72),                  # pipelined kernel, one column tile narrower than the tile
    ([300] * 20, 256, 200),                # 20 groups of 300 rows: many tile changes, K tail
])
def test_dgrad_small(pkg, dev, sizes, N, K):
    g = torch.Generator().manual_seed(sum(sizes) + 7 * N + K)
    dy = torch.randn(sum(sizes), N, generator=g).to(torch.bfloat16)
    w = (torch.randn(len(sizes), N, K, generator=g) * 0.05).to(torch.bfloat16)
    out = pkg.cases.case07_moe_grouped_gemm_fc1_dgrad.kernel_function(dy.to(dev), w.to(dev), sizes)
    assert out.shape == (sum(sizes), K)
    _check(out, ref_torch.grouped_gemm_dgrad_fp32(dy, w, sizes), f"dgrad sizes={sizes} N={N} K={K}")


def test_dgrad_scaled_identity_exact(pkg, dev):
    # dy @ (c I) with c a power of two is exact: bit-identical, on both tile heights.
    for sizes in ([100, 300, 200], [40, 60, 20]):
        dy = torch.randn(sum(sizes), 256).to(torch.bfloat16)
        w = torch.stack([torch.eye(256), 4 * torch.eye(256), 0.5 * torch.eye(256)]).to(torch.bfloat16)
        out = pkg.ops.grouped_gemm_dgrad(dy.to(dev), w.to(dev), _offsets(sizes, dev)).cpu()
        a, b = sizes[0], sizes[0] + sizes[1]
        assert_bits_equal(out[:a], dy[:a], f"identity {sizes}")
        assert_bits_equal(out[a:b], (4 * dy[a:b].float()).to(torch.bfloat16), f"4I {sizes}")
        assert_bits_equal(out[b:], (0.5 * dy[b:].float()).to(torch.bfloat16), f"I/2 {sizes}")


def test_dgrad_writes_only_grouped_rows(pkg, dev):
    # Rows past group_offsets[G] and bytes past dx keep their contents.
    M, N, K = 300, 64, 40
    dy = torch.randn(M, N, device=dev).to(torch.bfloat16)
    w = torch.randn(2, N, K, device=dev).to(torch.bfloat16)
    offs = torch.tensor([0, 100, 250], dtype=torch.int32, device=dev)
    buf = torch.full((M * K + 4096,), 7.0, dtype=torch.bfloat16, device=dev)
    out = buf[:M * K].view(M, K)
    pkg.ops.grouped_gemm_dgrad(dy, w, offs, out=out)
    assert torch.all(buf[250 * K:] == 7.0)
    ref = ref_torch.grouped_gemm_dgrad_fp32(dy[:250].cpu(), w.cpu(), [100, 150])
    _check(out[:250], ref, "dgrad rows")


def test_dgrad_empty_reduction_gives_zeros(pkg, dev):
    dy = torch.empty(10, 0, dtype=torch.bfloat16, device=dev)
    w = torch.empty(2, 0, 16, dtype=torch.bfloat16, device=dev)
    out = pkg.ops.grouped_gemm_dgrad(dy, w, _offsets([4, 6], dev), out=torch.full((10, 16), 3.0, dtype=torch.bfloat16,
                                                                                     device=dev))
    assert torch.count_nonzero(out) == 0


@pytest.mark.parametrize("case_name", ["case07_moe_grouped_gemm_fc1_dgrad", "case08_moe_grouped_gemm_fc2_dgrad",
                                       "case13_grouped_gemm_single_group_fc1_dgrad",
                                       "case19_grouped_gemm_single_group_fc2_dgrad"])
def test_dgrad_reference_case_shapes(pkg, dev, case_name):
    # The case's own Model and shapes (T=4096), every element against the CPU oracle, one group at a time.
    case = getattr(pkg.cases, case_name)
    dy, w = case.get_inputs(dev)
    out = case.Model()(dy, w)
    assert out.shape == (case.TOKENS, case.K)
    off = 0
    for gi, m in enumerate(case.group_sizes(case.TOKENS, case.NUM_GROUPS)):
        ref = ref_torch.grouped_gemm_dgrad_fp32(dy[off:off + m].cpu(), w[gi:gi + 1].cpu(), [m])
        _check(out[off:off + m], ref, f"{case_name} group {gi}")
        off += m


def test_case37_single_expert_dgrad(pkg, dev):
    # Seeded inputs identical to the reference's make_inputs; its fp32 golden and its own rule.
    case = pkg.cases.case37_ref_musa_asm_bf16_gemm_nn_256x384
    grad_output, weight = case.make_inputs(seed=0, device=dev)
    got = case.kernel_function(grad_output, weight)
    golden = ref_torch.grouped_gemm_dgrad_fp32(grad_output.cpu(), weight.cpu().unsqueeze(0), [case.M]).to(dev)
    diff = (got.float() - golden).abs()
    max_rel = (diff / golden.abs().clamp(min=1.0)).max().item()
    assert not (max_rel > 2e-2 and diff.max().item() > 2e-1)
    _check(got, golden, "case37")


def test_dgrad_split_reduction(pkg, dev):
    # One group with few output tiles (3 x 2 here) and a workspace: the reduction runs as 5 splits
    # (3, 3, 3, 3 and 4 steps of 64) into fp32 planes summed in split order. Only the group's rows
    # (offsets 40 .. 560 of 600) are written, the result matches the fp32 oracle, and a second
    # call is bit-identical (no atomics: the order is fixed).
    lib = pkg._lib.lib()
    M, N, K = 600, 1024, 512
    assert lib.moe_grouped_gemm_dgrad_workspace_size(M, N, K, 1) == 5 * M * K * 4
    g = torch.Generator().manual_seed(37)
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16)
    w = (torch.randn(1, N, K, generator=g) * 0.05).to(torch.bfloat16)
    offs = torch.tensor([40, 560], dtype=torch.int32, device=dev)
    outs = []
    for _ in range(2):
        buf = torch.full((M * K + 4096,), 7.0, dtype=torch.bfloat16, device=dev)
        out = buf[:M * K].view(M, K)
        pkg.ops.grouped_gemm_dgrad(dy.to(dev), w.to(dev), offs, out=out)
        assert torch.all(out[:40] == 7.0) and torch.all(buf[560 * K:] == 7.0)
        outs.append(out.cpu())
    _check(outs[0][40:560], ref_torch.grouped_gemm_dgrad_fp32(dy[40:560], w, [520]), "split dgrad")
    assert_bits_equal(outs[0], outs[1], "split dgrad repeat")


@pytest.mark.parametrize("sizes,N,K", [
    # tails of 1, 127, 128 (128-row tiles), 129, 255 (256-row tiles), whole tiles, an empty group; K tail
    ([1, 127, 128, 129, 255, 256, 512, 0, 385, 640], 4096, 520),
    ([3, 0, 70, 2000, 128, 4097], 7168, 2048),       # fc2 dgrad class: the benchmark's reduction and width
    ([100] * 100 + [2000] * 10, 4096, 512),          # 200 tail units over the persistent grid
    ([257] * 16, 4160, 8),                           # one-row tails, one narrow column tile, 65 steps
])
def test_dgrad_tail_tiles_match_full_tiles(pkg, dev, sizes, N, K):
    """With its workspace dgrad computes a group's last row tile of 1 to 128 rows as a 128-row
    tile, taken from a list after the 256-row tiles; without it every row tile has 256 rows. The
    per-element reduction order and rounding are the same: equal bit for bit."""
    lib = pkg._lib.lib()
    M, G = sum(sizes), len(sizes)
    assert lib.moe_grouped_gemm_dgrad_workspace_size(M, N, K, G) == (4 * (64 + G) + 255) // 256 * 256
    g = torch.Generator().manual_seed(M + N + K + 11)
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16)
    w = (torch.randn(G, N, K, generator=g) * 0.05).to(torch.bfloat16)
    offs = _offsets(sizes, dev)
    dyd, wd = dy.to(dev), w.to(dev)
    ws = torch.full((8192,), 0xAB, dtype=torch.uint8, device=dev)  # stale contents: the list kernel rewrites it
    tails = pkg.ops.grouped_gemm_dgrad(dyd, wd, offs, workspace=ws)
    tails2 = pkg.ops.grouped_gemm_dgrad(dyd, wd, offs, workspace=ws)  # the same workspace again
    full = pkg.ops.grouped_gemm_dgrad(dyd, wd, offs, workspace=torch.empty(0, dtype=torch.uint8, device=dev))
    torch.cuda.synchronize()
    what = f"sizes={sizes[:6]} N={N} K={K}"
    assert_bits_equal(tails.cpu(), tails2.cpu(), "tail dgrad repeat " + what)
    assert_bits_equal(tails.cpu(), full.cpu(), "tail vs full tiles " + what)
    _check(tails, ref_torch.grouped_gemm_dgrad_fp32(dy, w, sizes), "tail dgrad " + what)


# ------------------------------------------------------------------ wgrad
@pytest.mark.parametrize("sizes,N,K", [
    ([64], 256, 256),                       # one tile, one step
    ([1], 8, 8),                            # degenerate
    ([300, 0, 17, 513], 200, 264),          # ragged, empty group, N and K tails
    ([102] * 5, 520, 1024),                 # case05/09 group size, K tail in the reduction
    ([2048, 5], 128, 264),                  # long reduction
    ([1, 2, 0, 63, 64, 65, 127, 128, 129, 191, 192, 193] * 3, 136, 200),  # many small groups: 3-step minimum, zero steps
    ([5000, 0, 3000], 264, 520),            # long reductions of different lengths, N and K tails
])
def test_wgrad_small(pkg, dev, sizes, N, K):
    g = torch.Generator().manual_seed(3 * sum(sizes) + N + 5 * K)
    dy = torch.randn(sum(sizes), N, generator=g).to(torch.bfloat16)
    x = torch.randn(sum(sizes), K, generator=g).to(torch.bfloat16)
    out = pkg.cases.case09_moe_grouped_gemm_fc1_wgrad.kernel_function(dy.to(dev), x.to(dev), sizes, len(sizes))
    assert out.shape == (len(sizes), N, K)
    _check(out, ref_torch.grouped_gemm_wgrad_fp32(dy, x, sizes), f"wgrad sizes={sizes} N={N} K={K}")
    for gi, m in enumerate(sizes):
        if m == 0:
            assert torch.count_nonzero(out[gi]) == 0


@pytest.mark.parametrize("sizes,N,K", [
    ([3, 0, 700, 41, 700, 0, 1500, 64, 129, 5], 264, 520),
    # 80 skewed groups x 8 tiles = 640 tiles: three rounds on 256 CUs, the second dealt in reverse
    ([(37 * i * i) % 1500 for i in range(80)], 512, 1024),
])
def test_wgrad_group_order_is_bit_identical(pkg, dev, sizes, N, K):
    # With the workspace the tiles take the groups largest first (dealt in reverse on odd rounds);
    # without it, by index. Each tile's accumulation is the same either way, so dw is bit for bit
    # the same (skewed ragged groups, empty ones and ties included).
    lib, ptr = pkg._lib.lib(), pkg._lib.ptr
    g = torch.Generator().manual_seed(23)
    dy = torch.randn(sum(sizes), N, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(sum(sizes), K, generator=g).to(torch.bfloat16).to(dev)
    offs = _offsets(sizes, dev)
    assert lib.moe_grouped_gemm_wgrad_workspace_size(sum(sizes), N, K, len(sizes)) > 0
    ordered = pkg.ops.grouped_gemm_wgrad(dy, x, offs)
    plain = torch.empty_like(ordered)
    rc = lib.moe_grouped_gemm_wgrad(ptr(dy), ptr(x), sum(sizes), N, K, len(sizes), ptr(offs), ptr(plain), None, 0,
                                    pkg._lib.stream_handle())
    assert rc == 0
    torch.cuda.synchronize()
    assert_bits_equal(ordered, plain, "wgrad ordered vs by index")
    _check(ordered, ref_torch.grouped_gemm_wgrad_fp32(dy.cpu(), x.cpu(), sizes), "wgrad ordered")


@pytest.mark.parametrize("G", [1, 2, 5, 64, 1000, 4096])
def test_wgrad_group_order_matches_stable_sort(pkg, dev, G):
    # The workspace's group order (int16 [G]): groups by descending rows, ties by ascending index -- a
    # CPU stable sort of the clamped group sizes (ties, empty groups and a non-power-of-two G included).
    lib, ptr = pkg._lib.lib(), pkg._lib.ptr
    g = torch.Generator().manual_seed(G)
    sizes = torch.randint(0, 4, (G,), generator=g).tolist()
    N = K = 64
    M = sum(sizes)
    dy = torch.randn(max(M, 1), N, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(max(M, 1), K, generator=g).to(torch.bfloat16).to(dev)
    offs = _offsets(sizes, dev)
    nbytes = lib.moe_grouped_gemm_wgrad_workspace_size(M, N, K, G)
    if G == 1:
        assert nbytes == 0
        return
    ws = torch.full((nbytes,), 0x55, dtype=torch.uint8, device=dev)
    dw = pkg.ops.grouped_gemm_wgrad(dy[:M], x[:M], offs, workspace=ws)
    order = ws[:2 * G].view(torch.int16).cpu().long()
    want = sorted(range(G), key=lambda i: (-sizes[i], i))
    assert order.tolist() == want
    plain = pkg.ops.grouped_gemm_wgrad(dy[:M], x[:M], offs, workspace=torch.empty(0, dtype=torch.uint8, device=dev))
    assert_bits_equal(dw, plain, "wgrad with the workspace order vs by index")


@pytest.mark.parametrize("sizes,N,K", [
    ([3, 0, 700, 41, 128, 129, 1, 64, 100, 5] * 2, 264, 520),   # long groups mixed in, N and K tails
    ([3, 0, 700, 41, 128, 129, 1, 64, 100, 5] * 2, 520, 264),
    ([102] * 8 + [103] * 4, 384, 1032),                          # the case05/09 group sizes, a K tail
    ([102] * 8 + [103] * 4, 1032, 384),
    ([7] * 300, 136, 200),                                       # many tiny groups: units over many groups
    ([7] * 300, 136, 1800),                                      # units of 8 and 7 swept tiles
    ([102] * 8 + [103] * 4, 128, 1032),                          # one fixed tile per group
    ([50] * 6 + [200], 96, 120),                                 # N, K <= 128: one tile per group
    ([0, 0, 0], 136, 200),                                       # only empty groups: zeros
])
def test_wgrad_sweep_short_groups(pkg, dev, sizes, N, K):
    # Groups averaging under 256 rows: with the workspace the groups of at most 128 rows run in the
    # sweep kernel (the whole reduction in one LDS stage) and the longer ones in the ping-pong kernel.
    # Each output element is the same sequence of MFMAs as without the workspace (ping-pong only), so
    # dw is bit for bit the same; against the CPU oracle at the task tolerance; nothing past dw written.
    lib, ptr = pkg._lib.lib(), pkg._lib.ptr
    G, M = len(sizes), sum(sizes)
    assert M < 256 * G
    g = torch.Generator().manual_seed(M + 7 * N + K)
    dy = torch.randn(max(M, 1), N, generator=g).to(torch.bfloat16).to(dev)[:M]
    x = torch.randn(max(M, 1), K, generator=g).to(torch.bfloat16).to(dev)[:M]
    offs = _offsets(sizes, dev)
    buf = torch.full((G * N * K + 8192,), 3.0, dtype=torch.bfloat16, device=dev)
    swept = buf[:G * N * K].view(G, N, K)
    ws = torch.full((lib.moe_grouped_gemm_wgrad_workspace_size(M, N, K, G),), 0x55, dtype=torch.uint8, device=dev)
    pkg.ops.grouped_gemm_wgrad(dy, x, offs, out=swept, workspace=ws)
    again = pkg.ops.grouped_gemm_wgrad(dy, x, offs, workspace=ws)
    plain = torch.empty_like(swept)
    rc = lib.moe_grouped_gemm_wgrad(ptr(dy), ptr(x), M, N, K, G, ptr(offs), ptr(plain), None, 0,
                                    pkg._lib.stream_handle())
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.all(buf[G * N * K:] == 3.0), "written past dw"
    assert_bits_equal(swept, plain, "wgrad sweep + ping-pong vs ping-pong only")
    assert_bits_equal(again, swept, "wgrad sweep, second call")
    _check(swept, ref_torch.grouped_gemm_wgrad_fp32(dy.cpu(), x.cpu(), sizes), f"wgrad sweep sizes={sizes}")
    for gi, m in enumerate(sizes):
        if m == 0:
            assert torch.count_nonzero(swept[gi]) == 0


def test_wgrad_one_row_groups_exact(pkg, dev):
    # A group of one row is the outer product dy[r] x[r]^T: exact in fp32, one rounding.
    g = torch.Generator().manual_seed(91)
    dy = torch.randn(5, 264, generator=g).to(torch.bfloat16)
    x = torch.randn(5, 520, generator=g).to(torch.bfloat16)
    out = pkg.ops.grouped_gemm_wgrad(dy.to(dev), x.to(dev), _offsets([1] * 5, dev)).cpu()
    for r in range(5):
        assert_bits_equal(out[r], torch.outer(dy[r].float(), x[r].float()).to(torch.bfloat16), f"row {r}")


def test_wgrad_no_rows_gives_zeros_and_stays_in_bounds(pkg, dev):
    G, N, K = 3, 72, 40
    dy = torch.empty(0, N, dtype=torch.bfloat16, device=dev)
    x = torch.empty(0, K, dtype=torch.bfloat16, device=dev)
    buf = torch.full((G * N * K + 4096,), 5.0, dtype=torch.bfloat16, device=dev)
    out = buf[:G * N * K].view(G, N, K)
    pkg.ops.grouped_gemm_wgrad(dy, x, torch.zeros(G + 1, dtype=torch.int32, device=dev), out=out)
    assert torch.count_nonzero(out) == 0
    assert torch.all(buf[G * N * K:] == 5.0)


@pytest.mark.parametrize("case_name", ["case05_moe_grouped_gemm_fc2_wgrad", "case09_moe_grouped_gemm_fc1_wgrad"])
def test_wgrad_reference_case_shapes(pkg, dev, case_name):
    case = getattr(pkg.cases, case_name)
    dy, x = case.get_inputs(dev)
    out = case.Model()(dy, x)
    assert out.shape == (case.NUM_GROUPS, case.N, case.K)
    off = 0
    # every element against the CPU oracle, one group at a time
    for gi, m in enumerate(case.group_sizes(case.TOKENS, case.NUM_GROUPS)):
        ref = ref_torch.grouped_gemm_wgrad_fp32(dy[off:off + m].cpu(), x[off:off + m].cpu(), [m])[0]
        _check(out[gi], ref, f"{case_name} group {gi}")
        off += m
