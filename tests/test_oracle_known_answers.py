"""Pins the oracle to the reference's own known-answer vectors (CPU).

Each vector is restated as data from the reference file cited beside it.  Both
oracle restatements (eager torch, plain C) must reproduce it.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle_c, ref_torch

# 4 experts x 2 tokens: token 0 -> experts 0 and 2 (rows 0, 1), token 1 -> expert 1 (row 2).
# kernel_cases/case21_ref_permute_with_mask_map_trans.py:90-98 (same map in case22:109-117,
# case24:90-98 (int32), case30:80-88, case32:97-105 (int32)).
MAP_EM = torch.tensor([[0, -1], [-1, 2], [1, -1], [-1, -1]], dtype=torch.int64)


def test_permute_known_answer_case21():
    # case21...:88-103: inp = arange(8).reshape(2,4)+1 bf16; out rows = [inp0, inp0, inp1]
    inp = torch.arange(2 * 4, dtype=torch.bfloat16).reshape(2, 4) + 1
    out = ref_torch.permute_expert_major(inp, MAP_EM)
    assert out.shape == (3, 4)
    assert torch.equal(out, torch.stack([inp[0], inp[0], inp[1]]))
    out_c, _ = oracle_c.permute(inp.view(torch.int16).numpy(), MAP_EM.numpy(), 3, expert_major=True)
    assert np.array_equal(out_c, torch.stack([inp[0], inp[0], inp[1]]).view(torch.int16).numpy())


def test_permute_with_probs_known_answer_case22():
    # case22...:106-134: probs [[10,0,20,0],[0,30,0,0]] -> permuted_probs [10,20,30]; row not scaled.
    inp = torch.arange(2 * 4, dtype=torch.bfloat16).reshape(2, 4) + 1
    probs = torch.tensor([[10.0, 0.0, 20.0, 0.0], [0.0, 30.0, 0.0, 0.0]])
    out, pp = ref_torch.permute_expert_major(inp, MAP_EM, probs)
    assert torch.equal(pp, torch.tensor([10.0, 20.0, 30.0]))
    assert torch.equal(out[0], inp[0]) and not torch.equal(out[0], (inp[0].float() * 10).to(inp.dtype))
    out_c, pp_c = oracle_c.permute(inp.view(torch.int16).numpy(), MAP_EM.numpy(), 3, probs.numpy(),
                                   expert_major=True)
    assert np.array_equal(pp_c, np.array([10.0, 20.0, 30.0], np.float32))
    assert np.array_equal(out_c, out.view(torch.int16).numpy())


def test_permute_known_answer_case30():
    # case30...:77-98: same scatter, grad instead of inp; a pre-scaled grad changes the output.
    grad = torch.arange(2 * 4, dtype=torch.bfloat16).reshape(2, 4) + 1
    out = ref_torch.permute_expert_major(grad, MAP_EM)
    assert torch.equal(out, torch.stack([grad[0], grad[0], grad[1]]))
    scaled = ref_torch.permute_expert_major(grad * torch.full((2, 1), 0.25).to(grad.dtype), MAP_EM)
    assert not torch.equal(scaled, out)


def test_unpermute_known_answer_case24():
    # case24...:87-102: grad_in [[4,1],[4,1],[7,0]] -> [[8,2],[7,0]] (fp32 and bf16).
    grad_in = torch.tensor([[4, 1], [4, 1], [7, 0]], dtype=torch.bfloat16)
    acc, stored = ref_torch.unpermute_mask(grad_in, MAP_EM.to(torch.int32))
    expect = torch.tensor([[8.0, 2.0], [7.0, 0.0]])
    assert torch.equal(acc, expect) and torch.equal(stored, expect.to(torch.bfloat16))
    assert torch.equal(ref_torch.unpermute(grad_in, MAP_EM), expect.to(torch.bfloat16))
    out_c, acc_c = oracle_c.unpermute(grad_in.view(torch.int16).numpy().view(np.uint16), MAP_EM.numpy())
    assert np.array_equal(acc_c, expect.numpy())
    assert np.array_equal(out_c, expect.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


def test_unpermute_probgrad_known_answer_case32():
    # case32...:95-118: acc [[8,2],[7,0]], gathered [[10,0,20,0],[0,30,0,0]].
    grad_in = torch.tensor([[4, 1], [4, 1], [7, 0]], dtype=torch.bfloat16)
    prob_grad = torch.tensor([10.0, 20.0, 30.0])
    acc, stored, gathered = ref_torch.unpermute_mask_probgrad(grad_in, MAP_EM.to(torch.int32), prob_grad)
    expect_prob = torch.tensor([[10.0, 0.0, 20.0, 0.0], [0.0, 30.0, 0.0, 0.0]])
    assert torch.equal(acc, torch.tensor([[8.0, 2.0], [7.0, 0.0]]))
    assert torch.equal(gathered, expect_prob)
    dact, dprobs = ref_torch.permute_bwd(grad_in, prob_grad, MAP_EM)
    assert torch.equal(dact, stored) and torch.equal(dprobs, expect_prob)
    assert np.array_equal(oracle_c.prob_gather(prob_grad.numpy(), MAP_EM.numpy()), expect_prob.numpy())


def test_topk_known_answer_case23():
    # case23...:74-86: [[0.1,0.5,0.3,0.2],[4,1,3,2]], k=2 -> values [[0.5,0.3],[4,3]], idx [[1,2],[0,2]].
    inp = torch.tensor([[0.1, 0.5, 0.3, 0.2], [4.0, 1.0, 3.0, 2.0]], dtype=torch.float32)
    v, i = ref_torch.topk(inp, 2)
    assert torch.equal(v, torch.tensor([[0.5, 0.3], [4.0, 3.0]]))
    assert torch.equal(i, torch.tensor([[1, 2], [0, 2]]))
    vc, ic = oracle_c.topk(inp.numpy(), 2)
    assert np.array_equal(vc, v.numpy()) and np.array_equal(ic, i.numpy())


@pytest.mark.parametrize("bits_in,bits_out", [
    (0x3F808000, 0x3F80),  # tie, even LSB: rounds down (case25...:82-90)
    (0x3F818000, 0x3F82),  # tie, odd LSB: rounds up (case25...:92-99)
    (0x3F808001, 0x3F81),  # above the tie: up
    (0x3F807FFF, 0x3F80),  # below the tie: down
    (0x7F7FFFFF, 0x7F80),  # largest finite fp32 rounds to +inf
    (0xFF800000, 0xFF80),  # -inf stays -inf
    (0x80000000, 0x8000),  # -0 keeps its sign
    (0x7FC00001, 0x7FC0),  # NaN -> canonical quiet NaN
])
def test_bf16_rne_known_answers_case25(bits_in, bits_out):
    x = torch.tensor([bits_in], dtype=torch.int64).to(torch.int32).view(torch.float32)
    got = ref_torch.round_bf16_rne(x).view(torch.int16).item() & 0xFFFF
    assert got == bits_out
    assert oracle_c.bf16_rne(x.numpy())[0] == bits_out
    # torch's own conversion agrees on every non-NaN case (its vectorised CPU path
    # does not canonicalise NaN payloads; the kernels emit 0x7FC0 for any NaN).
    if not torch.isnan(x).any():
        assert (x.to(torch.bfloat16).view(torch.int16).item() & 0xFFFF) == bits_out


def test_row_id_map_case12_generator_total():
    # case12...:39 asserts R = 5 * 16384 + 16384/4 = 86016 for its seeded mask; the
    # row-id map must then be a bijection onto [0, 86016) (checked at a reduced size elsewhere).
    from conftest import load_pkg

    rm, _ = load_pkg().inputs.reference_routing_mask(16384, 320)
    assert int(rm.sum()) == 86016
    em, tm = ref_torch.row_id_map(rm)
    vals = tm[tm >= 0]
    assert vals.numel() == 86016 and torch.equal(vals.sort().values, torch.arange(86016))


def test_modular_map_invariants_case21():
    # case21...:126: with (t + k) mod E routing and E > topk, row_id_map[TOPK, 0] == -1.
    m = ref_torch.modular_row_id_map(64, 16, 8)
    assert m[8, 0].item() == -1
    assert int((m >= 0).sum()) == 64 * 8
