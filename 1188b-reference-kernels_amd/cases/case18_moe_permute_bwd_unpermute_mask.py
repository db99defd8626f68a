"""case18 moe_permute_bwd_unpermute_mask on gfx950.

The case has no optimized bundle; this is the drop-in for its Model.forward
(kernel_cases/case18_moe_permute_bwd_unpermute_mask.py:68-78):
`kernel_function(dperm_act, dpp, row_id_map) -> (dact [T,H] bf16, dprobs [T,E] fp32)`.
The reference generator (:85-92) is unseeded; get_inputs seeds it with
inputs.SEED_CASE18.
"""
from __future__ import annotations

import torch

from .. import inputs, ops

TOKENS = 4096
HID = 8192
NUM_EXPERTS = 320
TOPK = 8
NUM_OUT_TOKENS = TOKENS * TOPK

CASE = {"id": 18, "name": "moe_permute_bwd_unpermute_mask",
        "kernel": "moe_unpermute_mask<__mt_bfloat16, float, long, false, true, true, 8>",
        "upstream": "_moe_permute_mask_mapBackward", "backward": False}


def get_init_inputs():
    return [NUM_EXPERTS]


def get_inputs(device="cuda", tokens: int = TOKENS, hidden: int = HID, experts: int = NUM_EXPERTS,
               topk: int = TOPK, seed: int = inputs.SEED_CASE18):
    rm = inputs.case18_mask(tokens, experts, topk, seed)
    row_id_map = ops.row_id_map(rm.to(device), expert_major=True, token_major=False)["expert_major"]
    dperm_act = torch.randn(tokens * topk, hidden).to(torch.bfloat16)
    dpp = torch.randn(tokens * topk, dtype=torch.float32)
    return [dperm_act.to(device), dpp.to(device), row_id_map]


def kernel_function(dperm_act, dpp, row_id_map):
    """(dact [T,H], dprobs [T,E]) with dact[t] = sum_e dperm_act[map[e,t]], dprobs[t,e] = dpp[map[e,t]]."""
    return ops.permute_bwd(dperm_act, dpp, row_id_map, layout=ops.EXPERT_MAJOR)
