"""case24 deep_ep moe_unpermute_mask_kernel<bf16, 8, false> on gfx950 (combine forward).

Drop-in for reference_unpermute_mask
(kernel_cases/case24_ref_moe_unpermute_mask_kernel_false.py:45-68): returns
(fp32 hidden sum, bf16 stored grad_x); int32 expert-major map; ValueError
when the map points past grad_in.  make_row_id_map follows :71-84.
"""
from __future__ import annotations

import torch

from .. import inputs, ops
from ._common import expert_major_map

M = 16384
HIDDEN = 8192
NUM_EXPERTS = 320
TOPK = 8


def unpermute_mask(grad_in: torch.Tensor, row_id_map: torch.Tensor):
    """(acc fp32 [T,H], acc.to(bf16)) with acc[t] = sum_e float(grad_in[row_id_map[e,t]])."""
    if row_id_map.ndim != 2 or grad_in.ndim != 2:
        raise ValueError(f"shapes grad_in {tuple(grad_in.shape)} row_id_map {tuple(row_id_map.shape)}")
    if row_id_map.numel() and int(row_id_map.max().item()) >= grad_in.shape[0]:
        raise ValueError("row_id_map points past grad_in")
    return ops.unpermute(grad_in, row_id_map, layout=ops.EXPERT_MAJOR, with_acc=True)


def make_row_id_map(num_tokens: int = M, num_experts: int = NUM_EXPERTS, topk: int = TOPK, device="cuda"):
    """Expert-major int32 map. Token t goes to experts (t + k) mod num_experts."""
    return expert_major_map(inputs.modular_routing_mask(num_tokens, num_experts, topk), torch.int32, device)


kernel_function = unpermute_mask
