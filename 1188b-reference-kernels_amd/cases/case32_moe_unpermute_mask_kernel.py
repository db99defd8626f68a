"""case32 deep_ep moe_unpermute_mask_kernel<bf16, 8, true> on gfx950 (dispatch backward).

Drop-in for reference_unpermute_mask
(kernel_cases/case32_ref_moe_unpermute_mask_kernel.py:46-76): returns
(fp32 hidden sum, bf16 grad_x, grad_probs [T,E]); int32 expert-major map;
ValueError on mismatched prob_grad or a map pointing past grad_in.
"""
from __future__ import annotations

import torch

from .. import inputs, ops
from ._common import expert_major_map

M = 16384
HIDDEN = 8192
NUM_EXPERTS = 320
TOPK = 8


def unpermute_mask(grad_in: torch.Tensor, row_id_map: torch.Tensor, prob_grad: torch.Tensor):
    if row_id_map.ndim != 2 or grad_in.ndim != 2:
        raise ValueError(f"shapes grad_in {tuple(grad_in.shape)} row_id_map {tuple(row_id_map.shape)}")
    if prob_grad.ndim != 1 or prob_grad.shape[0] != grad_in.shape[0]:
        raise ValueError(f"prob_grad {tuple(prob_grad.shape)} does not match grad_in {tuple(grad_in.shape)}")
    if row_id_map.numel() and int(row_id_map.max().item()) >= grad_in.shape[0]:
        raise ValueError("row_id_map points past grad_in")
    return ops.permute_bwd(grad_in, prob_grad.float(), row_id_map, layout=ops.EXPERT_MAJOR, with_acc=True)


def make_row_id_map(num_tokens: int = M, num_experts: int = NUM_EXPERTS, topk: int = TOPK, device="cuda"):
    return expert_major_map(inputs.modular_routing_mask(num_tokens, num_experts, topk), torch.int32, device)


kernel_function = unpermute_mask
