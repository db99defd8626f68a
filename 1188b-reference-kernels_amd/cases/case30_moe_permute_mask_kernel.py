"""case30 deep_ep moe_permute_mask_kernel<bf16, false> on gfx950 (combine backward).

Drop-in for reference_permute_mask
(kernel_cases/case30_ref_moe_permute_mask_kernel.py:44-58): scatter grad[t]
to output[row_id_map[e, t]], num_out = max(row_id_map)+1, no probs.
"""
from __future__ import annotations

import torch

from .. import inputs, ops
from ._common import check_scatter_shapes, expert_major_map, permute_from_map

M = 16384
HIDDEN = 8192
NUM_EXPERTS = 320
TOPK = 8


def permute_mask(grad: torch.Tensor, row_id_map: torch.Tensor) -> torch.Tensor:
    check_scatter_shapes(grad, row_id_map)
    out, _ = permute_from_map(grad, row_id_map, None, ops.EXPERT_MAJOR)
    return out


def make_row_id_map(num_tokens: int = M, num_experts: int = NUM_EXPERTS, topk: int = TOPK, device="cuda"):
    return expert_major_map(inputs.modular_routing_mask(num_tokens, num_experts, topk), torch.int64, device)


kernel_function = permute_mask
