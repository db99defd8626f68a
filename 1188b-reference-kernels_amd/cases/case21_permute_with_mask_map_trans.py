"""case21 permute_with_mask_map_trans on gfx950 (TE unpermute backward, no probs).

Drop-in for reference_permute_with_mask_map_trans
(kernel_cases/case21_ref_permute_with_mask_map_trans.py:52-68): same arguments,
same ValueError on bad shapes, empty output when nothing is routed, num_out =
max(row_id_map)+1.  make_row_id_map follows :71-84 ((t + k) mod E routing).
"""
from __future__ import annotations

import torch

from .. import inputs, ops
from ._common import check_scatter_shapes, expert_major_map, permute_from_map

M = 16384
HIDDEN = 8192
NUM_EXPERTS = 320
TOPK = 8


def permute_with_mask_map_trans(inp: torch.Tensor, row_id_map: torch.Tensor) -> torch.Tensor:
    """Scatter inp[token] to output[row_id_map[expert, token]] when the id is not -1."""
    check_scatter_shapes(inp, row_id_map)
    out, _ = permute_from_map(inp, row_id_map, None, ops.EXPERT_MAJOR)
    return out


def make_row_id_map(num_tokens: int = M, num_experts: int = NUM_EXPERTS, topk: int = TOPK, device="cuda"):
    """Expert-major int64 map. Token t is routed to experts (t + k) mod num_experts."""
    return expert_major_map(inputs.modular_routing_mask(num_tokens, num_experts, topk), torch.int64, device)


kernel_function = permute_with_mask_map_trans
