"""case22 deep_ep moe_permute_mask_kernel<bf16, true> on gfx950 (dispatch with probs).

Drop-in for reference_permute_mask_with_probs
(kernel_cases/case22_ref_moe_permute_mask_kernel_true.py:47-69):
(out [num_out,H], permuted_probs [num_out]) with num_out = max(row_id_map)+1;
the hidden row is copied, not scaled.  make_probs follows :88-103; the routing
generator (:72-85) and the shape constants (:41-44) are case21's, taken from
its module.
"""
from __future__ import annotations

import torch

from .. import inputs, ops
from ._common import check_scatter_shapes, permute_from_map
from .case21_permute_with_mask_map_trans import HIDDEN, M, NUM_EXPERTS, TOPK, make_row_id_map  # noqa: F401


def permute_mask_with_probs(inp: torch.Tensor, row_id_map: torch.Tensor, probs: torch.Tensor):
    """Scatter inp[token] and probs[token, expert] to the destination rows."""
    check_scatter_shapes(inp, row_id_map)
    experts, tokens = row_id_map.shape
    if probs.shape != (tokens, experts):
        raise ValueError(f"probs {tuple(probs.shape)} expected {(tokens, experts)}")
    return permute_from_map(inp, row_id_map, probs, ops.EXPERT_MAJOR)


def make_probs(row_id_map: torch.Tensor, seed: int = 0, device="cuda") -> torch.Tensor:
    """fp32 probs on the routed (token, expert) pairs; zeros elsewhere."""
    return inputs.case22_probs((row_id_map >= 0).cpu(), seed).to(device)


kernel_function = permute_mask_with_probs
