"""case30 deep_ep moe_permute_mask_kernel<bf16, false> on gfx950 (combine backward).

Drop-in for reference_permute_mask
(kernel_cases/case30_ref_moe_permute_mask_kernel.py:44-58): scatter grad[t]
to output[row_id_map[e, t]], num_out = max(row_id_map)+1, no probs -- the same
scatter as case21's, and the same routing generator (case30...:61-74 is
case21...:71-84), so both come from case21's module.
"""
from __future__ import annotations

import torch

from .case21_permute_with_mask_map_trans import (HIDDEN, M, NUM_EXPERTS, TOPK,  # noqa: F401
                                                 make_row_id_map, permute_with_mask_map_trans)


def permute_mask(grad: torch.Tensor, row_id_map: torch.Tensor) -> torch.Tensor:
    """Scatter grad[token] to output[row_id_map[expert, token]] when the id is not -1."""
    return permute_with_mask_map_trans(grad, row_id_map)


kernel_function = permute_mask
