"""case17 moe_permute_with_mask_map on gfx950.

Drop-in for kernel_results/case17_moe_permute_with_mask_map/kernel.py:4-6
(`kernel_function(x, row_id_map, probs) -> (out [R,H] bf16, permuted_probs [R] fp32)`),
math kernel_cases/case17_moe_permute_with_mask_map.py:58-71, generator :30-48, :78-90.
Without `num_out` the row count is max(row_id_map)+1 (one scalar read back,
as in binding.cpp:24); with `num_out` (the case Model's num_out_tokens) rows
beyond the routed count are zero, as the Model's new_zeros leaves them.
"""
from __future__ import annotations

from .. import inputs, ops
from ._common import permute_from_map

TOKENS = 16384
HID = 8192
NUM_EXPERTS = 320

CASE = {"id": 17, "name": "moe_permute_with_mask_map",
        "kernel": "permute_with_mask_map<__mt_bfloat16, float, long, true>",
        "profiler_avg_ms": 3.11, "backward": False}


def make_routing_map(tokens: int = TOKENS, experts: int = NUM_EXPERTS):
    return inputs.reference_routing_mask(tokens, experts)


def make_row_id_map(routing_map, device="cuda"):
    """routing_map [T,E] -> row_id_map [T,E] int64 (non-trans), on the GPU."""
    return ops.row_id_map(routing_map.to(device), expert_major=False, token_major=True)["token_major"]


def get_init_inputs():
    return [NUM_EXPERTS, 86016]


def get_inputs(device="cuda", tokens: int = TOKENS, hidden: int = HID, experts: int = NUM_EXPERTS):
    rm, sel = make_routing_map(tokens, experts)
    row_id_map = make_row_id_map(rm, device)
    x, probs = inputs.case17_x_probs(sel, hidden, experts)
    return [x.to(device), row_id_map, probs.to(device)]


def kernel_function(x, row_id_map, probs, num_out=None):
    """(out [R,H] bf16, permuted_probs [R] fp32); R = num_out or max(row_id_map)+1."""
    if x.dim() != 2:
        raise RuntimeError("x must be [T,H]")
    if row_id_map.dim() != 2:
        raise RuntimeError("row_id_map must be [T,E]")
    if row_id_map.size(0) != x.size(0):
        raise RuntimeError("map/probs token dim mismatch")
    if num_out is None:
        return permute_from_map(x, row_id_map, probs.float(), ops.TOKEN_MAJOR)
    # num_out from the Model: no host read; the map is a row-id map (dense over its R rows),
    # and rows R..num_out-1 are zero-filled on the device.
    return ops.permute(x, row_id_map, probs.float(), num_out=num_out, layout=ops.TOKEN_MAJOR, zero_tail=True)


class Model:
    """The case's Model(num_experts, num_out_tokens) interface: forward(x, row_id_map, probs)."""

    def __init__(self, num_experts=NUM_EXPERTS, num_out_tokens=86016):
        self.num_experts = num_experts
        self.num_out = num_out_tokens

    def __call__(self, x, row_id_map, probs):
        return kernel_function(x, row_id_map, probs, num_out=self.num_out)

    forward = __call__
