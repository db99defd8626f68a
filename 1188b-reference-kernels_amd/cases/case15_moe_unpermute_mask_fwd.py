"""case15 moe_unpermute_mask_fwd on gfx950.

Drop-in for kernel_results/case15_moe_unpermute_mask_fwd/kernel.py:4-5
(`kernel_function(pin, row_id_map) -> out [T,H]`), math
kernel_cases/case15_moe_unpermute_mask_fwd.py:58-64, generator :30-49, :71-77.
Accumulation is fp32 in ascending expert order (the reference's index_add_
order), so the result is bit-identical to the reference on the CPU.
"""
from __future__ import annotations

from .. import inputs, ops

TOKENS = 16384
HID = 8192
NUM_EXPERTS = 320

CASE = {"id": 15, "name": "moe_unpermute_mask_fwd",
        "kernel": "moe_unpermute_mask<__mt_bfloat16, float, long, false, false, true, 8>",
        "profiler_avg_ms": 3.27, "backward": False}


def make_routing_map(tokens: int = TOKENS, experts: int = NUM_EXPERTS):
    return inputs.reference_routing_mask(tokens, experts)[0]


def make_row_id_map_trans(routing_map, device="cuda"):
    """routing_map [T,E] -> row_id_map [E,T] int64 (-1 = unselected), on the GPU."""
    return ops.row_id_map(routing_map.to(device), expert_major=True, token_major=False)["expert_major"]


def get_init_inputs():
    return [NUM_EXPERTS]


def get_inputs(device="cuda", tokens: int = TOKENS, hidden: int = HID, experts: int = NUM_EXPERTS):
    rm = make_routing_map(tokens, experts)
    row_id_map = make_row_id_map_trans(rm, device)
    pin = inputs.case15_pin(int(rm.sum()), hidden)
    return [pin.to(device), row_id_map]


def kernel_function(pin, row_id_map):
    """out[t] = bf16(sum_e float(pin[row_id_map[e, t]])) over selected experts."""
    return ops.unpermute(pin, row_id_map, layout=ops.EXPERT_MAJOR)
