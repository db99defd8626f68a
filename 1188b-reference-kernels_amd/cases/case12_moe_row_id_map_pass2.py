"""case12 moe_row_id_map_pass2 on gfx950.

Drop-in for kernel_results/case12_moe_row_id_map_pass2/kernel.py:4-6
(`kernel_function(routing_map) -> (row_id_map [E,T] int64, row_id_map_non_trans [T,E] int64)`),
math kernel_cases/case12_moe_row_id_map_pass2.py:43-61, generator :30-40.
"""
from __future__ import annotations

from .. import inputs, ops

TOKENS = 16384
NUM_EXPERTS = 320

CASE = {"id": 12, "name": "moe_row_id_map_pass2", "kernel": "_row_id_map_pass_2_kernel",
        "profiler_avg_ms": 4.24, "backward": False}


def make_routing_map(tokens: int = TOKENS, experts: int = NUM_EXPERTS):
    return inputs.reference_routing_mask(tokens, experts)[0]


def get_init_inputs():
    return []


def get_inputs(device="cuda"):
    return [make_routing_map().to(device)]


def kernel_function(routing_map):
    """routing_map [T,E] bool -> (row_id_map [E,T] int64, row_id_map_non_trans [T,E] int64)."""
    if routing_map.dim() != 2:
        raise RuntimeError("routing_map must be [T,E]")
    r = ops.row_id_map(routing_map, expert_major=True, token_major=True)
    return r["expert_major"], r["token_major"]
