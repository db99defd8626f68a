"""case06 cp_seq_chunk_index_select on gfx950 (row gather).

Drop-in for kernel_results/case06_cp_seq_chunk_index_select/kernel.py:4-7
(`kernel_function(k_ag, v_ag, index) -> (index_select(k_ag,0,index), index_select(v_ag,0,index))`),
math kernel_cases/case06_cp_seq_chunk_index_select.py:38-40, generator :47-52.

Out-of-range indices: torch.index_select (the case's Model) raises, and the
optimized bundle reads whatever memory the index points at (no bounds check,
kernel_results/case06_cp_seq_chunk_index_select/kernel.mu:9).  Here an index
outside [0, rows) gives a zero row: the kernel never reads out of bounds, and a
caller that needs the exception checks the index on the host first (one
min/max read, which the drop-in does not pay on every call).
"""
from __future__ import annotations

import torch

from .. import ops

CHUNKS = 2
TOK = 65536
HEADS = 16
DQK = 192
DV = 128

CASE = {"id": 6, "name": "cp_seq_chunk_index_select", "kernel": "triton_poi_fused_index_select_0",
        "profiler_avg_ms": 3.64, "backward": False}


def get_init_inputs():
    return []


def get_inputs(device="cuda", tok: int = TOK):
    torch.manual_seed(20261111)
    k_ag = torch.randn(CHUNKS, tok, HEADS, DQK).to(torch.bfloat16)
    v_ag = torch.randn(CHUNKS, tok, HEADS, DV).to(torch.bfloat16)
    index = torch.arange(CHUNKS, dtype=torch.int32)
    return [k_ag.to(device), v_ag.to(device), index.to(device)]


def kernel_function(k_ag, v_ag, index):
    return ops.index_select(k_ag, index), ops.index_select(v_ag, index)
