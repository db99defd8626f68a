"""case25 ref_unary_cast_fp32_to_bf16 on gfx950.

Drop-in for the op the case times, inp.to(torch.bfloat16)
(kernel_cases/case25_ref_unary_cast_fp32_to_bf16.py:107): fp32 -> bf16 with round to nearest
even, the case's golden `reference_cast_fp32_to_bf16` / `round_bf16_rne` (:56-72) for finite
values; any NaN becomes 0x7FC0 (torch's scalar conversion).  `make_inputs` draws the same seeded tensor as the
reference's (:74-79).
"""
from __future__ import annotations

import torch

from .. import ops

M = 16384
N = 8192

CASE = {"id": 25, "name": "ref_unary_cast_fp32_to_bf16", "dtype": "fp32 -> bf16 (RNE)", "backward": False}


def kernel_function(inp: torch.Tensor) -> torch.Tensor:
    if inp.dtype != torch.float32:
        raise ValueError(f"expected fp32 input, got {inp.dtype}")
    return ops.cast(inp, torch.bfloat16)


def make_inputs(m: int = M, n: int = N, seed: int = 0, device="cuda"):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    inp = torch.randn(m, n, generator=g, dtype=torch.float32) * 8
    return inp.to(device)
