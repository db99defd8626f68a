"""case11 router_bwd_cast_bf16_to_fp32 on gfx950.

The case has no optimized bundle; this is the drop-in for its Model
(kernel_cases/case11_router_bwd_cast_bf16_to_fp32.py:38-44): `Model().forward(x) = x.to(torch.float32)`,
x bf16 [4096, 8192] (:32-33).  The reference get_inputs (:51-52) is unseeded; get_inputs
here takes a seed.
"""
from __future__ import annotations

import torch

from .. import inputs, ops

TOKENS = 4096
HID = 8192

CASE = {"id": 11, "name": "router_bwd_cast_bf16_to_fp32", "dtype": "bf16 -> fp32", "backward": False}


def kernel_function(x: torch.Tensor) -> torch.Tensor:
    return ops.cast(x, torch.float32)


class Model:
    """Model().forward(x) = x.to(torch.float32)."""

    def __call__(self, x):
        return kernel_function(x)

    forward = __call__


def get_init_inputs():
    return []


def get_inputs(device="cuda", seed: int = inputs.SEED_CONFIG_BASE + 61, tokens: int = TOKENS, hid: int = HID):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(tokens, hid, generator=g).to(torch.bfloat16).to(device)]
