"""case31 ref_musa_asm_tf32_ssgemm_tn_128x256 on gfx950: the router wgrad in tf32.

Drop-in for the GEMM the case times (kernel_cases/case31_ref_musa_asm_tf32_ssgemm_tn_128x256.py:1-38,
`te_general_gemm(inp.to(fp32), grad_output, out_dtype=fp32, layout="NT", grad=True)`):
grad_weight [N, K] = tf32(grad_output [M, N])^T @ tf32(inp [M, K]), fp32 accumulate and out, its
golden `reference_tf32` (:61-68) with `round_tf32_rne` (:52-58).  `make_inputs` draws the same
seeded tensors as the reference's (:80-85).
"""
from __future__ import annotations

import torch

from .. import ops

M = 16384
N = 320   # num_experts, rows of grad_weight
K = 8192  # hidden, cols of grad_weight

CASE = {"id": 31, "name": "ref_musa_asm_tf32_ssgemm_tn_128x256", "dtype": "fp32 in (tf32 products) / fp32 out",
        "backward": False}


def kernel_function(grad_output: torch.Tensor, inp: torch.Tensor) -> torch.Tensor:
    return ops.router_wgrad_tf32(grad_output, inp)


def make_inputs(seed: int = 0, device="cuda", m: int = M, n: int = N, k: int = K):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    grad_output = torch.randn(m, n, generator=g, dtype=torch.float32)
    inp = torch.randn(m, k, generator=g, dtype=torch.bfloat16).float()
    return grad_output.to(device), inp.to(device)
