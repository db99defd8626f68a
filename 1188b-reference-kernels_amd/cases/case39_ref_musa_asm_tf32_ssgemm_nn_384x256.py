"""case39 ref_musa_asm_tf32_ssgemm_nn_384x256 on gfx950: the router dgrad in tf32.

Drop-in for the GEMM the case times (kernel_cases/case39_ref_musa_asm_tf32_ssgemm_nn_384x256.py:1-35,
`te_general_gemm(weight.to(fp32), grad_output, out_dtype=fp32, layout="NN", grad=True)`):
grad_input [M, N] = tf32(grad_output [M, K]) @ tf32(weight [K, N]), fp32 accumulate and out, its
golden `reference_tf32` (:61-68) with `round_tf32_rne` (:51-58).  `make_inputs` draws the same
seeded tensors as the reference's (:82-88).
"""
from __future__ import annotations

import torch

from .. import ops

M = 16384
K = 320   # num_experts
N = 8192  # hidden_size

CASE = {"id": 39, "name": "ref_musa_asm_tf32_ssgemm_nn_384x256", "dtype": "fp32 in (tf32 products) / fp32 out",
        "backward": False}


def kernel_function(grad_output: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return ops.router_dgrad_tf32(grad_output, weight)


def make_inputs(seed: int = 0, device="cuda", m: int = M, k: int = K, n: int = N):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    grad_output = torch.randn(m, k, generator=g, dtype=torch.float32)
    weight = torch.randn(k, n, generator=g, dtype=torch.bfloat16).float()
    return grad_output.to(device), weight.to(device)
