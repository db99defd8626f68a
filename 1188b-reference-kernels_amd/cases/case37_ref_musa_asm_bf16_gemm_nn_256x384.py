"""case37 ref_musa_asm_bf16_gemm_nn_256x384 on gfx950: one expert's fc1 dgrad.

Drop-in for the GEMM the case times (kernel_cases/case37_ref_musa_asm_bf16_gemm_nn_256x384.py:65,
`torch.matmul(grad_output, weight)`): dgrad [M, N] = grad_output [M, K] @ weight [K, N],
both row-major, bf16 in / fp32 accumulate / bf16 out, alpha 1, beta 0 (:1-12).  It is the
one-group case of the grouped dgrad.  `make_inputs` draws the same seeded tensors as the
reference's (:52-57); the fp32 golden and the tolerance rule (:47-49, :68-76) live in the
tests, not here.
"""
from __future__ import annotations

import torch

from ._common import grouped_dgrad

M = 288   # representative expert token count (:42)
K = 5120  # fc1 out_features, the reduction
N = 8192  # hidden size, the dgrad columns

CASE = {"id": 37, "name": "ref_musa_asm_bf16_gemm_nn_256x384", "dtype": "bf16 in / fp32 accumulate / bf16 out",
        "backward": False}


def kernel_function(grad_output: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """grad_output [M, K] @ weight [K, N] -> [M, N] bf16."""
    if grad_output.ndim != 2 or weight.ndim != 2 or grad_output.shape[1] != weight.shape[0]:
        raise ValueError(f"shapes grad_output {tuple(grad_output.shape)} weight {tuple(weight.shape)}: "
                         "need [M, K] @ [K, N]")
    return grouped_dgrad(grad_output, weight.unsqueeze(0), [grad_output.shape[0]])


def make_inputs(seed: int = 0, device="cuda", m: int = M, k: int = K, n: int = N):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    grad_output = torch.randn(m, k, generator=g, dtype=torch.bfloat16)
    weight = torch.randn(k, n, generator=g, dtype=torch.bfloat16)
    return grad_output.to(device), weight.to(device)
