"""case38 ref_musa_asm_bf16_ssgemm_nt_320x256 on gfx950: the router gate GEMM.

Drop-in for the GEMM the case times (kernel_cases/case38_ref_musa_asm_bf16_ssgemm_nt_320x256.py:1-35,
`te_general_gemm(weight, inp, out_dtype=torch.float32, layout="TN")`): logits [M, N] =
inp [M, K] @ weight [N, K]^T, bf16 in, fp32 accumulate, fp32 out (:8-13).  `make_inputs` draws
the same seeded tensors as the reference's (:56-61); its golden `reference_fp32` (:46-53) and
its explicit-sum check (:64-79) live in the tests.  `router_topk` is the same GEMM with the
router top-k, mask and merge probs fused into its epilogue.
"""
from __future__ import annotations

import torch

from .. import ops

M = 16384
K = 8192  # hidden_size
N = 320   # num_experts

CASE = {"id": 38, "name": "ref_musa_asm_bf16_ssgemm_nt_320x256", "dtype": "bf16 in / fp32 accumulate / fp32 out",
        "backward": False}


def kernel_function(inp: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """inp [M, K] bf16 @ weight [N, K]^T bf16 -> fp32 logits [M, N]."""
    return ops.router_logits(inp, weight)


def router_topk(inp: torch.Tensor, weight: torch.Tensor, k: int = 8):
    """(logits, values, indices, routing mask, merge probs) of the router in one kernel."""
    values, indices, logits, mask, probs = ops.router_topk(inp, weight, k, with_logits=True, with_mask=True,
                                                           with_probs=True)
    return logits, values, indices, mask, probs


def make_inputs(seed: int = 0, device="cuda", m: int = M, k: int = K, n: int = N):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    inp = torch.randn(m, k, generator=g, dtype=torch.bfloat16)
    weight = torch.randn(n, k, generator=g, dtype=torch.bfloat16)
    return inp.to(device), weight.to(device)
