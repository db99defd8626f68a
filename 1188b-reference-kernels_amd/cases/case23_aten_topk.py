"""case23 aten::topk on gfx950 (router top-k).

Drop-in for kernel_results/case23_aten_topk/kernel.py:14-25
(`kernel_function(input, k=8, dim=1, largest=True, sorted=True) -> (values, indices)`),
contract kernel_cases/case23_ref_aten_topk.py:47-62 (stable descending sort,
first k).  Same ValueErrors as the bundle; this build supports k <= 64
(the bundle stops at 8).
"""
from __future__ import annotations

import torch

from .. import inputs, ops

M = 16384
NUM_EXPERTS = 320
TOPK = 8
MAX_K = 64


def kernel_function(input, k=8, dim=1, largest=True, sorted=True):
    if not largest:
        raise ValueError("only largest=True is supported")
    if dim not in (1, -1):
        raise ValueError("only dim=1 is supported")
    if input.dim() != 2:
        raise ValueError(f"expected 2D input, got {input.dim()}D")
    n = int(input.shape[1])
    k = min(int(k), n)
    if k > MAX_K:
        raise ValueError(f"k={k} exceeds the {MAX_K} supported by this kernel")
    if input.dtype != torch.float32:
        raise RuntimeError("only float32 is supported")
    return ops.topk(input, k)


def make_inputs(seed: int = 0, device="cuda", m: int = M, n: int = NUM_EXPERTS):
    return inputs.case23_logits(m, n, seed).to(device)
