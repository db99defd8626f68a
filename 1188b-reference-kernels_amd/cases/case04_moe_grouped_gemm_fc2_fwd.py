"""case04 moe_grouped_gemm_fc2_fwd on gfx950.

The case has no optimized bundle; this is the drop-in for its Model
(kernel_cases/case04_moe_grouped_gemm_fc2_fwd.py:49-64):
`Model(num_groups, tokens).forward(x [T,K], w [G,N,K]) -> cat_g(x[seg_g] @ w[g].T)`
with the uniform group_sizes of :43-46, plus `kernel_function(x, w, m_splits=None)`
for ragged groups.  bf16 in / fp32 accumulate / bf16 out (:37).  The
reference get_inputs (:71-73) is unseeded; get_inputs here takes a seed.
"""
from __future__ import annotations

import torch

from .. import inputs, ops
from ._common import cached_offsets

NUM_GROUPS = 40
TOKENS = 4096
N = 8192
K = 2560

CASE = {"id": 4, "name": "moe_grouped_gemm_fc2_fwd", "dtype": "bf16 in / fp32 accumulate / bf16 out",
        "backward": False}


def group_sizes(total, groups):
    return inputs.uniform_group_sizes(total, groups)


def kernel_function(x, w, m_splits=None, swiglu=False):
    """out[seg_g] = x[seg_g] @ w[g].T for consecutive row segments of sizes m_splits."""
    if m_splits is None:
        m_splits = group_sizes(x.shape[0], w.shape[0])
    if len(m_splits) != w.shape[0] or sum(m_splits) != x.shape[0]:
        raise ValueError(f"m_splits (len {len(m_splits)}, sum {sum(m_splits)}) does not match x {tuple(x.shape)} "
                         f"and w {tuple(w.shape)}")
    offsets = cached_offsets(m_splits, x.device)
    return ops.grouped_gemm(x, w, offsets, swiglu=swiglu)


class Model:
    """Model(num_groups, tokens).forward(x, w) with uniform group sizes."""

    def __init__(self, num_groups=NUM_GROUPS, tokens=TOKENS):
        self.num_groups = num_groups
        self.sizes = group_sizes(tokens, num_groups)

    def __call__(self, x, w):
        return kernel_function(x, w, self.sizes)

    forward = __call__


def get_init_inputs():
    return [NUM_GROUPS, TOKENS]


def get_inputs(device="cuda", seed: int = inputs.SEED_CASE04, tokens: int = TOKENS, groups: int = NUM_GROUPS,
               n: int = N, k: int = K):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, k, generator=g).to(torch.bfloat16)
    w = torch.randn(groups, n, k, generator=g).to(torch.bfloat16)
    return [x.to(device), w.to(device)]
