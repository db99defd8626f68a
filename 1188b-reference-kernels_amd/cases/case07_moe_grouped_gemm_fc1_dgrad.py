"""case07 moe_grouped_gemm_fc1_dgrad on gfx950.

The case has no optimized bundle; this is the drop-in for its Model
(kernel_cases/case07_moe_grouped_gemm_fc1_dgrad.py:49-64):
`Model(num_groups, tokens).forward(dy [T,N], w [G,N,K]) -> cat_g(dy[seg_g] @ w[g])`
(the input gradient of a grouped linear layer, layout "NN") with the uniform
group_sizes of :43-46, plus `kernel_function(dy, w, m_splits=None)` for ragged
groups.  bf16 in / fp32 accumulate / bf16 out (:37).  The reference
get_inputs (:71-73) is unseeded; get_inputs here takes a seed.
"""
from __future__ import annotations

import torch

from .. import inputs
from ._common import grouped_dgrad

NUM_GROUPS = 40
TOKENS = 4096
N = 5120
K = 8192

CASE = {"id": 7, "name": "moe_grouped_gemm_fc1_dgrad", "dtype": "bf16 in / fp32 accumulate / bf16 out",
        "backward": False}


def group_sizes(total, groups):
    return inputs.uniform_group_sizes(total, groups)


def kernel_function(dy, w, m_splits=None):
    """dx[seg_g] = dy[seg_g] @ w[g] for consecutive row segments of sizes m_splits."""
    if m_splits is None:
        m_splits = group_sizes(dy.shape[0], w.shape[0])
    return grouped_dgrad(dy, w, m_splits)


class Model:
    """Model(num_groups, tokens).forward(dy, w) with uniform group sizes."""

    def __init__(self, num_groups=NUM_GROUPS, tokens=TOKENS):
        self.num_groups = num_groups
        self.sizes = group_sizes(tokens, num_groups)

    def __call__(self, dy, w):
        return kernel_function(dy, w, self.sizes)

    forward = __call__


def get_init_inputs():
    return [NUM_GROUPS, TOKENS]


def get_inputs(device="cuda", seed: int = inputs.SEED_CONFIG_BASE + 57, tokens: int = TOKENS, groups: int = NUM_GROUPS,
               n: int = N, k: int = K):
    g = torch.Generator().manual_seed(seed)
    dy = torch.randn(tokens, n, generator=g).to(torch.bfloat16)
    w = torch.randn(groups, n, k, generator=g).to(torch.bfloat16)
    return [dy.to(device), w.to(device)]
