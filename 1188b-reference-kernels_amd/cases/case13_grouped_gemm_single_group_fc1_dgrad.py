"""case13 grouped_gemm_single_group_fc1_dgrad on gfx950.

The case has no optimized bundle; this is the drop-in for its Model
(kernel_cases/case13_grouped_gemm_single_group_fc1_dgrad.py:49-64):
`Model(num_groups, tokens).forward(dy [T,N], w [G,N,K]) -> cat_g(dy[seg_g] @ w[g])`
(the input gradient of a grouped linear layer, layout "NN") with the uniform
group_sizes of :43-46, plus `kernel_function(dy, w, m_splits=None)` for ragged
groups.  bf16 in / fp32 accumulate / bf16 out (:37).  The reference
get_inputs (:71-73) is unseeded; get_inputs here takes a seed.
"""
from __future__ import annotations

from .. import inputs
from ._common import grouped_gemm_case

_CASE = grouped_gemm_case("dgrad", case_id=13, name="grouped_gemm_single_group_fc1_dgrad", num_groups=1, tokens=4096,
                          n=5120, k=8192, seed=inputs.SEED_CONFIG_BASE + 63)
NUM_GROUPS, TOKENS, N, K, CASE = _CASE.NUM_GROUPS, _CASE.TOKENS, _CASE.N, _CASE.K, _CASE.CASE
group_sizes = _CASE.group_sizes
kernel_function = _CASE.kernel_function
Model = _CASE.Model
get_init_inputs = _CASE.get_init_inputs
get_inputs = _CASE.get_inputs
