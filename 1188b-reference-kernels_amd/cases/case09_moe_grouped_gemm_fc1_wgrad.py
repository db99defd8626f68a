"""case09 moe_grouped_gemm_fc1_wgrad on gfx950.

The case has no optimized bundle; this is the drop-in for its Model
(kernel_cases/case09_moe_grouped_gemm_fc1_wgrad.py:49-64):
`Model(num_groups, tokens).forward(dy [T,N], x [T,K]) -> stack_g(dy[seg_g].T @ x[seg_g])`
(the weight gradient of a grouped linear layer, layout "TN") with the uniform
group_sizes of :43-46, plus `kernel_function(dy, x, m_splits=None, num_groups=None)`
for ragged groups (a group without rows gets a zero gradient).  bf16 in /
fp32 accumulate / bf16 out (:37).  The reference get_inputs (:71-73) is
unseeded; get_inputs here takes a seed.
"""
from __future__ import annotations

from .. import inputs
from ._common import grouped_gemm_case

_CASE = grouped_gemm_case("wgrad", case_id=9, name="moe_grouped_gemm_fc1_wgrad", num_groups=40, tokens=4096,
                          n=5120, k=8192, seed=inputs.SEED_CONFIG_BASE + 59)
NUM_GROUPS, TOKENS, N, K, CASE = _CASE.NUM_GROUPS, _CASE.TOKENS, _CASE.N, _CASE.K, _CASE.CASE
group_sizes = _CASE.group_sizes
kernel_function = _CASE.kernel_function
Model = _CASE.Model
get_init_inputs = _CASE.get_init_inputs
get_inputs = _CASE.get_inputs
