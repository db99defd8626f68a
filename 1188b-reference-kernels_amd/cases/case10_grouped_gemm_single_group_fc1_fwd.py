"""case10 grouped_gemm_single_group_fc1_fwd on gfx950.

The case has no optimized bundle; this is the drop-in for its Model
(kernel_cases/case10_grouped_gemm_single_group_fc1_fwd.py:49-64):
`Model(num_groups, tokens).forward(x [T,K], w [G,N,K]) -> cat_g(x[seg_g] @ w[g].T)`
with one group of all 4096 rows (NUM_GROUPS = 1, :25-28) and the uniform
group_sizes of :43-46, plus `kernel_function(x, w, m_splits=None)` for ragged
groups.  bf16 in / fp32 accumulate / bf16 out (:37).  The reference
get_inputs (:71-73) is unseeded; get_inputs here takes a seed.
"""
from __future__ import annotations

from .. import inputs
from ._common import grouped_gemm_case

_CASE = grouped_gemm_case("fwd", case_id=10, name="grouped_gemm_single_group_fc1_fwd", num_groups=1, tokens=4096,
                          n=5120, k=8192, seed=inputs.SEED_CONFIG_BASE + 60)
NUM_GROUPS, TOKENS, N, K, CASE = _CASE.NUM_GROUPS, _CASE.TOKENS, _CASE.N, _CASE.K, _CASE.CASE
group_sizes = _CASE.group_sizes
kernel_function = _CASE.kernel_function
Model = _CASE.Model
get_init_inputs = _CASE.get_init_inputs
get_inputs = _CASE.get_inputs
