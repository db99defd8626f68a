"""Oracle: a CPU restatement of the reference's MoE dispatch math.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import anything here, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or shipped.
The product path (the HIP library and its Python layer) does not import it.

Two independent restatements:
  * ref_torch -- eager PyTorch on the CPU, following the reference cases op for
    op (cumsum row-id map, index_select + index_copy_ permute, index_add_
    unpermute in ascending expert order, per-group torch.mm, stable-sort top-k).
    This is also the CPU baseline of bench.py.
  * oracle_c  -- plain C loops (moe_oracle.c, built by gcc into liboracle.so)
    for the integer/byte work and the ordered fp32 sums, wrapped for numpy.

Each function cites the reference file:line it follows.  How each one is
pinned (golden vectors, brute force, invariants) is stated in the test that
pins it (tests/test_oracle_*.py).
"""
