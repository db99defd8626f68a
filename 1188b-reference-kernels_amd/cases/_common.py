"""Helpers shared by the case modules."""
from __future__ import annotations

from types import SimpleNamespace

import torch

from .. import inputs, ops


def scatter_rows(row_id_map: torch.Tensor) -> tuple[int, bool]:
    """(num_out, dense): num_out = max(row_id_map) + 1 (0 if no entry is >= 0), the reference
    functions' output row count, and whether the entries >= 0 name every output row exactly once
    (as a row-id map's do), so that a scatter writes every row. A map with repeated entries is
    never dense, whatever its count.

    One pass over the map (moe_map_extent) and one read-back, where the reference reads its max
    (kernel_cases/case21_ref_permute_with_mask_map_trans.py:64,
    kernel_results/case17_moe_permute_with_mask_map/binding.cpp:24).
    """
    if row_id_map.numel() == 0:
        return 0, True
    mx, _, bijective = ops.map_extent(row_id_map)
    return mx + 1, bijective


def permute_from_map(inp: torch.Tensor, row_id_map: torch.Tensor, probs, layout: str):
    """The reference scatter with num_out = max(row_id_map) + 1 and zero-initialised outputs
    (new_zeros, kernel_cases/case22_ref_moe_permute_mask_kernel_true.py:63-67): a dense map
    writes every row, so the outputs are not cleared first; any other map gets zeroed outputs,
    so the rows no entry names stay zero.  Returns (out, permuted_probs or None)."""
    num_out, dense = scatter_rows(row_id_map)
    if num_out == 0:
        return inp.new_empty((0, inp.shape[1])), (None if probs is None else probs.new_empty((0,), dtype=torch.float32))
    out = pp = None
    if not dense:
        out = torch.zeros(num_out, inp.shape[1], dtype=inp.dtype, device=inp.device)
        if probs is not None:
            pp = torch.zeros(num_out, dtype=torch.float32, device=inp.device)
    return ops.permute(inp, row_id_map, probs, num_out=num_out, layout=layout, zero_tail=False, out=out,
                       permuted_probs=pp)


def expert_major_map(selected_em: torch.Tensor, dtype=torch.int64, device="cuda") -> torch.Tensor:
    """Expert-major row-id map [E, T] of an expert-major selection, built by the GPU kernel."""
    mask_tm = selected_em.t().contiguous().to(device)
    maps = ops.row_id_map(mask_tm, expert_major=dtype == torch.int64, token_major=False,
                          expert_major_i32=dtype == torch.int32)
    return maps["expert_major"] if dtype == torch.int64 else maps["expert_major_i32"]


def check_scatter_shapes(inp: torch.Tensor, row_id_map: torch.Tensor) -> None:
    if row_id_map.ndim != 2 or inp.ndim != 2 or row_id_map.shape[1] != inp.shape[0]:
        raise ValueError(f"shapes inp {tuple(inp.shape)} row_id_map {tuple(row_id_map.shape)}")


_OFFSETS_CACHE: dict = {}


def cached_offsets(m_splits, device) -> torch.Tensor:
    """Device int32 [G+1] offsets of host group sizes, uploaded once per (sizes, device).

    The case Models call their kernels with the same fixed sizes every time; the kernels only
    read the offsets, so one copy per device serves every call.
    """
    key = (tuple(int(m) for m in m_splits), str(torch.device(device)))
    t = _OFFSETS_CACHE.get(key)
    if t is None:
        if len(_OFFSETS_CACHE) >= 64:
            _OFFSETS_CACHE.clear()
        t = ops.group_offsets_from_splits(m_splits, device)
        _OFFSETS_CACHE[key] = t
    return t


def _split_offsets(m_splits, total: int, groups: int, what: str, device):
    if len(m_splits) != groups or sum(m_splits) != total:
        raise ValueError(f"m_splits (len {len(m_splits)}, sum {sum(m_splits)}) does not match {what}")
    return cached_offsets(m_splits, device)


def grouped_dgrad(dy: torch.Tensor, w: torch.Tensor, m_splits) -> torch.Tensor:
    """cat_g(dy[seg_g] @ w[g]) for consecutive row segments of sizes m_splits."""
    offsets = _split_offsets(m_splits, dy.shape[0], w.shape[0], f"dy {tuple(dy.shape)} and w {tuple(w.shape)}",
                             dy.device)
    return ops.grouped_gemm_dgrad(dy, w, offsets)


def grouped_wgrad(dy: torch.Tensor, x: torch.Tensor, m_splits) -> torch.Tensor:
    """stack_g(dy[seg_g].T @ x[seg_g]) for consecutive row segments of sizes m_splits."""
    offsets = _split_offsets(m_splits, dy.shape[0], len(m_splits), f"dy {tuple(dy.shape)} and x {tuple(x.shape)}",
                             dy.device)
    return ops.grouped_gemm_wgrad(dy, x, offsets)


def grouped_gemm_case(kind: str, *, case_id: int, name: str, num_groups: int, tokens: int, n: int, k: int,
                      seed: int) -> SimpleNamespace:
    """The module attributes of a grouped-GEMM case (the reference cases 03/04 "fwd", 07/08/13/19 "dgrad",
    05/09 "wgrad" share one shape: kernel_cases/case07_moe_grouped_gemm_fc1_dgrad.py:37-73 and its siblings):

    * NUM_GROUPS, TOKENS, N, K, CASE and group_sizes (uniform m_splits, the first `total % groups` one larger, :43-46);
    * kernel_function for ragged groups -- fwd: (x [T,K], w [G,N,K], m_splits=None, swiglu=False) ->
      cat_g(x[seg_g] @ w[g].T); dgrad: (dy [T,N], w [G,N,K], m_splits=None) -> cat_g(dy[seg_g] @ w[g]);
      wgrad: (dy [T,N], x [T,K], m_splits=None, num_groups=NUM_GROUPS) -> stack_g(dy[seg_g].T @ x[seg_g]);
    * Model(num_groups, tokens) whose forward is kernel_function with the uniform sizes (:49-64);
    * get_init_inputs and a seeded get_inputs (the reference's :71-73 is unseeded), N(0,1) bf16 tensors drawn in
      the order of the forward's arguments.
    """
    if kind not in ("fwd", "dgrad", "wgrad"):
        raise ValueError(f"kind {kind!r}")

    def group_sizes(total, groups):
        return inputs.uniform_group_sizes(total, groups)

    if kind == "fwd":
        def kernel_function(x, w, m_splits=None, swiglu=False):
            """out[seg_g] = x[seg_g] @ w[g].T for consecutive row segments of sizes m_splits."""
            if m_splits is None:
                m_splits = group_sizes(x.shape[0], w.shape[0])
            offsets = _split_offsets(m_splits, x.shape[0], w.shape[0], f"x {tuple(x.shape)} and w {tuple(w.shape)}",
                                     x.device)
            return ops.grouped_gemm(x, w, offsets, swiglu=swiglu)
    elif kind == "dgrad":
        def kernel_function(dy, w, m_splits=None):
            """dx[seg_g] = dy[seg_g] @ w[g] for consecutive row segments of sizes m_splits."""
            if m_splits is None:
                m_splits = group_sizes(dy.shape[0], w.shape[0])
            return grouped_dgrad(dy, w, m_splits)
    else:
        def kernel_function(dy, x, m_splits=None, num_groups=num_groups):
            """dw[g] = dy[seg_g].T @ x[seg_g] for consecutive row segments of sizes m_splits."""
            if m_splits is None:
                m_splits = group_sizes(dy.shape[0], num_groups)
            return grouped_wgrad(dy, x, m_splits)

    class Model:
        """Model(num_groups, tokens).forward(a, b) with uniform group sizes."""

        def __init__(self, num_groups=num_groups, tokens=tokens):
            self.num_groups = num_groups
            self.sizes = group_sizes(tokens, num_groups)

        def __call__(self, a, b):
            return kernel_function(a, b, self.sizes)

        forward = __call__

    def get_init_inputs():
        return [num_groups, tokens]

    if kind == "wgrad":
        def get_inputs(device="cuda", seed: int = seed, tokens: int = tokens, n: int = n, k: int = k):
            g = torch.Generator().manual_seed(seed)
            dy = torch.randn(tokens, n, generator=g).to(torch.bfloat16)
            x = torch.randn(tokens, k, generator=g).to(torch.bfloat16)
            return [dy.to(device), x.to(device)]
    else:
        def get_inputs(device="cuda", seed: int = seed, tokens: int = tokens, groups: int = num_groups, n: int = n,
                       k: int = k):
            g = torch.Generator().manual_seed(seed)
            a = torch.randn(tokens, k if kind == "fwd" else n, generator=g).to(torch.bfloat16)
            w = torch.randn(groups, n, k, generator=g).to(torch.bfloat16)
            return [a.to(device), w.to(device)]

    case = {"id": case_id, "name": name, "dtype": "bf16 in / fp32 accumulate / bf16 out", "backward": False}
    return SimpleNamespace(NUM_GROUPS=num_groups, TOKENS=tokens, N=n, K=k, CASE=case, group_sizes=group_sizes,
                           kernel_function=kernel_function, Model=Model, get_init_inputs=get_init_inputs,
                           get_inputs=get_inputs)
