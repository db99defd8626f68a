"""Eager-PyTorch CPU restatement of the reference's MoE dispatch math.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Every function runs on
whatever device its inputs are on, but is meant for CPU tensors.  Paths are
relative to the reference repository.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch


# ------------------------------------------------------------------ bf16 RNE
def round_bf16_rne(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 by round-to-nearest-even on the top 16 bits.

    kernel_cases/case25_ref_unary_cast_fp32_to_bf16.py:56-66 (bit formula),
    with NaN mapped to 0x7FC0 like torch's own conversion.
    """
    bits = x.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) >> 16) & 0xFFFF
    nan = torch.isnan(x)
    rounded = torch.where(nan, torch.full_like(rounded, 0x7FC0), rounded)
    return rounded.to(torch.int32).to(torch.int16).view(torch.bfloat16).view_as(x)


# ------------------------------------------------------------- row-id map
def row_id_map(routing_map: torch.Tensor):
    """(row_id_map [E,T] int64, row_id_map_non_trans [T,E] int64).

    kernel_cases/case12_moe_row_id_map_pass2.py:43-50 (make_row_id_map) and
    :59-61 (Model.forward returns (row.t().contiguous(), row)).
    """
    mask = routing_map.to(torch.int64)
    within = torch.cumsum(mask, dim=0) - 1
    counts = mask.sum(dim=0)
    offset = torch.cumsum(counts, dim=0) - counts
    row = torch.where(mask > 0, within + offset.unsqueeze(0), torch.full_like(within, -1))
    return row.t().contiguous(), row.contiguous()


def expert_offsets(routing_map: torch.Tensor) -> torch.Tensor:
    """int32 [E+1]: first row of each expert and the routed total (cumsum of counts)."""
    counts = routing_map.to(torch.int64).sum(dim=0)
    return torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(counts, 0)]).to(torch.int32)


def modular_row_id_map(num_tokens: int, num_experts: int, topk: int) -> torch.Tensor:
    """Expert-major int64 map for (t + k) mod E routing.

    kernel_cases/case21_ref_permute_with_mask_map_trans.py:71-84 (same body in
    case22...:72-85, case24...:71-84 (int32), case30...:61-74, case32...:79-92 (int32)).
    """
    choice = (torch.arange(num_tokens)[:, None] + torch.arange(topk)) % num_experts
    selected = torch.zeros(num_experts, num_tokens, dtype=torch.bool)
    selected.scatter_(0, choice.t(), True)
    counts = selected.sum(dim=1)
    offset = torch.cumsum(counts, 0) - counts
    within = selected.long().cumsum(dim=1) - 1
    empty = torch.full((num_experts, num_tokens), -1, dtype=torch.int64)
    return torch.where(selected, within + offset[:, None], empty)


# ------------------------------------------------------------------ permute
def permute_token_major(x: torch.Tensor, row_id_map: torch.Tensor, probs: torch.Tensor, num_out: int):
    """(out [num_out,H], permuted_probs [num_out]) for a token-major [T,E] map.

    kernel_cases/case17_moe_permute_with_mask_map.py:58-71 (Model.forward).
    """
    n, e = row_id_map.shape
    dst = row_id_map.reshape(-1)
    keep = dst >= 0
    tok = torch.arange(n, device=x.device).repeat_interleave(e)
    src_rows = tok[keep]
    dst_rows = dst[keep]
    out = x.new_zeros((num_out, x.shape[1]))
    out.index_copy_(0, dst_rows, x.index_select(0, src_rows))
    permuted_probs = probs.new_zeros(num_out)
    permuted_probs.index_copy_(0, dst_rows, probs.reshape(-1)[keep])
    return out, permuted_probs


def source_tokens(row_id_map: torch.Tensor, num_out: int) -> torch.Tensor:
    """int32 [num_out]: the token each permuted row is copied from (-1 where no entry names the row).

    No reference function: the inverse of the token-major map of case12
    (kernel_cases/case12_moe_row_id_map_pass2.py:43-61), i.e. the index_select
    source of case17's permute (kernel_cases/case17_moe_permute_with_mask_map.py:58-71):
    permute_token_major(x, map, ...)[0][p] == x[source_tokens(map)[p]].
    """
    n, e = row_id_map.shape
    dst = row_id_map.reshape(-1)
    keep = (dst >= 0) & (dst < num_out)
    tok = torch.arange(n, dtype=torch.int32).repeat_interleave(e)
    out = torch.full((num_out,), -1, dtype=torch.int32)
    out[dst[keep]] = tok[keep]
    return out


def permute_expert_major(inp: torch.Tensor, row_id_map: torch.Tensor, probs: Optional[torch.Tensor] = None):
    """Scatter for an expert-major [E,T] map, num_out = max + 1.

    kernel_cases/case21_ref_permute_with_mask_map_trans.py:52-68 (no probs),
    kernel_cases/case22_ref_moe_permute_mask_kernel_true.py:47-69 (with probs),
    kernel_cases/case30_ref_moe_permute_mask_kernel.py:44-58 (no probs).
    Returns out, or (out, permuted_probs) when probs is given.
    """
    if row_id_map.ndim != 2 or inp.ndim != 2 or row_id_map.shape[1] != inp.shape[0]:
        raise ValueError(f"shapes inp {tuple(inp.shape)} row_id_map {tuple(row_id_map.shape)}")
    experts, tokens = row_id_map.shape
    if probs is not None and probs.shape != (tokens, experts):
        raise ValueError(f"probs {tuple(probs.shape)} expected {(tokens, experts)}")
    valid = row_id_map >= 0
    if not bool(valid.any()):
        empty = inp.new_empty((0, inp.shape[1]))
        return empty if probs is None else (empty, probs.new_empty((0,)))
    dest = row_id_map[valid]
    num_out = int(dest.max().item()) + 1
    token = torch.arange(tokens).view(1, -1).expand_as(row_id_map)[valid]
    out = inp.new_zeros((num_out, inp.shape[1]))
    out[dest] = inp[token]
    if probs is None:
        return out
    expert = torch.arange(experts).view(-1, 1).expand_as(row_id_map)[valid]
    permuted_probs = probs.new_zeros((num_out,))
    permuted_probs[dest] = probs[token, expert]
    return out, permuted_probs


# ---------------------------------------------------------------- unpermute
def unpermute(pin: torch.Tensor, row_id_map: torch.Tensor) -> torch.Tensor:
    """out[t] = bf16(sum_e float(pin[row_id_map[e,t]])) for an expert-major map.

    kernel_cases/case15_moe_unpermute_mask_fwd.py:58-64 (Model.forward).
    """
    valid = row_id_map >= 0
    src = row_id_map[valid]
    dst = valid.nonzero(as_tuple=True)[1]
    out = torch.zeros(row_id_map.shape[1], pin.shape[1], dtype=torch.float32, device=pin.device)
    out.index_add_(0, dst, pin.index_select(0, src).float())
    return out.to(pin.dtype)


def unpermute_merge(pin: torch.Tensor, row_id_map: torch.Tensor, probs: torch.Tensor, *,
                    expert_major: bool = True, with_acc: bool = False):
    """out[t] = bf16(sum_{e asc} probs[t,e] * float(pin[map(t,e)])): the merge form.

    No reference function (TE's with_merging_probs); closed form of case15's
    Model.forward (kernel_cases/case15_moe_unpermute_mask_fwd.py:58-64) with each
    gathered row scaled by its prob before index_add_ -- multiply, then add,
    in the same ascending-expert order.
    """
    m = row_id_map if expert_major else row_id_map.t()
    valid = m >= 0
    e_idx, dst = valid.nonzero(as_tuple=True)
    src = m[valid]
    w = probs[dst, e_idx].float()
    acc = torch.zeros(m.shape[1], pin.shape[1], dtype=torch.float32, device=pin.device)
    acc.index_add_(0, dst, pin.index_select(0, src).float() * w[:, None])
    return (acc, acc.to(pin.dtype)) if with_acc else acc.to(pin.dtype)


def unpermute_mask(grad_in: torch.Tensor, row_id_map: torch.Tensor):
    """(acc fp32, acc.to(bf16)): per-expert index_add_ loop.

    kernel_cases/case24_ref_moe_unpermute_mask_kernel_false.py:45-68.
    """
    if row_id_map.ndim != 2 or grad_in.ndim != 2:
        raise ValueError(f"shapes grad_in {tuple(grad_in.shape)} row_id_map {tuple(row_id_map.shape)}")
    experts, tokens = row_id_map.shape
    if row_id_map.numel() and int(row_id_map.max().item()) >= grad_in.shape[0]:
        raise ValueError("row_id_map points past grad_in")
    acc = torch.zeros(tokens, grad_in.shape[1], dtype=torch.float32)
    token_ids = torch.arange(tokens)
    for expert in range(experts):
        src_row = row_id_map[expert]
        mask = src_row >= 0
        if not bool(mask.any()):
            continue
        rows = src_row[mask].long()
        acc.index_add_(0, token_ids[mask], grad_in.index_select(0, rows).float())
    return acc, acc.to(grad_in.dtype)


def permute_bwd(dperm_act: torch.Tensor, dpp: torch.Tensor, row_id_map: torch.Tensor):
    """(dact [T,H] bf16, dprobs [T,E] fp32).

    kernel_cases/case18_moe_permute_bwd_unpermute_mask.py:68-78 (Model.forward).
    """
    e, n = row_id_map.shape
    h = dperm_act.shape[1]
    valid = row_id_map >= 0
    e_idx, dst = valid.nonzero(as_tuple=True)
    src = row_id_map[e_idx, dst]
    dact = torch.zeros(n, h, dtype=torch.float32, device=dperm_act.device)
    dact.index_add_(0, dst, dperm_act.index_select(0, src).float())
    dprobs = torch.zeros(n * e, dtype=torch.float32, device=dperm_act.device)
    dprobs.index_copy_(0, dst * e + e_idx, dpp.index_select(0, src))
    return dact.to(dperm_act.dtype), dprobs.view(n, e)


def unpermute_mask_probgrad(grad_in: torch.Tensor, row_id_map: torch.Tensor, prob_grad: torch.Tensor):
    """(acc fp32, bf16, grad_probs [T,E]).

    kernel_cases/case32_ref_moe_unpermute_mask_kernel.py:46-76.
    """
    if row_id_map.ndim != 2 or grad_in.ndim != 2:
        raise ValueError(f"shapes grad_in {tuple(grad_in.shape)} row_id_map {tuple(row_id_map.shape)}")
    experts, tokens = row_id_map.shape
    if prob_grad.ndim != 1 or prob_grad.shape[0] != grad_in.shape[0]:
        raise ValueError(f"prob_grad {tuple(prob_grad.shape)} does not match grad_in {tuple(grad_in.shape)}")
    if row_id_map.numel() and int(row_id_map.max().item()) >= grad_in.shape[0]:
        raise ValueError("row_id_map points past grad_in")
    acc = torch.zeros(tokens, grad_in.shape[1], dtype=torch.float32)
    gathered = torch.zeros(tokens, experts, dtype=torch.float32)
    token_ids = torch.arange(tokens)
    for expert in range(experts):
        src_row = row_id_map[expert]
        mask = src_row >= 0
        if not bool(mask.any()):
            continue
        rows = src_row[mask].long()
        acc.index_add_(0, token_ids[mask], grad_in.index_select(0, rows).float())
        gathered[mask, expert] = prob_grad.index_select(0, rows).float()
    return acc, acc.to(grad_in.dtype), gathered


# -------------------------------------------------------------------- top-k
def topk(inp: torch.Tensor, k: int):
    """(values, indices): first k of a stable descending sort of each row.

    kernel_cases/case23_ref_aten_topk.py:47-62 (reference_topk).
    """
    if inp.ndim != 2:
        raise ValueError(f"expected 2D input, got {tuple(inp.shape)}")
    if not (1 <= k <= inp.shape[1]):
        raise ValueError(f"k={k} out of range for N={inp.shape[1]}")
    values, indices = torch.sort(inp, dim=1, descending=True, stable=True)
    return values[:, :k].contiguous(), indices[:, :k].contiguous()


def mask_and_probs(values: torch.Tensor, indices: torch.Tensor, num_experts: int):
    """(routing_map bool [T,E], probs fp32 [T,E]) from top-k results.

    Mask: zeros(T,E,bool).scatter_(1, idx, True)
    (kernel_cases/case18_moe_permute_bwd_unpermute_mask.py:86-88).  Probs:
    softmax over the k selected values, scattered (closed form; no reference function).
    """
    T = values.shape[0]
    rm = torch.zeros(T, num_experts, dtype=torch.bool)
    rm.scatter_(1, indices, True)
    probs = torch.zeros(T, num_experts, dtype=torch.float32)
    probs.scatter_(1, indices, torch.softmax(values.float(), dim=-1))
    return rm, probs


# ------------------------------------------------------------- grouped GEMM
def grouped_gemm(x: torch.Tensor, w: torch.Tensor, sizes: Sequence[int]) -> torch.Tensor:
    """cat_g(x[seg_g] @ w[g].T) in the inputs' dtype (per-group torch.mm, then cat).

    kernel_cases/case03_moe_grouped_gemm_fc1_fwd.py:57-64 (= case04...:57-64).
    """
    outs, off = [], 0
    for i, m in enumerate(sizes):
        outs.append(torch.mm(x[off:off + m], w[i].t()))
        off += m
    return torch.cat(outs, dim=0)


def grouped_gemm_fp32(x: torch.Tensor, w: torch.Tensor, sizes: Sequence[int]) -> torch.Tensor:
    """fp32-accumulated golden: cat_g(x[seg_g].float() @ w[g].float().T), fp32 out.

    kernel_cases/case35_ref_musa_asm_bf16_gemm_nt_256x384.py:41-48 (reference_fp32)
    applied per group of case03/case04's Model.forward.
    """
    outs, off = [], 0
    for i, m in enumerate(sizes):
        outs.append(x[off:off + m].float().matmul(w[i].float().t()))
        off += m
    if not outs:
        return torch.zeros(0, w.shape[1], dtype=torch.float32)
    return torch.cat(outs, dim=0)


def grouped_gemm_dgrad(dy: torch.Tensor, w: torch.Tensor, sizes: Sequence[int]) -> torch.Tensor:
    """cat_g(dy[seg_g] @ w[g]) in the inputs' dtype (per-group torch.mm, then cat).

    kernel_cases/case07_moe_grouped_gemm_fc1_dgrad.py:57-64 (= case08, case13, case19 :57-64).
    """
    outs, off = [], 0
    for i, m in enumerate(sizes):
        outs.append(torch.mm(dy[off:off + m], w[i]))
        off += m
    return torch.cat(outs, dim=0)


def grouped_gemm_dgrad_fp32(dy: torch.Tensor, w: torch.Tensor, sizes: Sequence[int]) -> torch.Tensor:
    """fp32-accumulated golden of the dgrad: cat_g(dy[seg_g].float() @ w[g].float()), fp32 out.

    kernel_cases/case37_ref_musa_asm_bf16_gemm_nn_256x384.py:47-49 (reference_fp32, one group)
    applied per group of case07's Model.forward.
    """
    outs, off = [], 0
    for i, m in enumerate(sizes):
        outs.append(dy[off:off + m].float().matmul(w[i].float()))
        off += m
    if not outs:
        return torch.zeros(0, w.shape[2], dtype=torch.float32)
    return torch.cat(outs, dim=0)


def grouped_gemm_wgrad(dy: torch.Tensor, x: torch.Tensor, sizes: Sequence[int]) -> torch.Tensor:
    """stack_g(dy[seg_g].T @ x[seg_g]) in the inputs' dtype (per-group torch.mm, then stack).

    kernel_cases/case09_moe_grouped_gemm_fc1_wgrad.py:57-64 (= case05 :57-64).
    """
    outs, off = [], 0
    for m in sizes:
        outs.append(torch.mm(dy[off:off + m].t(), x[off:off + m]))
        off += m
    return torch.stack(outs, dim=0)


def grouped_gemm_wgrad_fp32(dy: torch.Tensor, x: torch.Tensor, sizes: Sequence[int]) -> torch.Tensor:
    """fp32-accumulated golden of the wgrad: stack_g(dy[seg_g].float().T @ x[seg_g].float()), fp32 out.

    The fp32 form of case09's Model.forward (case37...:47-49's reference_fp32 rule).
    """
    outs, off = [], 0
    for m in sizes:
        outs.append(dy[off:off + m].float().t().matmul(x[off:off + m].float()))
        off += m
    return torch.stack(outs, dim=0)


def router_logits_fp32(inp: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fp32-accumulated router logits: inp.float() @ weight.float().T.

    kernel_cases/case38_ref_musa_asm_bf16_ssgemm_nt_320x256.py:46-53 (reference_fp32).
    """
    return inp.float().matmul(weight.float().t())


def round_tf32_rne(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> tf32 (10 mantissa bits), ties to even, as fp32 values.

    kernel_cases/case39_ref_musa_asm_tf32_ssgemm_nn_384x256.py:51-58 (= case31...:52-58):
    add 0x1000 unless the 13 dropped bits are exactly 0x1000 with an even kept LSB, then clear them.
    """
    bits = x.float().contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    low = bits & 0x1FFF
    lsb = (bits >> 13) & 1
    add = torch.where((low == 0x1000) & (lsb == 0), torch.zeros_like(bits), torch.full_like(bits, 0x1000))
    out = ((bits + add) & 0xFFFFE000) & 0xFFFFFFFF
    out = torch.where(out >= 2 ** 31, out - 2 ** 32, out)
    return out.to(torch.int32).view(torch.float32).view_as(x)


def router_dgrad_tf32(grad_output: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """tf32(grad_output) @ tf32(weight) in fp32: case39...:61-68 (reference_tf32)."""
    return round_tf32_rne(grad_output).matmul(round_tf32_rne(weight))


def router_wgrad_tf32(grad_output: torch.Tensor, inp: torch.Tensor) -> torch.Tensor:
    """tf32(grad_output)^T @ tf32(inp) in fp32: case31...:61-68 (reference_tf32)."""
    return round_tf32_rne(grad_output).transpose(0, 1).matmul(round_tf32_rne(inp))


def swiglu(y: torch.Tensor) -> torch.Tensor:
    """silu(y[:, :F]) * y[:, F:] in fp32, F = N/2 (gate first).  No reference function."""
    f = y.shape[1] // 2
    g, u = y[:, :f].float(), y[:, f:].float()
    return g * torch.sigmoid(g) * u


# ---------------------------------------------------------------- row gather
def index_select(src: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """kernel_cases/case06_cp_seq_chunk_index_select.py:38-40."""
    return torch.index_select(src, 0, index)


# ----------------------------------------------------------- MoE FFN forward
def moe_ffn_forward(x: torch.Tensor, logits: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, topk_k: int):
    """Composed forward (the reference has no entry point; chain of its cases):
    top-k (case23) -> mask/probs -> row-id map (case12) -> permute (case17) ->
    per-group torch.mm fc1 (case03) -> SwiGLU -> fc2 (case04) -> merge
    unpermute (case15 + probs).  bf16 GEMMs as the reference's Model does them.
    """
    E = logits.shape[1]
    values, indices = topk(logits, topk_k)
    rm, probs = mask_and_probs(values, indices, E)
    row_em, row_tm = row_id_map(rm)
    R = int(rm.sum())
    xp, _ = permute_token_major(x, row_tm, probs, R)
    sizes = rm.sum(dim=0).tolist()
    y = grouped_gemm(xp, w1, sizes)
    h = swiglu(y).to(torch.bfloat16)
    z = grouped_gemm(h, w2, sizes)
    return unpermute_merge(z, row_em, probs)


def moe_ffn_forward_fp32(x: torch.Tensor, logits: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, topk_k: int):
    """moe_ffn_forward with fp32-accumulated GEMMs (the golden of the bf16 tolerance checks).

    Same chain as moe_ffn_forward, each grouped GEMM as grouped_gemm_fp32
    (kernel_cases/case35_ref_musa_asm_bf16_gemm_nt_256x384.py:41-48 per group of
    kernel_cases/case03_moe_grouped_gemm_fc1_fwd.py:57-64 and case04...:57-64),
    rounded to bf16 where the layer stores its intermediates: h after SwiGLU
    and z after fc2; then the merge of unpermute_merge.  Every output row
    depends only on its own token, so a subset of tokens gives those tokens'
    rows of the full layer.
    """
    E = logits.shape[1]
    values, indices = topk(logits, topk_k)
    rm, probs = mask_and_probs(values, indices, E)
    row_em, row_tm = row_id_map(rm)
    R = int(rm.sum())
    xp, _ = permute_token_major(x, row_tm, probs, R)
    sizes = rm.sum(dim=0).tolist()
    h = swiglu(grouped_gemm_fp32(xp, w1, sizes)).to(torch.bfloat16)
    z = grouped_gemm_fp32(h, w2, sizes).to(torch.bfloat16)
    return unpermute_merge(z, row_em, probs)
