"""Tensor-level API over the C ABI: validates, allocates outputs, launches.

Every function runs its HIP kernels on torch's current stream of the input's
device; torch tensors are only containers (allocation and streams).  There is
no CPU or eager-torch fallback: inputs must live on the GPU and the native
library must be built.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import (MOE_EPILOGUE_NONE, MOE_EPILOGUE_SWIGLU, MOE_IDX_I32, MOE_IDX_I64,
                   MOE_MAP_EXPERT_MAJOR, MOE_MAP_TOKEN_MAJOR, call, ptr, stream_handle)

TOKEN_MAJOR = "token_major"    # map [T, E]  (case12 non-trans, case17)
EXPERT_MAJOR = "expert_major"  # map [E, T]  (case12 trans, case15/18/21/22/24/30/32)

_LAYOUTS = {TOKEN_MAJOR: MOE_MAP_TOKEN_MAJOR, EXPERT_MAJOR: MOE_MAP_EXPERT_MAJOR}
_IDX = {torch.int32: MOE_IDX_I32, torch.int64: MOE_IDX_I64}


def _on_gpu(name: str, t: torch.Tensor) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device}); there is no CPU path")


def _dtype(name: str, t: torch.Tensor, *dtypes: torch.dtype) -> None:
    if t.dtype not in dtypes:
        raise TypeError(f"{name} must have dtype {' or '.join(map(str, dtypes))}, got {t.dtype}")


def _out(out: Optional[torch.Tensor], shape: tuple, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A caller-provided output (checked: GPU, dtype, shape, contiguous) or a new one."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    _on_gpu("out", out)
    _dtype("out", out, dtype)
    if tuple(out.shape) != tuple(shape) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {tuple(shape)} tensor, got {tuple(out.shape)}"
                         f"{'' if out.is_contiguous() else ' (non-contiguous)'}")
    return out


def _map_dims(row_id_map: torch.Tensor, layout: str) -> tuple[int, int]:
    """(tokens, experts) of a 2-D map in the given layout."""
    if row_id_map.ndim != 2:
        raise ValueError(f"row_id_map must be 2-D, got shape {tuple(row_id_map.shape)}")
    if layout not in _LAYOUTS:
        raise ValueError(f"map layout must be {TOKEN_MAJOR!r} or {EXPERT_MAJOR!r}, got {layout!r}")
    a, b = row_id_map.shape
    return (a, b) if layout == TOKEN_MAJOR else (b, a)


# --------------------------------------------------------------------- top-k
def topk(logits: torch.Tensor, k: int, *, with_mask: bool = False, with_probs: bool = False):
    """Row-wise top-k of fp32 router logits (torch.topk(dim=1, largest, sorted)).

    Returns (values fp32 [T,k], indices int64 [T,k]) and, on request, the
    routing mask bool [T,E] and the merge probs fp32 [T,E] (softmax over the k
    selected values, scattered; 0 elsewhere).
    """
    _on_gpu("logits", logits)
    _dtype("logits", logits, torch.float32)
    if logits.ndim != 2:
        raise ValueError(f"expected 2D input, got {tuple(logits.shape)}")
    T, E = logits.shape
    if not (1 <= k <= E):
        raise ValueError(f"k={k} out of range for N={E}")
    x = logits.contiguous()
    values = torch.empty(T, k, dtype=torch.float32, device=x.device)
    indices = torch.empty(T, k, dtype=torch.int64, device=x.device)
    mask = torch.empty(T, E, dtype=torch.bool, device=x.device) if with_mask else None
    probs = torch.empty(T, E, dtype=torch.float32, device=x.device) if with_probs else None
    call("moe_topk", ptr(x), T, E, k, ptr(values), ptr(indices),
         ptr(mask.view(torch.uint8)) if mask is not None else None, ptr(probs), stream_handle())
    out = [values, indices]
    if with_mask:
        out.append(mask)
    if with_probs:
        out.append(probs)
    return tuple(out)


def router_logits(inp: torch.Tensor, weight: torch.Tensor, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Router gate GEMM: inp [M, K] bf16 @ weight [N, K]^T bf16 -> fp32 logits [M, N] (fp32 accumulate)."""
    _on_gpu("inp", inp)
    _on_gpu("weight", weight)
    _dtype("inp", inp, torch.bfloat16)
    _dtype("weight", weight, torch.bfloat16)
    if inp.ndim != 2 or weight.ndim != 2 or inp.shape[1] != weight.shape[1]:
        raise ValueError(f"shapes inp {tuple(inp.shape)} weight {tuple(weight.shape)}: need [M,K] and [N,K]")
    M, K = inp.shape
    N = weight.shape[0]
    ic, wc = inp.contiguous(), weight.contiguous()
    out = _out(out, (M, N), torch.float32, inp.device)
    call("moe_router_logits", ptr(ic), M, K, ptr(wc), N, ptr(out), None, 0, stream_handle())
    return out


def router_topk(inp: torch.Tensor, weight: torch.Tensor, k: int, *, with_logits: bool = False,
                with_mask: bool = False, with_probs: bool = False):
    """router_logits followed by topk on its rows (two kernels, one call).

    Returns (values, indices) and, on request and in this order, the fp32 logits [M, N],
    the routing mask bool [M, N] and the merge probs fp32 [M, N] -- the outputs of topk.
    """
    _on_gpu("inp", inp)
    _on_gpu("weight", weight)
    _dtype("inp", inp, torch.bfloat16)
    _dtype("weight", weight, torch.bfloat16)
    if inp.ndim != 2 or weight.ndim != 2 or inp.shape[1] != weight.shape[1]:
        raise ValueError(f"shapes inp {tuple(inp.shape)} weight {tuple(weight.shape)}: need [M,K] and [N,K]")
    M, K = inp.shape
    N = weight.shape[0]
    if not (1 <= k <= N):
        raise ValueError(f"k={k} out of range for N={N}")
    ic, wc = inp.contiguous(), weight.contiguous()
    dev = inp.device
    values = torch.empty(M, k, dtype=torch.float32, device=dev)
    indices = torch.empty(M, k, dtype=torch.int64, device=dev)
    logits = torch.empty(M, N, dtype=torch.float32, device=dev) if with_logits else None
    mask = torch.empty(M, N, dtype=torch.bool, device=dev) if with_mask else None
    probs = torch.empty(M, N, dtype=torch.float32, device=dev) if with_probs else None
    ws_bytes = 0 if with_logits else _lib.lib().moe_router_workspace_size(M, K, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    call("moe_router_topk", ptr(ic), M, K, ptr(wc), N, k, ptr(logits), ptr(values), ptr(indices),
         ptr(mask.view(torch.uint8)) if mask is not None else None, ptr(probs), ptr(ws), ws_bytes, stream_handle())
    out = [values, indices]
    if with_logits:
        out.append(logits)
    if with_mask:
        out.append(mask)
    if with_probs:
        out.append(probs)
    return tuple(out)


def cast(x: torch.Tensor, dtype: torch.dtype, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x.to(dtype) for bf16 -> fp32 (exact) and fp32 -> bf16 (round to nearest even, any NaN -> 0x7FC0)."""
    _on_gpu("x", x)
    pairs = {(torch.bfloat16, torch.float32): "moe_cast_bf16_to_f32", (torch.float32, torch.bfloat16): "moe_cast_f32_to_bf16"}
    fn = pairs.get((x.dtype, dtype))
    if fn is None:
        raise TypeError(f"cast supports bfloat16 -> float32 and float32 -> bfloat16, got {x.dtype} -> {dtype}")
    xc = x.contiguous()
    if out is None:
        out = torch.empty(x.shape, dtype=dtype, device=x.device)
    elif out.dtype != dtype or out.shape != x.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of the input's shape and the target dtype")
    call(fn, ptr(xc), xc.numel(), ptr(out), stream_handle())
    return out


def _ws(nbytes: int, device) -> Optional[torch.Tensor]:
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes else None


def router_dgrad_tf32(grad_output: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """grad_input [M, N] = tf32(grad_output [M, K]) @ tf32(weight [K, N]), fp32 in/accumulate/out."""
    for n, t in (("grad_output", grad_output), ("weight", weight)):
        _on_gpu(n, t)
        _dtype(n, t, torch.float32)
    if grad_output.ndim != 2 or weight.ndim != 2 or grad_output.shape[1] != weight.shape[0]:
        raise ValueError(f"shapes grad_output {tuple(grad_output.shape)} weight {tuple(weight.shape)}: need [M,K] @ [K,N]")
    M, K = grad_output.shape
    N = weight.shape[1]
    go, wc = grad_output.contiguous(), weight.contiguous()
    out = torch.empty(M, N, dtype=torch.float32, device=go.device)
    nbytes = _lib.lib().moe_router_dgrad_tf32_workspace_size(M, K, N)
    ws = _ws(nbytes, go.device)
    call("moe_router_dgrad_tf32", ptr(go), M, K, ptr(wc), N, ptr(out), ptr(ws), nbytes, stream_handle())
    return out


def router_wgrad_tf32(grad_output: torch.Tensor, inp: torch.Tensor) -> torch.Tensor:
    """grad_weight [N, K] = tf32(grad_output [M, N])^T @ tf32(inp [M, K]), fp32 in/accumulate/out."""
    for n, t in (("grad_output", grad_output), ("inp", inp)):
        _on_gpu(n, t)
        _dtype(n, t, torch.float32)
    if grad_output.ndim != 2 or inp.ndim != 2 or grad_output.shape[0] != inp.shape[0]:
        raise ValueError(f"shapes grad_output {tuple(grad_output.shape)} inp {tuple(inp.shape)}: need [M,N] and [M,K]")
    M, N = grad_output.shape
    K = inp.shape[1]
    go, ic = grad_output.contiguous(), inp.contiguous()
    out = torch.empty(N, K, dtype=torch.float32, device=go.device)
    nbytes = _lib.lib().moe_router_wgrad_tf32_workspace_size(M, N, K)
    ws = _ws(nbytes, go.device)
    call("moe_router_wgrad_tf32", ptr(go), M, N, ptr(ic), K, ptr(out), ptr(ws), nbytes, stream_handle())
    return out


def map_extent(row_id_map: torch.Tensor) -> tuple[int, int, bool]:
    """(max(-1, largest entry), number of entries >= 0, whether those entries name every row of [0, max] exactly
    once) of a row-id map (any layout, int32 or int64), read back to the host after one pass over the map; the
    scatter functions' output row count is the first + 1."""
    _on_gpu("row_id_map", row_id_map)
    if row_id_map.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"row_id_map dtype {row_id_map.dtype}: int32 or int64 expected")
    m = row_id_map.contiguous()
    n = m.numel()
    res = torch.empty(3, dtype=torch.int64, device=m.device)
    nbytes = _lib.lib().moe_map_extent_workspace_size(n)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=m.device)
    call("moe_map_extent", ptr(m), MOE_IDX_I64 if m.dtype == torch.int64 else MOE_IDX_I32, n, ptr(res), ptr(ws), nbytes,
         stream_handle())
    mx, cnt, bijective = res.tolist()
    return int(mx), int(cnt), bool(bijective)


# ---------------------------------------------------------------- row-id map
def row_id_map(routing_map: torch.Tensor, *, expert_major: bool = True, token_major: bool = True,
               expert_major_i32: bool = False, expert_offsets: bool = False, src_rows: Optional[int] = None,
               src_out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> dict:
    """Row-id map of a bool/uint8 routing mask [T, E].

    Returns a dict with the requested outputs: "expert_major" int64 [E,T],
    "token_major" int64 [T,E], "expert_major_i32" int32 [E,T],
    "expert_offsets" int32 [E+1] (offsets[e] = first row of expert e,
    offsets[E] = number of routed rows R) and, with `src_rows` (or `src_out`),
    "src_token" int32 [src_rows]: the source token of each permuted row
    (src_token[map(t, e)] = t; src_rows = R, e.g. T * k for top-k routing,
    gives every row; rows >= R are left unwritten).
    """
    _on_gpu("routing_map", routing_map)
    _dtype("routing_map", routing_map, torch.bool, torch.uint8)
    if routing_map.ndim != 2:
        raise ValueError("routing_map must be [T,E]")
    T, E = routing_map.shape
    m = routing_map.contiguous().view(torch.uint8)
    dev = m.device
    res = {}
    if expert_major:
        res["expert_major"] = torch.empty(E, T, dtype=torch.int64, device=dev)
    if token_major:
        res["token_major"] = torch.empty(T, E, dtype=torch.int64, device=dev)
    if expert_major_i32:
        res["expert_major_i32"] = torch.empty(E, T, dtype=torch.int32, device=dev)
    if expert_offsets:
        res["expert_offsets"] = torch.empty(E + 1, dtype=torch.int32, device=dev)
    if src_out is not None:
        if src_out.dtype != torch.int32 or not src_out.is_contiguous() or src_out.ndim != 1:
            raise ValueError("src_out must be a contiguous 1-d int32 tensor")
        res["src_token"] = src_out
    elif src_rows is not None:
        if src_rows < 0:
            raise ValueError(f"src_rows must be >= 0, got {src_rows}")
        res["src_token"] = torch.empty(src_rows, dtype=torch.int32, device=dev)
    src = res.get("src_token")
    ws_bytes = _lib.lib().moe_row_id_map_workspace_size(T, E)
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    call("moe_row_id_map", ptr(m), T, E, ptr(res.get("expert_major")), ptr(res.get("token_major")),
         ptr(res.get("expert_major_i32")), ptr(res.get("expert_offsets")), ptr(src),
         0 if src is None else src.numel(), ptr(workspace), workspace.numel() * workspace.element_size(),
         stream_handle())
    return res


# ------------------------------------------------------------------- permute
def permute(x: torch.Tensor, row_id_map: torch.Tensor, probs: Optional[torch.Tensor] = None, *,
            num_out: int, layout: str = TOKEN_MAJOR, zero_tail: bool = True,
            out: Optional[torch.Tensor] = None, permuted_probs: Optional[torch.Tensor] = None):
    """out[map(t,e)] = x[t]; permuted_probs[map(t,e)] = probs[t,e] for map >= 0.

    Rows of `out` at index >= R (R = number of entries >= 0) are zero when
    `zero_tail` (the reference's new_zeros); that assumes the entries name the
    rows 0..R-1, as a row-id map's do -- for other maps pass zeroed `out` /
    `permuted_probs` and zero_tail=False (rows no entry names are left as they
    are).  Pass zero_tail=False when num_out is known to equal R.
    Returns (out, permuted_probs or None).
    """
    _on_gpu("x", x)
    _on_gpu("row_id_map", row_id_map)
    _dtype("x", x, torch.bfloat16)
    _dtype("row_id_map", row_id_map, torch.int32, torch.int64)
    if x.ndim != 2:
        raise ValueError(f"x must be [T,H], got {tuple(x.shape)}")
    T, E = _map_dims(row_id_map, layout)
    if T != x.shape[0]:
        raise ValueError(f"shapes inp {tuple(x.shape)} row_id_map {tuple(row_id_map.shape)}")
    H = x.shape[1]
    xc, mc = x.contiguous(), row_id_map.contiguous()
    pc = None
    if probs is not None:
        _on_gpu("probs", probs)
        if tuple(probs.shape) != (T, E):
            raise ValueError(f"probs {tuple(probs.shape)} expected {(T, E)}")
        pc = probs.contiguous().to(torch.float32)
    out = _out(out, (num_out, H), x.dtype, x.device)
    if pc is not None and permuted_probs is None:
        permuted_probs = torch.empty(num_out, dtype=torch.float32, device=x.device)
    ws = None
    ws_bytes = 0
    if zero_tail:
        ws_bytes = _lib.lib().moe_permute_workspace_size(T)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    call("moe_permute", ptr(xc), T, H, ptr(mc), _IDX[mc.dtype], _LAYOUTS[layout], E, ptr(pc), ptr(out),
         ptr(permuted_probs) if pc is not None else None, num_out, int(zero_tail), ptr(ws), ws_bytes,
         stream_handle())
    return out, (permuted_probs if pc is not None else None)


# ----------------------------------------------------------------- unpermute
def unpermute(pin: torch.Tensor, row_id_map: torch.Tensor, merge_probs: Optional[torch.Tensor] = None, *,
              layout: str = EXPERT_MAJOR, out: Optional[torch.Tensor] = None, with_acc: bool = False):
    """out[t] = bf16(sum_{e asc} [merge_probs[t,e] *] float(pin[map(t,e)])), fp32 accumulate.

    Returns out, or (acc fp32 [T,H], out) with `with_acc`.
    """
    _on_gpu("pin", pin)
    _on_gpu("row_id_map", row_id_map)
    _dtype("pin", pin, torch.bfloat16)
    _dtype("row_id_map", row_id_map, torch.int32, torch.int64)
    if pin.ndim != 2:
        raise ValueError(f"pin must be [R,H], got {tuple(pin.shape)}")
    T, E = _map_dims(row_id_map, layout)
    R, H = pin.shape
    pc, mc = pin.contiguous(), row_id_map.contiguous()
    wc = None
    if merge_probs is not None:
        _on_gpu("merge_probs", merge_probs)
        if tuple(merge_probs.shape) != (T, E):
            raise ValueError(f"merge_probs {tuple(merge_probs.shape)} expected {(T, E)}")
        wc = merge_probs.contiguous().to(torch.float32)
    out = _out(out, (T, H), pin.dtype, pin.device)
    acc = torch.empty(T, H, dtype=torch.float32, device=pin.device) if with_acc else None
    call("moe_unpermute", ptr(pc), R, H, ptr(mc), _IDX[mc.dtype], _LAYOUTS[layout], E, T, ptr(wc), ptr(out),
         ptr(acc), stream_handle())
    return (acc, out) if with_acc else out


def permute_bwd(dperm_act: torch.Tensor, dpp: torch.Tensor, row_id_map: torch.Tensor, *,
                layout: str = EXPERT_MAJOR, with_acc: bool = False):
    """(dact [T,H] bf16, dprobs [T,E] fp32) of the permute backward (case18 math).

    With `with_acc`: (acc fp32 [T,H], dact, dprobs).
    """
    _on_gpu("dperm_act", dperm_act)
    _on_gpu("dpp", dpp)
    _on_gpu("row_id_map", row_id_map)
    _dtype("dperm_act", dperm_act, torch.bfloat16)
    _dtype("dpp", dpp, torch.float32)
    _dtype("row_id_map", row_id_map, torch.int32, torch.int64)
    if dperm_act.ndim != 2:
        raise ValueError(f"dperm_act must be [R,H], got {tuple(dperm_act.shape)}")
    T, E = _map_dims(row_id_map, layout)
    R, H = dperm_act.shape
    if dpp.ndim != 1 or dpp.shape[0] != R:
        raise ValueError(f"dpp {tuple(dpp.shape)} does not match dperm_act {tuple(dperm_act.shape)}")
    ac, pc, mc = dperm_act.contiguous(), dpp.contiguous(), row_id_map.contiguous()
    dact = torch.empty(T, H, dtype=dperm_act.dtype, device=dperm_act.device)
    dprobs = torch.empty(T, E, dtype=torch.float32, device=dperm_act.device)
    acc = torch.empty(T, H, dtype=torch.float32, device=dperm_act.device) if with_acc else None
    call("moe_permute_bwd", ptr(ac), R, H, ptr(pc), ptr(mc), _IDX[mc.dtype], _LAYOUTS[layout], E, T,
         ptr(dact), ptr(dprobs), ptr(acc), stream_handle())
    return (acc, dact, dprobs) if with_acc else (dact, dprobs)


# -------------------------------------------------------------- index_select
def index_select(src: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """torch.index_select(src, 0, index) for bf16 src and int32/int64 index."""
    _on_gpu("src", src)
    _on_gpu("index", index)
    _dtype("src", src, torch.bfloat16)
    _dtype("index", index, torch.int32, torch.int64)
    if src.ndim < 1:
        raise ValueError("src must have at least one dimension")
    if index.ndim != 1:
        raise ValueError("index must be one-dimensional")
    sc, ic = src.contiguous(), index.contiguous()
    row = 1
    for d in sc.shape[1:]:
        row *= d
    out = torch.empty((ic.shape[0], *sc.shape[1:]), dtype=sc.dtype, device=sc.device)
    call("moe_index_select", ptr(sc), sc.shape[0], row, ptr(ic), _IDX[ic.dtype], ic.shape[0], ptr(out),
         stream_handle())
    return out


# -------------------------------------------------------------- grouped GEMM
def group_offsets_from_splits(m_splits: Sequence[int], device) -> torch.Tensor:
    """int32 [G+1] exclusive prefix of host m_splits, on `device`."""
    offs = [0]
    for m in m_splits:
        if m < 0:
            raise ValueError(f"negative group size {m}")
        offs.append(offs[-1] + int(m))
    return torch.tensor(offs, dtype=torch.int32).to(device, non_blocking=True)


def _gemm_workspace(M: int, K: int, N: int, G: int, workspace: Optional[torch.Tensor], device):
    """The grouped GEMM's workspace (the list of groups whose last row tile has at most 128 rows):
    allocated when None; an empty tensor runs without one (every row tile 256 rows)."""
    nbytes = _lib.lib().moe_grouped_gemm_workspace_size(M, K, N, G)
    if nbytes == 0 or (workspace is not None and workspace.numel() == 0):
        return None, 0
    if workspace is None or workspace.numel() * workspace.element_size() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
    return workspace, workspace.numel() * workspace.element_size()


def grouped_gemm(a: torch.Tensor, w: torch.Tensor, group_offsets: torch.Tensor, *, swiglu: bool = False,
                 out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[rows of g] = a[rows of g] @ w[g]^T (bf16 in, fp32 accumulate, bf16 out).

    a bf16 [M, K]; w bf16 [G, N, K]; group_offsets int32 [G+1] on the device.
    With swiglu, out[:, j] = silu(y[:, j]) * y[:, N/2 + j] and out is [M, N/2].
    workspace: uint8 device tensor (moe_grouped_gemm_workspace_size bytes; allocated when None,
    an empty tensor: none).
    """
    _on_gpu("a", a)
    _on_gpu("w", w)
    _on_gpu("group_offsets", group_offsets)
    _dtype("a", a, torch.bfloat16)
    _dtype("w", w, torch.bfloat16)
    _dtype("group_offsets", group_offsets, torch.int32)
    if a.ndim != 2 or w.ndim != 3 or a.shape[1] != w.shape[2]:
        raise ValueError(f"shapes a {tuple(a.shape)} w {tuple(w.shape)}: need a [M,K], w [G,N,K]")
    G, N, K = w.shape
    if group_offsets.shape != (G + 1,):
        raise ValueError(f"group_offsets {tuple(group_offsets.shape)} expected ({G + 1},)")
    M = a.shape[0]
    ac, wc, oc = a.contiguous(), w.contiguous(), group_offsets.contiguous()
    ncols = N // 2 if swiglu else N
    out = _out(out, (M, ncols), torch.bfloat16, a.device)
    ws, ws_bytes = _gemm_workspace(M, K, N, G, workspace, a.device)
    call("moe_grouped_gemm", ptr(ac), M, K, ptr(wc), G, N, ptr(oc),
         MOE_EPILOGUE_SWIGLU if swiglu else MOE_EPILOGUE_NONE, ptr(out), ptr(ws), ws_bytes, stream_handle())
    return out


def permute_index(row_id_map: torch.Tensor, num_out: int, *, layout: str = TOKEN_MAJOR, fill: bool = True,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Source token of each permuted row: out[map(t, e)] = t (int32 [num_out]).

    The inverse of a row-id map; with fill, rows that no map entry names are -1.
    """
    _on_gpu("row_id_map", row_id_map)
    _dtype("row_id_map", row_id_map, torch.int32, torch.int64)
    T, E = _map_dims(row_id_map, layout)
    if num_out < 0:
        raise ValueError(f"num_out must be >= 0, got {num_out}")
    if out is None:
        out = torch.empty(num_out, dtype=torch.int32, device=row_id_map.device)
    elif out.dtype != torch.int32 or out.numel() < num_out or not out.is_contiguous():
        raise ValueError("out must be a contiguous int32 tensor of at least num_out elements")
    m = row_id_map.contiguous()
    call("moe_permute_index", ptr(m), _IDX[m.dtype], _LAYOUTS[layout], T, E, ptr(out), num_out, int(fill),
         stream_handle())
    return out


def grouped_gemm_gather(x: torch.Tensor, a_rows: torch.Tensor, w: torch.Tensor, group_offsets: torch.Tensor, *,
                        swiglu: bool = False, out: Optional[torch.Tensor] = None,
                        workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """grouped_gemm(x[a_rows], w, group_offsets) without materialising x[a_rows].

    x bf16 [X, K]; a_rows int32 [M] (an index outside [0, X) reads a zero row).
    """
    _on_gpu("x", x)
    _on_gpu("a_rows", a_rows)
    _on_gpu("w", w)
    _on_gpu("group_offsets", group_offsets)
    _dtype("x", x, torch.bfloat16)
    _dtype("a_rows", a_rows, torch.int32)
    _dtype("w", w, torch.bfloat16)
    _dtype("group_offsets", group_offsets, torch.int32)
    if x.ndim != 2 or w.ndim != 3 or x.shape[1] != w.shape[2] or a_rows.ndim != 1:
        raise ValueError(f"shapes x {tuple(x.shape)} a_rows {tuple(a_rows.shape)} w {tuple(w.shape)}: "
                         "need x [X,K], a_rows [M], w [G,N,K]")
    G, N, K = w.shape
    if group_offsets.shape != (G + 1,):
        raise ValueError(f"group_offsets {tuple(group_offsets.shape)} expected ({G + 1},)")
    M = a_rows.shape[0]
    xc, rc, wc, oc = x.contiguous(), a_rows.contiguous(), w.contiguous(), group_offsets.contiguous()
    ncols = N // 2 if swiglu else N
    out = _out(out, (M, ncols), torch.bfloat16, x.device)
    ws, ws_bytes = _gemm_workspace(M, K, N, G, workspace, x.device)
    call("moe_grouped_gemm_gather", ptr(xc), x.shape[0], ptr(rc), M, K, ptr(wc), G, N, ptr(oc),
         MOE_EPILOGUE_SWIGLU if swiglu else MOE_EPILOGUE_NONE, ptr(out), ptr(ws), ws_bytes, stream_handle())
    return out


def grouped_gemm_dgrad(dy: torch.Tensor, w: torch.Tensor, group_offsets: torch.Tensor, *,
                       out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dx[rows of g] = dy[rows of g] @ w[g] (bf16 in, fp32 accumulate, bf16 out).

    dy bf16 [M, N]; w bf16 [G, N, K] (the forward's weights); group_offsets int32 [G+1] on the device.
    workspace: uint8 device tensor of moe_grouped_gemm_dgrad_workspace_size bytes (a one-group split's
    fp32 partials, or the list of groups whose last row tile has at most 128 rows); allocated when
    None or smaller than that size; an empty tensor runs without one.
    """
    _on_gpu("dy", dy)
    _on_gpu("w", w)
    _on_gpu("group_offsets", group_offsets)
    _dtype("dy", dy, torch.bfloat16)
    _dtype("w", w, torch.bfloat16)
    _dtype("group_offsets", group_offsets, torch.int32)
    if dy.ndim != 2 or w.ndim != 3 or dy.shape[1] != w.shape[1]:
        raise ValueError(f"shapes dy {tuple(dy.shape)} w {tuple(w.shape)}: need dy [M,N], w [G,N,K]")
    G, N, K = w.shape
    if group_offsets.shape != (G + 1,):
        raise ValueError(f"group_offsets {tuple(group_offsets.shape)} expected ({G + 1},)")
    M = dy.shape[0]
    dyc, wc, oc = dy.contiguous(), w.contiguous(), group_offsets.contiguous()
    out = _out(out, (M, K), torch.bfloat16, dy.device)
    # A one-group dgrad with few output tiles splits its reduction into fp32 partials in a workspace;
    # with long reductions the workspace lists the group tails of at most 128 rows.
    nbytes = _lib.lib().moe_grouped_gemm_dgrad_workspace_size(M, N, K, G)
    if workspace is not None and workspace.numel() == 0:
        nbytes = 0
    if workspace is None or workspace.numel() * workspace.element_size() < nbytes:
        ws = _ws(nbytes, dy.device)
    else:
        ws, nbytes = workspace, workspace.numel() * workspace.element_size()
    call("moe_grouped_gemm_dgrad", ptr(dyc), M, N, ptr(wc), G, K, ptr(oc), ptr(out), ptr(ws), nbytes, stream_handle())
    return out


def grouped_gemm_wgrad(dy: torch.Tensor, x: torch.Tensor, group_offsets: torch.Tensor, *,
                       out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dw[g] = dy[rows of g]^T @ x[rows of g] (bf16 in, fp32 accumulate, bf16 out); empty groups give zeros.

    dy bf16 [M, N]; x bf16 [M, K]; group_offsets int32 [G+1] on the device; returns dw bf16 [G, N, K].
    workspace: uint8 device tensor of moe_grouped_gemm_wgrad_workspace_size bytes for the group order (largest
    first; the same result bit for bit); allocated when None, an empty tensor runs without it.
    """
    _on_gpu("dy", dy)
    _on_gpu("x", x)
    _on_gpu("group_offsets", group_offsets)
    _dtype("dy", dy, torch.bfloat16)
    _dtype("x", x, torch.bfloat16)
    _dtype("group_offsets", group_offsets, torch.int32)
    if dy.ndim != 2 or x.ndim != 2 or dy.shape[0] != x.shape[0] or group_offsets.ndim != 1:
        raise ValueError(f"shapes dy {tuple(dy.shape)} x {tuple(x.shape)}: need dy [M,N], x [M,K]")
    G = group_offsets.shape[0] - 1
    M, N = dy.shape
    K = x.shape[1]
    dyc, xc, oc = dy.contiguous(), x.contiguous(), group_offsets.contiguous()
    out = _out(out, (G, N, K), torch.bfloat16, dy.device)
    # The group order (largest first) that balances the tiles over the workgroups for skewed group sizes.
    nbytes = _lib.lib().moe_grouped_gemm_wgrad_workspace_size(M, N, K, G)
    if workspace is not None and workspace.numel() == 0:
        nbytes = 0
    if workspace is None or workspace.numel() * workspace.element_size() < nbytes:
        ws = _ws(nbytes, dy.device)
    else:
        ws, nbytes = workspace, workspace.numel() * workspace.element_size()
    call("moe_grouped_gemm_wgrad", ptr(dyc), ptr(xc), M, N, K, G, ptr(oc), ptr(out), ptr(ws), nbytes, stream_handle())
    return out
