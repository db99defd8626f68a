"""MoE FFN forward layer on one GPU, composed from this package's kernels.

The reference has no entry point for the composed layer; it is the chain of
its cases: router top-k (case23) -> mask map -> row-id map (case12) ->
permute (case17) -> grouped GEMM fc1 (case03) + SwiGLU -> grouped GEMM fc2
(case04) -> unpermute with probability-weighted merge (case15 + merge probs).

Data layout in HBM (T tokens, H hidden, F ffn, E experts, k top-k, R = T*k):
  x        bf16 [T, H]        token-major activations (input)
  logits   fp32 [T, E]        router logits (input; the router GEMM is not part of this path)
  mask     bool [T, E]        1 at the k selected experts
  probs    fp32 [T, E]        softmax over the k selected logits, 0 elsewhere
  row_map  int64 [T, E]       token-major destination row, -1 if unselected
  offsets  int32 [E + 1]      first permuted row of each expert; offsets[E] = R
  src      int32 [R]          source token of each permuted row (inverse of row_map; written
                              by the row-id map's fill pass)
  xp       bf16 [R, H]        permuted rows x[src], expert-major (expert e = rows offsets[e]..);
                              only materialised with fused_permute=False — by default fc1
                              gathers its A rows from x through src (moe_grouped_gemm_gather)
  h        bf16 [R, F]        silu(xp @ W1_gate^T) * (xp @ W1_up^T)
  z        bf16 [R, H]        h @ W2^T
  out      bf16 [T, H]        sum_e probs[t, e] * z[row_map[t, e]]  (fp32, ascending e)
  W1       bf16 [E, 2F, H]    gate rows [0, F), up rows [F, 2F)  (out x in)
  W2       bf16 [E, H, F]
The intermediates (src, h, z, the row-id-map and GEMM workspaces) are allocated once per
token count and reused by later calls; the output is a new tensor on every call
(or the caller's `out=`), so a result stays valid across later forward() calls.
No host synchronisation happens inside forward() (R = T * k is known on the host).
"""
from __future__ import annotations

import torch

from . import ops


class MoEFFN:
    """forward(x, logits) -> out for fixed weights W1 [E, 2F, H], W2 [E, H, F]."""

    def __init__(self, w1: torch.Tensor, w2: torch.Tensor, topk: int, *, fused_permute: bool = True):
        if w1.ndim != 3 or w2.ndim != 3:
            raise ValueError("w1 must be [E, 2F, H] and w2 [E, H, F]")
        E, F2, H = w1.shape
        if w2.shape != (E, H, F2 // 2) or F2 % 2:
            raise ValueError(f"w2 {tuple(w2.shape)} does not match w1 {tuple(w1.shape)}")
        self.w1, self.w2 = w1, w2
        self.E, self.H, self.F, self.k = E, H, F2 // 2, topk
        self.fused_permute = fused_permute
        self._bufs = None
        self.last = {}

    def _buffers(self, T: int, device) -> dict:
        if self._bufs is None or self._bufs["T"] != T:
            R = T * self.k
            bf = dict(dtype=torch.bfloat16, device=device)
            self._bufs = {
                "T": T,
                "xp": None if self.fused_permute else torch.empty(R, self.H, **bf),
                "src": torch.empty(R, dtype=torch.int32, device=device),
                "h": torch.empty(R, self.F, **bf),
                "z": torch.empty(R, self.H, **bf),
                "ws": torch.empty(ops._lib.lib().moe_row_id_map_workspace_size(T, self.E), dtype=torch.uint8,
                                  device=device),
                # the grouped GEMMs' tail list (fc1 and fc2 run one after the other)
                "gemm_ws": torch.empty(max(ops._lib.lib().moe_grouped_gemm_workspace_size(R, self.H, 2 * self.F, self.E),
                                           ops._lib.lib().moe_grouped_gemm_workspace_size(R, self.F, self.H, self.E), 1),
                                       dtype=torch.uint8, device=device),
            }
        return self._bufs

    def route(self, logits: torch.Tensor):
        """(mask, probs, token-major row map, expert offsets) for router logits [T, E]; the
        source token of every permuted row lands in the cached `src` buffer."""
        b = self._buffers(logits.shape[0], logits.device)
        _, _, mask, probs = ops.topk(logits, self.k, with_mask=True, with_probs=True)
        maps = ops.row_id_map(mask, expert_major=False, token_major=True, expert_offsets=True, src_out=b["src"],
                              workspace=b["ws"])
        return mask, probs, maps["token_major"], maps["expert_offsets"]

    def forward(self, x: torch.Tensor, logits: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
        """out [T, H] bf16 for x [T, H] and router logits [T, E]; `out` may be given (contiguous bf16 [T, H])."""
        T = x.shape[0]
        if logits.shape != (T, self.E):
            raise ValueError(f"logits {tuple(logits.shape)} expected {(T, self.E)}")
        b = self._buffers(T, x.device)
        if out is None:
            out = torch.empty(T, self.H, dtype=torch.bfloat16, device=x.device)
        mask, probs, row_map, offsets = self.route(logits)
        if self.fused_permute:
            # src holds the source token of every permuted row (R = T * k rows, all named by the map)
            ops.grouped_gemm_gather(x, b["src"], self.w1, offsets, swiglu=True, out=b["h"], workspace=b["gemm_ws"])
        else:
            ops.permute(x, row_map, num_out=T * self.k, layout=ops.TOKEN_MAJOR, zero_tail=False, out=b["xp"])
            ops.grouped_gemm(b["xp"], self.w1, offsets, swiglu=True, out=b["h"], workspace=b["gemm_ws"])
        ops.grouped_gemm(b["h"], self.w2, offsets, out=b["z"], workspace=b["gemm_ws"])
        ops.unpermute(b["z"], row_map, probs, layout=ops.TOKEN_MAJOR, out=out)
        self.last = {"mask": mask, "probs": probs, "row_map": row_map, "offsets": offsets}
        return out

    __call__ = forward
