"""Seeded synthetic inputs: the reference cases' generators and the five
benchmark configurations.

Reference-case generators reproduce the reference's own construction call for
call (same seeds, same torch CPU RNG calls), so their tensors are the
reference's tensors:
  * routing mask of case12/15/17: kernel_cases/case12_moe_row_id_map_pass2.py:30-40
    (= case15...:30-39, case17...:30-39), seed 20261112;
  * case17 x / probs: kernel_cases/case17_moe_permute_with_mask_map.py:78-90, seed 20261114;
  * case15 pin: kernel_cases/case15_moe_unpermute_mask_fwd.py:71-77, seed 20261113;
  * case21/22/24/30/32 modular routing (t + k) mod E: case21...:71-84;
  * case22 probs: case22...:88-103; case23 logits: case23...:65-71;
  * case06: case06...:47-52, seed 20261111.
Generators the reference leaves unseeded (case03/04/18 get_inputs) take the
seeds below.  Benchmark configurations use seed 20261200 + config number.

Row-id maps that are inputs of a case (case15/17/18) are built from the mask
by this package's own GPU row-id-map kernel (ops.row_id_map).
"""
from __future__ import annotations

import torch

SEED_CASE18 = 20261118
SEED_CASE03 = 20261103
SEED_CASE04 = 20261104
SEED_CONFIG_BASE = 20261200


# ------------------------------------------------------------ reference cases
def reference_routing_mask(tokens: int = 16384, experts: int = 320, seed: int = 20261112):
    """case12/15/17 routing mask [T, E] bool (5 experts per token, 6 when t % 4 == 1) and the
    6 candidate experts per token `sel` [T, 6] (case17 uses them for probs)."""
    torch.manual_seed(seed)
    sel = torch.argsort(torch.rand(tokens, experts), dim=-1)[:, :6]
    rm = torch.zeros(tokens, experts, dtype=torch.bool)
    rm.scatter_(1, sel[:, :5], True)
    extra = torch.arange(tokens) % 4 == 1
    extra_rows = extra.nonzero(as_tuple=True)[0]
    rm[extra_rows] = rm[extra_rows].scatter(1, sel[extra_rows, 5:6], True)
    return rm, sel


def case17_x_probs(sel: torch.Tensor, hidden: int = 8192, experts: int = 320, seed: int = 20261114):
    """case17 x bf16 [T, H] and sparse probs fp32 [T, E] (CPU RNG, same calls as the reference)."""
    tokens = sel.shape[0]
    torch.manual_seed(seed)
    x = torch.randn(tokens, hidden).to(torch.bfloat16)
    probs = torch.zeros(tokens, experts, dtype=torch.float32)
    vals = torch.rand(tokens, 5, dtype=torch.float32)
    probs.scatter_(1, sel[:, :5], vals)
    extra = torch.arange(tokens) % 4 == 1
    probs[extra] = probs[extra].scatter(1, sel[extra, 5:6], torch.rand(int(extra.sum()), 1))
    return x, probs


def case15_pin(rows: int, hidden: int = 8192, seed: int = 20261113):
    torch.manual_seed(seed)
    return torch.randn(rows, hidden).to(torch.bfloat16)


def modular_routing_mask(tokens: int, experts: int, topk: int) -> torch.Tensor:
    """Expert-major selection [E, T] bool: token t goes to experts (t + k) mod E, k < topk."""
    choice = (torch.arange(tokens)[:, None] + torch.arange(topk)) % experts
    selected = torch.zeros(experts, tokens, dtype=torch.bool)
    selected.scatter_(0, choice.t(), True)
    return selected


def case22_probs(selected_em: torch.Tensor, seed: int = 0) -> torch.Tensor:
    """fp32 probs [T, E] on the routed pairs of an expert-major selection (rand + 0.1)."""
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    experts, tokens = selected_em.shape
    probs = torch.zeros(tokens, experts, dtype=torch.float32)
    token = torch.arange(tokens).view(1, -1).expand_as(selected_em)[selected_em]
    expert = torch.arange(experts).view(-1, 1).expand_as(selected_em)[selected_em]
    raw = torch.rand(int(selected_em.sum().item()), generator=g, dtype=torch.float32) + 0.1
    probs[token, expert] = raw
    return probs


def case23_logits(tokens: int = 16384, experts: int = 320, seed: int = 0) -> torch.Tensor:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return torch.randn(tokens, experts, generator=g, dtype=torch.float32)


def case18_mask(tokens: int = 4096, experts: int = 320, topk: int = 8, seed: int = SEED_CASE18):
    """case18 routing: argsort(rand)[:, :topk] per token (the reference draws it unseeded)."""
    torch.manual_seed(seed)
    rm = torch.zeros(tokens, experts, dtype=torch.bool)
    idx = torch.argsort(torch.rand(tokens, experts), dim=-1)[:, :topk]
    rm.scatter_(1, idx, True)
    return rm


def uniform_group_sizes(total: int, groups: int) -> list[int]:
    """case03/04 group_sizes: uniform m_splits, the first `total % groups` one larger."""
    base, rem = divmod(total, groups)
    return [base + (1 if i < rem else 0) for i in range(groups)]


# ------------------------------------------------------- benchmark configs
def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def router_logits(tokens: int, experts: int, *, skew: float, seed: int, device="cpu") -> torch.Tensor:
    """fp32 logits [T, E] ~ N(0,1) plus a per-expert bias ~ N(0, skew) (skew 0: no bias)."""
    g = _gen(device, seed)
    logits = torch.randn(tokens, experts, generator=g, device=device, dtype=torch.float32)
    if skew:
        bias = torch.randn(experts, generator=g, device=device, dtype=torch.float32) * skew
        logits = logits + bias
    return logits


def zipf_group_sizes(total: int, groups: int, *, s: float = 1.1, zero_expert: int = -1,
                     seed: int = SEED_CONFIG_BASE + 3) -> list[int]:
    """Ragged m_splits: multinomial(total, p) with p_e ~ (e+1)^-s, expert `zero_expert` forced to 0."""
    p = torch.arange(1, groups + 1, dtype=torch.float64) ** (-s)
    if zero_expert is not None:
        p[zero_expert] = 0.0
    p = p / p.sum()
    g = _gen("cpu", seed)
    draws = torch.multinomial(p, total, replacement=True, generator=g)
    return torch.bincount(draws, minlength=groups).tolist()


def randn_bf16(shape, *, std: float = 1.0, seed: int, device="cpu") -> torch.Tensor:
    g = _gen(device, seed)
    t = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    return t.to(torch.bfloat16)


CONFIGS = {
    # name: (tokens, hidden, experts, topk, skew)
    "c1": dict(tokens=4096, hidden=2048, experts=8, topk=2, skew=0.0),
    "c2": dict(tokens=8192, hidden=7168, experts=64, topk=8, skew=1.5),
    "c5": dict(tokens=16384, hidden=7168, experts=64, topk=8, skew=1.5, ffn=2048),
}
GEMM_CONFIGS = {
    # fc1 + SwiGLU: 16 experts, sum M = 16384 * 8 / 4, K = 7168, N = 4096 (gate || up)
    "c3": dict(groups=16, total=16384 * 8 // 4, K=7168, N=4096, swiglu=True),
    # fc2: same ragged M, K = 2048, N = 7168
    "c4": dict(groups=16, total=16384 * 8 // 4, K=2048, N=7168, swiglu=False),
}
