"""MoE expert routing and grouped per-expert Hessians.

Token routing follows ``modeling/moe/linear_experts.py:244-277``: for expert
e the tokens are ``torch.where(one_hot(top_k_index)[..., e].T)`` - ordered by
top-k position, then token index.  Outside ``moe_calibration_context`` an
expert sees only its routed tokens (ragged inputs); inside it every expert
sees all tokens (``modeling/moe/context.py:6-18``).  Each expert call adds 1
to that expert's ``num_samples`` (2-D input, ``gptq_quantize.py:70-73``),
also when no token is routed to it.

``accumulate_expert_hessians`` replaces the per-expert hook calls with one
grouped syrk launch over (expert, tile, token-split) work items.
"""
from __future__ import annotations

import contextlib

import torch

from . import ops

_CALIBRATE_ALL_EXPERTS = False


def get_calibrate_all_experts_flag() -> bool:
    return _CALIBRATE_ALL_EXPERTS


@contextlib.contextmanager
def moe_calibration_context():
    global _CALIBRATE_ALL_EXPERTS
    restore, _CALIBRATE_ALL_EXPERTS = _CALIBRATE_ALL_EXPERTS, True
    try:
        yield
    finally:
        _CALIBRATE_ALL_EXPERTS = restore


def route_tokens(top_k_index: torch.Tensor, num_experts: int, num_tokens: int | None = None):
    """Token lists per expert in the reference's order.

    ``num_tokens`` is the number of hidden-state rows (all of them reach
    every expert under ``moe_calibration_context``); it defaults to the
    rows of ``top_k_index``.

    Returns (rows int32 [sum n_e] token indices grouped by expert,
    offsets list[int] of length E + 1, top_k_pos int64 [sum n_e]).
    """
    tokens, k = top_k_index.shape
    dev = top_k_index.device
    if get_calibrate_all_experts_flag():
        nt = tokens if num_tokens is None else num_tokens
        rows = torch.arange(nt, device=dev, dtype=torch.int32).repeat(num_experts)
        offsets = [e * nt for e in range(num_experts + 1)]
        return rows, offsets, None
    # key = expert * (k * T) + pos * T + token  ->  sort = reference order
    pos = torch.arange(k, device=dev).unsqueeze(0).expand(tokens, k)
    tok = torch.arange(tokens, device=dev).unsqueeze(1).expand(tokens, k)
    key = top_k_index.long() * (k * tokens) + pos * tokens + tok
    order = torch.argsort(key.reshape(-1))
    sorted_tok = tok.reshape(-1)[order]
    counts = torch.bincount(top_k_index.reshape(-1).long(), minlength=num_experts)
    offsets = [0] + torch.cumsum(counts, 0).tolist()
    return sorted_tok.to(torch.int32), offsets, pos.reshape(-1)[order]


def accumulate_expert_hessians(x: torch.Tensor, rows: torch.Tensor | None, offsets, H: torch.Tensor,
                               num_samples: torch.Tensor, calls: int = 1):
    """H[e] += 2 * sum over the expert's rows of x x^T; num_samples[e] += calls.

    ``rows`` None: x is already grouped by expert (expert e owns the rows
    offsets[e] .. offsets[e+1] - 1, as ``expert_intermediate`` returns them).
    ``offsets`` is a list or an int64 tensor (on the device the call waits
    for nothing)."""
    ops.hessian_grouped_syrk_(H, x, rows, offsets, alpha=2.0)
    num_samples += calls
    return H, num_samples


def expert_intermediate(hidden: torch.Tensor, rows: torch.Tensor, offsets: list[int], gate: torch.Tensor,
                        up: torch.Tensor, act=torch.nn.functional.silu) -> torch.Tensor:
    """Concatenated down-projection inputs act(x W_g^T) * (x W_u^T) per expert
    (bf16), in the same grouped order as ``rows``."""
    outs = []
    for e in range(len(offsets) - 1):
        a, b = offsets[e], offsets[e + 1]
        if b == a:
            continue
        xe = hidden[rows[a:b].long()]
        outs.append(act(xe @ gate[e].t()) * (xe @ up[e].t()))
    if not outs:
        return torch.empty((0, gate.shape[1]), dtype=hidden.dtype, device=hidden.device)
    return torch.cat(outs, 0).contiguous()
