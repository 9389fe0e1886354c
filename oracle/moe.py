"""MoE token routing, restated for the CPU oracle.

``modeling/moe/linear_experts.py:244-277``: ``expert_mask =
one_hot(top_k_index, E).permute(2, 1, 0)``; for each expert,
``top_k_pos, token_indices = torch.where(expert_mask[e])``; with the
calibrate-all flag (``modeling/moe/context.py:6-18``) the expert runs on all
tokens, otherwise on ``hidden_states[token_indices]``.  Pinned by
``tests/llmcompressor/modeling/test_linear_experts.py:12-100`` (routed = 1
token per expert with a one-expert-per-token routing; calibrate-all = all).
"""
from __future__ import annotations

import torch


def expert_token_lists(top_k_index: torch.Tensor, num_experts: int, calibrate_all: bool = False,
                       num_tokens: int | None = None):
    tokens = top_k_index.shape[0] if num_tokens is None else num_tokens
    mask = torch.nn.functional.one_hot(top_k_index.long(), num_experts).permute(2, 1, 0)
    out = []
    for e in range(num_experts):
        top_k_pos, token_indices = torch.where(mask[e])
        out.append(torch.arange(tokens) if calibrate_all else token_indices)
    return out


def expert_hessians(hidden: torch.Tensor, top_k_index: torch.Tensor, num_experts: int,
                    calibrate_all: bool = False):
    """Per-expert (H_e, num_samples_e) for a gate/up input, fp32 on the CPU,
    following ``gptq_quantize.py:63-97`` for each expert's 2-D input."""
    from .gptq import accumulate_hessian, make_empty_hessian
    d = hidden.shape[1]
    Hs, ns = [], []
    for idx in expert_token_lists(top_k_index, num_experts, calibrate_all, hidden.shape[0]):
        H = make_empty_hessian(d)
        n = torch.zeros(())
        H, n = accumulate_hessian(hidden[idx], H, n)
        Hs.append(H)
        ns.append(n)
    return torch.stack(Hs), torch.stack(ns)
