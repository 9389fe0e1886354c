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
import re

import torch

from . import ops
from .staging import hold, held

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
                               num_samples: torch.Tensor, calls: int = 1, fresh: bool = False):
    """H[e] += 2 * sum over the expert's rows of x x^T; num_samples[e] += calls.

    ``rows`` None: x is already grouped by expert (expert e owns the rows
    offsets[e] .. offsets[e+1] - 1, as ``expert_intermediate`` returns them).
    ``offsets`` is a list or an int64 tensor (on the device the call waits
    for nothing).  ``fresh``: H holds no earlier sum (it may be freshly
    allocated, uncleared): its upper triangles are written, not read."""
    ops.hessian_grouped_syrk_(H, x, rows, offsets, alpha=2.0, beta=0.0 if fresh else 1.0)
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


class ExpertMLP(torch.nn.Module):
    """One expert of a gated MoE MLP: ``down_proj(act(gate_proj(h)) *
    up_proj(h))`` as separate ``nn.Linear`` modules, so that calibration
    hooks see each projection (``modeling/moe/linear_experts.py:26-95``,
    ``ExpertMLPWithGate``; its gate is applied to the concatenation
    [gate, up], which multiplies the same two halves)."""

    def __init__(self, hidden: int, intermediate: int, bias: bool = False, act=torch.nn.functional.silu,
                 dtype=None, device=None):
        super().__init__()
        self.intermediate_size = intermediate
        self.gate_proj = torch.nn.Linear(hidden, intermediate, bias=bias, dtype=dtype, device=device)
        self.up_proj = torch.nn.Linear(hidden, intermediate, bias=bias, dtype=dtype, device=device)
        self.down_proj = torch.nn.Linear(intermediate, hidden, bias=bias, dtype=dtype, device=device)
        self.act = act

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return self.down_proj(self.act(self.gate_proj(hidden_states)) * self.up_proj(hidden_states))


class LinearExperts(torch.nn.ModuleList):
    """The experts of an MoE layer as a list of ``ExpertMLP`` with the
    reference's calibration forward (``modeling/moe/linear_experts.py:159-277``,
    ``LinearExperts2D``): for each expert in index order its routed tokens
    ``torch.where(one_hot(top_k_index)[..., e].T)`` (all tokens under
    ``moe_calibration_context``, the outputs then taken at the routed rows),
    weighted by their top-k weights and summed into the output with
    ``index_add_``."""

    def __init__(self, num_experts: int, hidden: int, intermediate: int, bias: bool = False,
                 act=torch.nn.functional.silu, dtype=None, device=None):
        super().__init__([ExpertMLP(hidden, intermediate, bias, act, dtype, device) for _ in range(num_experts)])
        self.num_experts = num_experts
        self.intermediate_size = intermediate

    @classmethod
    @torch.no_grad()
    def from_stacked(cls, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor, act=torch.nn.functional.silu):
        """Experts from stacked weights gate / up [E, I, H] and down [E, H, I]
        (``copy_from_experts_module``, ``linear_experts.py:51-74``)."""
        E, inter, hidden = gate.shape
        self = cls(E, hidden, inter, act=act, dtype=gate.dtype, device=gate.device)
        for e, expert in enumerate(self):
            expert.gate_proj.weight.data = gate[e].contiguous()
            expert.up_proj.weight.data = up[e].contiguous()
            expert.down_proj.weight.data = down[e].contiguous()
        return self

    def forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                top_k_weights: torch.Tensor) -> torch.Tensor:
        final = torch.zeros_like(hidden_states)
        with torch.no_grad():
            mask = torch.nn.functional.one_hot(top_k_index, self.num_experts).permute(2, 1, 0)
        for e in range(self.num_experts):
            top_k_pos, token_indices = torch.where(mask[e])
            expert = self[e]
            if get_calibrate_all_experts_flag():
                out = expert(hidden_states)[token_indices]
            else:
                out = expert(hidden_states[token_indices])
            weighted = out * top_k_weights[token_indices, top_k_pos, None]
            final.index_add_(0, token_indices, weighted.to(final.dtype))
        return final


class ExpertFamily:
    """Same-shaped modules of one expert list that share quantization
    arguments (``experts.<e>.gate_proj`` for every e): their Hessians live
    in one [E, d, d] tensor, and the rows their forward hooks receive are
    held until a flush hands them, grouped by expert, to one grouped syrk
    launch (instead of one accumulation per expert call).  Rows are held as
    references to the hooks' inputs (``staging.hold``: a flush raises if one
    was modified in place since), up to ``budget`` bytes; a flush copies
    them into one grouped buffer.  Repeated calls of one expert before a
    flush go into the same group (another order of fp32 additions)."""

    def __init__(self, key: str, members: list, budget: int):
        self.key = key
        self.members = list(members)
        self.slot = {m: i for i, m in enumerate(self.members)}
        self.budget = budget
        self.H: torch.Tensor | None = None
        self._fresh = False        # H allocated, nothing accumulated yet
        self.samples = [0] * len(self.members)
        self._parts: list = []      # (slot, call index, rows)
        self._held = 0

    def hessian(self, module) -> torch.Tensor:
        """The member's [d, d] view of the family's Hessians (allocated with
        the first call of any member)."""
        if self.H is None:
            w = self.members[0].weight
            d = w.shape[1]
            # uncleared: the first grouped syrk writes every upper triangle
            self.H = torch.empty((len(self.members), d, d), dtype=torch.float32, device=w.device)
            self._fresh = True
        return self.H[self.slot[module]]

    def add(self, module, rows: torch.Tensor, samples: int) -> None:
        slot = self.slot[module]
        self.samples[slot] += samples
        if rows.shape[0] == 0:
            return
        nbytes = rows.numel() * rows.element_size()
        if self._parts and self._held + nbytes > self.budget:
            self.flush()
        x, version = hold(rows)
        self._parts.append((slot, len(self._parts), x, version))
        self._held += nbytes

    def flush(self) -> None:
        """Accumulates the held rows: one grouped syrk over the experts (the
        first one writes the upper triangles of the uncleared stack, experts
        without rows as zeros)."""
        if not self._parts:
            if self._fresh:
                self.H.zero_()
                self._fresh = False
            return
        parts = [(slot, i, held(x, v)) for slot, i, x, v in sorted(self._parts, key=lambda p: (p[0], p[1]))]
        self._parts, self._held = [], 0
        counts = [0] * len(self.members)
        for slot, _, rows in parts:
            counts[slot] += rows.shape[0]
        offsets = [0]
        for c in counts:
            offsets.append(offsets[-1] + c)
        dtypes = {rows.dtype for _, _, rows in parts}
        dt = dtypes.pop() if len(dtypes) == 1 else torch.float32
        x = torch.cat([rows.to(dt) for _, _, rows in parts]) if len(parts) > 1 else parts[0][2]
        ops.hessian_grouped_syrk_(self.H, x, None, offsets, alpha=2.0, beta=0.0 if self._fresh else 1.0)
        self._fresh = False

    def release(self) -> None:
        self._parts, self._held = [], 0
        self.H = None
        self._fresh = False
        self.samples = [0] * len(self.members)


_INDEXED = re.compile(r"(?:^|\.)(\d+)(?=\.|$)")


def expert_families(named_modules, targets, args_of, budget: int) -> dict:
    """{module: ExpertFamily} for the ``targets`` among ``named_modules``
    that belong to expert lists: modules named ``<list>.<e>.<rest>`` where
    ``<list>`` is a module with an integer ``num_experts`` or whose name ends
    in ``experts``, grouped by (``<list>``, ``<rest>``) when at least two
    share one weight shape, dtype, device and quantization arguments
    (``args_of(module)``)."""
    modules = dict(named_modules)
    groups: dict = {}
    for name, m in modules.items():
        if m not in targets:
            continue
        found = list(_INDEXED.finditer(name))
        if not found or not isinstance(getattr(m, "weight", None), torch.Tensor) or m.weight.dim() != 2:
            continue
        f = found[-1]
        parent = name[:f.start()]
        container = modules.get(parent)
        is_experts = parent.split(".")[-1] == "experts" or isinstance(getattr(container, "num_experts", None), int)
        if not is_experts:
            continue
        w = m.weight
        key = (parent, name[f.end():], tuple(w.shape), w.dtype, str(w.device))
        groups.setdefault(key, []).append((int(f.group(1)), m))
    out: dict = {}
    for key, items in groups.items():
        if len(items) < 2:
            continue
        items.sort(key=lambda t: t[0])
        members = [m for _, m in items]
        a0 = args_of(members[0])
        if any(args_of(m) != a0 for m in members[1:]):
            continue
        fam = ExpertFamily(f"{key[0]}.*{key[1]}" if key[0] else f"*{key[1]}", members, budget)
        for m in members:
            out[m] = fam
    return out
