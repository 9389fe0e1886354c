"""SparseGPT Hessian accumulation and pruning solve, restated for the CPU oracle.

Test infrastructure only: what the GPU path is compared against.
Follows ``modifiers/pruning/sparsegpt/sgpt_sparsify.py`` line by line:

* ``make_empty_hessian``  - ``:10-16``
* ``accumulate_hessian``  - ``:19-55`` (Linear / Conv1D branch: a running mean,
  ``H *= n / (n + added)`` then ``H += (sqrt(2 / n') X)^T (sqrt(2 / n') X)``)
* ``sparsify_weight``     - ``:58-213`` (dead columns ``:97-100``, damping and
  Cholesky chain with the identity fallback ``:102-117``, base mask
  ``:119-135``, blocked sweep with unstructured ``:150-165`` or N:M
  ``:166-186`` masks, lazy update ``:198-206``)

Working precision fp32 (``SGPT_PRECISION``, ``:7``); linear algebra is torch's
CPU LAPACK.

Pinning: the compensation update by an fp64 sequential optimal-brain-surgeon
brute force with explicit inverses of the trailing Hessian blocks (no
Cholesky factor); Hinv = I by plain magnitude pruning; the masks by their
invariants (per-block pruned set = every value at or below the k-th
smallest, k = int(numel * sparsity); N:M: at least n zeros in every group of
m); preserve_sparsity_mask by mask containment and its ValueError.
"""
from __future__ import annotations

import math

import torch

SGPT_PRECISION = torch.float32


def make_empty_hessian(num_columns: int, device="cpu") -> torch.Tensor:
    return torch.zeros((num_columns, num_columns), device=device, dtype=SGPT_PRECISION)


def accumulate_hessian(inp: torch.Tensor, H: torch.Tensor, num_samples: int):
    """Linear / Conv1D branch of ``sgpt_sparsify.py:19-55``."""
    inp = inp.to(device=H.device)
    if len(inp.shape) == 2:
        inp = inp.unsqueeze(0)
    num_added = inp.shape[0]
    if len(inp.shape) == 3:
        inp = inp.reshape((-1, inp.shape[-1]))
    inp = inp.t()
    H *= num_samples / (num_samples + num_added)
    num_samples += num_added
    inp = inp.to(dtype=SGPT_PRECISION)
    inp = math.sqrt(2 / num_samples) * inp
    H += inp.matmul(inp.t())
    return H, num_samples


def hinv_chain(H: torch.Tensor, dampening_frac: float):
    """Dead columns, damping and the Cholesky chain (``:97-117``).  Returns
    (Hinv upper, dead mask, ok)."""
    H = H.clone()
    dead = torch.diag(H) == 0
    H[dead, dead] = 1
    try:
        damp = dampening_frac * torch.mean(torch.diag(H))
        diag = torch.arange(H.shape[0], device=H.device)
        H[diag, diag] += damp
        H = torch.linalg.cholesky(H)
        H = torch.cholesky_inverse(H)
        H = torch.linalg.cholesky(H, upper=True)
        return H, dead, True
    except torch._C._LinAlgError:
        return torch.eye(H.shape[0], dtype=H.dtype, device=H.device), dead, False


def sparsify_weight(weight: torch.Tensor, H: torch.Tensor, sparsity: float, prune_n: int, prune_m: int,
                    block_size: int, dampening_frac: float, preserve_sparsity_mask: bool, hinv=None):
    """``sgpt_sparsify.py:58-213`` for a Linear weight.  Returns (loss, W in
    the weight's dtype, Hinv used, ok).  ``hinv`` replaces the Cholesky chain
    (the caller's upper factor; dead columns are still zeroed)."""
    final_dtype = weight.dtype
    W = weight.clone().to(dtype=SGPT_PRECISION)
    num_rows, num_columns = W.shape
    Hc, dead, ok = hinv_chain(H, dampening_frac)
    Hinv = Hc if hinv is None else hinv
    W[:, dead] = 0

    mask = None
    if preserve_sparsity_mask:
        mask = torch.where(W == 0, torch.tensor(1, dtype=torch.bool), torch.tensor(0, dtype=torch.bool))
        current_sparsity = mask.sum() / W.numel()
        if current_sparsity > sparsity:
            raise ValueError("The target sparsity is lower than the sparsity of the base model. Please retry "
                             "after turning preserve_sparsity_mask=False")

    losses = torch.zeros(num_rows)
    for i1 in range(0, num_columns, block_size):
        i2 = min(i1 + block_size, num_columns)
        count = i2 - i1
        W1 = W[:, i1:i2].clone()
        Q1 = torch.zeros_like(W1)
        Err1 = torch.zeros_like(W1)
        Losses1 = torch.zeros_like(W1)
        Hinv1 = Hinv[i1:i2, i1:i2]

        if prune_n == 0:
            if mask is not None:
                mask1 = mask[:, i1:i2]
                if int(W1.numel() * sparsity) > mask1.sum():
                    tmp = (~mask[:, i1:i2]) * W1 ** 2 / (torch.diag(Hinv1).reshape((1, -1))) ** 2
                    thresh = torch.sort(tmp.flatten())[0][int(tmp.numel() * sparsity)]
                    mask1 = tmp <= thresh
            else:
                tmp = W1 ** 2 / (torch.diag(Hinv1).reshape((1, -1))) ** 2
                thresh = torch.sort(tmp.flatten())[0][int(tmp.numel() * sparsity)]
                mask1 = tmp <= thresh
        else:
            mask1 = mask[:, i1:i2] if mask is not None else torch.zeros_like(W1) == 1

        for i in range(count):
            w = W1[:, i]
            d = Hinv1[i, i]
            if prune_n != 0 and i % prune_m == 0:
                tmp = W1[:, i:(i + prune_m)] ** 2 / (torch.diag(Hinv1)[i:(i + prune_m)].reshape((1, -1))) ** 2
                if mask is not None:
                    tmp = tmp * (~mask[:, i:(i + prune_m)])
                mask1.scatter_(1, i + _topk_smallest(tmp, prune_n), True)
            q = w.clone()
            q[mask1[:, i]] = 0
            Q1[:, i] = q
            Losses1[:, i] = (w - q) ** 2 / d ** 2
            err1 = (w - q) / d
            W1[:, i:] -= err1.unsqueeze(1).matmul(Hinv1[i, i:].unsqueeze(0))
            Err1[:, i] = err1

        W[:, i1:i2] = Q1
        losses += torch.sum(Losses1, 1) / 2
        if preserve_sparsity_mask:
            W[:, i2:] -= (~mask[:, i2:]) * Err1.matmul(Hinv[i1:i2, i2:])
        else:
            W[:, i2:] -= Err1.matmul(Hinv[i1:i2, i2:])

    loss = torch.sum(losses).item()
    return loss, W.to(final_dtype), Hinv, ok


def _topk_smallest(tmp: torch.Tensor, n: int) -> torch.Tensor:
    """Indices of the n smallest values per row (``torch.topk(tmp, n, dim=1,
    largest=False)[1]``, ``:185``).  torch leaves the order of equal values
    unspecified; here the lower column wins a tie (a stable sort), the rule the
    GPU kernel implements."""
    if n > tmp.shape[1]:
        raise RuntimeError("selected index k out of range")
    return torch.sort(tmp, dim=1, stable=True)[1][:, :n]
