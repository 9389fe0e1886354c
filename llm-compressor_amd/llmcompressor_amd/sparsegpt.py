"""SparseGPT Hessian accumulation and pruning solve on the GPU (drop-in functions).

Same names, signatures, return values and error behaviour as
``modifiers/pruning/sparsegpt/sgpt_sparsify.py``:

* ``make_empty_hessian(module, device=None)``                       (``:10-16``)
* ``accumulate_hessian(inp, module, H, num_samples)``                (``:19-55``)
* ``sparsify_weight(module, hessians_dict, sparsity, prune_n, prune_m,
  block_size, dampening_frac, preserve_sparsity_mask)``             (``:58-213``)

As for GPTQ, ``accumulate_hessian`` maintains the upper triangle of the
running-mean Hessian (diagonal included) and ``sparsify_weight`` reads only
that triangle.  Conv2d inputs are unfolded into their patches for the
Hessian, as the reference does; pruning a Conv2d weight, block sizes above
128 and N:M groups wider than 16 columns raise instead of computing.
"""
from __future__ import annotations

import logging

import torch

from . import _lib, ops
from ._lib import UNSUPPORTED, Mi355qError
from .gptq import _is_linear_like, conv2d_rows

logger = logging.getLogger("llmcompressor_amd")

SGPT_PRECISION = torch.float32

__all__ = ["make_empty_hessian", "accumulate_hessian", "sparsify_weight", "SparsifyResult", "sparsegpt_prune"]


def make_empty_hessian(module: torch.nn.Module, device: torch.device | None = None) -> torch.Tensor:
    weight = module.weight
    num_columns = weight.shape[1]
    device = device if device is not None else weight.device
    return torch.zeros((num_columns, num_columns), device=device, dtype=SGPT_PRECISION)


def accumulate_hessian(inp: torch.Tensor, module: torch.nn.Module, H: torch.Tensor,
                       num_samples: int) -> tuple[torch.Tensor, int]:
    """Running mean: H *= n / (n + added); H += (2 / (n + added)) X^T X (upper
    triangle, in place; one kernel call), ``added`` = the leading dimension
    after a 2-D input is unsqueezed to 3-D."""
    x, num_added = hessian_rows(inp, module, H.device)
    return H, fold_rows(H, x, num_samples, num_added)


def hessian_rows(inp: torch.Tensor, module: torch.nn.Module, device) -> tuple[torch.Tensor, int]:
    """The 2-D rows of one accumulation call on ``device`` and the
    reference's sample count for it (the leading dimension after a 2-D input
    is unsqueezed to 3-D)."""
    inp = inp.to(device=device)
    if len(inp.shape) == 2:
        inp = inp.unsqueeze(0)
    if isinstance(module, torch.nn.Conv2d):   # sgpt_sparsify.py:37-45: the unfolded patches
        return conv2d_rows(inp, module), inp.shape[0]
    if not _is_linear_like(module):
        raise NotImplementedError(f"SparseGPT Hessian for {type(module).__name__} is not provided by this build")
    return inp.reshape(-1, inp.shape[-1]), inp.shape[0]


def fold_rows(H: torch.Tensor, x, num_samples: int, num_added: int) -> int:
    """The running mean over ``num_samples`` samples extended by the rows x (a
    2-D tensor, or a list of them summed as one) of ``num_added`` more;
    returns the new count."""
    beta = num_samples / (num_samples + num_added)
    num_samples += num_added
    ops.hessian_syrk_segments_(H, list(x) if isinstance(x, (list, tuple)) else [x], alpha=2 / num_samples,
                               beta=beta)
    return num_samples


class SparsifyResult:
    """Pruned weight (original dtype and shape), loss, and whether the damped
    Hessian was positive definite (else Hinv = identity, as the reference)."""

    def __init__(self, loss: float, weight: torch.Tensor, hinv_ok: bool):
        self.loss, self.weight, self.hinv_ok = loss, weight, hinv_ok


def _check_blocks(rows: int, cols: int, sparsity, prune_n: int, prune_m: int, block_size: int, preserve: bool):
    """The reference's own failures (an index past the sorted block, a topk
    wider than its group, a group and its preserved-mask window of different
    widths), raised as the same exception types before any kernel runs."""
    if block_size > 128:
        raise NotImplementedError("SparseGPT block sizes above 128 are not provided by this build")
    if prune_n != 0 and prune_m > 16:
        raise NotImplementedError("N:M groups wider than 16 columns are not provided by this build")
    for i1 in range(0, cols, block_size):
        count = min(i1 + block_size, cols) - i1
        if prune_n == 0:
            k = int(rows * count * sparsity)
            if k >= rows * count:
                raise IndexError(f"index {k} is out of bounds for dimension 0 with size {rows * count}")
        else:
            j = ((count - 1) // prune_m) * prune_m
            if count - j < prune_n or prune_m < prune_n:
                raise RuntimeError("selected index k out of range")
            if preserve and min(j + prune_m, cols) - j != count - j:
                raise RuntimeError(f"The size of tensor a ({count - j}) must match the size of tensor b "
                                   f"({min(j + prune_m, cols) - j}) at non-singleton dimension 1")


def sparsegpt_prune(weight: torch.Tensor, hessian: torch.Tensor, sparsity, prune_n: int = 0, prune_m: int = 0,
                    block_size: int = 128, dampening_frac: float = 0.01,
                    preserve_sparsity_mask: bool = False) -> SparsifyResult:
    """The solve of ``sgpt_sparsify.py:81-213`` for a [rows, cols] weight and
    its running-mean Hessian (upper triangle read)."""
    rows, cols = weight.shape
    _check_blocks(rows, cols, sparsity, prune_n, prune_m, block_size, preserve_sparsity_mask)
    hinv, dead, status = ops.gptq_hinv_rtn(hessian, None, 1.0, dampening_frac)
    w_work = ops.gptq_load_weight(weight, None, dead)
    mask = None
    if preserve_sparsity_mask:
        mask, count = ops.sparsegpt_base_mask(w_work)
        current_sparsity = torch.tensor(int(count.cpu().to(torch.int64)[0]) & 0xFFFFFFFF) / w_work.numel()
        if current_sparsity > sparsity:
            raise ValueError("The target sparsity is lower than the sparsity of the base model. Please retry "
                             "after turning preserve_sparsity_mask=False")
    try:
        losses = ops.sparsegpt_sweep_(w_work, hinv, sparsity if prune_n == 0 else 0.0, prune_n, prune_m,
                                      block_size, mask)
    except Mi355qError as e:
        if e.status == UNSUPPORTED:
            raise NotImplementedError(str(e)) from e
        raise
    w_out, _ = ops.gptq_store_weight(w_work, None, weight.dtype)
    loss_st = torch.stack([torch.sum(losses), status[0].float()]).cpu()  # the one sync
    _lib.check_hinv_status([loss_st[1]])
    loss_ok = torch.stack([loss_st[0], (loss_st[1] == 0).float()])
    ok = bool(loss_ok[1])
    if not ok:
        logger.warning("Failed to invert hessian due to numerical instability. Consider increasing "
                       "SparseGPTModifier.dampening_frac, increasing the number of calibration samples, or "
                       "shuffling the calibration dataset")
    return SparsifyResult(float(loss_ok[0]), w_out, ok)


def sparsify_weight(module: torch.nn.Module, hessians_dict: dict, sparsity: float, prune_n: int, prune_m: int,
                    block_size: int, dampening_frac: float, preserve_sparsity_mask: bool):
    """Drop-in for ``sgpt_sparsify.sparsify_weight``: returns ``(loss,
    sparsified weight)`` in the module weight's shape and dtype and removes
    the module's Hessian from ``hessians_dict``."""
    final_shape = module.weight.shape
    H = hessians_dict[module]
    del hessians_dict[module]
    if isinstance(module, torch.nn.Conv2d) or not _is_linear_like(module):
        raise NotImplementedError(f"SparseGPT for {type(module).__name__} is not provided by this build")
    W = module.weight
    conv1d = not isinstance(module, torch.nn.Linear)  # transformers.Conv1D keeps [in, out]
    if conv1d:
        W = W.t().contiguous()
    res = sparsegpt_prune(W, H, sparsity, prune_n, prune_m, block_size, dampening_frac, preserve_sparsity_mask)
    out = res.weight
    if conv1d:
        out = out.t()
    return res.loss, out.reshape(final_shape)
