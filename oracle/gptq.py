"""GPTQ Hessian accumulation and solve, restated for the CPU oracle.

Follows ``modifiers/gptq/gptq_quantize.py`` line by line (environment flags
``LLM_COMPRESSOR_USE_INPLACE_*`` off, their default):

* ``make_empty_hessian``   - ``:54-60``
* ``accumulate_hessian``   - ``:63-97`` (Linear branch; ``num_samples`` counts
  the leading dim after a 2-D input is unsqueezed to 3-D, ``:70-73,91``)
* ``quantize_weight``      - ``:100-296`` (actorder ``:130-166,279-282,299-310``,
  dead-column mask ``:35-38,178``, damping + Cholesky chain with the RTN
  fallback ``:181-196``, blocked sweep ``:199-277``)
* ``normalise_hessian``    - ``modifiers/gptq/base.py:594`` (``H / num_samples``)

Working precision is fp32 as in the reference (``GPTQ_PRECISION``,
``:15``); linear algebra is torch's CPU LAPACK (spotrf/spotri).

Pinning: the Hessian is pinned by its closed form against an fp64
brute-force sum; the Cholesky chain by the identity U^T U (H + lambda I) = I
and by its non-PD fallback; the sweep by the special cases Hinv = I
(GPTQ == round-to-nearest), block-size invariance, a diagonal Hessian (no
cross-column feedback), an fp64 brute-force OBQ on small shapes, and the
shape contracts of ``tests/llmcompressor/modifiers/gptq/test_gptq_quantize.py:21-132``.
"""
from __future__ import annotations

import math

import torch

from .fake_quant import fake_quantize, float_codes
from .observers import OMinMax
from .qargs import OArgs

GPTQ_PRECISION = torch.float32


def make_empty_hessian(num_columns: int, device="cpu") -> torch.Tensor:
    return torch.zeros((num_columns, num_columns), device=device, dtype=GPTQ_PRECISION)


def accumulate_hessian_conv2d(inp: torch.Tensor, H: torch.Tensor, num_samples: torch.Tensor, kernel_size,
                              dilation=1, padding=0, stride=1):
    """Conv2d branch of ``gptq_quantize.py:63-97`` (``:80-89``): the input
    [B, C, h, w] unfolded into its patches, features x samples."""
    inp = inp.to(device=H.device)
    num_added = inp.shape[0]
    unfold = torch.nn.Unfold(kernel_size, dilation=dilation, padding=padding, stride=stride)
    inp = unfold(inp)
    inp = inp.permute([1, 0, 2])
    inp = inp.flatten(1)
    num_samples += num_added
    inp = inp.to(dtype=GPTQ_PRECISION)
    inp = math.sqrt(2) * inp
    H += inp.matmul(inp.t())
    return H, num_samples


def accumulate_hessian(inp: torch.Tensor, H: torch.Tensor, num_samples: torch.Tensor):
    """Linear / Conv1D branch of ``gptq_quantize.py:63-97``."""
    inp = inp.to(device=H.device)
    if inp.dim() == 2:
        inp = inp.unsqueeze(0)
    num_added = inp.shape[0]
    if inp.dim() == 3:
        inp = inp.reshape((-1, inp.shape[-1]))
    inp = inp.t()
    num_samples += num_added
    inp = inp.to(dtype=GPTQ_PRECISION)
    inp = math.sqrt(2) * inp
    H += inp.matmul(inp.t())
    return H, num_samples


def normalise_hessian(H: torch.Tensor, num_samples: torch.Tensor) -> torch.Tensor:
    """``modifiers/gptq/base.py:594``."""
    return H / num_samples


def apply_activation_ordering(W, H, stable=True):
    """``gptq_quantize.py:299-310``.  torch.argsort there is not stable; the
    oracle uses the stable order so exact ties keep column order."""
    perm = torch.argsort(torch.diag(H), descending=True, stable=stable)
    return W[:, perm], H[perm][:, perm], perm


def cholesky_chain(H: torch.Tensor, percdamp: float):
    """Damping + ``cholesky`` -> ``cholesky_inverse`` -> ``cholesky(upper)``.

    Returns (Hinv_upper, ok).  ``ok`` is False when LAPACK reports a non
    positive definite matrix; Hinv is then the identity (``:189-196``).
    """
    H = H.clone()
    damp = percdamp * torch.mean(torch.diag(H))
    diag = torch.arange(H.shape[0])
    H[diag, diag] += damp
    try:
        H = torch.linalg.cholesky(H)
        H = torch.cholesky_inverse(H)
        H = torch.linalg.cholesky(H, upper=True)
        return H, True
    except torch._C._LinAlgError:
        return torch.eye(H.shape[0], dtype=H.dtype), False


def quantize_weight(weight: torch.Tensor, args: OArgs, hessian: torch.Tensor,
                    observer: OMinMax | None = None, blocksize: int = 128,
                    percdamp: float = 0.01, mx_rule: str = "ct",
                    dequant_in_scale_dtype: bool = True, return_codes: bool = False):
    """``gptq_quantize.py:100-296``.

    ``weight`` is the module's weight (bf16), ``observer`` a weight observer
    that has already seen it (``calibration.observe``); when omitted one is
    created and run here.  Returns ``(loss, q_param_dict)`` with the
    reference's keys; with ``return_codes`` also the integer codes
    ``round((Q - zp) / scale)`` in original column order and the Hinv used.
    """
    strategy, actorder = args.strategy, args.actorder
    final_shape, final_dtype = weight.shape, weight.dtype
    if observer is None:
        observer = OMinMax("memoryless_minmax", "weight", args)
        observer(weight)
    W = weight.clone().to(dtype=GPTQ_PRECISION)
    H = hessian.clone()
    num_rows, num_columns = W.shape

    if actorder == "group" and strategy not in ("group", "tensor_group"):
        actorder = None
    perm = None
    if actorder:
        W, H, perm = apply_activation_ordering(W, H)
    if actorder == "group":
        observer.min_vals = observer.max_vals = None
        observer(W)

    g_idx = None
    if strategy in ("group", "tensor_group", "block"):
        divisor = args.group_size if strategy != "block" else args.block_structure[1]
        g_idx = torch.arange(num_columns, dtype=torch.int) // divisor
        if actorder == "weight":
            g_idx = g_idx[perm]

    qp = observer.get_qparams(mx_rule=mx_rule)
    scale, zero_point, global_scale = qp["scale"], qp["zero_point"], qp["global_scale"]

    losses = torch.zeros(num_rows, dtype=GPTQ_PRECISION)

    dead = torch.diag(H) == 0
    H[dead, dead] = 1
    W[:, dead] = 0

    Hinv, ok = cholesky_chain(H, percdamp)

    def qcol(q, col):
        if strategy == "tensor":
            return fake_quantize(q, scale, zero_point, args, global_scale, dequant_in_scale_dtype)
        if strategy == "channel":
            return fake_quantize(q, scale[:, 0], zero_point[:, 0], args, global_scale,
                                 dequant_in_scale_dtype)
        if strategy in ("group", "tensor_group"):
            g = int(g_idx[col])
            return fake_quantize(q, scale[:, g], zero_point[:, g], args, global_scale,
                                 dequant_in_scale_dtype)
        if strategy == "block":
            b = int(g_idx[col])
            bh = args.block_structure[0]
            s = scale[:, b].repeat_interleave(bh)[:num_rows]
            z = zero_point[:, b].repeat_interleave(bh)[:num_rows]
            return fake_quantize(q, s, z, args, global_scale, dequant_in_scale_dtype)
        raise ValueError(f"Quantization strategy is not supported for GPTQ: {strategy}")

    for i1 in range(0, num_columns, blocksize):
        i2 = min(i1 + blocksize, num_columns)
        count = i2 - i1
        W1 = W[:, i1:i2].clone()
        Q1 = torch.zeros_like(W1)
        Err1 = torch.zeros_like(W1)
        losses1 = torch.zeros_like(W1)
        Hinv1 = Hinv[i1:i2, i1:i2]
        for i in range(count):
            w = W1[:, i]
            d = Hinv1[i, i]
            q = qcol(w.clone(), i1 + i)
            Q1[:, i] = q
            losses1[:, i] = (w - q) ** 2 / d ** 2
            err1 = (w - q) / d
            W1[:, i:] -= err1.unsqueeze(1).matmul(Hinv1[i, i:].unsqueeze(0))
            Err1[:, i] = err1
        W[:, i1:i2] = Q1
        losses += torch.sum(losses1, 1) / 2
        W[:, i2:] -= Err1.matmul(Hinv[i1:i2, i2:])

    invperm = None
    if actorder:
        invperm = torch.argsort(perm)
        W = W[:, invperm]
    W32 = W
    W = W.reshape(final_shape).to(final_dtype)
    loss = torch.sum(losses).item()
    out = {
        "weight": W,
        "weight_scale": scale.to(dtype=final_dtype),
        "weight_zero_point": zero_point.to(dtype=args.zp_dtype),
    }
    if global_scale is not None:
        out["weight_global_scale"] = global_scale.to(dtype=final_dtype)
    if actorder == "group":
        out["weight_g_idx"] = g_idx[invperm]
    if not return_codes:
        return loss, out
    codes = weight_codes(W32 if args.type == "float" else W, scale, zero_point, args, g_idx, perm, invperm,
                         global_scale)
    return loss, out, {"codes": codes, "hinv": Hinv, "ok": ok, "perm": perm,
                       "scale_used": scale, "losses": losses}


def weight_codes(Wq, scale, zero_point, args: OArgs, g_idx, perm, invperm, global_scale=None):
    """Codes of the fake-quantised weight, original column order: integers,
    or for float types ``fake_quant.float_codes`` of the fp32 values."""
    rows, cols = Wq.shape
    if args.strategy == "tensor":
        s = scale.float().reshape(1, 1).expand(rows, cols)
        z = zero_point.float().reshape(1, 1).expand(rows, cols)
    elif args.strategy == "channel":
        s = scale.float().reshape(rows, 1).expand(rows, cols)
        z = zero_point.float().reshape(rows, 1).expand(rows, cols)
    else:
        gi = g_idx if perm is None else g_idx[invperm]
        if args.strategy == "block":
            bh = args.block_structure[0]
            s = scale.float().repeat_interleave(bh, 0)[:rows][:, gi.long()]
            z = zero_point.float().repeat_interleave(bh, 0)[:rows][:, gi.long()]
        else:
            s = scale.float()[:, gi.long()]
            z = zero_point.float()[:, gi.long()]
    if args.type == "float":
        s_eff = s if global_scale is None else s / global_scale.to(torch.float32)
        return float_codes(Wq, s_eff, args)
    return torch.round(Wq.float() / s + z).to(torch.int32)
