"""Quantize / dequantize / fake-quantize, restated for the CPU oracle.

The reference calls compressed-tensors (CT, pinned ``==0.17.1``,
``setup.py:143-147``; absent from this image) at
``modifiers/gptq/gptq_quantize.py:215-257`` (``fake_quantize``) and at save
time (``quantize`` inside the compressors).  This module restates the
published CT algorithm in torch-CPU code:

* ``quantize``:  ``q = round_to_type(clamp(x / scale + zp, q_min, q_max))``
  where the division happens in the promoted dtype of ``x`` and ``scale``
  (bf16 for a bf16 weight with a bf16 scale; fp32 for GPTQ's fp32 working
  copy), ``round`` is ``torch.round`` (half to even), fp8 rounding is the
  RNE cast to ``float8_e4m3fn``, fp4 rounding is ``cast_to_fp4`` below.
* ``dequantize``: ``(q.to(scale.dtype) - zp) * scale`` - the result is in
  the scale's dtype, so GPTQ's fp32 column is dequantised to bf16 values
  (switch ``dequant_in_scale_dtype``).

Pinning: the int paths are pinned by the reference's known-answer tables
``tests/llmcompressor/modifiers/calibration/test_lifecycle.py:16-165``
(weights: tensor/channel/group-3/block) and ``:168-273`` (activations);
``cast_to_fp4`` is pinned by the fp4 tensor-group rows of the same tables
and by a brute-force nearest-grid-point check over every bf16 value; the
fp8 path is torch's own cast.  The bf16 rounding of GPTQ's dequantised fp32
column (``dequant_in_scale_dtype=True``) is parity unpinned: no reference
test has an fp32 input with a bf16 scale.
"""
from __future__ import annotations

import torch

from .qargs import OArgs

FP4_GRID = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def cast_to_fp4(x: torch.Tensor) -> torch.Tensor:
    """Round to the e2m1 grid, ties to even, saturating at 6 (CT ``cast_to_fp4``).

    Magnitude thresholds: <=0.25 -> 0, <0.75 -> 0.5, <=1.25 -> 1, <1.75 -> 1.5,
    <=2.5 -> 2, <3.5 -> 3, <=5 -> 4, else 6; the sign is re-applied by
    multiplying with ``sign(x)``, so values in (-0.25, 0) become -0.0.
    """
    sign = torch.sign(x)
    a = torch.abs(x)
    out = torch.full_like(a, 6.0)
    out = torch.where(a <= 5.0, torch.full_like(a, 4.0), out)
    out = torch.where(a < 3.5, torch.full_like(a, 3.0), out)
    out = torch.where(a <= 2.5, torch.full_like(a, 2.0), out)
    out = torch.where(a < 1.75, torch.full_like(a, 1.5), out)
    out = torch.where(a <= 1.25, torch.full_like(a, 1.0), out)
    out = torch.where(a < 0.75, torch.full_like(a, 0.5), out)
    out = torch.where(a <= 0.25, torch.zeros_like(a), out)
    return out * sign


def round_to_type(t: torch.Tensor, args: OArgs, q_min: float, q_max: float) -> torch.Tensor:
    """CT ``round_to_quantized_type_args``: clamp, then round in the type's grid."""
    dt = t.dtype
    t = torch.clamp(t, q_min, q_max)
    if args.type == "float":
        if args.num_bits == 8:
            r = t.to(torch.float8_e4m3fn)
        elif args.num_bits == 4:
            r = cast_to_fp4(t)
        else:
            raise NotImplementedError("float bits must be 4 or 8")
    else:
        r = torch.round(t)
    return r.to(dt)


def quantize(x, scale, zero_point, args: OArgs, global_scale=None):
    """Returns rounded values in the promoted dtype of ``x / scale``."""
    q_min, q_max = args.q_range()
    if global_scale is not None:
        scale = scale.to(global_scale.dtype) / global_scale
    scaled = x / scale
    if zero_point is not None:
        scaled = scaled + zero_point.to(scaled.dtype)
    return round_to_type(scaled, args, q_min, q_max)


def dequantize(x_q, scale, zero_point=None, global_scale=None, dequant_in_scale_dtype=True):
    if global_scale is not None:
        scale = scale.to(global_scale.dtype) / global_scale
    dt = scale.dtype if dequant_in_scale_dtype else torch.promote_types(x_q.dtype, scale.dtype)
    v = x_q.to(dt)
    if zero_point is not None:
        v = v - zero_point.to(dt)
    return v * scale.to(dt)


def fake_quantize(x, scale, zero_point, args: OArgs, global_scale=None,
                  dequant_in_scale_dtype=True):
    """Elementwise QDQ; ``scale``/``zero_point`` must broadcast against ``x``."""
    q = quantize(x, scale, zero_point, args, global_scale)
    return dequantize(q, scale, zero_point, global_scale, dequant_in_scale_dtype)


def float_codes(wq: torch.Tensor, s_eff: torch.Tensor, args: OArgs) -> torch.Tensor:
    """Codes of fake-quantised float values ``wq`` (int32): float8_e4m3fn bit
    patterns, or e2m1 codes sign << 3 | index in ``FP4_GRID``.  ``s_eff`` is
    the effective scale per element (scale / global_scale); the grid value is
    recovered as the nearest point to wq / s_eff (the dequantisation rounding
    is far below the grid spacing)."""
    q = wq.to(torch.float32) / s_eff.to(torch.float32)
    sign = torch.signbit(q).to(torch.int32)
    if args.num_bits == 8:
        return q.to(torch.float8_e4m3fn).view(torch.uint8).to(torch.int32)
    grid = torch.tensor(FP4_GRID, dtype=torch.float32)
    idx = torch.argmin((q.abs().unsqueeze(-1) - grid).abs(), dim=-1).to(torch.int32)
    return (sign << 3) | idx


def signed_grid_index(codes: torch.Tensor, args: OArgs) -> torch.Tensor:
    """Float codes as signed positions on the type's grid (monotonic in the
    value), so one code step is one grid step."""
    c = codes.to(torch.int32) & 0xFF
    if args.num_bits == 8:
        mag, sign = c & 0x7F, (c >> 7) & 1
    else:
        mag, sign = c & 0x7, (c >> 3) & 1
    return torch.where(sign == 1, -mag, mag)


def expand_qparams(t: torch.Tensor, shape, args: OArgs) -> torch.Tensor:
    """Expand a [rows, n] qparam tensor to per-element [rows, cols] for ``args.strategy``.

    Equivalent to CT's reshape-based group/block application because every
    step of QDQ is elementwise.
    """
    rows, cols = shape
    if args.strategy == "tensor":
        return t.reshape(1, 1).expand(rows, cols)
    if args.strategy in ("channel", "token"):
        return t.reshape(rows, 1).expand(rows, cols)
    if args.strategy in ("group", "tensor_group"):
        gs = args.group_size
        return t.reshape(rows, -1).repeat_interleave(gs, dim=1)[:, :cols]
    if args.strategy == "block":
        bh, bw = args.block_structure
        return t.repeat_interleave(bh, dim=0).repeat_interleave(bw, dim=1)[:rows, :cols]
    raise ValueError(args.strategy)


def fake_quantize_weight(w, scale, zero_point, args: OArgs, global_scale=None):
    """Whole-weight QDQ as the forward pass of a quantized Linear applies it.

    The group/tensor-group path of CT casts the result back to ``w.dtype``.
    """
    s = expand_qparams(scale, w.shape, args)
    z = expand_qparams(zero_point, w.shape, args) if zero_point is not None else None
    out = fake_quantize(w, s, z, args, global_scale)
    return out.to(w.dtype)
