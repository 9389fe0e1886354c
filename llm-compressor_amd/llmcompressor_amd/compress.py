"""Quantize + pack of calibrated weights into compressed-tensors layouts.

Replaces the compressor step of the save path
(``transformers/compression/compressed_tensors_utils.py:172-191``,
``entrypoints/model_free/process.py:114``) and the in-repo nibble packer
(``utils/pack_int4_to_int8.py:13-28``).  Each function takes the module's
fake-quantised weight and its qparams and returns the tensors a
compressed-tensors checkpoint stores for that format:

* ``pack_quantized`` (int4 W4A16): ``weight_packed`` int32 [rows, cols/8]
  (offset-binary nibbles, element k at bits 4k), ``weight_scale``,
  ``weight_zero_point``, ``weight_shape``.
* ``int_quantized`` (int8): ``weight`` int8 codes.
* ``mxfp4_pack_quantized``: ``weight_packed`` uint8 [rows, cols/2] e2m1
  pairs (even column in the low nibble) and ``weight_scale`` uint8 e8m0
  [rows, cols/32].
* ``float_quantized`` (fp8 e4m3): ``weight`` float8_e4m3fn.
"""
from __future__ import annotations

import torch

from . import ops
from .quant_args import QuantizationArgs, QuantizationType


def _codes(weight, scale, zero_point, args: QuantizationArgs, g_idx=None):
    return ops.quantize_int(weight, scale, zero_point if not args.symmetric else None, args.strategy.value,
                            args.num_bits, args.group_size, g_idx=g_idx, block_structure=args.block_structure)


def pack_quantized(weight, scale, zero_point, args: QuantizationArgs, g_idx=None) -> dict:
    if args.type != QuantizationType.INT or args.num_bits > 8:
        raise ValueError("pack_quantized needs an integer format of at most 8 bits")
    codes = _codes(weight, scale, zero_point, args, g_idx)
    out = {"weight_scale": scale, "weight_shape": torch.tensor(list(weight.shape), dtype=torch.int64)}
    if args.num_bits == 4:
        out["weight_packed"] = ops.pack_int4_int32(codes)
    else:
        out["weight"] = codes
    if not args.symmetric:
        out["weight_zero_point"] = zero_point
    if g_idx is not None:
        out["weight_g_idx"] = g_idx
    return out


def int_quantized(weight, scale, zero_point, args: QuantizationArgs) -> dict:
    return {"weight": _codes(weight, scale, zero_point, args), "weight_scale": scale}


def pack_int4_to_int8(codes: torch.Tensor) -> torch.Tensor:
    """``utils/pack_int4_to_int8.py:13-28`` (two signed nibbles per int8)."""
    return ops.pack_int4_int8(codes)


def mxfp4_pack_quantized(weight: torch.Tensor, rule: str = "ct") -> dict:
    codes, e8 = ops.mxfp4_quantize_pack(weight, rule)
    return {"weight_packed": codes, "weight_scale": e8}


def float_quantized(weight, scale, args: QuantizationArgs) -> dict:
    return {"weight": ops.quantize_fp8(weight, scale, args.strategy.value, args.group_size),
            "weight_scale": scale}
