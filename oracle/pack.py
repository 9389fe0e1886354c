"""Quantize + pack byte layouts, restated in numpy for the CPU oracle.

* ``pack_int4_to_int8``  - ``utils/pack_int4_to_int8.py:13-28`` (in-repo):
  low nibble = even column, high nibble = odd column, rows never mixed;
  odd column counts raise.  Pinned by
  ``tests/llmcompressor/utils/test_pack_int4_to_int8.py:25-46``.
* ``pack_to_int32``      - compressed-tensors ``pack_to_int32`` (the
  ``pack_quantized`` format of W4A16): codes offset by 2^(b-1), eight
  4-bit fields per int32, field k at bits 4k along the column axis
  (``packed_dim=0``: along the rows, as CT packs asymmetric group / channel
  zero points).  Parity unpinned against the reference (CT absent, no
  reference test); pinned by a hand-computed vector and the unpack round
  trip.
* ``mxfp4_quantize_pack`` - MXFP4 codes and e8m0 scales from bf16 bit
  patterns: shared exponent by the rule in ``oracle.observers.mx_scale_exponent``
  ("ct" default, "ocp" switch), e2m1 rounding with compressed-tensors
  ``cast_to_fp4`` thresholds, code = sign << 3 | grid index, two codes per
  byte with the even column in the low nibble (CT ``pack_fp4_to_uint8``).
  Parity unpinned against the reference (no test, CT absent); pinned
  against the torch fake-quant path of this oracle and a brute-force
  nearest-grid-point search with ties to even.
* ``fp4_group_quantize_pack`` - the NVFP4 ``weight_packed`` tensor: the same
  codes and layout for x / (scale / global_scale) with given fp8 group
  scales.  Format name and tensor names pinned by
  ``tests/llmcompressor/entrypoints/model_free/test_convert_checkpoint.py:81-109``;
  the code layout parity unpinned as for MXFP4, and pinned the same way.
"""
from __future__ import annotations

import numpy as np

E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)


def pack_int4_to_int8(t: np.ndarray) -> np.ndarray:
    if t.ndim != 2:
        raise ValueError(f"Expected 2D tensor, but got {t.ndim}D")
    rows, cols = t.shape
    if cols % 2 != 0:
        raise ValueError(f"Expected even number of columns for int4 packing, but got shape {t.shape}")
    u = t.astype(np.int8).view(np.uint8)
    low = u[:, 0::2] & 0x0F
    high = u[:, 1::2] & 0x0F
    return ((high << 4) | low).astype(np.uint8).view(np.int8).reshape(rows, cols // 2)


def pack_to_int32(codes: np.ndarray, num_bits: int = 4, packed_dim: int = 1) -> np.ndarray:
    if packed_dim == 0:   # fields along the rows (CT's group / channel zero points)
        return np.ascontiguousarray(pack_to_int32(np.ascontiguousarray(codes.T), num_bits).T)
    rows, cols = codes.shape
    per = 32 // num_bits
    v = (codes.astype(np.int32) + (1 << (num_bits - 1))).astype(np.uint32) & ((1 << num_bits) - 1)
    if cols % per:   # padded after the offset: unused positions hold 0
        v = np.pad(v, ((0, 0), (0, per - cols % per)))
    v = v.reshape(rows, -1, per)
    shifts = (np.arange(per, dtype=np.uint32) * num_bits)
    return np.bitwise_or.reduce(v << shifts, axis=2).astype(np.uint32).view(np.int32)


def unpack_from_int32(packed: np.ndarray, cols: int, num_bits: int = 4, packed_dim: int = 1) -> np.ndarray:
    if packed_dim == 0:
        return np.ascontiguousarray(unpack_from_int32(np.ascontiguousarray(packed.T), cols, num_bits).T)
    per = 32 // num_bits
    u = packed.view(np.uint32)
    shifts = (np.arange(per, dtype=np.uint32) * num_bits)
    v = (u[:, :, None] >> shifts) & ((1 << num_bits) - 1)
    return (v.reshape(packed.shape[0], -1)[:, :cols].astype(np.int32) - (1 << (num_bits - 1))).astype(np.int8)


def _mx_exponent(amax_bits: np.ndarray, rule: str) -> np.ndarray:
    """e8m0 byte from bf16 absmax bit patterns (uint16, sign clear)."""
    b = amax_bits.astype(np.int64)
    if rule == "ct":
        r = (b + (1 << 5)) & 0xFF80
        e = ((r >> 7) & 0xFF) - 127
    elif rule == "ocp":
        e = ((b >> 7) & 0xFF) - 127
    else:
        raise ValueError(rule)
    e8 = np.clip(e + 127 - 2, 0, 254)
    return np.where(b == 0, 0, e8).astype(np.uint8)


def e2m1_codes(v: np.ndarray) -> np.ndarray:
    """CT cast_to_fp4 thresholds -> 4-bit codes (sign bit for v < 0)."""
    a = np.minimum(np.abs(v), 6.0)
    idx = np.select(
        [a <= 0.25, a < 0.75, a <= 1.25, a < 1.75, a <= 2.5, a < 3.5, a <= 5.0],
        [0, 1, 2, 3, 4, 5, 6], default=7).astype(np.uint8)
    return idx | np.where(v < 0, 8, 0).astype(np.uint8)


def mxfp4_quantize_pack(x_bits: np.ndarray, rule: str = "ct"):
    """x_bits: uint16 bf16 patterns [rows, cols] -> (codes uint8 [rows, cols/2], e8m0 [rows, cols/32])."""
    rows, cols = x_bits.shape
    if cols % 32:
        raise ValueError("cols must be a multiple of 32")
    g = x_bits.reshape(rows, cols // 32, 32)
    amax = (g & 0x7FFF).max(axis=2)
    e8 = _mx_exponent(amax, rule)
    xf = (x_bits.astype(np.uint32) << 16).view(np.float32).reshape(rows, cols // 32, 32)
    scale_inv = np.ldexp(np.float32(1.0), (127 - e8.astype(np.int32)))[..., None].astype(np.float32)
    v = (xf * scale_inv).reshape(rows, cols)
    c = e2m1_codes(v)
    packed = (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)
    return packed, e8


def fp4_group_quantize_pack(x: np.ndarray, scale: np.ndarray, group: int, global_scale=None) -> np.ndarray:
    """NVFP4 weight codes (``nvfp4-pack-quantized``): e2m1 codes of
    x / (scale / global_scale), the effective scale and the quotient in
    float32 as the oracle's ``fake_quant.quantize`` forms them; x float32
    [rows, cols], scale float32 [rows, ceil(cols / group)].  Packed as
    ``mxfp4_quantize_pack``."""
    s = scale.astype(np.float32)
    if global_scale is not None:
        s = (s / np.float32(global_scale)).astype(np.float32)
    cols = x.shape[1]
    v = (x.astype(np.float32) / s[:, np.arange(cols) // group]).astype(np.float32)
    c = e2m1_codes(v)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)


def fp4_unpack(packed: np.ndarray) -> np.ndarray:
    """e2m1 grid values (float32) of packed codes [rows, cols / 2]."""
    rows, half = packed.shape
    c = np.empty((rows, half * 2), dtype=np.uint8)
    c[:, 0::2], c[:, 1::2] = packed & 0x0F, packed >> 4
    return (E2M1_GRID[c & 7] * np.where(c & 8, -1.0, 1.0)).astype(np.float32)


def mxfp4_unpack(packed: np.ndarray, e8: np.ndarray) -> np.ndarray:
    rows, half = packed.shape
    lo, hi = packed & 0x0F, packed >> 4
    c = np.empty((rows, half * 2), dtype=np.uint8)
    c[:, 0::2], c[:, 1::2] = lo, hi
    v = E2M1_GRID[c & 7] * np.where(c & 8, -1.0, 1.0)
    s = np.ldexp(np.float32(1.0), e8.astype(np.int32) - 127).repeat(32, axis=1)
    return (v * s).astype(np.float32)
