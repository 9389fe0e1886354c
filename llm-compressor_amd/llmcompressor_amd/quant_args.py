"""Quantization arguments and schemes.

Mirrors the parts of compressed-tensors' ``QuantizationArgs`` /
``QuantizationScheme`` / preset schemes that the reference's hot path reads
(``modifiers/gptq/gptq_quantize.py:117-166``, ``observers/helpers.py:63-131``,
``modifiers/quantization/calibration.py:36-83``), with the same field names,
enum values and defaulting rules, so recipes written for the reference
construct the same arguments here.
"""
from __future__ import annotations

import copy
from dataclasses import dataclass, field
from enum import Enum

import torch


class QuantizationType(str, Enum):
    INT = "int"
    FLOAT = "float"


class QuantizationStrategy(str, Enum):
    TENSOR = "tensor"
    CHANNEL = "channel"
    GROUP = "group"
    BLOCK = "block"
    TOKEN = "token"
    TENSOR_GROUP = "tensor_group"
    ATTN_HEAD = "attn_head"


class ActivationOrdering(str, Enum):
    """``GROUP`` re-observes the permuted weight; ``WEIGHT`` keeps the
    original group scales.  ``DYNAMIC`` / ``STATIC`` are the aliases the
    reference accepts (``modifiers/gptq/base.py:131``)."""
    GROUP = "group"
    WEIGHT = "weight"
    DYNAMIC = "dynamic"
    STATIC = "static"


def _norm_actorder(a):
    if a is None or a is False:
        return None
    if a is True:
        return ActivationOrdering.GROUP
    a = ActivationOrdering(a.value if isinstance(a, ActivationOrdering) else str(a).lower())
    if a == ActivationOrdering.DYNAMIC:
        return ActivationOrdering.GROUP
    if a == ActivationOrdering.STATIC:
        return ActivationOrdering.WEIGHT
    return a


@dataclass
class QuantizationArgs:
    num_bits: int = 8
    type: QuantizationType | str = QuantizationType.INT
    symmetric: bool = True
    group_size: int | None = None
    strategy: QuantizationStrategy | str | None = None
    block_structure: list[int] | None = None
    dynamic: bool | str = False
    actorder: ActivationOrdering | str | bool | None = None
    scale_dtype: torch.dtype | None = None
    zp_dtype: torch.dtype | None = None
    observer: str | None = "minmax"
    observer_kwargs: dict = field(default_factory=dict)

    def __post_init__(self):
        self.type = QuantizationType(self.type.value if isinstance(self.type, QuantizationType) else self.type)
        if self.strategy is not None:
            self.strategy = QuantizationStrategy(
                self.strategy.value if isinstance(self.strategy, QuantizationStrategy) else self.strategy)
        gs = self.group_size
        if gs is not None:
            if gs > 0:
                if self.strategy is None:
                    self.strategy = QuantizationStrategy.GROUP
                elif self.strategy not in (QuantizationStrategy.GROUP, QuantizationStrategy.TENSOR_GROUP):
                    raise ValueError(f"group_size requires strategy group, got {self.strategy}")
            elif gs == -1:
                self.strategy = QuantizationStrategy.CHANNEL
                self.group_size = None
            else:
                raise ValueError(f"invalid group_size {gs}")
        if self.strategy is None:
            self.strategy = QuantizationStrategy.TENSOR
        if self.strategy == QuantizationStrategy.BLOCK and not self.block_structure:
            raise ValueError("block strategy requires block_structure")
        self.actorder = _norm_actorder(self.actorder)
        if self.dynamic and self.observer == "minmax":
            self.observer = None
        if self.zp_dtype is None:
            self.zp_dtype = torch.int8 if self.type == QuantizationType.INT else (
                torch.float8_e4m3fn if self.num_bits == 8 else torch.uint8)

    @property
    def is_mx(self) -> bool:
        """MXFP4: 4-bit float, group 32, power-of-two (e8m0) scales."""
        return (self.type == QuantizationType.FLOAT and self.num_bits == 4 and self.group_size == 32
                and self.scale_dtype == torch.uint8)

    def q_range(self) -> tuple[float, float]:
        if self.type == QuantizationType.INT:
            return float(-(1 << (self.num_bits - 1))), float((1 << (self.num_bits - 1)) - 1)
        if self.num_bits == 8:
            return -448.0, 448.0
        if self.num_bits == 4:
            return -6.0, 6.0
        raise ValueError(f"unsupported float num_bits {self.num_bits}")

    def model_copy(self):
        return copy.deepcopy(self)


# The members of compressed-tensors' ``QuantizationArgs`` this package reads
# from a caller's arguments object; ``resolve_args`` reads nothing else.
CT_ARG_FIELDS = ("num_bits", "type", "symmetric", "group_size", "strategy", "block_structure", "dynamic",
                 "actorder", "scale_dtype", "zp_dtype", "observer", "observer_kwargs")


def _plain(v):
    """An enum member's value (compressed-tensors' str enums, or any other
    enum class), else the value itself."""
    return v.value if isinstance(v, Enum) else v


def resolve_args(args) -> QuantizationArgs:
    """This package's ``QuantizationArgs`` for ``args``.

    ``args`` is returned as it is when it already is one; any other object
    (compressed-tensors' ``QuantizationArgs``, as the reference hands to
    ``quantize_weight`` at ``modifiers/gptq/base.py:591-597``, or a namespace
    with the same field names) is read through the fields in
    ``CT_ARG_FIELDS`` only, enum members by their values, into a new
    dataclass that derives the integer / float range and the MX layout from
    them.  Missing fields take compressed-tensors' defaults.  The caller's
    object is never modified."""
    if isinstance(args, QuantizationArgs):
        return args
    kw = {}
    for f in CT_ARG_FIELDS:
        if hasattr(args, f):
            kw[f] = getattr(args, f)
    for f in ("type", "strategy", "dynamic", "observer"):
        if f in kw:
            kw[f] = _plain(kw[f])
    if "actorder" in kw:
        kw["actorder"] = _plain(kw["actorder"])
    if kw.get("block_structure") is not None:
        kw["block_structure"] = [int(v) for v in kw["block_structure"]]
    kw["observer_kwargs"] = dict(kw.get("observer_kwargs") or {})
    if kw.get("zp_dtype", 0) is None:
        del kw["zp_dtype"]     # filled by type and width, as compressed-tensors does
    return QuantizationArgs(**kw)


@dataclass
class QuantizationScheme:
    targets: list[str] = field(default_factory=lambda: ["Linear"])
    weights: QuantizationArgs | None = None
    input_activations: QuantizationArgs | None = None
    output_activations: QuantizationArgs | None = None


def _w4a16(sym=True):
    return QuantizationScheme(weights=QuantizationArgs(num_bits=4, type="int", symmetric=sym, strategy="group",
                                                       group_size=128))


PRESET_SCHEMES = {
    "W4A16": lambda: _w4a16(True),
    "W4A16_ASYM": lambda: _w4a16(False),
    "W8A16": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=8, type="int", symmetric=True, strategy="channel")),
    "W8A8": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=8, type="int", symmetric=True, strategy="channel"),
        input_activations=QuantizationArgs(num_bits=8, type="int", symmetric=True, strategy="token",
                                           dynamic=True)),
    "FP8_DYNAMIC": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=8, type="float", symmetric=True, strategy="channel"),
        input_activations=QuantizationArgs(num_bits=8, type="float", symmetric=True, strategy="token",
                                           dynamic=True)),
    "FP8": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=8, type="float", symmetric=True, strategy="tensor"),
        input_activations=QuantizationArgs(num_bits=8, type="float", symmetric=True, strategy="tensor")),
    "NVFP4A16": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=4, type="float", symmetric=True, strategy="tensor_group", group_size=16,
                                 scale_dtype=torch.float8_e4m3fn, zp_dtype=torch.float8_e4m3fn)),
    "NVFP4": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=4, type="float", symmetric=True, strategy="tensor_group", group_size=16,
                                 scale_dtype=torch.float8_e4m3fn, zp_dtype=torch.float8_e4m3fn),
        input_activations=QuantizationArgs(num_bits=4, type="float", symmetric=True, strategy="tensor_group",
                                           group_size=16, dynamic="local", scale_dtype=torch.float8_e4m3fn,
                                           zp_dtype=torch.float8_e4m3fn)),
    "MXFP4A16": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=4, type="float", symmetric=True, strategy="group", group_size=32,
                                 scale_dtype=torch.uint8, zp_dtype=torch.uint8)),
    "MXFP4": lambda: QuantizationScheme(
        weights=QuantizationArgs(num_bits=4, type="float", symmetric=True, strategy="group", group_size=32,
                                 scale_dtype=torch.uint8, zp_dtype=torch.uint8),
        input_activations=QuantizationArgs(num_bits=4, type="float", symmetric=True, strategy="group",
                                           group_size=32, dynamic=True, scale_dtype=torch.uint8,
                                           zp_dtype=torch.uint8)),
}


def preset_name_to_scheme(name: str, targets: list[str]) -> QuantizationScheme:
    try:
        s = PRESET_SCHEMES[name.upper()]()
    except KeyError:
        raise KeyError(f"Unknown preset scheme {name}; available: {sorted(PRESET_SCHEMES)}") from None
    s.targets = list(targets)
    return s
