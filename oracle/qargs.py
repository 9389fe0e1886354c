"""Quantization arguments used by the oracle.

Restates the fields of compressed-tensors ``QuantizationArgs`` that the
reference hot path reads (``modifiers/gptq/gptq_quantize.py:117-166``,
``observers/helpers.py:63-101``, ``observers/min_max.py:34-49``).  This is
plain data; it has no behaviour to pin.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class OArgs:
    num_bits: int = 8
    type: str = "int"               # "int" | "float"
    symmetric: bool = True
    strategy: str = "tensor"        # tensor|channel|group|tensor_group|block|token
    group_size: int | None = None
    block_structure: list[int] | None = None
    actorder: str | None = None     # None | "weight" | "group"
    dynamic: bool | str = False
    observer: str = "minmax"
    scale_dtype: torch.dtype | None = None
    observer_kwargs: dict = field(default_factory=dict)
    # MXFP4: group-32 power-of-two scales (no global scale)
    is_mx: bool = False

    @property
    def zp_dtype(self) -> torch.dtype:
        if self.type == "int":
            return torch.int8
        return torch.float8_e4m3fn if self.num_bits == 8 else torch.bfloat16

    def q_range(self) -> tuple[float, float]:
        """(q_min, q_max) as compressed-tensors ``calculate_range`` gives them."""
        if self.type == "int":
            return float(-(1 << (self.num_bits - 1))), float((1 << (self.num_bits - 1)) - 1)
        if self.num_bits == 8:
            return -448.0, 448.0
        if self.num_bits == 4:
            return -6.0, 6.0
        raise ValueError(f"unsupported float bits {self.num_bits}")
