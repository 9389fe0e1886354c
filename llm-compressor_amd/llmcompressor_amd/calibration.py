"""Observer attachment and qparam updates on modules.

Mirrors ``modifiers/quantization/calibration.py:36-157``: weight observers
named ``minmax`` / ``static_minmax`` are replaced by ``memoryless_minmax``
(``:64-71``), dynamic arguments get no observer (``:80``), ``observe`` runs
the observer on ``module.<base_name>``, and ``update_qparams`` stores
``<base>_scale`` / ``<base>_zero_point`` (skipping scale/zp for dynamic
arguments) when the module has those parameters.
"""
from __future__ import annotations

from collections.abc import Iterable
from itertools import product

import torch
from torch.nn import Module

from .observers import Observer
from .quant_args import QuantizationScheme, resolve_args

__all__ = ["initialize_observer", "observe", "update_qparams", "initialize_module_for_quantization"]


def initialize_module_for_quantization(module: Module, scheme: QuantizationScheme) -> None:
    """Attach ``quantization_scheme`` and empty ``weight_scale`` /
    ``weight_zero_point`` parameters shaped for the weight strategy (and
    ``weight_global_scale`` for tensor groups)."""
    module.quantization_scheme = scheme
    if scheme.weights is None or not hasattr(module, "weight"):
        return
    wa = resolve_args(scheme.weights)
    rows, cols = module.weight.shape
    s = wa.strategy.value
    if s == "tensor":
        shape = (1,)
    elif s == "channel":
        shape = (rows, 1)
    elif s in ("group", "tensor_group"):
        shape = (rows, -(-cols // wa.group_size))
    elif s == "block":
        bh, bw = wa.block_structure
        shape = (-(-rows // bh), -(-cols // bw))
    else:
        raise ValueError(f"strategy {s} cannot quantize weights")
    dev = module.weight.device
    sdt = wa.scale_dtype if wa.scale_dtype is not None else module.weight.dtype
    module.register_parameter("weight_scale", torch.nn.Parameter(torch.empty(shape, dtype=sdt, device=dev),
                                                                 requires_grad=False))
    module.register_parameter("weight_zero_point", torch.nn.Parameter(
        torch.zeros(shape, dtype=wa.zp_dtype, device=dev), requires_grad=False))
    if s == "tensor_group":   # NVFP4: the per-tensor global scale beside the group scales
        module.register_parameter("weight_global_scale", torch.nn.Parameter(
            torch.ones((1,), dtype=torch.float32, device=dev), requires_grad=False))
    if wa.actorder is not None and wa.actorder.value == "group":
        module.register_parameter("weight_g_idx", torch.nn.Parameter(
            torch.full((cols,), -1, dtype=torch.int, device=dev), requires_grad=False))


def initialize_observer(module: Module, base_name: str) -> None:
    arg_name = {"weight": "weights", "output": "output_activations"}.get(base_name, "input_activations")
    scheme = getattr(module, "quantization_scheme", None)
    args = getattr(scheme, arg_name, None) if scheme is not None else None
    if args is None:
        return
    args = resolve_args(args)
    observer = args.observer
    if base_name == "weight" and observer in ("static_minmax", "minmax"):
        observer = "memoryless_minmax"
    if base_name == "weight" and observer == "mse":
        observer = "memoryless_mse"
    if args.dynamic is not True:
        obs = Observer.load_from_registry(observer, base_name=base_name, args=args)
        module.register_module(f"{base_name}_observer", obs)


def observe(module: Module | Iterable[Module], base_name: str) -> None:
    if isinstance(module, Iterable):
        for m in module:
            observe(m, base_name)
        return
    observer = getattr(module, f"{base_name}_observer", None)
    if observer is None:
        return
    observer(getattr(module, base_name))


def update_qparams(module: Module | Iterable[Module], base_name: str | Iterable[str],
                   only_update_onload: bool = False) -> None:
    if isinstance(module, Iterable) or not isinstance(base_name, str):
        modules = [module] if not isinstance(module, Iterable) else module
        names = [base_name] if isinstance(base_name, str) else base_name
        for m, b in product(modules, names):
            update_qparams(m, b, only_update_onload=only_update_onload)
        return
    observer = getattr(module, f"{base_name}_observer", None)
    if observer is None or not observer.has_statistics:
        return
    args = observer.args
    is_dynamic = getattr(args, "dynamic", False) in (True, "local")
    qparams = observer.get_qparams()
    for name, val in qparams.items():
        if val is None or (is_dynamic and name in ("scale", "zero_point")):
            continue
        full = f"{base_name}_{name}"
        if hasattr(module, full):
            p = getattr(module, full)
            if p.shape != val.shape or p.dtype != val.dtype:
                setattr(module, full, torch.nn.Parameter(val.detach().clone(), requires_grad=False))
            else:
                p.data.copy_(val)
