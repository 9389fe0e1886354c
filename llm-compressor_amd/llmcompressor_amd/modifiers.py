"""GPTQModifier / QuantizationModifier: the calling order around the kernels.

These mirror the reference's modifiers at the level the hot path needs
(``modifiers/gptq/base.py:50-674``,
``modifiers/quantization/quantization/base.py:26-137``):

* ``on_initialize``: attach the scheme + weight qparams + observers to every
  targeted ``nn.Linear`` (``QuantizationMixin.initialize_quantization``);
* ``on_calibration_start``: register the ``calibrate_module`` forward hook
  (``base.py:255-289``) that lazily creates H and ``num_samples`` and calls
  ``accumulate_hessian``;
* ``on_sequential_epoch_end``: ``observe(weight)`` then ``compress_modules``
  -> ``quantize_weight`` on H / num_samples (``base.py:578-601``), writing
  ``weight`` / ``weight_scale`` / ``weight_zero_point`` / ``weight_g_idx``;
* ``QuantizationModifier``: RTN - observe + update_qparams of weights
  (``quantization/base.py:85-96``).

``GPTQModifier.apply(model, batches)`` runs one calibration pass over the
batches (the basic pipeline: every target sees its inputs in one pass) and
compresses every module.
"""
from __future__ import annotations

import logging
import re
import time

import torch

from .calibration import initialize_module_for_quantization, initialize_observer, observe, update_qparams
from .gptq import accumulate_hessian, gptq_quantize, make_empty_hessian
from .quant_args import ActivationOrdering, QuantizationArgs, QuantizationScheme, preset_name_to_scheme

logger = logging.getLogger("llmcompressor_amd")


def _matches(name: str, module: torch.nn.Module, patterns) -> bool:
    for p in patterns:
        if p.startswith("re:"):
            if re.match(p[3:], name):
                return True
        elif p == type(module).__name__ or p == name:
            return True
    return False


class QuantizationModifier:
    def __init__(self, scheme: str | dict | None = None, targets=("Linear",), ignore=("lm_head",),
                 config_groups: dict | None = None):
        self.targets = list(targets)
        self.ignore = list(ignore)
        self.scheme = scheme
        self.config_groups = config_groups

    def resolve_schemes(self) -> list[QuantizationScheme]:
        if self.config_groups:
            out = []
            for g in self.config_groups.values():
                if isinstance(g, QuantizationScheme):
                    out.append(g)
                else:
                    w = g.get("weights")
                    out.append(QuantizationScheme(targets=g.get("targets", self.targets),
                                                  weights=w if isinstance(w, QuantizationArgs) or w is None
                                                  else QuantizationArgs(**w)))
            return out
        if isinstance(self.scheme, str):
            return [preset_name_to_scheme(self.scheme, self.targets)]
        if isinstance(self.scheme, QuantizationScheme):
            return [self.scheme]
        raise ValueError("a scheme or config_groups is required")

    def target_modules(self, model: torch.nn.Module):
        for name, m in model.named_modules():
            for sch in self.resolve_schemes():
                if _matches(name, m, sch.targets) and not _matches(name, m, self.ignore):
                    yield name, m, sch
                    break

    def on_initialize(self, model):
        self._modules = {}
        for name, m, sch in self.target_modules(model):
            sch = QuantizationScheme(targets=sch.targets, weights=sch.weights.model_copy() if sch.weights else None,
                                     input_activations=sch.input_activations, output_activations=sch.output_activations)
            self._resolve_actorder(sch)
            initialize_module_for_quantization(m, sch)
            initialize_observer(m, "weight")
            self._modules[m] = name
        return True

    def _resolve_actorder(self, sch):
        pass

    def on_sequential_epoch_end(self, modules):
        observe(modules, "weight")
        update_qparams(modules, "weight")

    def apply(self, model, batches=None):
        self.on_initialize(model)
        self.on_sequential_epoch_end(list(self._modules))
        return model


class GPTQModifier(QuantizationModifier):
    def __init__(self, scheme=None, targets=("Linear",), ignore=("lm_head",), config_groups=None,
                 block_size: int = 128, dampening_frac: float | None = 0.01, actorder="static",
                 offload_hessians: bool = False):
        super().__init__(scheme, targets, ignore, config_groups)
        self.block_size = block_size
        self.dampening_frac = dampening_frac
        self.actorder = actorder
        self.offload_hessians = offload_hessians
        self._hessians: dict = {}
        self._num_samples: dict = {}
        self._hooks = []
        self.timings: dict[str, float] = {}

    def _resolve_actorder(self, sch):
        """``base.py:137-193``: the sentinel default ``static`` only fills an unset actorder."""
        w = sch.weights
        if w is None:
            return
        if self.actorder == "static":
            w.actorder = ActivationOrdering.WEIGHT if w.actorder is None else w.actorder
        elif self.actorder is not None:
            mine = QuantizationArgs(actorder=self.actorder).actorder
            if w.actorder is not None and w.actorder != mine:
                raise ValueError("Cannot resolve activation ordering when both GPTQModifier.actorder and "
                                 "QuantizationScheme.actorder are provided and differ")
            w.actorder = mine
        if w.actorder == ActivationOrdering.GROUP and w.strategy.value not in ("group", "tensor_group"):
            w.actorder = None

    def calibrate_module(self, module, args, _output):
        inp = args[0]
        if module not in self._num_samples:
            dev = module.weight.device
            self._hessians[module] = make_empty_hessian(module, device="cpu" if self.offload_hessians else dev)
            self._num_samples[module] = torch.zeros(tuple(), device=dev)
        H = self._hessians[module]
        if self.offload_hessians:
            H = H.to(module.weight.device)
        H, self._num_samples[module] = accumulate_hessian(inp, module, H, self._num_samples[module])
        self._hessians[module] = H.to("cpu") if self.offload_hessians else H

    def on_calibration_start(self, model):
        for m in self._modules:
            if getattr(m.quantization_scheme, "weights", None) is not None:
                self._hooks.append(m.register_forward_hook(self.calibrate_module))
        if not self._hooks:
            raise ValueError("GPTQModifier was unable to find any modules to quantize. Please check "
                             "quantization `config_groups` and `targets` in recipe")

    def on_sequential_epoch_end(self, modules):
        modules = [m for m in modules if getattr(m, "quantization_scheme", None) is not None]
        observe(modules, "weight")
        self.compress_modules()

    def compress_modules(self):
        for module in list(self._num_samples):
            name = self._modules[module]
            n = float(self._num_samples.pop(module).item())
            H = self._hessians.pop(module).to(module.weight.device)
            qa = module.quantization_scheme.weights
            t0 = time.perf_counter()
            with torch.no_grad():
                res = gptq_quantize(module.weight, qa, H, module.weight_observer, self.block_size,
                                    self.dampening_frac, num_samples=n)
            self.timings[name] = time.perf_counter() - t0
            logger.info("Quantized %s using %d samples, loss %.4f", name, int(n), res.loss)
            with torch.no_grad():
                module.weight.data.copy_(res.weight)
                update = {"weight_scale": res.scale.to(module.weight.dtype),
                          "weight_zero_point": res.zero_point.to(qa.zp_dtype)}
                if qa.actorder == ActivationOrdering.GROUP:
                    update["weight_g_idx"] = res.g_idx[torch.argsort(res.perm)]
                for k, v in update.items():
                    setattr(module, k, torch.nn.Parameter(v, requires_grad=False))
            module.gptq_codes = res.codes

    def on_calibration_end(self):
        for h in self._hooks:
            h.remove()
        self._hooks = []

    def on_finalize(self):
        if self._num_samples:
            raise ValueError(f"Failed to compress {len(self._num_samples)} modules")
        return True

    def apply(self, model, batches):
        """Initialize, hook, run the calibration batches, compress."""
        self.on_initialize(model)
        self.on_calibration_start(model)
        with torch.no_grad():
            for b in batches:
                model(b)
        self.on_calibration_end()
        self.on_sequential_epoch_end(list(self._modules))
        self.on_finalize()
        return model
