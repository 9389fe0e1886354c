"""compressed-tensors checkpoints from calibrated modules: the save step.

Replaces the compress-and-write half of ``modify_save_pretrained``
(``transformers/compression/compressed_tensors_utils.py:127-228``: the
compressor's ``compress_model`` and ``update_config``) for the formats the
calibration path produces, with this package's kernels doing the quantize and
pack, and the in-repo int4 shard rewriter ``utils/pack_int4_to_int8.py:31-212``
(``QuantConfigParser``, ``Int8Packer``, its command line).

Format of a module (``infer_quantization_format``), as
``tests/llmcompressor/transformers/compression/test_compress_tensor_utils.py:289-322``
fixes it: W8A8 int -> ``int-quantized``, W4A16 / W8A16 int -> ``pack-quantized``,
W8A8 fp8 -> ``float-quantized``, weight-only fp8 -> ``naive-quantized``; MXFP4 ->
``mxfp4-pack-quantized`` (``docs/guides/compression_schemes.md:68-77``).

Tensors written per format follow compressed-tensors as recalled (parity
unpinned: the library is absent and no reference test holds a checkpoint):

* ``pack-quantized``: ``weight_packed`` int32 [rows, ceil(cols * b / 32)]
  (offset-binary b-bit fields along columns, field e at bits b * e),
  ``weight_shape`` int64 [2], ``weight_scale``, ``weight_zero_point`` when
  asymmetric, ``weight_g_idx`` with group activation order;
* ``int-quantized`` / ``naive-quantized`` (int): ``weight`` int8 codes,
  ``weight_scale``, ``weight_zero_point`` when asymmetric;
* ``float-quantized`` / ``naive-quantized`` (fp8): ``weight`` float8_e4m3fn,
  ``weight_scale``;
* ``mxfp4-pack-quantized``: ``weight_packed`` uint8 [rows, cols / 2] (even
  column in the low nibble), ``weight_scale`` uint8 e8m0 [rows, cols / 32].
"""
from __future__ import annotations

import argparse
import json
import os
import re
import shutil

import torch

from . import ops
from .quant_args import QuantizationArgs, QuantizationScheme, QuantizationType

__all__ = ["infer_quantization_format", "compress_module", "quantization_config", "save_compressed",
           "QuantConfigParser", "Int8Packer"]

QUANTIZATION_CONFIG_NAME = "quantization_config"
_VERSION = "llmcompressor_amd-1"


def infer_quantization_format(scheme: QuantizationScheme | None) -> str | None:
    """On-disk format of a module quantized with ``scheme`` (None: not quantized)."""
    w = getattr(scheme, "weights", None)
    if w is None:
        return None
    if w.is_mx:
        return "mxfp4-pack-quantized"
    a = scheme.input_activations
    if w.type == QuantizationType.INT:
        if a is None or w.num_bits < 8:
            return "pack-quantized"
        return "int-quantized"
    if w.num_bits == 8 and a is not None and a.type == QuantizationType.FLOAT and a.num_bits == 8:
        return "float-quantized"
    return "naive-quantized"


def _codes(module, w: QuantizationArgs) -> torch.Tensor:
    g_idx = getattr(module, "weight_g_idx", None)
    return ops.quantize_int(module.weight, module.weight_scale, None if w.symmetric else module.weight_zero_point,
                            w.strategy.value, w.num_bits, w.group_size, g_idx=g_idx,
                            block_structure=w.block_structure)


def compress_module(module: torch.nn.Module, fmt: str | None = None) -> dict[str, torch.Tensor]:
    """The tensors ``fmt`` stores for ``module``'s weight (names without the
    module prefix), computed on the module's GPU by this package's kernels."""
    scheme = module.quantization_scheme
    w = scheme.weights
    fmt = fmt or infer_quantization_format(scheme)
    if fmt == "mxfp4-pack-quantized":
        codes, e8 = ops.mxfp4_quantize_pack(module.weight)
        return {"weight_packed": codes, "weight_scale": e8}
    out = {"weight_scale": module.weight_scale.data}
    if w.type == QuantizationType.INT:
        codes = _codes(module, w)
        if fmt == "pack-quantized":
            out["weight_packed"] = ops.pack_int32(codes, w.num_bits)
            out["weight_shape"] = torch.tensor(list(module.weight.shape), dtype=torch.int64)
            g_idx = getattr(module, "weight_g_idx", None)
            if g_idx is not None:
                out["weight_g_idx"] = g_idx.data
        elif fmt in ("int-quantized", "naive-quantized"):
            out["weight"] = codes
        else:
            raise ValueError(f"format {fmt} cannot hold integer weights")
        if not w.symmetric:
            out["weight_zero_point"] = module.weight_zero_point.data
        return out
    if w.num_bits == 8 and fmt in ("float-quantized", "naive-quantized"):
        out["weight"] = ops.quantize_fp8(module.weight, module.weight_scale, w.strategy.value, w.group_size)
        return out
    raise NotImplementedError(f"format {fmt} for {w.type.value}{w.num_bits} weights is not provided by this build")


def _args_dict(a: QuantizationArgs | None):
    if a is None:
        return None
    dt = lambda t: None if t is None else str(t).replace("torch.", "")  # noqa: E731
    return {"num_bits": a.num_bits, "type": a.type.value, "symmetric": a.symmetric, "group_size": a.group_size,
            "strategy": a.strategy.value, "block_structure": a.block_structure, "dynamic": a.dynamic,
            "actorder": None if a.actorder is None else a.actorder.value, "observer": a.observer,
            "observer_kwargs": a.observer_kwargs, "scale_dtype": dt(a.scale_dtype), "zp_dtype": dt(a.zp_dtype)}


def _quantized_modules(model):
    for name, m in model.named_modules():
        if getattr(getattr(m, "quantization_scheme", None), "weights", None) is not None:
            yield name, m


def quantization_config(model: torch.nn.Module, quantization_format: str | None = None) -> dict:
    """The ``quantization_config`` entry of ``config.json``: one config group
    per distinct scheme, the overall format (``mixed-precision`` when groups
    differ), and the Linear layers left unquantized as ``ignore``."""
    groups, formats = {}, set()
    for _, m in _quantized_modules(model):
        s = m.quantization_scheme
        fmt = quantization_format or infer_quantization_format(s)
        formats.add(fmt)
        g = {"targets": list(s.targets), "weights": _args_dict(s.weights),
             "input_activations": _args_dict(s.input_activations),
             "output_activations": _args_dict(s.output_activations), "format": fmt}
        key = json.dumps(g, sort_keys=True)
        if key not in groups:
            groups[key] = g
    ignore = [name for name, m in model.named_modules()
              if isinstance(m, torch.nn.Linear) and getattr(m, "quantization_scheme", None) is None]
    fmt = (formats.pop() if len(formats) == 1 else "mixed-precision") if formats else "dense"
    return {"config_groups": {f"group_{i}": g for i, g in enumerate(groups.values())}, "format": fmt,
            "ignore": ignore, "quant_method": "compressed-tensors", "quantization_status": "compressed",
            "kv_cache_scheme": None, "global_compression_ratio": None, "sparsity_config": {},
            "transform_config": {}, "version": _VERSION}


def _state_dict(model, quantization_format):
    """(name -> CPU tensor) of the checkpoint: compressed tensors for every
    quantized module, the remaining parameters and buffers as they are."""
    out, taken = {}, set()
    for name, m in _quantized_modules(model):
        prefix = f"{name}." if name else ""
        with torch.no_grad():
            for k, v in compress_module(m, quantization_format).items():
                out[prefix + k] = v.detach().to("cpu").contiguous()
        taken |= {prefix + k for k in ("weight", "weight_scale", "weight_zero_point", "weight_g_idx")}
    for k, v in list(model.state_dict().items()):
        if k in taken or k in out or "_observer." in k:
            continue
        out[k] = v.detach().to("cpu").contiguous()
    return out


def save_compressed(model: torch.nn.Module, save_directory: str, quantization_format: str | None = None,
                    max_shard_size: int = 5 * 2 ** 30, config: dict | None = None) -> dict:
    """Write ``model`` as a compressed-tensors checkpoint: safetensors shards
    (``model.safetensors``, or ``model-0000i-of-0000n.safetensors`` plus
    ``model.safetensors.index.json`` above ``max_shard_size`` bytes) and
    ``config.json`` = the model's config (``model.config.to_dict()`` when it
    has one, else ``config``) with ``quantization_config``.  Returns the index
    (``metadata.total_size`` and ``weight_map``)."""
    from safetensors.torch import save_file

    os.makedirs(save_directory, exist_ok=True)
    state = _state_dict(model, quantization_format)
    shards, cur, cur_size = [], {}, 0
    for k in sorted(state):
        n = state[k].numel() * state[k].element_size()
        if cur and cur_size + n > max_shard_size:
            shards.append(cur)
            cur, cur_size = {}, 0
        cur[k] = state[k]
        cur_size += n
    shards.append(cur)
    weight_map, total = {}, 0
    for i, sh in enumerate(shards):
        fname = "model.safetensors" if len(shards) == 1 else f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors"
        save_file(sh, os.path.join(save_directory, fname), metadata={"format": "pt"})
        for k, v in sh.items():
            weight_map[k] = fname
            total += v.numel() * v.element_size()
    index = {"metadata": {"total_size": total}, "weight_map": weight_map}
    if len(shards) > 1:
        with open(os.path.join(save_directory, "model.safetensors.index.json"), "w") as f:
            json.dump(index, f, indent=2, sort_keys=True)
    cfg = getattr(model, "config", None)
    data = cfg.to_dict() if hasattr(cfg, "to_dict") else dict(config or {})
    data[QUANTIZATION_CONFIG_NAME] = quantization_config(model, quantization_format)
    with open(os.path.join(save_directory, "config.json"), "w") as f:
        json.dump(data, f, indent=2, sort_keys=True)
    return index


# ---------------------------------------------------------------- int4 shard rewriter
class QuantConfigParser:
    """Which int8 weights of a checkpoint hold int4 codes, from its
    ``config.json`` ``quantization_config`` (``pack_int4_to_int8.py:74-141``)."""

    def __init__(self, model_path) -> None:
        config_path = os.path.join(model_path, "config.json")
        if not os.path.exists(config_path):
            raise ValueError("config.json not found in model path")
        with open(config_path, "r") as f:
            self.config = json.load(f).get("quantization_config", {})
            if not self.config:
                raise ValueError("quantization_config not found in config.json")

    @staticmethod
    def _as_module_name(layer_name):
        return layer_name[: -len(".weight")] if layer_name.endswith(".weight") else layer_name

    @staticmethod
    def _int4_condition(weights_scheme):
        if not isinstance(weights_scheme, dict):
            return False
        num_bits_value = weights_scheme.get("num_bits")
        if num_bits_value is None:
            return False
        try:
            num_bits = int(num_bits_value)
        except (TypeError, ValueError):
            return False
        return num_bits == 4 and str(weights_scheme.get("type", "int")).lower() == "int"

    def is_int4_layer(self, layer_name):
        module_name = self._as_module_name(layer_name)
        for group in self.config.get("config_groups", {}).values():
            if not isinstance(group, dict) or not self._int4_condition(group.get("weights", {})):
                continue
            targets = group.get("targets", [])
            if isinstance(targets, str):
                targets = [targets]
            if not isinstance(targets, list):
                continue
            for target in targets:
                if not isinstance(target, str):
                    continue
                if target == "Linear":   # the broad recipe target matches linear weights
                    return True
                if target.startswith("re:"):
                    if re.match(target[3:], module_name) or re.match(target[3:], layer_name):
                        return True
                elif target in (module_name, layer_name):
                    return True
        return False


class Int8Packer:
    """Rewrites a checkpoint whose int4 layers hold one code per int8 into two
    codes per int8 (``pack_int4_to_int8.py:144-200``); the packing runs on the
    GPU (``mi355q_pack_int4_int8``), shard by shard."""

    def __init__(self, model_path, save_path, bias32=False, rename=False, device="cuda"):
        self.bias32, self.rename, self.device = bias32, rename, device
        self.model_path, self.save_path = model_path, save_path
        if not os.path.exists(self.model_path) or not os.path.isdir(self.model_path):
            raise ValueError("Invalid model path")
        os.makedirs(self.save_path, exist_ok=True)
        self.quant_config_parser = QuantConfigParser(model_path)
        self.model_tensors = sorted(f for f in os.listdir(self.model_path) if f.endswith(".safetensors"))
        if not self.model_tensors:
            raise ValueError("No .safetensors files found in model path")

    def _process(self, tensor_name):
        from safetensors import safe_open
        from safetensors.torch import save_file

        index, packed, total = {}, {}, 0
        with safe_open(os.path.join(self.model_path, tensor_name), framework="pt") as f:
            for key in f.keys():
                t = f.get_tensor(key)
                if not key.endswith("weight") or t.dtype != torch.int8 or t.ndim != 2:
                    packed[key] = t.to(torch.float32) if key.endswith("bias") and self.bias32 else t
                    index[key] = tensor_name
                    continue
                if self.quant_config_parser.is_int4_layer(key):
                    if t.shape[1] % 2:
                        raise ValueError(
                            f"Expected even number of columns for int4 packing, but got shape {t.shape}")
                    new_key = f"{key[:-len('weight')]}weight_packed" if self.rename else key
                    packed[new_key] = ops.pack_int4_int8(t.to(self.device)).cpu()
                    index[new_key] = tensor_name
                else:
                    packed[key] = t
                    index[key] = tensor_name
        for t in packed.values():
            total += t.numel() * t.element_size()
        save_file(packed, os.path.join(self.save_path, tensor_name))
        return index, total

    def save(self):
        final_map, final_size = {}, 0
        for name in self.model_tensors:
            m, n = self._process(name)
            final_map.update(m)
            final_size += n
        org = os.path.join(self.model_path, "model.safetensors.index.json")
        if os.path.exists(org):
            with open(org, "r") as f:
                idx = json.load(f)
            idx["weight_map"] = final_map
            meta = idx.get("metadata", {})
            if not isinstance(meta, dict):
                meta = {}
            meta["total_size"] = final_size
            idx["metadata"] = meta
            with open(os.path.join(self.save_path, "model.safetensors.index.json"), "w") as f:
                json.dump(idx, f, sort_keys=True, indent=2)
        for file in os.listdir(self.model_path):
            if file.endswith(".safetensors") or file == "model.safetensors.index.json":
                continue
            src = os.path.join(self.model_path, file)
            if os.path.isfile(src):
                shutil.copy(src, os.path.join(self.save_path, file))


def main(argv=None):
    """``python -m llmcompressor_amd.save -i <model> -o <out> [-bias32] [-rename_packed]``
    (the reference's ``python -m llmcompressor.utils.pack_int4_to_int8``)."""
    parser = argparse.ArgumentParser()
    parser.add_argument("-i", "--model_path", type=str, required=True)
    parser.add_argument("-o", "--save_path", type=str, required=True)
    parser.add_argument("-bias32", action="store_true", default=False)
    parser.add_argument("-rename_packed", action="store_true", default=False,
                        help="Whether to rename packed int8 weight keys to *weight_packed*")
    args = parser.parse_args(argv)
    Int8Packer(args.model_path, args.save_path, args.bias32, args.rename_packed).save()


if __name__ == "__main__":
    main()
