"""compressed-tensors checkpoints from calibrated modules: the save step.

Replaces the compress-and-write half of ``modify_save_pretrained``
(``transformers/compression/compressed_tensors_utils.py:127-228``: the
compressor's ``compress_model`` and ``update_config``) for the formats the
calibration path produces, with this package's kernels doing the quantize and
pack, and the int4 shard rewriter of ``utils/pack_int4_to_int8.py:31-212``
(``QuantConfigParser``, ``Int8Packer``, its command line).

Format of a module (``infer_quantization_format``), as
``tests/llmcompressor/transformers/compression/test_compress_tensor_utils.py:289-322``
fixes it: W8A8 int -> ``int-quantized``, W4A16 / W8A16 int -> ``pack-quantized``,
W8A8 fp8 -> ``float-quantized``, weight-only fp8 -> ``naive-quantized``; MXFP4 ->
``mxfp4-pack-quantized`` (``docs/guides/compression_schemes.md:68-77``); NVFP4
(fp4 tensor-group weights) -> ``nvfp4-pack-quantized`` (its tensor names pinned
by ``tests/llmcompressor/entrypoints/model_free/test_convert_checkpoint.py:81-109``).

Tensors written per format follow compressed-tensors as recalled (parity
unpinned: the library is absent and no reference test holds a checkpoint):

* ``pack-quantized``: ``weight_packed`` int32 [rows, ceil(cols * b / 32)]
  (offset-binary b-bit fields along columns, field e at bits b * e),
  ``weight_shape`` int64 [2], ``weight_scale``, ``weight_zero_point`` when
  asymmetric (group / channel zero points packed the same way along the
  output dimension: int32 [ceil(rows * b / 32), groups]), ``weight_g_idx``
  with group activation order;
* ``int-quantized`` / ``naive-quantized`` (int): ``weight`` int8 codes,
  ``weight_scale``, ``weight_zero_point`` when asymmetric;
* ``float-quantized`` / ``naive-quantized`` (fp8): ``weight`` float8_e4m3fn,
  ``weight_scale``;
* ``mxfp4-pack-quantized``: ``weight_packed`` uint8 [rows, cols / 2] (even
  column in the low nibble), ``weight_scale`` uint8 e8m0 [rows, cols / 32];
* ``nvfp4-pack-quantized``: ``weight_packed`` uint8 [rows, cols / 2] (the
  same code layout, e2m1 of weight / (scale / global_scale)),
  ``weight_scale`` float8_e4m3fn [rows, cols / 16], ``weight_global_scale``
  [1] in the module's dtype for it.
"""
from __future__ import annotations

import argparse
import json
import os
import shutil

import torch

from . import ops
from .quant_args import QuantizationArgs, QuantizationScheme, QuantizationStrategy, QuantizationType, resolve_args

__all__ = ["infer_quantization_format", "compress_module", "quantization_config", "save_compressed",
           "QuantConfigParser", "Int8Packer"]

QUANTIZATION_CONFIG_NAME = "quantization_config"
_VERSION = "llmcompressor_amd-1"


def infer_quantization_format(scheme: QuantizationScheme | None) -> str | None:
    """On-disk format of a module quantized with ``scheme`` (None: not quantized)."""
    w = getattr(scheme, "weights", None)
    if w is None:
        return None
    w = resolve_args(w)
    if w.is_mx:
        return "mxfp4-pack-quantized"
    if w.type == QuantizationType.FLOAT and w.num_bits == 4 and w.strategy == QuantizationStrategy.TENSOR_GROUP:
        return "nvfp4-pack-quantized"
    a = getattr(scheme, "input_activations", None)
    a = None if a is None else resolve_args(a)
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
    w = resolve_args(scheme.weights)
    fmt = fmt or infer_quantization_format(scheme)
    if fmt == "mxfp4-pack-quantized":
        codes, e8 = ops.mxfp4_quantize_pack(module.weight)
        return {"weight_packed": codes, "weight_scale": e8}
    if fmt == "nvfp4-pack-quantized":
        gs = getattr(module, "weight_global_scale", None)
        if gs is None:
            raise ValueError("nvfp4-pack-quantized needs the module's weight_global_scale")
        scale = module.weight_scale.data
        packed = ops.fp4_quantize_pack(module.weight, scale, w.group_size, gs.data)
        # the group scales are fp8 values held in a wider dtype: the cast is
        # exact; the global scale is written as the module holds it (its fp32
        # parameter), as a parameter the compressor passes through
        return {"weight_packed": packed, "weight_scale": scale.to(torch.float8_e4m3fn),
                "weight_global_scale": gs.data.reshape(1)}
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
            zp = module.weight_zero_point.data
            if fmt == "pack-quantized" and w.strategy in (QuantizationStrategy.GROUP, QuantizationStrategy.CHANNEL):
                zp = ops.pack_int32(zp.to(torch.int8).t().contiguous(), w.num_bits).t().contiguous()
            out["weight_zero_point"] = zp
        return out
    if w.num_bits == 8 and fmt in ("float-quantized", "naive-quantized"):
        out["weight"] = ops.quantize_fp8(module.weight, module.weight_scale, w.strategy.value, w.group_size)
        return out
    raise NotImplementedError(f"format {fmt} for {w.type.value}{w.num_bits} weights is not provided by this build")


def _args_dict(a: QuantizationArgs | None):
    if a is None:
        return None
    a = resolve_args(a)
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
# Interface kept from utils/pack_int4_to_int8.py:69-212 (class and method
# names, constructor arguments, the command-line flags and the ValueError
# conditions its tests pin); the selection reuses the recipe target matcher
# and the rewrite streams one shard at a time with the nibble pack on the GPU.

def _int4_int_weights(weights) -> bool:
    """A config group's weight arguments describe 4-bit integers (type int by
    default, num_bits given as anything int() accepts)."""
    if not isinstance(weights, dict):
        return False
    try:
        bits = int(weights["num_bits"])
    except (KeyError, TypeError, ValueError):
        return False
    return bits == 4 and str(weights.get("type", "int")).lower() == "int"


def _target_list(targets) -> list[str]:
    if isinstance(targets, str):
        return [targets]
    return [t for t in targets if isinstance(t, str)] if isinstance(targets, list) else []


class QuantConfigParser:
    """Which tensors of a checkpoint hold int4 codes one per int8, from the
    ``quantization_config`` of its ``config.json``: the targets of every
    config group with 4-bit integer weights, matched like recipe targets
    against the tensor's module name (``re:`` patterns also against the
    tensor name).  A checkpoint records no module classes; its quantized
    2-D weights come from Linear layers, so a ``Linear`` target takes them
    all."""

    def __init__(self, model_path) -> None:
        path = os.path.join(model_path, "config.json")
        if not os.path.exists(path):
            raise ValueError("config.json not found in model path")
        with open(path) as f:
            qc = json.load(f).get(QUANTIZATION_CONFIG_NAME) or {}
        if not qc:
            raise ValueError("quantization_config not found in config.json")
        self.config = qc
        groups = qc.get("config_groups") or {}
        self.int4_targets = [t for g in groups.values()
                             if isinstance(g, dict) and _int4_int_weights(g.get("weights"))
                             for t in _target_list(g.get("targets", []))]

    def is_int4_layer(self, layer_name) -> bool:
        from .modifiers import matches_target

        module = layer_name.removesuffix(".weight")
        return (matches_target(module, "Linear", self.int4_targets)
                or matches_target(layer_name, None, self.int4_targets))


class Int8Packer:
    """Rewrites a safetensors checkpoint whose int4 layers hold one code per
    int8 into two codes per int8 (even column in the low nibble,
    ``mi355q_pack_int4_int8``), shard by shard; optionally widens biases to
    fp32 and renames packed weights to ``*.weight_packed``.  The index, if
    any, gets the new weight map and total size; every other file is copied."""

    def __init__(self, model_path, save_path, bias32=False, rename=False, device="cuda"):
        if not os.path.isdir(model_path):
            raise ValueError("Invalid model path")
        self.model_path, self.save_path = model_path, save_path
        self.bias32, self.rename, self.device = bias32, rename, device
        os.makedirs(save_path, exist_ok=True)
        self.quant_config_parser = QuantConfigParser(model_path)
        self.shards = sorted(n for n in os.listdir(model_path) if n.endswith(".safetensors"))
        if not self.shards:
            raise ValueError("No .safetensors files found in model path")

    def _packable(self, key: str, t: torch.Tensor) -> bool:
        return (key.endswith("weight") and t.dtype == torch.int8 and t.dim() == 2
                and self.quant_config_parser.is_int4_layer(key))

    def _rewrite_shard(self, shard: str) -> tuple[dict, int]:
        from safetensors.torch import load_file, save_file

        tensors = load_file(os.path.join(self.model_path, shard))
        out = {}
        for key, t in tensors.items():
            if self._packable(key, t):
                key = key.removesuffix("weight") + "weight_packed" if self.rename else key
                t = ops.pack_int4_int8(t.to(self.device)).cpu()    # odd widths raise ValueError
            elif self.bias32 and key.endswith("bias"):
                t = t.to(torch.float32)
            out[key] = t
        save_file(out, os.path.join(self.save_path, shard))
        return dict.fromkeys(out, shard), sum(t.numel() * t.element_size() for t in out.values())

    def save(self) -> None:
        weight_map, size = {}, 0
        for shard in self.shards:
            m, n = self._rewrite_shard(shard)
            weight_map.update(m)
            size += n
        index = "model.safetensors.index.json"
        if os.path.exists(os.path.join(self.model_path, index)):
            with open(os.path.join(self.model_path, index)) as f:
                idx = json.load(f)
            meta = idx.get("metadata") if isinstance(idx.get("metadata"), dict) else {}
            idx.update(weight_map=weight_map, metadata={**meta, "total_size": size})
            with open(os.path.join(self.save_path, index), "w") as f:
                json.dump(idx, f, indent=2, sort_keys=True)
        for name in os.listdir(self.model_path):
            src = os.path.join(self.model_path, name)
            if os.path.isfile(src) and not name.endswith(".safetensors") and name != index:
                shutil.copy(src, os.path.join(self.save_path, name))


def main(argv=None):
    """Command line of the rewriter, with the reference's flags:
    ``python -m llmcompressor_amd.save -i <checkpoint> -o <out> [-bias32] [-rename_packed]``."""
    ap = argparse.ArgumentParser(description="pack int4-in-int8 checkpoint weights two codes per byte (GPU)")
    ap.add_argument("-i", "--model_path", type=str, required=True, help="checkpoint directory to read")
    ap.add_argument("-o", "--save_path", type=str, required=True, help="directory to write")
    ap.add_argument("-bias32", action="store_true", default=False, help="store biases as fp32")
    ap.add_argument("-rename_packed", action="store_true", default=False,
                    help="store packed weights as <module>.weight_packed")
    a = ap.parse_args(argv)
    Int8Packer(a.model_path, a.save_path, a.bias32, a.rename_packed).save()


if __name__ == "__main__":
    main()
