"""The save step's host logic (CPU only): format inference, quantization_config,
the int4 shard rewriter's config parsing and validation."""
import json

import pytest
import torch

from llmcompressor_amd import QuantizationArgs, QuantizationScheme, preset_name_to_scheme
from llmcompressor_amd.calibration import initialize_module_for_quantization
from llmcompressor_amd.save import Int8Packer, QuantConfigParser, infer_quantization_format, quantization_config


def _scheme(w_bits, q_type, quantize_activations):
    """test_compress_tensor_utils.py:250-287: channel weights, tensor activations."""
    w = QuantizationArgs(num_bits=w_bits, type=q_type, strategy="channel")
    a = QuantizationArgs(num_bits=8, type=q_type, strategy="tensor") if quantize_activations else None
    return QuantizationScheme(targets=["Linear"], weights=w, input_activations=a)


@pytest.mark.parametrize("style,q_type,expected", [
    ("W8A8", "int", "int-quantized"), ("W4A16", "int", "pack-quantized"), ("W8A16", "int", "pack-quantized"),
    ("W8A8", "float", "float-quantized"), ("W8A16", "float", "naive-quantized")])
def test_format_inference_as_reference(style, q_type, expected):
    """tests/llmcompressor/transformers/compression/test_compress_tensor_utils.py:289-322."""
    w_bits, a_bits = int(style[1]), int(style[3:])
    assert infer_quantization_format(_scheme(w_bits, q_type, a_bits < 16)) == expected


def test_format_of_presets():
    assert infer_quantization_format(preset_name_to_scheme("MXFP4", ["Linear"])) == "mxfp4-pack-quantized"
    assert infer_quantization_format(preset_name_to_scheme("W4A16", ["Linear"])) == "pack-quantized"
    assert infer_quantization_format(preset_name_to_scheme("FP8_DYNAMIC", ["Linear"])) == "float-quantized"
    assert infer_quantization_format(None) is None


def test_quantization_config_groups_and_ignore():
    model = torch.nn.Sequential(torch.nn.Linear(64, 64), torch.nn.Linear(64, 64), torch.nn.Linear(64, 8))
    for m in (model[0], model[1]):
        initialize_module_for_quantization(m, preset_name_to_scheme("W4A16", ["Linear"]))
    q = quantization_config(model)
    assert q["format"] == "pack-quantized" and q["quant_method"] == "compressed-tensors"
    assert q["quantization_status"] == "compressed" and q["ignore"] == ["2"]
    assert list(q["config_groups"]) == ["group_0"]
    g = q["config_groups"]["group_0"]
    assert g["targets"] == ["Linear"] and g["weights"]["num_bits"] == 4 and g["weights"]["group_size"] == 128
    assert g["weights"]["strategy"] == "group" and g["input_activations"] is None
    initialize_module_for_quantization(model[2], preset_name_to_scheme("W8A8", ["Linear"]))
    q = quantization_config(model)
    assert q["format"] == "mixed-precision" and len(q["config_groups"]) == 2 and q["ignore"] == []
    json.dumps(q)


def _write_config(path, qc):
    (path / "config.json").write_text(json.dumps({"quantization_config": qc}))


def test_quant_config_parser_matches_reference_rules(tmp_path):
    """pack_int4_to_int8.py:74-141: int4 int groups only; Linear, re: and exact targets."""
    _write_config(tmp_path, {"config_groups": {
        "a": {"targets": ["re:.*experts\\.\\d+\\.(up|down)_proj$"], "weights": {"num_bits": 4, "type": "int"}},
        "b": {"targets": "model.layers.0.self_attn.q_proj", "weights": {"num_bits": "4"}},
        "c": {"targets": ["re:.*o_proj$"], "weights": {"num_bits": 8, "type": "int"}},
        "d": {"targets": ["re:.*k_proj$"], "weights": {"num_bits": 4, "type": "float"}},
        "e": "not a group"}})
    p = QuantConfigParser(str(tmp_path))
    assert p.is_int4_layer("model.layers.3.mlp.experts.7.up_proj.weight")
    assert p.is_int4_layer("model.layers.0.self_attn.q_proj.weight")
    assert not p.is_int4_layer("model.layers.1.self_attn.q_proj.weight")
    assert not p.is_int4_layer("model.layers.0.self_attn.o_proj.weight")
    assert not p.is_int4_layer("model.layers.0.self_attn.k_proj.weight")
    _write_config(tmp_path, {"config_groups": {"g": {"targets": ["Linear"], "weights": {"num_bits": 4}}}})
    assert QuantConfigParser(str(tmp_path)).is_int4_layer("anything.weight")


def test_packer_validation(tmp_path):
    with pytest.raises(ValueError, match="Invalid model path"):
        Int8Packer(str(tmp_path / "missing"), str(tmp_path / "out"))
    with pytest.raises(ValueError, match="config.json not found"):
        Int8Packer(str(tmp_path), str(tmp_path / "out"))
    (tmp_path / "config.json").write_text(json.dumps({"architectures": ["X"]}))
    with pytest.raises(ValueError, match="quantization_config not found"):
        Int8Packer(str(tmp_path), str(tmp_path / "out"))
    _write_config(tmp_path, {})
    with pytest.raises(ValueError, match="quantization_config not found"):
        Int8Packer(str(tmp_path), str(tmp_path / "out"))
    _write_config(tmp_path, {"format": "pack-quantized"})
    with pytest.raises(ValueError, match="No .safetensors"):
        Int8Packer(str(tmp_path), str(tmp_path / "out"))


def test_quant_config_parser_reference_fixtures(tmp_path):
    """The reference's parser cases (test_pack_int4_to_int8.py:47-86), from the golden fixture."""
    from pathlib import Path
    gold = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
    for case in gold["quant_config_parser"]["cases"]:
        _write_config(tmp_path, case["quantization_config"])
        p = QuantConfigParser(str(tmp_path))
        assert all(p.is_int4_layer(n) for n in case["int4"])
        assert not any(p.is_int4_layer(n) for n in case["not_int4"])
