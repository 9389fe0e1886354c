"""GPU: the checkpoint writer and the int4 shard rewriter produce the oracle's
bytes (codes, packing, scales), and the files they write are complete."""
import json

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from llmcompressor_amd import QuantizationModifier, ops
from llmcompressor_amd.save import Int8Packer, save_compressed
from oracle import fake_quant as ofq
from oracle import pack as opack
from oracle.qargs import OArgs

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _load_dir(path):
    out = {}
    for f in sorted(path.glob("*.safetensors")):
        with safe_open(str(f), framework="pt") as h:
            for k in h.keys():
                out[k] = h.get_tensor(k)
    return out


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_int32_matches_oracle(dev, bits):
    say(f"pack_int32 bits={bits}")
    for cols in (64, 37, 100):
        r = np.random.default_rng(bits + cols).integers(-(1 << (bits - 1)), 1 << (bits - 1),
                                                        size=(33, cols)).astype(np.int8)
        got = ops.pack_int32(torch.from_numpy(r).to(dev), bits).cpu().numpy()
        assert np.array_equal(got, opack.pack_to_int32(r, bits))
        assert np.array_equal(opack.unpack_from_int32(got, cols, bits), r)


def _model(dev):
    torch.manual_seed(0)
    m = torch.nn.Sequential(torch.nn.Linear(256, 128, bias=True), torch.nn.ReLU(),
                            torch.nn.Linear(128, 64, bias=False), torch.nn.Linear(64, 32))
    return m.to(dev).to(torch.bfloat16)


def _oracle_codes(lin, oa):
    w = lin.weight.detach().cpu()
    s = ofq.expand_qparams(lin.weight_scale.detach().cpu(), w.shape, oa)
    z = None if oa.symmetric else ofq.expand_qparams(lin.weight_zero_point.detach().cpu(), w.shape, oa)
    return ofq.quantize(w, s, z, oa)


def test_save_w4a16_checkpoint(dev, tmp_path):
    say("save W4A16")
    model = _model(dev)
    QuantizationModifier(scheme="W4A16", targets=("Linear",), ignore=("3",)).apply(model)
    idx = save_compressed(model, str(tmp_path), max_shard_size=8_000, config={"architectures": ["Tiny"]})
    t = _load_dir(tmp_path)
    assert (tmp_path / "model.safetensors.index.json").exists() and len(list(tmp_path.glob("*.safetensors"))) > 1
    assert set(idx["weight_map"]) == set(t)
    assert idx["metadata"]["total_size"] == sum(v.numel() * v.element_size() for v in t.values())
    oa = OArgs(num_bits=4, strategy="group", group_size=128)
    for name in ("0", "2"):
        lin = model[int(name)]
        rows, cols = lin.weight.shape
        assert t[f"{name}.weight_shape"].tolist() == [rows, cols]
        codes = opack.unpack_from_int32(t[f"{name}.weight_packed"].numpy(), cols, 4)
        assert np.array_equal(codes, _oracle_codes(lin, oa).to(torch.int8).numpy())
        assert torch.equal(t[f"{name}.weight_scale"], lin.weight_scale.detach().cpu())
        assert f"{name}.weight" not in t and f"{name}.weight_zero_point" not in t
    assert torch.equal(t["0.bias"], model[0].bias.detach().cpu())
    assert torch.equal(t["3.weight"], model[3].weight.detach().cpu())
    cfg = json.loads((tmp_path / "config.json").read_text())
    assert cfg["architectures"] == ["Tiny"]
    q = cfg["quantization_config"]
    assert q["format"] == "pack-quantized" and q["ignore"] == ["3"] and q["quant_method"] == "compressed-tensors"


@pytest.mark.parametrize("scheme,fmt", [("W8A8", "int-quantized"), ("FP8_DYNAMIC", "float-quantized"),
                                        ("MXFP4", "mxfp4-pack-quantized"), ("W4A16_ASYM", "pack-quantized"),
                                        ("NVFP4A16", "nvfp4-pack-quantized")])
def test_save_formats(dev, tmp_path, scheme, fmt):
    say(f"save {scheme}")
    model = _model(dev)
    grouped = scheme.startswith("W4A16")   # group 128: the 64-column layer stays unquantized
    QuantizationModifier(scheme=scheme, targets=("Linear",), ignore=("3",) if grouped else ()).apply(model)
    save_compressed(model, str(tmp_path))
    t = _load_dir(tmp_path)
    assert json.loads((tmp_path / "config.json").read_text())["quantization_config"]["format"] == fmt
    for i in ((0, 2) if grouped else (0, 2, 3)):
        lin, p = model[i], f"{i}."
        if scheme == "MXFP4":
            bits = lin.weight.detach().cpu().view(torch.int16).numpy().view(np.uint16)
            oc, os_ = opack.mxfp4_quantize_pack(bits, "ct")
            assert np.array_equal(t[p + "weight_packed"].numpy(), oc)
            assert np.array_equal(t[p + "weight_scale"].numpy(), os_)
            # the module keeps the scales as float powers of two, the file as e8m0
            e8 = t[p + "weight_scale"].to(torch.float32)
            assert torch.equal(torch.exp2(e8 - 127), lin.weight_scale.detach().cpu().float())
        elif scheme == "NVFP4A16":
            w = lin.weight.detach().cpu().float().numpy()
            sc = lin.weight_scale.detach().cpu().float().numpy()
            gs = lin.weight_global_scale.detach().cpu().float()
            assert np.array_equal(t[p + "weight_packed"].numpy(), opack.fp4_group_quantize_pack(w, sc, 16, float(gs)))
            assert t[p + "weight_scale"].dtype == torch.float8_e4m3fn
            assert torch.equal(t[p + "weight_scale"].float(), torch.from_numpy(sc))
            assert t[p + "weight_global_scale"].dtype == torch.float32
            assert torch.equal(t[p + "weight_global_scale"], gs.reshape(1))
            # decoded codes x effective scales = the oracle's fake-quantized weight
            idx = np.arange(w.shape[1]) // 16
            dec = opack.fp4_unpack(t[p + "weight_packed"].numpy()) * (sc / np.float32(gs)).astype(np.float32)[:, idx]
            oa = OArgs(num_bits=4, type="float", strategy="tensor_group", group_size=16)
            fq = ofq.fake_quantize(torch.from_numpy(w), torch.from_numpy(sc[:, idx]), None, oa,
                                   global_scale=gs.reshape(1))
            assert np.array_equal(dec, fq.numpy())
        elif scheme == "W8A8":
            oa = OArgs(num_bits=8, strategy="channel")
            assert torch.equal(t[p + "weight"], _oracle_codes(lin, oa).to(torch.int8))
        elif scheme == "FP8_DYNAMIC":
            oa = OArgs(num_bits=8, type="float", strategy="channel")
            assert t[p + "weight"].dtype == torch.float8_e4m3fn
            assert torch.equal(t[p + "weight"].float(), _oracle_codes(lin, oa).float())
        else:
            oa = OArgs(num_bits=4, strategy="group", group_size=128, symmetric=False)
            codes = opack.unpack_from_int32(t[p + "weight_packed"].numpy(), lin.weight.shape[1], 4)
            assert np.array_equal(codes, _oracle_codes(lin, oa).to(torch.int8).numpy())
            zp = lin.weight_zero_point.detach().cpu()
            packed_zp = t[p + "weight_zero_point"]
            assert packed_zp.dtype == torch.int32 and packed_zp.shape == ((zp.shape[0] + 7) // 8, zp.shape[1])
            assert np.array_equal(packed_zp.numpy(), opack.pack_to_int32(zp.numpy(), 4, packed_dim=0))
            assert np.array_equal(opack.unpack_from_int32(packed_zp.numpy(), zp.shape[0], 4, packed_dim=0),
                                  zp.numpy())


def test_fp4_quantize_pack_matches_oracle(dev):
    """NVFP4 weight codes with given scales against the oracle, bit for bit:
    bf16 and fp32 inputs, quotients on and next to every rounding threshold,
    negative values rounding to zero, zeros of both signs."""
    say("fp4_quantize_pack vs oracle")
    rng = np.random.default_rng(21)
    rows, cols, g = 37, 96, 16
    sc = (2.0 ** rng.integers(-6, 3, size=(rows, cols // g))).astype(np.float32) * \
        rng.choice(np.array([1.0, 1.125, 1.5, 1.75], np.float32), size=(rows, cols // g))
    gs = np.float32(448.0 * 6.0 / 3.7)
    s_eff = (sc / gs).astype(np.float32)[:, np.arange(cols) // g]
    thr = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 7.0, 0.1], np.float32)
    t = rng.choice(thr, size=(rows, cols)) * rng.choice(np.array([1.0, 1.0 + 2 ** -20, 1.0 - 2 ** -20], np.float32),
                                                      size=(rows, cols))
    t *= rng.choice(np.array([1.0, -1.0], np.float32), size=(rows, cols))
    x = (t * s_eff).astype(np.float32)
    x[0, :4] = [0.0, -0.0, -1e-30, 1e-30]
    for dtype in (torch.float32, torch.bfloat16):
        xt = torch.from_numpy(x).to(dtype)
        got = ops.fp4_quantize_pack(xt.to(dev), torch.from_numpy(sc).to(dev), g, torch.tensor([gs]).to(dev))
        want = opack.fp4_group_quantize_pack(xt.float().numpy(), sc, g, float(gs))
        assert np.array_equal(got.cpu().numpy(), want), dtype
    # a global scale held on the host is moved to the weight's device
    host_gs = ops.fp4_quantize_pack(torch.from_numpy(x).to(dev), torch.from_numpy(sc).to(dev), g, torch.tensor([gs]))
    assert np.array_equal(host_gs.cpu().numpy(), opack.fp4_group_quantize_pack(x, sc, g, float(gs)))
    none = ops.fp4_quantize_pack(torch.from_numpy(x).to(dev), torch.from_numpy(sc).to(dev), g)
    assert np.array_equal(none.cpu().numpy(), opack.fp4_group_quantize_pack(x, sc, g))


def test_save_gptq_nvfp4_checkpoint(dev, tmp_path):
    """GPTQ with NVFP4 weights, then the checkpoint: the file's codes are
    the oracle's codes of the stored weight, group scales and global scale
    (the global scale rounded to the weight dtype, as the reference's
    ``quantize_weight`` returns it, and written into the fp32 parameter, as
    ``update_offload_parameter`` writes it: fp32 in every NVFP4 checkpoint),
    and they decode to the GPTQ weight the module holds, on the fp4
    grid, up to the rounding of the stored global scale and of the weight
    to bf16 (2^-8 each)."""
    from llmcompressor_amd import GPTQModifier
    say("save GPTQ NVFP4A16")
    model = _model(dev)
    g = torch.Generator(device=dev).manual_seed(3)
    batches = [torch.randn(4, 64, 256, device=dev, generator=g).to(torch.bfloat16) for _ in range(4)]
    GPTQModifier(scheme="NVFP4A16", targets=("Linear",), ignore=()).apply(model, batches)
    save_compressed(model, str(tmp_path))
    t = _load_dir(tmp_path)
    assert json.loads((tmp_path / "config.json").read_text())["quantization_config"]["format"] == \
        "nvfp4-pack-quantized"
    for i in (0, 2, 3):
        lin, p = model[i], f"{i}."
        w = lin.weight.detach().cpu().float().numpy()
        sc = lin.weight_scale.detach().cpu().float().numpy()
        gs = float(lin.weight_global_scale.detach().cpu().float())
        packed = t[p + "weight_packed"].numpy()
        assert np.array_equal(packed, opack.fp4_group_quantize_pack(w, sc, 16, gs))
        assert t[p + "weight_scale"].dtype == torch.float8_e4m3fn
        assert t[p + "weight_global_scale"].tolist() == [gs]
        assert t[p + "weight_global_scale"].dtype == torch.float32
        assert lin.weight_global_scale.dtype == torch.float32
        assert gs == float(torch.tensor(gs).to(torch.bfloat16).float())   # rounded to bf16 first
        dec = opack.fp4_unpack(packed) * (sc / np.float32(gs)).astype(np.float32)[:, np.arange(w.shape[1]) // 16]
        err = np.abs(dec - w)
        say(f"  layer {i}: decoded vs GPTQ weight, max rel {float(np.max(err / np.maximum(np.abs(w), 1e-30))):.2e}")
        assert bool(np.all(err <= 2.0 ** -7 * np.abs(w))), i


def test_int8_packer_rewrites_int4_layers(dev, tmp_path):
    """pack_int4_to_int8.py:31-200 on a two-shard checkpoint (rename, bias32)."""
    say("Int8Packer")
    src, out = tmp_path / "src", tmp_path / "out"
    src.mkdir()
    cfg = {"architectures": ["X"], "quantization_config": {"config_groups": {"g": {
        "targets": ["re:.*q_proj$"], "weights": {"num_bits": 4, "type": "int"}}}, "format": "int-quantized"}}
    (src / "config.json").write_text(json.dumps(cfg))
    (src / "tokenizer.json").write_text("{}")
    rng = np.random.default_rng(0)
    q = torch.from_numpy(rng.integers(-8, 8, size=(64, 128)).astype(np.int8))
    k = torch.from_numpy(rng.integers(-128, 128, size=(32, 64)).astype(np.int8))
    b = torch.randn(64).to(torch.bfloat16)
    n = torch.ones(32, dtype=torch.bfloat16)
    s1, s2 = "model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"
    save_file({"l.q_proj.weight": q, "l.q_proj.bias": b}, str(src / s1))
    save_file({"l.k_proj.weight": k, "l.norm.weight": n}, str(src / s2))
    (src / "model.safetensors.index.json").write_text(json.dumps(
        {"metadata": {"total_size": 0}, "weight_map": {"l.q_proj.weight": s1, "l.q_proj.bias": s1,
                                                        "l.k_proj.weight": s2, "l.norm.weight": s2}}))
    Int8Packer(str(src), str(out), bias32=True, rename=True).save()
    t = _load_dir(out)
    assert np.array_equal(t["l.q_proj.weight_packed"].numpy(), opack.pack_int4_to_int8(q.numpy()))
    assert "l.q_proj.weight" not in t
    assert torch.equal(t["l.k_proj.weight"], k) and torch.equal(t["l.norm.weight"], n)
    assert t["l.q_proj.bias"].dtype == torch.float32 and torch.equal(t["l.q_proj.bias"], b.float())
    idx = json.loads((out / "model.safetensors.index.json").read_text())
    assert idx["weight_map"] == {"l.q_proj.weight_packed": s1, "l.q_proj.bias": s1, "l.k_proj.weight": s2,
                                 "l.norm.weight": s2}
    assert idx["metadata"]["total_size"] == sum(v.numel() * v.element_size() for v in t.values())
    assert (out / "tokenizer.json").exists() and json.loads((out / "config.json").read_text()) == cfg
    # the reference's known answer (test_pack_int4_to_int8.py:25-38), through a shard
    src2, out2 = tmp_path / "src2", tmp_path / "out2"
    src2.mkdir()
    (src2 / "config.json").write_text(json.dumps({"quantization_config": {"config_groups": {"g": {
        "targets": ["Linear"], "weights": {"num_bits": 4}}}}}))
    save_file({"a.weight": torch.tensor([[1, 2, -1, 0], [3, 4, 5, 6]], dtype=torch.int8)},
              str(src2 / "model.safetensors"))
    Int8Packer(str(src2), str(out2)).save()
    got = _load_dir(out2)["a.weight"]
    assert got.tolist() == [[0x21, 0x0F], [0x43, 0x65]]
    save_file({"a.weight": torch.zeros(2, 3, dtype=torch.int8)}, str(src2 / "model.safetensors"))
    with pytest.raises(ValueError, match="even number of columns"):
        Int8Packer(str(src2), str(out2)).save()
