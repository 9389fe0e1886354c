"""GPU MSE observers (memoryless_mse / mse) against the oracle's grid search.

Bars: the reference's known-answer losses (test_mse.py:9-43) to 1e-10 on the
fp32 table input; on random bf16 / fp32 weights the chosen min / max equal the
oracle's in every group (bit-exact), so the fake-quantised loss is the
oracle's.
"""
import json
from pathlib import Path

import pytest
import torch

from llmcompressor_amd.observers import Observer
from llmcompressor_amd.quant_args import QuantizationArgs
from oracle import fake_quant as ofq
from oracle import observers as oobs
from oracle.qargs import OArgs

pytestmark = pytest.mark.gpu

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("case", GOLD["mse_observer"]["cases"], ids=lambda c: f"{c['strategy']}-{c['symmetric']}")
def test_mse_known_losses_on_gpu(dev, case):
    g = GOLD["mse_observer"]
    st = case["strategy"]
    kw = dict(num_bits=g["num_bits"], strategy=st, symmetric=case["symmetric"],
              group_size=g["group_size_for_group"] if st == "group" else None,
              block_structure=g["block_structure_for_block"] if st == "block" else None)
    t = torch.arange(24).reshape((6, 4)) / 24
    obs = Observer.load_from_registry("mse", base_name="weight", args=QuantizationArgs(observer="mse", **kw))
    qp = obs(t.to(dev)).get_qparams()
    a = OArgs(observer="mse", **kw)
    q = ofq.fake_quantize_weight(t, qp["scale"].cpu(), qp["zero_point"].cpu(), a)
    loss = (torch.sum((t - q).abs().pow(2)) / t.numel()).item()
    say(f"mse {st} sym={case['symmetric']} loss {loss:.6e} vs {case['exp_loss']:.4e}")
    assert loss == pytest.approx(case["exp_loss"], abs=g["abs_tol"])


CASES = [dict(num_bits=4, strategy="group", group_size=128), dict(num_bits=4, strategy="group", group_size=32),
         dict(num_bits=4, strategy="group", group_size=128, symmetric=False),
         dict(num_bits=8, strategy="channel"), dict(num_bits=8, strategy="channel", symmetric=False),
         dict(num_bits=8, strategy="tensor"), dict(num_bits=8, strategy="block", block_structure=[64, 96]),
         dict(num_bits=4, strategy="group", group_size=512)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_mse_observer_matches_oracle(dev, case, dtype):
    g = torch.Generator().manual_seed(11)
    w = torch.randn(192, 1024, generator=g) * 0.02
    w[torch.rand(192, 1024, generator=g) < 0.002] *= 12       # outliers: shrinking pays
    w = w.to(dtype)
    say(f"mse observer {case} {dtype}")
    obs = Observer.load_from_registry("memoryless_mse", base_name="weight",
                                      args=QuantizationArgs(observer="memoryless_mse", **case))
    obs(w.to(dev))
    mn, mx = obs.min_vals.cpu(), obs.max_vals.cpu()
    qp = obs.get_qparams()
    a = OArgs(observer="mse", **case)
    omn, omx = oobs.mse_grid_search(oobs.flatten_weight(w, a), a)
    agree = ((mn == omn.reshape(mn.shape)) & (mx == omx.reshape(mx.shape))).float().mean().item()
    s_o, z_o = oobs.calculate_qparams(omn, omx, a)
    q_gpu = ofq.fake_quantize_weight(w, qp["scale"].cpu().reshape(s_o.shape), qp["zero_point"].cpu().reshape(s_o.shape), a)
    q_ora = ofq.fake_quantize_weight(w, s_o, z_o, a)
    l_gpu = (q_gpu.double() - w.double()).pow(2).sum().item()
    l_ora = (q_ora.double() - w.double()).pow(2).sum().item()
    say(f"  agreement {agree:.5f} loss {l_gpu:.6e} vs {l_ora:.6e}")
    assert agree == 1.0
    assert l_gpu == l_ora


FP8_CASES = [dict(strategy="channel"), dict(strategy="tensor"), dict(strategy="group", group_size=128),
             dict(strategy="block", block_structure=[64, 128])]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", FP8_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_mse_observer_fp8_matches_oracle(dev, case, dtype):
    """The search on the fp8 e4m3 grid (mse_quant.py:255-262 with float
    args: scale max|x| / 448, fake-quantised through float8_e4m3fn): the
    chosen min / max equal the oracle's in every cell."""
    g = torch.Generator().manual_seed(17)
    w = torch.randn(192, 1024, generator=g) * torch.exp(torch.randn(192, 1, generator=g))
    w[torch.rand(192, 1024, generator=g) < 0.002] *= 40       # outliers: shrinking pays
    w = w.to(dtype)
    say(f"mse observer fp8 {case} {dtype}")
    kw = dict(num_bits=8, type="float", symmetric=True, **case)
    obs = Observer.load_from_registry("memoryless_mse", base_name="weight",
                                      args=QuantizationArgs(observer="memoryless_mse", **kw))
    obs(w.to(dev))
    mn, mx = obs.min_vals.cpu(), obs.max_vals.cpu()
    qp = obs.get_qparams()
    a = OArgs(observer="mse", **kw)
    omn, omx, steps = oobs.mse_grid_search(oobs.flatten_weight(w, a), a, return_steps=True)
    agree = ((mn == omn.reshape(mn.shape)) & (mx == omx.reshape(mx.shape))).float().mean().item()
    shrunk = ((omx.abs() < oobs.flatten_weight(w, a).abs().amax(dim=(0, -1))).float().mean().item())
    s_o, z_o = oobs.calculate_qparams(omn, omx, a)
    assert torch.equal(qp["scale"].cpu().reshape(s_o.shape).float(), s_o.float())
    say(f"  agreement {agree:.5f} over {steps} steps, {shrunk:.3f} of the cells shrunk")
    assert agree == 1.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_imatrix_fp8_matches_oracle(dev, dtype):
    say(f"imatrix fp8 channel {dtype}")
    g = torch.Generator().manual_seed(6)
    w = (torch.randn(192, 1024, generator=g) * 0.02).to(dtype)
    s2 = torch.exp(2 * torch.randn(1024, generator=g))
    args = QuantizationArgs(num_bits=8, type="float", symmetric=True, strategy="channel", observer="imatrix_mse")
    obs = Observer.load_from_registry("imatrix_mse", base_name="weight", args=args)
    obs._imatrix_sum, obs._imatrix_count = s2.clone().to(dev), torch.tensor(3, dtype=torch.int64)
    obs(w.to(dev))
    mn, mx = obs.min_vals.cpu(), obs.max_vals.cpu()
    a = OArgs(num_bits=8, type="float", symmetric=True, strategy="channel", observer="imatrix_mse")
    flat = oobs.flatten_weight(w, a)
    imp = oobs.imatrix_importance(s2, 3, flat, a)
    omn, omx = oobs.imatrix_grid_search(flat, a, importance=imp)
    agree = ((mn == omn.reshape(mn.shape)) & (mx == omx.reshape(mx.shape))).float().mean().item()
    say(f"  agreement {agree:.5f}")
    assert agree == 1.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", [dict(strategy="tensor_group", group_size=16), dict(strategy="group", group_size=32)],
                         ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_mse_observer_fp4_matches_oracle(dev, case, dtype):
    """The search on the e2m1 grid (scale max|x| / 6 per candidate, CT
    cast_to_fp4): the chosen min / max equal the oracle's in every group.
    For tensor groups the global scale and fp8 group scales then come from
    these statistics (observers/base.py:78-123)."""
    g = torch.Generator().manual_seed(23)
    w = (torch.randn(192, 1024, generator=g) * torch.exp(torch.randn(192, 1, generator=g))).to(dtype)
    say(f"mse observer fp4 {case} {dtype}")
    kw = dict(num_bits=4, type="float", symmetric=True, **case)
    obs = Observer.load_from_registry("memoryless_mse", base_name="weight",
                                      args=QuantizationArgs(observer="memoryless_mse", **kw))
    obs(w.to(dev))
    mn, mx = obs.min_vals.cpu(), obs.max_vals.cpu()
    a = OArgs(observer="mse", **kw)
    flat = oobs.flatten_weight(w, a)
    omn, omx, steps = oobs.mse_grid_search(flat, a, return_steps=True)
    agree = ((mn == omn.reshape(mn.shape)) & (mx == omx.reshape(mx.shape))).float().mean().item()
    shrunk = (omx.abs() < flat.abs().amax(dim=(0, -1))).float().mean().item()
    say(f"  agreement {agree:.5f} over {steps} steps, {shrunk:.3f} of the groups shrunk")
    assert agree == 1.0
    if case["strategy"] == "tensor_group":
        qp = obs.get_qparams()
        gs = oobs.global_scale_from_stats([(omn, omx)])
        s_o, _ = oobs.calculate_qparams(omn, omx, a, global_scale=gs)
        assert torch.equal(qp["global_scale"].cpu().float().reshape(1), gs.float().reshape(1))
        assert torch.equal(qp["scale"].cpu().float().reshape(s_o.shape), s_o.float())


def test_mse_observer_fp8_scaled_fp4_refused(dev):
    """fp4 with fp8 scales (the NVFP4 preset) is not searched: the observer
    raises."""
    args = QuantizationArgs(num_bits=4, type="float", symmetric=True, observer="memoryless_mse",
                            strategy="tensor_group", group_size=16, scale_dtype=torch.float8_e4m3fn)
    obs = Observer.load_from_registry("memoryless_mse", base_name="weight", args=args)
    with pytest.raises(NotImplementedError):
        obs(torch.randn(32, 64, device=dev))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_mse_observer_mxfp4_matches_oracle(dev, dtype):
    """MXFP4 (group 32): each candidate's scale is the power of two of the
    e8m0 exponent of its shrunk absmax (calculate_qparams' MX branch, CT
    rule); the chosen min / max equal the oracle's in every group, and so do
    the resulting e8m0 scales."""
    g = torch.Generator().manual_seed(29)
    w = (torch.randn(192, 1024, generator=g) * torch.exp(torch.randn(192, 1, generator=g) * 2)).to(dtype)
    say(f"mse observer mxfp4 {dtype}")
    args = QuantizationArgs(num_bits=4, type="float", symmetric=True, strategy="group", group_size=32,
                            scale_dtype=torch.uint8, zp_dtype=torch.uint8, observer="memoryless_mse")
    obs = Observer.load_from_registry("memoryless_mse", base_name="weight", args=args)
    obs(w.to(dev))
    mn, mx = obs.min_vals.cpu(), obs.max_vals.cpu()
    qp = obs.get_qparams()
    a = OArgs(num_bits=4, type="float", symmetric=True, strategy="group", group_size=32, is_mx=True,
              observer="mse")
    flat = oobs.flatten_weight(w, a)
    omn, omx, steps = oobs.mse_grid_search(flat, a, return_steps=True)
    agree = ((mn == omn.reshape(mn.shape)) & (mx == omx.reshape(mx.shape))).float().mean().item()
    shrunk = (omx.abs() < flat.abs().amax(dim=(0, -1))).float().mean().item()
    say(f"  agreement {agree:.5f} over {steps} steps, {shrunk:.3f} of the groups shrunk")
    assert agree == 1.0
    s_o, _ = oobs.calculate_qparams(omn, omx, a)
    assert torch.equal(qp["scale"].cpu().float().reshape(s_o.shape), s_o.float())


@pytest.mark.parametrize("strategy", ["tensor", "group"])
def test_mse_activation_moving_average(dev, strategy):
    say(f"mse activations {strategy}")
    kw = dict(num_bits=8, strategy=strategy, group_size=128 if strategy == "group" else None)
    obs = Observer.load_from_registry("mse", base_name="input", args=QuantizationArgs(observer="mse", **kw))
    ora = oobs.OMSE("mse", "input", OArgs(observer="mse", **kw))
    for seed in (1, 2):
        x = (torch.randn(2, 64, 512, generator=torch.Generator().manual_seed(seed)) * 2).to(torch.bfloat16)
        obs(x.to(dev))
        ora(x)
        mn, mx = obs.min_vals.cpu().reshape(-1), obs.max_vals.cpu().reshape(-1)
        omn, omx = ora.min_vals.reshape(-1), ora.max_vals.reshape(-1)
        say(f"  after call {seed}: dtypes {mn.dtype} / {omn.dtype}, min equal {(mn == omn).float().mean():.4f}, "
            f"max equal {(mx == omx).float().mean():.4f}; gpu {mn[:4].tolist()} {mx[:4].tolist()} oracle "
            f"{omn[:4].tolist()} {omx[:4].tolist()}")
        assert mn.dtype == omn.dtype
        assert torch.equal(mn, omn) and torch.equal(mx, omx)


# ---------------------------------------------------------------- imatrix_mse
def _imatrix_obs(strategy="channel", group_size=None, **kw):
    args = QuantizationArgs(num_bits=4, symmetric=kw.pop("symmetric", True), strategy=strategy,
                            group_size=group_size, observer="imatrix_mse", observer_kwargs=kw)
    return Observer.load_from_registry("imatrix_mse", base_name="weight", args=args)


def test_imatrix_uniform_importance_matches_memoryless_mse(dev):
    """test_imatrix.py:175-212 on the GPU."""
    say("imatrix uniform == memoryless_mse")
    torch.manual_seed(123)
    lin = torch.nn.Linear(8, 4).to(dev)
    lin._imatrix_sum = torch.ones(8)
    lin._imatrix_count = torch.tensor(1, dtype=torch.int64)
    oi = _imatrix_obs(norm=2.4, maxshrink=0.20)
    oi.attach(lin)
    ou = Observer.load_from_registry("memoryless_mse", base_name="weight", args=QuantizationArgs(
        num_bits=4, symmetric=True, strategy="channel", observer="memoryless_mse", observer_kwargs={"grid": 20}))
    qi = oi(lin.weight.detach()).get_qparams()
    qu = ou(lin.weight.detach()).get_qparams()
    assert torch.allclose(qi["scale"], qu["scale"]) and torch.equal(qi["zero_point"], qu["zero_point"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", [dict(strategy="channel"), dict(strategy="group", group_size=128),
                                  dict(strategy="group", group_size=32, symmetric=False)],
                         ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_imatrix_matches_oracle(dev, case, dtype):
    say(f"imatrix {case} {dtype}")
    g = torch.Generator().manual_seed(5)
    w = (torch.randn(192, 1024, generator=g) * 0.02).to(dtype)
    s2 = torch.exp(2 * torch.randn(1024, generator=g))        # skewed E[x^2]
    obs = _imatrix_obs(**dict(case))
    obs._imatrix_sum, obs._imatrix_count = s2.clone().to(dev), torch.tensor(3, dtype=torch.int64)
    obs(w.to(dev))
    mn, mx = obs.min_vals.cpu(), obs.max_vals.cpu()
    a = OArgs(num_bits=4, observer="imatrix_mse", **case)
    flat = oobs.flatten_weight(w, a)
    imp = oobs.imatrix_importance(s2, 3, flat, a)
    omn, omx = oobs.imatrix_grid_search(flat, a, importance=imp)
    agree = ((mn == omn.reshape(mn.shape)) & (mx == omx.reshape(mx.shape))).float().mean().item()
    say(f"  agreement {agree:.5f}")
    assert agree == 1.0


def test_imatrix_hook_accumulates_and_hands_over(dev, caplog):
    say("imatrix hook")
    lin = torch.nn.Linear(256, 64).to(dev).to(torch.bfloat16)
    obs = _imatrix_obs()
    obs.attach(lin)
    xs = [(torch.randn(2, 50, 256, generator=torch.Generator().manual_seed(s)) * 3).to(torch.bfloat16)
          for s in (1, 2)]
    with torch.no_grad():
        for x in xs:
            lin(x.to(dev))
    exp = sum(x.float().pow(2).sum(dim=(0, 1)) for x in xs)
    assert int(lin._imatrix_count) == 200
    assert torch.allclose(lin._imatrix_sum.cpu(), exp, rtol=1e-5)
    obs.detach(lin)
    second = _imatrix_obs()
    second.attach(lin)                          # takes the accumulators
    assert not hasattr(lin, "_imatrix_sum") and int(second._imatrix_count) == 200
    qp = second(lin.weight.detach()).get_qparams()
    assert torch.isfinite(qp["scale"]).all()
    bare = _imatrix_obs()
    with caplog.at_level("WARNING", logger="llmcompressor_amd"):
        bare(lin.weight.detach()).get_qparams()
    assert "no importance data available" in caplog.text
    with pytest.raises(ValueError):
        _imatrix_obs(strict=True)(lin.weight.detach())
