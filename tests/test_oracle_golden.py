"""Pin the CPU oracle against the reference's own known-answer tests and
against what the mathematics fixes (CPU only)."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fake_quant as ofq
from oracle import moe as omoe
from oracle import observers as oobs
from oracle import pack as opack
from oracle.qargs import OArgs

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def _args(d):
    d = dict(d)
    if d.get("scale_dtype") == "float8_e4m3fn":
        d["scale_dtype"] = torch.float8_e4m3fn
    return OArgs(**d)


@pytest.mark.parametrize("case", GOLD["static_weight_quantization"]["cases"],
                         ids=lambda c: c["args"]["strategy"])
def test_static_weight_quantization_table(case):
    """test_lifecycle.py:16-165 - observer stats + fake-quant forward."""
    args = _args(case["args"])
    w = torch.arange(24, dtype=torch.bfloat16).reshape(4, 6)
    obs = oobs.OMinMax("memoryless_minmax", "weight", args)
    obs(w)
    assert torch.equal(obs.min_vals.float(), torch.tensor(case["min"], dtype=torch.float32))
    assert torch.equal(obs.max_vals.float(), torch.tensor(case["max"], dtype=torch.float32))
    qp = obs.get_qparams()
    out = ofq.fake_quantize_weight(w, qp["scale"], qp["zero_point"], args, qp["global_scale"])
    exp = torch.tensor(case["quant"], dtype=torch.bfloat16)
    # the reference compares the bf16 forward output with allclose at default tolerances
    assert torch.allclose(out.float(), exp.float())
    assert torch.nn.functional.mse_loss(out.float(), w.float()) <= case["loss"]


def test_static_activation_quantization_table():
    """test_lifecycle.py:168-273 (int tensor row)."""
    case = GOLD["static_activation_quantization"]["cases"][0]
    args = _args(case["args"])
    x = torch.arange(12, dtype=torch.bfloat16).reshape(1, 2, 6)
    obs = oobs.OMinMax("memoryless_minmax", "input", args)
    obs(x)
    assert torch.equal(obs.min_vals.float(), torch.tensor(case["min"]))
    assert torch.equal(obs.max_vals.float(), torch.tensor(case["max"]))
    qp = obs.get_qparams()
    out = ofq.fake_quantize(x, qp["scale"], qp["zero_point"], args)
    # the reference converts the 4-decimal table to the output dtype (bf16) first
    assert torch.allclose(out.float(), torch.tensor(case["quant"]).to(torch.bfloat16).float())


@pytest.mark.parametrize("case", GOLD["min_max_observer"]["cases"], ids=lambda c: str(c["symmetric"]))
def test_min_max_observer_scale(case):
    """test_min_max.py:8-29."""
    args = OArgs(num_bits=8, symmetric=case["symmetric"])
    obs = oobs.OMinMax("memoryless_minmax", "weight", args)
    qp = obs(torch.tensor(GOLD["min_max_observer"]["input"])).get_qparams()
    assert round(qp["scale"].item(), 4) == case["scale"]
    assert round(qp["zero_point"].item(), 4) == case["zero_point"]


def test_min_max_value_update():
    """test_min_max.py:49-86 (moving average, base 'input')."""
    g = GOLD["min_max_value_update"]
    obs = oobs.OMinMax("minmax", "input", OArgs(num_bits=8, strategy="tensor"))
    cmax = cmin = 1
    for t, emax, emin in zip(g["inputs"], g["expected_running_max_after"], g["expected_running_min_after"]):
        obs(torch.tensor(t))
        cmax = max(obs.max_vals[0].item(), cmax)
        cmin = min(obs.min_vals[0].item(), cmin)
        assert abs(cmax - emax) < 1e-6 and abs(cmin - emin) < 1e-6


@pytest.mark.parametrize("case", GOLD["observer_min_max_vals"]["cases"], ids=lambda c: c["name"])
def test_observer_min_max_vals(case):
    """test_observers.py:66-123."""
    obs = oobs.OMinMax(case["name"], "input", OArgs(strategy="tensor", observer_kwargs=case["kwargs"]))
    mins, maxs = [], []
    for o in GOLD["observer_min_max_vals"]["observed"]:
        obs(torch.tensor(o))
        mins.append(obs.min_vals)
        maxs.append(obs.max_vals)
    assert torch.allclose(torch.stack(mins), torch.tensor(case["min"]))
    assert torch.allclose(torch.stack(maxs), torch.tensor(case["max"]))


def test_strict_symmetric():
    """test_strict_symmetric.py:13-71."""
    g = GOLD["strict_symmetric"]
    args = OArgs(num_bits=8, strategy="channel")
    obs = oobs.OMinMax("strict_symmetric_minmax", "weight", args)
    qp = obs(torch.tensor(g["observed"], dtype=torch.float32)).get_qparams()
    assert qp["scale"].dtype == torch.float32
    assert qp["scale"].flatten().tolist() == pytest.approx(g["scale"])
    obs2 = oobs.OMinMax("strict_symmetric_minmax", "weight", args)
    assert obs2(torch.zeros(2, 3)).get_qparams()["scale"].flatten().tolist() == pytest.approx(g["zeros_scale"])


def test_pack_int4_to_int8_table():
    """test_pack_int4_to_int8.py:25-46."""
    g = GOLD["pack_int4_to_int8"]
    out = opack.pack_int4_to_int8(np.array(g["input"], dtype=np.int8))
    assert np.array_equal(out, np.array(g["expected"], dtype=np.int8))
    with pytest.raises(ValueError, match=g["odd_error"]):
        opack.pack_int4_to_int8(np.array(g["odd_input"], dtype=np.int8))


def test_linear_experts_routing_counts():
    """test_linear_experts.py:12-100."""
    g = GOLD["linear_experts_routing"]
    idx = torch.tensor(g["top_k_index"])
    routed = omoe.expert_token_lists(idx, g["num_experts"], False, g["num_tokens"])
    assert all(len(r) == g["routed_tokens_per_expert"] for r in routed)
    alls = omoe.expert_token_lists(idx, g["num_experts"], True, g["num_tokens"])
    assert all(len(r) == g["calibrate_all_tokens_per_expert"] for r in alls)


# ---------------------------------------------------------------- math pins
def _all_finite_bf16():
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = (b.astype(np.uint32) << 16).view(np.float32)
    return b[np.isfinite(f)]


def test_cast_to_fp4_is_nearest_ties_even_brute_force():
    """cast_to_fp4 == nearest e2m1 grid point, ties to the even mantissa, for every bf16 in [-6, 6]."""
    bits = _all_finite_bf16()
    x = torch.from_numpy((bits.astype(np.uint32) << 16).view(np.float32).copy())
    x = x[(x.abs() <= 6)]
    got = ofq.cast_to_fp4(x)
    grid = torch.tensor(ofq.FP4_GRID)
    a = x.abs()
    dist = (a.unsqueeze(1) - grid.unsqueeze(0)).abs()
    best = dist.min(dim=1).values
    cand = dist == best.unsqueeze(1)
    # even mantissa: grid indices 0,2,4,6 (0, 1, 2, 4) win ties
    even = torch.tensor([1, 0, 1, 0, 1, 0, 1, 0], dtype=torch.bool)
    pick = torch.where((cand & even).any(1), (cand & even).float().argmax(1), cand.float().argmax(1))
    exp = grid[pick] * torch.sign(x)
    assert torch.equal(got, exp)


def test_mxfp4_numpy_matches_torch_fake_quant_path():
    """The numpy byte packer and the torch observer + cast_to_fp4 path agree."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(64, 256, generator=g) * torch.exp(torch.randn(64, 1, generator=g) * 3)).to(torch.bfloat16)
    x[0, :32] = 0
    x[1, :32] = -0.0
    x[2, 5] = 1e-30
    bits = x.view(torch.int16).numpy().view(np.uint16)
    for rule in ("ct", "ocp"):
        codes, e8 = opack.mxfp4_quantize_pack(bits, rule)
        args = OArgs(num_bits=4, type="float", strategy="group", group_size=32, is_mx=True)
        obs = oobs.OMinMax("memoryless_minmax", "weight", args)
        qp = obs(x).get_qparams(mx_rule=rule)
        deq = ofq.fake_quantize_weight(x.float(), qp["scale"], None, args)
        back = opack.mxfp4_unpack(codes, e8)
        assert np.array_equal(back, deq.numpy()), rule
        assert np.array_equal(oobs.mx_scale_exponent(
            torch.max(obs_abs := x.float().abs().reshape(64, 8, 32), dim=2).values, rule).numpy(), e8.astype(np.int32))
        del obs_abs


def test_nvfp4_packer_matches_torch_fake_quant_path():
    """The numpy NVFP4 packer (codes of x / (scale / global_scale)) decodes to
    the torch ``fake_quantize`` of the same weight with the same fp8 group
    scales and global scale, element for element, and each code is the
    nearest e2m1 value of its quotient (ties to even)."""
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(48, 128, generator=g) * torch.exp(torch.randn(48, 1, generator=g) * 2)).to(torch.bfloat16)
    x[0, :16] = 0
    x[1, 3] = -1e-30
    xf = x.float()
    amax = xf.abs().reshape(48, 8, 16).amax(dim=2)
    gs = torch.tensor([448.0 * 6.0], dtype=torch.float32) / xf.abs().max()
    sc = (gs * amax / 6.0).clamp(min=2.0 ** -9).to(torch.float8_e4m3fn).float()
    packed = opack.fp4_group_quantize_pack(xf.numpy(), sc.numpy(), 16, float(gs))
    assert packed.shape == (48, 64) and packed.dtype == np.uint8
    s_full = sc.repeat_interleave(16, dim=1)
    args = OArgs(num_bits=4, type="float", strategy="tensor_group", group_size=16)
    fq = ofq.fake_quantize(xf, s_full, None, args, global_scale=gs)
    s_eff = s_full / gs
    back = opack.fp4_unpack(packed) * s_eff.numpy()
    assert np.array_equal(back, fq.numpy())
    # brute force: the decoded grid value is the nearest to the clamped quotient
    q = (xf / s_eff).clamp(-6, 6)
    grid = torch.tensor([-6, -4, -3, -2, -1.5, -1, -0.5, 0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=torch.float32)
    dist = (q.reshape(-1, 1) - grid).abs().min(dim=1).values.reshape(q.shape)
    assert torch.equal((q - torch.from_numpy(opack.fp4_unpack(packed))).abs(), dist)
    # without a global scale the quotient is x / scale
    p1 = opack.fp4_group_quantize_pack(xf.numpy(), (sc / gs).numpy(), 16)
    assert np.array_equal(p1, packed)


def test_mx_scale_rules_bound_the_group():
    """OCP: amax / scale in [4, 8); CT rule: amax / scale in [3.5, 7)."""
    bits = _all_finite_bf16()
    bits = bits[(bits & 0x7FFF) != 0]
    amax = torch.from_numpy((bits.astype(np.uint32) << 16).view(np.float32).copy()).abs()
    amax = amax[(amax > 2.0 ** -100) & (amax < 2.0 ** 100)]
    for rule, lo, hi in (("ocp", 4.0, 8.0), ("ct", 3.5, 7.0)):
        s = oobs.e8m0_to_float(oobs.mx_scale_exponent(amax, rule))
        r = amax / s
        assert bool(((r >= lo) & (r < hi)).all()), rule


def test_int32_pack_known_vector_and_round_trip():
    codes = np.array([[-8, -7, -1, 0, 1, 2, 6, 7]], dtype=np.int8)
    # offset-binary nibbles 0,1,7,8,9,10,14,15 at bits 0,4,...,28
    exp = np.array([0xFEA98710], dtype=np.uint32).view(np.int32)
    assert np.array_equal(opack.pack_to_int32(codes), exp.reshape(1, 1))
    r = np.random.default_rng(0).integers(-8, 8, size=(16, 64)).astype(np.int8)
    assert np.array_equal(opack.unpack_from_int32(opack.pack_to_int32(r), 64), r)
    # along the rows (zero points [rows, groups]): the same fields, transposed; ragged rows pad with 0
    z = np.random.default_rng(1).integers(-8, 8, size=(13, 5)).astype(np.int8)
    pz = opack.pack_to_int32(z, 4, packed_dim=0)
    assert pz.shape == (2, 5)
    assert np.array_equal(pz[:, 0:1].T, opack.pack_to_int32(np.ascontiguousarray(z[:, 0:1].T)))
    assert np.array_equal(pz[0, :], np.stack([opack.pack_to_int32(np.ascontiguousarray(z[:8, g][None]))[0, 0]
                                              for g in range(5)]))
    assert np.array_equal(opack.unpack_from_int32(pz, 13, 4, packed_dim=0), z)


def test_fp8_cast_is_torch_rne():
    x = torch.tensor([464.0, 448.0, 1.5 * 2 ** -10, -0.0, 2 ** -10])
    args = OArgs(num_bits=8, type="float")
    q = ofq.round_to_type(x, args, -448.0, 448.0)
    assert q.tolist()[:3] == [448.0, 448.0, 2 ** -9]
    assert torch.signbit(q[3])


def test_int_round_half_even_and_clamp():
    args = OArgs(num_bits=4)
    q = ofq.quantize(torch.tensor([0.5, 1.5, 2.5, -0.5, 7.6, -9.0]), torch.tensor(1.0), None, args)
    assert q.tolist() == [0.0, 2.0, 2.0, -0.0, 7.0, -8.0]


@pytest.mark.parametrize("case", GOLD["mse_observer"]["cases"], ids=lambda c: f"{c['strategy']}-{c['symmetric']}")
def test_mse_observer_known_losses(case):
    """test_mse.py:9-43: the MSE observer's qparams give the table's loss."""
    from oracle.fake_quant import fake_quantize_weight
    from oracle.observers import OMSE
    g = GOLD["mse_observer"]
    st = case["strategy"]
    a = OArgs(num_bits=g["num_bits"], strategy=st, symmetric=case["symmetric"],
              group_size=g["group_size_for_group"] if st == "group" else None,
              block_structure=g["block_structure_for_block"] if st == "block" else None, observer="mse")
    t = torch.arange(24).reshape((6, 4)) / 24
    qp = OMSE("mse", "weight", a)(t).get_qparams()
    q = fake_quantize_weight(t, qp["scale"], qp["zero_point"], a)
    loss = (torch.sum((t - q).abs().pow(2)) / t.numel()).item()
    assert loss == pytest.approx(case["exp_loss"], abs=g["abs_tol"])


def _mse_candidates_fp64(w, a, p_list, norm):
    """Error of every shrink candidate per group, evaluated in fp64 from the
    weight QDQ path (the lifecycle-pinned one), independent of the search."""
    flat = oobs.flatten_weight(w, a)
    mn, mx = torch.amin(flat, dim=(0, -1)), torch.amax(flat, dim=(0, -1))
    errs = []
    for p in p_list:
        s, z = oobs.calculate_qparams(mn * p, mx * p, a)
        q = ofq.fake_quantize_weight(w, s, z, a)
        d = (q.double() - w.double()).abs().pow(norm)
        errs.append(oobs.flatten_weight(d, a).sum(dim=(0, -1)))
    return torch.stack(errs)  # [candidates, *groups]


@pytest.mark.parametrize("symmetric", [True, False])
def test_mse_search_picks_the_smallest_candidate(symmetric):
    w = (torch.randn(16, 256, generator=torch.Generator().manual_seed(7)) * 0.02).to(torch.bfloat16)
    w[3, 5] = 0.3   # an outlier group, where shrinking pays
    a = OArgs(num_bits=4, strategy="group", group_size=32, symmetric=symmetric)
    mn, mx, steps = oobs.mse_grid_search(oobs.flatten_weight(w, a), a, return_steps=True)
    ps = [1 - i / 100.0 for i in range(steps)]
    errs = _mse_candidates_fp64(w, a, ps, 2.4)
    flat = oobs.flatten_weight(w, a)
    mn0, mx0 = torch.amin(flat, dim=(0, -1)), torch.amax(flat, dim=(0, -1))
    chosen = torch.stack([(mn0 * p == mn) & (mx0 * p == mx) for p in ps]).float().argmax(0)
    got = errs.gather(0, chosen.unsqueeze(0))[0]
    # bf16 sums decide the search: within their resolution of the true minimum
    assert torch.all(got <= errs.min(0).values * 1.01 + 1e-30)


def test_mse_search_stops_after_patience_without_improvement():
    """A constant group: shrinking only moves the clamped code further away,
    so step 0 is best, the search stops after 1 + patience steps and keeps
    min / max."""
    a = OArgs(num_bits=8, strategy="channel", symmetric=True)
    w = torch.full((4, 64), 0.25)
    mn, mx, steps = oobs.mse_grid_search(oobs.flatten_weight(w, a), a, patience=5, return_steps=True)
    assert steps == 6 and torch.equal(mx, torch.full((4, 1), 0.25)) and torch.equal(mn, mx)
    assert oobs.mse_grid_search(oobs.flatten_weight(w, a), a, maxshrink=0.0, return_steps=True)[2] == 0


def _imatrix_case(seed=123):
    torch.manual_seed(seed)
    return torch.nn.Linear(8, 4).weight.detach().clone()


def test_imatrix_uniform_importance_matches_memoryless_mse():
    """test_imatrix.py:175-212: all-ones importance, norm 2.4, maxshrink 0.2,
    grid 20 gives the memoryless_mse qparams (fp32 weights)."""
    w = _imatrix_case()
    a = OArgs(num_bits=4, strategy="channel")
    flat = oobs.flatten_weight(w, a)
    imp = oobs.imatrix_importance(torch.ones(8), 1, flat, a)
    mi, xi = oobs.imatrix_grid_search(flat, a, maxshrink=0.20, norm=2.4, importance=imp)
    mu, xu = oobs.mse_grid_search(flat, a, grid=20)
    si, zi = oobs.calculate_qparams(mi, xi, a)
    su, zu = oobs.calculate_qparams(mu, xu, a)
    assert torch.allclose(si, su) and torch.equal(zi, zu)


def test_imatrix_importance_changes_and_weights_the_choice():
    """test_imatrix.py:150-173, and the chosen candidate minimises the
    importance-weighted fp64 error over the candidates."""
    w = _imatrix_case()
    a = OArgs(num_bits=4, strategy="channel")
    flat = oobs.flatten_weight(w, a)
    imp = oobs.imatrix_importance(torch.tensor([1000.0] * 4 + [0.01] * 4), 1, flat, a)
    mw, xw = oobs.imatrix_grid_search(flat, a, importance=imp)
    mu, xu = oobs.imatrix_grid_search(flat, a, importance=None)
    assert not torch.allclose(oobs.calculate_qparams(mw, xw, a)[0], oobs.calculate_qparams(mu, xu, a)[0])
    mn0, mx0 = torch.amin(flat, dim=(0, -1)), torch.amax(flat, dim=(0, -1))
    errs = []
    for i in range(20):
        p = 1 - i / 20
        s, z = oobs.calculate_qparams(p * mn0, p * mx0, a)
        q = ofq.fake_quantize_weight(w, s, z, a)
        errs.append(((q.double() - w.double()).abs().pow(3) * imp.reshape(w.shape).double()).sum(-1))
    errs = torch.stack(errs)
    s_w = oobs.calculate_qparams(mw, xw, a)
    qw = ofq.fake_quantize_weight(w, s_w[0], s_w[1], a)
    got = ((qw.double() - w.double()).abs().pow(3) * imp.reshape(w.shape).double()).sum(-1)
    assert torch.all(got <= errs.min(0).values * (1 + 1e-5))


def test_imatrix_importance_validation():
    w = _imatrix_case()
    a = OArgs(num_bits=4, strategy="channel")
    flat = oobs.flatten_weight(w, a)
    assert oobs.imatrix_importance(None, 0, flat, a) is None
    for bad in (torch.full((8,), float("nan")), -torch.ones(8), torch.zeros(8), torch.ones(7)):
        assert oobs.imatrix_importance(bad, 1, flat, a) is None
    assert oobs.imatrix_importance(torch.ones(8), 1, flat, OArgs(num_bits=4, strategy="tensor")) is None
    assert oobs.imatrix_importance(torch.ones(8), 1, flat, a, base_name="input") is None
    imp = oobs.imatrix_importance(torch.arange(1.0, 9.0), 2, flat, a)
    assert torch.allclose(imp[0, 0, 0], torch.arange(1.0, 9.0) / 4.5)
