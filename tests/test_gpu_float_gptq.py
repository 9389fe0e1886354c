"""GPU: GPTQ on float weights (FP8 e4m3 per channel / per tensor, MXFP4 group
32 with power-of-two scales, NVFP4 tensor-group 16 with fp8 group scales and
a global scale) against the oracle.

The sweep rounds each column with CT's float rounding (RNE to the e4m3 or
e2m1 grid after ``x / (scale / global_scale)``, gptq_quantize.py:215-247) and
feeds the error back exactly as for int codes.  Codes compare as signed grid
positions (one code step = one grid step): the given-Hinv sweep within one
step of the oracle's for nearly every row (an fp8 row whose first code flips
by one step can cascade further, as the oracle's own rows do under a changed
fp32 summation), end to end within the cascade-aware bar of the int cases
(2 % of rows for fp8).  Scales and global scales are equal bit for bit.
"""
import pytest
import torch

from llmcompressor_amd import gptq, workloads
from llmcompressor_amd.observers import Observer
from llmcompressor_amd.quant_args import QuantizationArgs
from oracle import gptq as og
from oracle.fake_quant import signed_grid_index
from oracle.observers import OMinMax
from oracle.qargs import OArgs
from parity_util import code_agreement, code_bar

pytestmark = pytest.mark.gpu

E4 = torch.float8_e4m3fn
FLOAT_CASES = {
    "nvfp4": (dict(num_bits=4, type="float", strategy="tensor_group", group_size=16, scale_dtype=E4, zp_dtype=E4),
              dict(num_bits=4, type="float", strategy="tensor_group", group_size=16, scale_dtype=E4)),
    "nvfp4-actorder": (dict(num_bits=4, type="float", strategy="tensor_group", group_size=16, scale_dtype=E4,
                            zp_dtype=E4, actorder="weight"),
                       dict(num_bits=4, type="float", strategy="tensor_group", group_size=16, scale_dtype=E4,
                            actorder="weight")),
    "mxfp4": (dict(num_bits=4, type="float", strategy="group", group_size=32, scale_dtype=torch.uint8,
                   zp_dtype=torch.uint8),
              dict(num_bits=4, type="float", strategy="group", group_size=32, is_mx=True)),
    "fp8-channel": (dict(num_bits=8, type="float", strategy="channel", actorder="weight"),
                    dict(num_bits=8, type="float", strategy="channel", actorder="weight")),
    "fp8-tensor": (dict(num_bits=8, type="float", strategy="tensor"),
                   dict(num_bits=8, type="float", strategy="tensor")),
}


def say(*a):
    print(*a, flush=True)


def _grid(codes, oa):
    return signed_grid_index(codes.cpu().to(torch.int32), oa)


def _layer_err(W, Q, X):
    Xf = X.reshape(-1, X.shape[-1]).float()
    return (Xf @ (W.float() - Q.float()).t()).norm().item()


def _check_qparams(res, ex, out_o):
    assert torch.equal(res.scale.cpu().float().reshape(ex["scale_used"].shape), ex["scale_used"].float())
    if "weight_global_scale" in out_o:
        assert res.global_scale is not None
        assert float(res.global_scale) == float(out_o["weight_global_scale"])
    else:
        assert res.global_scale is None


@pytest.mark.parametrize("name", list(FLOAT_CASES))
def test_float_sweep_given_oracle_hinv(dev, name):
    """Sweep with the oracle's Hinv: every code within one grid step of the
    oracle's, nearly all equal; loss within 1e-4."""
    qk, ok = FLOAT_CASES[name]
    rows, cols, tokens = 384, 1024, 4096
    say(f"float gptq sweep given the oracle's hinv {name}")
    W = workloads.gptq_weight(rows, cols, seed=43)
    X = workloads.heavy_tailed_activations((2, tokens // 2, cols), seed=44)
    Ho, no = og.accumulate_hessian(X, og.make_empty_hessian(cols), torch.zeros(()))
    Ho = og.normalise_hessian(Ho, no)
    Ho[9, :] = 0
    Ho[:, 9] = 0   # a dead column
    oa = OArgs(**ok)
    loss_o, out_o, ex = og.quantize_weight(W, oa, Ho, return_codes=True)
    qa = QuantizationArgs(**qk)
    perm = None if ex["perm"] is None else ex["perm"].to(dev)
    Hp = Ho if perm is None else Ho[ex["perm"]][:, ex["perm"]]
    dead = (torch.diag(Hp) == 0).to(torch.int32).to(dev)
    prep = gptq.PreparedHessian(gptq._effective_actorder(qa), perm, None if perm is None else torch.argsort(perm),
                                ex["hinv"].to(dev), dead, torch.zeros(1, dtype=torch.int32, device=dev))
    Wd = W.to(dev)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(Wd)
    res = gptq.gptq_quantize(Wd, qa, torch.triu(Ho).to(dev), obs, prepared=prep)
    _check_qparams(res, ex, out_o)
    st = code_agreement(_grid(res.codes, oa), _grid(ex["codes"], oa))
    say(f"  {st} loss {res.loss:.6g} vs {loss_o:.6g}")
    assert code_bar(st, rows) and st["agree"] >= 0.9995
    assert abs(res.loss - loss_o) <= 1e-4 * abs(loss_o) + 1e-6


@pytest.mark.parametrize("name", list(FLOAT_CASES))
def test_float_gptq_end_to_end_parity(dev, name):
    qk, ok = FLOAT_CASES[name]
    rows, cols, tokens = 384, 1024, 4096
    say(f"float gptq e2e {name}")
    W = workloads.gptq_weight(rows, cols, seed=41)
    X = workloads.heavy_tailed_activations((2, tokens // 2, cols), seed=42)
    qa = QuantizationArgs(**qk)
    lin = torch.nn.Linear(cols, rows, bias=False).to(dev)
    lin.weight.data = W.to(dev)
    H = gptq.make_empty_hessian(lin)
    n = torch.zeros((), device=dev)
    H, n = gptq.accumulate_hessian(X.to(dev), lin, H, n)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(lin.weight)
    res = gptq.gptq_quantize(lin.weight, qa, H, obs, num_samples=float(n.item()))
    oa = OArgs(**ok)
    Ho, no = og.accumulate_hessian(X, og.make_empty_hessian(cols), torch.zeros(()))
    loss_o, out_o, ex = og.quantize_weight(W, oa, og.normalise_hessian(Ho, no), return_codes=True)
    _check_qparams(res, ex, out_o)
    st = code_agreement(_grid(res.codes, oa), _grid(ex["codes"], oa))
    e_gpu = _layer_err(W, res.weight.cpu(), X)
    e_ora = _layer_err(W, out_o["weight"], X)
    say(f"  {st} err_gpu={e_gpu:.6g} err_oracle={e_ora:.6g} loss {res.loss:.6g} vs {loss_o:.6g}")
    assert code_bar(st, rows, 0.02 if qk["num_bits"] == 8 else 0.01)
    assert abs(e_gpu - e_ora) <= 0.005 * e_ora
    assert abs(res.loss - loss_o) <= 1e-3 * abs(loss_o) + 1e-6


@pytest.mark.parametrize("name", ["nvfp4", "mxfp4", "fp8-channel"])
def test_float_gptq_batched_equals_single(dev, name):
    """The batched solve gives each member what its own solve gives,
    including per-member global scales (NVFP4)."""
    qk, _ = FLOAT_CASES[name]
    say(f"float gptq batched {name}")
    B, rows, d = 3, 200, 384
    qa = QuantizationArgs(**qk)
    g = torch.Generator().manual_seed(5)
    Ws = [workloads.gptq_weight(rows, d, seed=60 + b) * (b + 1) for b in range(B)]
    Hs = []
    for b in range(B):
        X = torch.randn(1024, d, generator=g)
        Hs.append(torch.triu(X.t() @ X / 1024 + 0.01 * torch.eye(d)))
    W = torch.stack(Ws).to(dev)
    H = torch.stack(Hs).to(dev)
    res = gptq.gptq_quantize_batched(W, qa, H.clone(), num_samples=1.0)
    for b in range(B):
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
        obs(W[b])
        single = gptq.gptq_quantize(W[b], qa, H[b].clone(), obs, num_samples=1.0)
        assert torch.equal(res[b].codes, single.codes)
        assert torch.equal(res[b].weight, single.weight)
        assert torch.equal(res[b].scale.reshape(single.scale.shape), single.scale)
        if single.global_scale is not None:
            assert torch.equal(res[b].global_scale, single.global_scale)


def test_tensor_group_golden_table_on_gpu(dev):
    """The reference's fp4 tensor-group known answer (test_lifecycle.py, group
    3 over arange(24)): GPU observer statistics, global and fp8 group scales,
    and the fake-quantised weight GPTQ writes with a diagonal Hessian (no
    error feedback, so GPTQ is round-to-nearest)."""
    import json
    from pathlib import Path
    gold = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
    case = next(c for c in gold["static_weight_quantization"]["cases"] if c["args"]["type"] == "float")
    a = dict(case["args"], scale_dtype=E4, zp_dtype=E4)
    qa = QuantizationArgs(**a)
    w = torch.arange(24, dtype=torch.bfloat16).reshape(4, 6).to(dev)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(w)
    assert torch.equal(obs.min_vals.float().cpu(), torch.tensor(case["min"], dtype=torch.float32))
    assert torch.equal(obs.max_vals.float().cpu(), torch.tensor(case["max"], dtype=torch.float32))
    res = gptq.gptq_quantize(w, qa, torch.eye(6, device=dev), obs)
    exp = torch.tensor(case["quant"], dtype=torch.bfloat16)
    assert torch.allclose(res.weight.float().cpu(), exp.float()), (res.weight, exp)
    oobs = OMinMax("memoryless_minmax", "weight", OArgs(**dict(case["args"], scale_dtype=E4)))
    qp = oobs(w.cpu()).get_qparams()
    assert float(res.global_scale) == float(qp["global_scale"])
    assert torch.equal(res.scale.float().cpu(), qp["scale"].float())
