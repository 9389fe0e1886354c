"""The drop-in ``quantize_weight`` called as the reference calls it.

``modifiers/gptq/base.py:591-597`` hands ``quantize_weight`` compressed-tensors'
``QuantizationArgs`` and leaves the reference's own observer on
``module.weight_observer``.  Neither object is this package's: here the
arguments are a namespace holding only compressed-tensors' field names with
str-enum values of a foreign enum class, and the observer is an object with
only ``__call__`` / ``get_qparams`` / ``delete_statistics`` whose statistics
and qparams come from the oracle's restatement of the reference's min-max
observer (``observers/min_max.py:16-25``, ``observers/base.py:99-145``).
The results meet the oracle's GPTQ under the end-to-end code bar, and equal
bit for bit what the same call gives with this package's own arguments and
observer.
"""
from enum import Enum
from types import SimpleNamespace

import pytest
import torch

from llmcompressor_amd import CT_ARG_FIELDS, gptq, workloads
from llmcompressor_amd.observers import Observer
from llmcompressor_amd.quant_args import QuantizationArgs
from oracle import gptq as og
from oracle import observers as oobs
from oracle.qargs import OArgs
from parity_util import code_agreement, code_bar

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


class CTType(str, Enum):
    INT = "int"
    FLOAT = "float"


class CTStrategy(str, Enum):
    TENSOR = "tensor"
    CHANNEL = "channel"
    GROUP = "group"
    BLOCK = "block"
    TENSOR_GROUP = "tensor_group"


class CTActOrder(str, Enum):
    GROUP = "group"
    WEIGHT = "weight"
    DYNAMIC = "dynamic"
    STATIC = "static"


def ct_args(num_bits, type, strategy, symmetric=True, group_size=None, actorder=None, scale_dtype=None,
            zp_dtype=None):
    """A namespace with exactly compressed-tensors' field names."""
    ns = SimpleNamespace(num_bits=num_bits, type=CTType(type), symmetric=symmetric, group_size=group_size,
                         strategy=CTStrategy(strategy), block_structure=None, dynamic=False,
                         actorder=None if actorder is None else CTActOrder(actorder), scale_dtype=scale_dtype,
                         zp_dtype=zp_dtype, observer="minmax", observer_kwargs={})
    assert set(vars(ns)) == set(CT_ARG_FIELDS)
    return ns


class ForeignObserver:
    """The reference observer's surface and nothing more; statistics and
    qparams from the oracle's min-max observer, returned on the device."""

    def __init__(self, oargs: OArgs, device):
        self._obs = oobs.OMinMax("memoryless_minmax", "weight", oargs)
        self._dev = device
        self.log = []

    def __call__(self, observed):
        self.log.append(("observe", tuple(observed.shape), observed.dtype))
        self._obs(observed.detach().cpu())
        return self

    def get_qparams(self):
        self.log.append(("get_qparams",))
        return {k: None if v is None else v.to(self._dev) for k, v in self._obs.get_qparams().items()}

    def delete_statistics(self, check_fused=True):
        self.log.append(("delete", check_fused))
        self._obs.min_vals = self._obs.max_vals = None


class OwnObserverProxy:
    """This package's observer behind the same three members."""

    def __init__(self, obs):
        self._obs = obs

    def __call__(self, observed):
        self._obs(observed)
        return self

    def get_qparams(self):
        return self._obs.get_qparams()

    def delete_statistics(self, check_fused=True):
        self._obs.delete_statistics(check_fused=check_fused)


def _int_codes(w, scale, zp, g_idx, group_size):
    """Integer codes round(w / scale) + zp of a fake-quantised weight."""
    w = w.float()
    cols = w.shape[1]
    if g_idx is None:
        g_idx = torch.arange(cols) // group_size if group_size else torch.zeros(cols, dtype=torch.long)
    s = scale.float()[:, g_idx.long()]
    z = zp.float()[:, g_idx.long()]
    return (torch.round(w / s) + z).to(torch.int32)


INT_CASES = [
    dict(num_bits=4, type="int", strategy="group", group_size=128),
    dict(num_bits=4, type="int", strategy="group", group_size=128, actorder="static"),
    dict(num_bits=4, type="int", strategy="group", group_size=128, actorder="dynamic"),
    dict(num_bits=4, type="int", strategy="group", group_size=128, symmetric=False, actorder="group"),
    dict(num_bits=8, type="int", strategy="channel", actorder="weight"),
]


def _layer(dev, rows, cols, tokens, seed):
    W = workloads.gptq_weight(rows, cols, seed=seed)
    X = workloads.heavy_tailed_activations((2, tokens // 2, cols), seed=seed + 1)
    lin = torch.nn.Linear(cols, rows, bias=False).to(dev)
    lin.weight.data = W.to(dev)
    H = gptq.make_empty_hessian(lin)
    n = torch.zeros((), device=dev)
    H, n = gptq.accumulate_hessian(X.to(dev), lin, H, n)
    return W, X, lin, H / n


def _oargs(case):
    c = dict(case)
    a = c.pop("actorder", None)
    a = {"static": "weight", "dynamic": "group"}.get(a, a)
    return OArgs(actorder=a, **c)


@pytest.mark.parametrize("case", INT_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_dropin_with_compressed_tensors_args_and_observer(dev, case):
    rows, cols, tokens = 384, 1024, 4096
    say(f"drop-in with CT-shaped args {case}")
    W, X, lin, H = _layer(dev, rows, cols, tokens, seed=41)
    oa = _oargs(case)
    lin.weight_observer = ForeignObserver(oa, dev)
    lin.weight_observer(lin.weight)              # observe(module, "weight"), as base.py runs it
    args = ct_args(**case)
    snapshot = dict(vars(args))
    loss, q = gptq.quantize_weight(module=lin, quant_args=args, hessian=H.clone())
    assert dict(vars(args)) == snapshot          # the caller's arguments are not modified
    log = lin.weight_observer.log
    if oa.actorder == "group":                   # gptq_quantize.py:145-148: re-observe the permuted fp32 weight
        assert log[1:] == [("delete", False), ("observe", (rows, cols), torch.float32), ("get_qparams",)]
    else:
        assert log[1:] == [("get_qparams",)]
    Ho = torch.triu(H.cpu())
    Ho = Ho + torch.triu(Ho, 1).t()
    loss_o, out_o, ex = og.quantize_weight(W, oa, Ho, return_codes=True)
    assert q["weight"].dtype == torch.bfloat16 and q["weight"].shape == W.shape
    assert torch.equal(q["weight_scale"].cpu(), out_o["weight_scale"])
    assert q["weight_zero_point"].dtype == torch.int8
    assert torch.equal(q["weight_zero_point"].cpu(), out_o["weight_zero_point"])
    assert ("weight_g_idx" in q) == (oa.actorder == "group")
    if "weight_g_idx" in q:
        assert torch.equal(q["weight_g_idx"].cpu(), out_o["weight_g_idx"])
    g_idx = out_o.get("weight_g_idx")
    codes = _int_codes(q["weight"].cpu(), q["weight_scale"].cpu(), q["weight_zero_point"].cpu(), g_idx,
                       oa.group_size)
    codes_o = _int_codes(out_o["weight"], out_o["weight_scale"], out_o["weight_zero_point"], g_idx, oa.group_size)
    assert torch.equal(codes_o, ex["codes"])     # the recovery reads the oracle's own codes back
    st = code_agreement(codes, codes_o)
    e_gpu = (X.reshape(-1, cols).float() @ (W.float() - q["weight"].cpu().float()).t()).norm().item()
    e_ora = (X.reshape(-1, cols).float() @ (W.float() - out_o["weight"].float()).t()).norm().item()
    say(f"  {st} err_gpu={e_gpu:.6g} err_oracle={e_ora:.6g} loss {loss:.6g} vs {loss_o:.6g}")
    assert code_bar(st, rows)
    assert abs(e_gpu - e_ora) <= 0.005 * e_ora
    assert abs(loss - loss_o) <= 1e-3 * abs(loss_o) + 1e-6


SAME_CASES = INT_CASES + [
    dict(num_bits=8, type="float", strategy="channel", actorder="static"),
    dict(num_bits=4, type="float", strategy="tensor_group", group_size=16, scale_dtype=torch.float8_e4m3fn,
         zp_dtype=torch.float8_e4m3fn, actorder="dynamic"),
    dict(num_bits=4, type="float", strategy="group", group_size=32, scale_dtype=torch.uint8, zp_dtype=torch.uint8),
]


@pytest.mark.parametrize("case", SAME_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_dropin_ct_args_equal_own_args(dev, case):
    """Foreign arguments and a three-member observer give bit for bit what
    this package's own arguments and observer give (integer, FP8, NVFP4 and
    MXFP4 weights)."""
    rows, cols, tokens = 256, 512, 2048
    say(f"drop-in CT args == own args {case}")
    W, X, lin, H = _layer(dev, rows, cols, tokens, seed=43)
    c = dict(case)
    own = QuantizationArgs(**c)
    outs = []
    for args in (own, ct_args(**case)):
        obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=own)
        obs(lin.weight)
        lin.weight_observer = OwnObserverProxy(obs)
        outs.append(gptq.quantize_weight(module=lin, quant_args=args, hessian=H.clone()))
    (l0, q0), (l1, q1) = outs
    assert l0 == l1 and q0.keys() == q1.keys()
    for k in q0:
        assert q0[k].dtype == q1[k].dtype and torch.equal(q0[k], q1[k]), k
    if case.get("zp_dtype") is not None:
        assert q1["weight_zero_point"].dtype == case["zp_dtype"]
