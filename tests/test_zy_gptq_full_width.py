"""Config-0 shape end to end: 4096 x 4096 W4A16 g128 against the oracle.

Its own module, collected after the other GPU parity tests, so that a
failure here hides none of them under ``pytest -x``.  Bars as
test_gpu_parity.py's end-to-end GPTQ tests (and why a strict +-1 bound on
every code is not one of them: tests/gptq_code_spread.py).
"""
import pytest
import torch

from llmcompressor_amd import gptq, workloads
from llmcompressor_amd.observers import Observer
from llmcompressor_amd.quant_args import QuantizationArgs
from oracle import gptq as og
from oracle.qargs import OArgs
from parity_util import code_agreement, code_bar

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _layer_err(W, Q, X):
    Xf = X.reshape(-1, X.shape[-1]).float()
    return (Xf @ (W.float() - Q.float()).t()).norm().item()


def test_gptq_full_width_4096(dev):
    """Config-0 shape: 4096 x 4096 W4A16 g128 (8192 calibration tokens)."""
    rows = cols = 4096
    say("gptq 4096x4096")
    W = workloads.gptq_weight(rows, cols, seed=0)
    X = workloads.heavy_tailed_activations((4, 2048, cols), seed=1)
    qa = QuantizationArgs(num_bits=4, strategy="group", group_size=128)
    lin = torch.nn.Linear(cols, rows, bias=False).to(dev)
    lin.weight.data = W.to(dev)
    H = gptq.make_empty_hessian(lin)
    n = torch.zeros((), device=dev)
    H, n = gptq.accumulate_hessian(X.to(dev), lin, H, n)
    Hc = H.cpu()
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(lin.weight)
    res = gptq.gptq_quantize(lin.weight, qa, H, obs, num_samples=float(n.item()))
    # oracle solve on the GPU-accumulated Hessian (mirrored), checked separately above
    Hf = torch.triu(Hc) + torch.triu(Hc, 1).t()
    _, out_o, ex = og.quantize_weight(W, OArgs(num_bits=4, strategy="group", group_size=128), Hf / float(n.item()),
                                      return_codes=True)
    codes = res.codes.cpu().to(torch.int32)
    st = code_agreement(codes, ex["codes"])
    Xs = X[:1]
    e_gpu, e_ora = _layer_err(W, res.weight.cpu(), Xs), _layer_err(W, out_o["weight"], Xs)
    say(f"  {st} err {e_gpu:.6g} vs {e_ora:.6g}")
    assert code_bar(st, rows)
    assert abs(e_gpu - e_ora) <= 0.005 * e_ora


