"""The GPTQ configurations at their own shapes against the oracle.

* 4096 x 4096 W4A16 g128 (8192 calibration tokens, and the full 64 x 2048);
* 14336 x 4096 W8A8 int8 per-channel symmetric, actorder=weight (4 x 2048
  tokens): the 14336-row solve takes the pushed lazy-update schedule and the
  wide sweep blocks;
* the Llama-3-8B down projection, 4096 x 14336 W4A16 g128 (d = 14336:
  the 112-block Cholesky chain and 112 sweep blocks).

The GPU accumulates the Hessian and solves; the oracle solves on the GPU's
Hessian (mirrored), so the codes compare the solves.  Its own module,
collected after the other GPU parity tests, so that a failure here hides
none of them under ``pytest -x``.  Bars as test_gpu_parity.py's end-to-end
GPTQ tests (and why a strict +-1 bound on every code is not one of them:
tests/gptq_code_spread.py): code bar, equal scales, layer error within 0.5 %.
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


def _gpu_heavy(shape, seed, dev, nu=4):
    """Student-t(nu) x lognormal(0, 1) per column, bf16, generated on the GPU
    in slices of 8192 rows."""
    g = torch.Generator(device=dev).manual_seed(seed)
    rows, cols = shape
    c = torch.exp(torch.randn(cols, generator=g, device=dev))
    out = torch.empty(rows, cols, dtype=torch.bfloat16, device=dev)
    for r0 in range(0, rows, 8192):
        m = min(8192, rows - r0)
        z = torch.randn(m, cols, generator=g, device=dev)
        chi = sum(torch.randn(m, cols, generator=g, device=dev) ** 2 for _ in range(nu))
        out[r0:r0 + m] = (z / torch.sqrt(chi / nu) * c).to(torch.bfloat16)
    return out


def _solve_vs_oracle(dev, W, X, qa, oa, tag, rows_frac=0.01):
    """GPU Hessian + solve of W on calibration rows X [tokens, cols] (one
    sample per 2048 tokens), the oracle's solve on that Hessian, the bars
    (``rows_frac``: the share of rows whose codes may diverge at all)."""
    rows, cols = W.shape
    lin = torch.nn.Linear(cols, rows, bias=False, device=dev, dtype=torch.bfloat16)
    lin.weight.data = W.to(dev)
    H = gptq.make_empty_hessian(lin)
    n = torch.zeros((), device=dev)
    H, n = gptq.accumulate_hessian(X.reshape(-1, 2048, cols), lin, H, n)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(lin.weight)
    res = gptq.gptq_quantize(lin.weight, qa, H, obs, num_samples=float(n.item()))
    Hc = H.cpu()
    del H
    say(f"  {tag}: GPU solve done, oracle solve ...")
    Hf = torch.triu(Hc) + torch.triu(Hc, 1).t()
    del Hc
    Wc = W.cpu()
    _, out_o, ex = og.quantize_weight(Wc, oa, Hf / float(n.item()), return_codes=True)
    del Hf
    st = code_agreement(res.codes.cpu().to(torch.int32), ex["codes"])
    Xs = X[:2048].cpu()
    e_gpu, e_ora = _layer_err(Wc, res.weight.cpu(), Xs), _layer_err(Wc, out_o["weight"], Xs)
    say(f"  {tag}: {st} err {e_gpu:.6g} vs {e_ora:.6g} (ratio {e_gpu / e_ora:.6f})")
    assert torch.equal(res.scale.cpu().to(torch.bfloat16).reshape(out_o["weight_scale"].shape),
                       out_o["weight_scale"]), tag
    assert code_bar(st, rows, rows_frac), tag
    assert abs(e_gpu - e_ora) <= 0.005 * e_ora, tag


# Longer rows (14336 columns) and finer grids (int8) give each row more
# chances to meet a rounding boundary: the oracle against itself with only
# its Cholesky chain's fp32 order changed (flip identity or fp64) diverges in
# 172-190 of 14336 rows (1.2-1.3 %) at the W8A8 shape and in 57-69 of 4096
# rows (1.4-1.7 %, codes up to 3 apart) at the down projection's
# (tests/gptq_code_spread.py --configs, seeds 4 and 9).  Those two allow
# 2.5 % of the rows to diverge; agreement >= 99.9 %, +-1 first divergences
# and the layer error bound are unchanged.
WIDE_ROWS_FRAC = 0.025


def test_gptq_full_width_4096_all_tokens(dev):
    """Config-0 exactly: 4096 x 4096 W4A16 g128 on 64 x 2048 tokens."""
    say("gptq 4096x4096, 64 x 2048 tokens")
    W = workloads.gptq_weight(4096, 4096, seed=0)
    X = _gpu_heavy((64 * 2048, 4096), 1, dev)
    _solve_vs_oracle(dev, W, X, QuantizationArgs(num_bits=4, strategy="group", group_size=128),
                     OArgs(num_bits=4, strategy="group", group_size=128), "C0 131072 tokens")


def test_gptq_w8a8_channel_actorder_14336x4096(dev):
    """W8A8 weights: 14336 x 4096 int8 per-channel symmetric, actorder=weight."""
    say("gptq W8A8 14336x4096 actorder=weight, 4 x 2048 tokens")
    g = torch.Generator(device=dev).manual_seed(4)
    W = (torch.randn(14336, 4096, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    X = _gpu_heavy((4 * 2048, 4096), 5, dev)
    _solve_vs_oracle(dev, W, X, QuantizationArgs(num_bits=8, strategy="channel", actorder="weight"),
                     OArgs(num_bits=8, strategy="channel", actorder="weight"), "C2 14336x4096", WIDE_ROWS_FRAC)


def test_gptq_down_projection_4096x14336(dev):
    """The Llama-3-8B down projection: 4096 x 14336 W4A16 g128, actorder=weight
    (the GPTQModifier default), 8 x 2048 tokens."""
    say("gptq down projection 4096x14336 actorder=weight, 8 x 2048 tokens")
    g = torch.Generator(device=dev).manual_seed(9)
    W = (torch.randn(4096, 14336, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    X = _gpu_heavy((8 * 2048, 14336), 10, dev)
    _solve_vs_oracle(dev, W, X, QuantizationArgs(num_bits=4, strategy="group", group_size=128, actorder="weight"),
                     OArgs(num_bits=4, strategy="group", group_size=128, actorder="weight"), "C4 down 4096x14336",
                     WIDE_ROWS_FRAC)


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


