"""GPU: the allocation-free sweep entry point against the one with a caller
workspace, through the C ABI: bit-identical codes, dequantised weights and
losses on two calls in a row (the second smaller), and the size limit."""
import ctypes as C

import pytest
import torch

from llmcompressor_amd import _lib as L
from llmcompressor_amd import ops, workloads
from llmcompressor_amd.observers import Observer
from llmcompressor_amd.quant_args import QuantizationArgs

pytestmark = pytest.mark.gpu


def _problem(dev, rows, cols, seed, case):
    W = workloads.gptq_weight(rows, cols, seed=seed).to(dev)
    x = workloads.heavy_tailed_activations((2 * cols, cols), seed=seed + 1).to(dev)
    H = torch.zeros(cols, cols, device=dev)
    ops.hessian_syrk_(H, x, alpha=2.0)
    hinv, _, ok = ops.gptq_hinv(H, None, float(2 * cols), 0.01)
    assert ok
    qa = QuantizationArgs(**case)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    qp = obs(W).get_qparams()
    s = qp["scale"].to(torch.float32).reshape(rows, -1).contiguous()
    z = None if qa.symmetric else qp["zero_point"].to(torch.float32).reshape(s.shape).contiguous()
    gs = qa.group_size if qa.strategy.value == "group" else None
    g_idx = (torch.arange(cols, device=dev, dtype=torch.int32) // gs) if gs else None
    qmin, qmax = qa.q_range()
    return ops.gptq_load_weight(W), hinv, s, z, g_idx, qa.strategy.value, qmin, qmax


def _noalloc(w, hinv, s, z, g_idx, strategy, qmin, qmax, blocksize=128):
    rows, cols = w.shape
    codes = torch.empty((rows, cols), dtype=torch.int8, device=w.device)
    losses = torch.zeros(rows, dtype=torch.float32, device=w.device)
    L.check(L.lib().mi355q_gptq_sweep_noalloc(
        w.data_ptr(), rows, cols, hinv.data_ptr(), s.data_ptr(), L.ptr(z), s.stride(0), L.ptr(g_idx),
        ops.STRATEGY_CODE[strategy], 1, C.c_float(qmin), C.c_float(qmax), 1, blocksize, codes.data_ptr(),
        losses.data_ptr(), L.stream_of(w)))
    return codes, losses


@pytest.mark.parametrize("shapes", [[(512, 2048, 1, dict(num_bits=4, strategy="group", group_size=128)),
                                     (200, 640, 2, dict(num_bits=8, strategy="channel", symmetric=False))]],
                         ids=["512x2048-then-200x640"])
def test_sweep_noalloc_matches_workspace_entry(dev, shapes):
    for rows, cols, seed, case in shapes:
        print(f"sweep noalloc {rows}x{cols} {case}", flush=True)
        w0, hinv, s, z, g_idx, strategy, qmin, qmax = _problem(dev, rows, cols, seed, case)
        w_ref, w_na = w0.clone(), w0.clone()
        codes_ref, losses_ref = ops.gptq_sweep_(w_ref, hinv, s, z, strategy, g_idx, qmin, qmax, dequant_bf16=True)
        codes_na, losses_na = _noalloc(w_na, hinv, s, z, g_idx, strategy, qmin, qmax)
        torch.cuda.synchronize()
        assert torch.equal(codes_na, codes_ref)
        assert torch.equal(w_na, w_ref)
        assert torch.equal(losses_na, losses_ref)


def test_sweep_noalloc_rejects_shapes_above_the_scratch(dev):
    cap = L.lib().mi355q_gptq_sweep_noalloc_max_bytes()
    assert cap == 64 << 20
    rows = cap // (1024 * 4) + 1                 # one row more than the array holds at 1024 error columns
    status = L.lib().mi355q_gptq_sweep_noalloc(None, rows, 4096, None, None, None, 1, None, ops.STRATEGY_CODE["channel"],
                                               1, C.c_float(-8), C.c_float(7), 1, 128, None, None, None)
    assert status == L.INVALID_ARGUMENT
    assert b"scratch" in L.lib().mi355q_last_error()
