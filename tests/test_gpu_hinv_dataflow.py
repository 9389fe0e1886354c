"""GPU: the dataflow factorisation (one persistent launch for the Cholesky
chain and L^-1, orders that are multiples of 128 with 4..64 blocks, batches
of at most 8) against the blocked chain (MI355Q_HINV_DAG=0) and against
float64, the reference's cholesky -> cholesky_inverse -> cholesky(upper)
(modifiers/gptq/gptq_quantize.py:181-188).  Repeated calls give identical
bits (each tile accumulates in a fixed order whatever the schedule), a
Hessian that is not positive definite reports it as the chain does, and a
wait forced past its limit from the host raises instead of falling back."""
import os

import pytest
import torch

from llmcompressor_amd import _lib as L
from llmcompressor_amd import ops, workloads

pytestmark = pytest.mark.gpu


def _hessian(d, seed, dev):
    x = workloads.heavy_tailed_activations((1, 2 * d, d), seed=seed).to(dev).reshape(-1, d).float()
    return 2.0 * x.t() @ x, float(2 * d)


def _f64_hinv(H, n, damp=0.01):
    h = H.double().cpu() / n
    h = h + torch.diag(torch.where(torch.diagonal(h) == 0, torch.ones(()), torch.zeros(())).double())
    h = h + damp * torch.mean(torch.diagonal(h)) * torch.eye(h.shape[0], dtype=torch.float64)
    return torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(h)), upper=True)


def _rel(a, b):
    return float(torch.linalg.norm(a.double().cpu() - b.double().cpu()) / torch.linalg.norm(b.double().cpu()))


def _with_env(key, value, fn):
    old = os.environ.get(key)
    os.environ[key] = value
    try:
        return fn()
    finally:
        if old is None:
            del os.environ[key]
        else:
            os.environ[key] = old


@pytest.mark.parametrize("d", [512, 1024, 2048, 4096])
def test_dataflow_single_matches_chain_and_f64(dev, d):
    print(f"dataflow hinv d={d}", flush=True)
    H, n = _hessian(d, 11 + d, dev)
    h1, dead1, ok1 = ops.gptq_hinv(H, None, n, 0.01)
    h1b, _, _ = ops.gptq_hinv(H, None, n, 0.01)
    h0, dead0, ok0 = _with_env("MI355Q_HINV_DAG", "0", lambda: ops.gptq_hinv(H, None, n, 0.01))
    assert ok1 and ok0 and torch.equal(dead1, dead0)
    assert torch.equal(h1, h1b)                       # deterministic across calls
    assert torch.equal(h1, torch.triu(h1))
    r_chain, r_f64 = _rel(h1, h0), _rel(h1, _f64_hinv(H, n))
    print(f"  rel vs chain {r_chain:.3g}, vs f64 {r_f64:.3g} (chain vs f64 {_rel(h0, _f64_hinv(H, n)):.3g})")
    assert r_chain <= 2e-5 and r_f64 <= 1e-4


@pytest.mark.parametrize("d,B", [(512, 3), (1024, 8), (2048, 2)])
def test_dataflow_batched_matches_single(dev, d, B):
    print(f"dataflow hinv batched d={d} B={B}", flush=True)
    Hs, ns = zip(*[_hessian(d, 100 + b, dev) for b in range(B)])
    H = torch.stack(Hs)
    hb, deadb, okb = ops.gptq_hinv_batched(H, None, torch.tensor(ns), 0.01)
    assert bool(okb.all())
    for b in range(B):
        hs, _, _ = ops.gptq_hinv(Hs[b], None, ns[b], 0.01)
        assert torch.equal(hb[b], hs), b              # batch members computed as single matrices
    h0, _, _ = _with_env("MI355Q_HINV_DAG", "0", lambda: ops.gptq_hinv_batched(H, None, torch.tensor(ns), 0.01))
    assert _rel(hb, h0) <= 2e-5


def test_dataflow_not_positive_definite(dev):
    print("dataflow hinv: not positive definite", flush=True)
    d = 512
    H, n = _hessian(d, 7, dev)
    H[300, 300] = -1e6 * n                            # a negative pivot
    _, _, ok = ops.gptq_hinv(H, None, n, 0.01)
    _, _, ok0 = _with_env("MI355Q_HINV_DAG", "0", lambda: ops.gptq_hinv(H, None, n, 0.01))
    assert not ok and not ok0
    h, _, status = ops.gptq_hinv_rtn(H, None, n, 0.01)
    assert int(status.cpu()[0]) == L.NOT_POSITIVE_DEFINITE
    assert torch.equal(h, torch.eye(d, device=dev))  # the reference's fallback


def test_dataflow_forced_timeout_raises_then_recovers(dev):
    """Waits bounded at 0 us: every waiting workgroup gives up, the launch
    drains, and the host raises; the next call runs normally."""
    print("dataflow hinv: forced time-out", flush=True)
    d = 1024
    H, n = _hessian(d, 5, dev)
    with pytest.raises(L.Mi355qError) as e:
        _with_env("MI355Q_HINV_DAG_TIMEOUT_US", "0", lambda: ops.gptq_hinv(H, None, n, 0.01))
    assert e.value.status == L.TIMEOUT
    torch.cuda.synchronize()
    h1, _, ok = ops.gptq_hinv(H, None, n, 0.01)
    assert ok and _rel(h1, _f64_hinv(H, n)) <= 1e-4
