"""GPU: the library is reentrant — no handles, locks or mutable global state
(the allocation-free sweep's scratch array aside) — so two host threads, each
on its own HIP stream, can run Hessian accumulation and GPTQ solves at the
same time.  Each thread's results must be bit-identical to the same work run
alone on the default stream."""
import threading

import pytest
import torch

from llmcompressor_amd import gptq, ops, workloads
from llmcompressor_amd.observers import Observer
from llmcompressor_amd.quant_args import QuantizationArgs

pytestmark = pytest.mark.gpu


def _run(W, X, qa):
    H = torch.zeros(W.shape[1], W.shape[1], device=W.device)
    ops.hessian_syrk_(H, X, alpha=2.0)
    obs = Observer.load_from_registry("memoryless_minmax", base_name="weight", args=qa)
    obs(W)
    res = gptq.gptq_quantize(W, qa, H, obs, num_samples=float(X.shape[0]))
    return H, res.codes, res.weight


def test_two_threads_two_streams_match_sequential(dev):
    print("two host threads on two streams vs sequential", flush=True)
    qas = [QuantizationArgs(num_bits=4, type="int", symmetric=True, strategy="group", group_size=128),
           QuantizationArgs(num_bits=8, type="int", symmetric=True, strategy="channel", actorder="weight")]
    ins = []
    for i in range(2):
        W = workloads.gptq_weight(512 + 128 * i, 1024, seed=70 + i).to(dev)
        X = workloads.heavy_tailed_activations((4096 + 1000 * i, 1024), seed=80 + i).to(dev)
        ins.append((W, X, qas[i]))
    seq = [_run(*a) for a in ins]
    torch.cuda.synchronize()
    out, errs = [None, None], []

    def worker(i):
        try:
            s = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(s):
                for _ in range(6):
                    r = _run(*ins[i])
                s.synchronize()
            out[i] = r
        except Exception as e:   # surfaced after join
            errs.append(e)

    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs, errs
    for i in range(2):
        for a, b in zip(out[i], seq[i]):
            assert torch.equal(a, b), i


def test_hinv_beside_a_busy_stream_is_unchanged(dev):
    """The Cholesky panel solve overwrites the panel in place; every
    workgroup owns whole rows of it, so the result must not depend on which
    workgroups run together.  Here a second stream keeps the CUs busy with
    Hessian accumulations while the solve runs, which scatters the solve's
    workgroups in time; the inverse must stay bit-identical to a solo run."""
    print("gptq_hinv d=4096 beside Hessian accumulations on a second stream", flush=True)
    d = 4096
    X = workloads.heavy_tailed_activations((8192, d), seed=91).to(dev)
    H = torch.zeros(d, d, device=dev)
    ops.hessian_syrk_(H, X, alpha=2.0)
    ref, _, ok = ops.gptq_hinv(H, None, float(X.shape[0]), 0.01)
    assert ok
    Xb = torch.randn(65536, d, device=dev, generator=torch.Generator(device=dev).manual_seed(92)).to(torch.bfloat16)
    Hb = torch.zeros(d, d, device=dev)
    busy, main = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()
    for rep in range(3):
        with torch.cuda.stream(busy):
            for _ in range(4):
                ops.hessian_syrk_(Hb, Xb, alpha=1.0)
        with torch.cuda.stream(main):
            got, _, ok = ops.gptq_hinv(H, None, float(X.shape[0]), 0.01)
        torch.cuda.synchronize()
        assert ok
        assert torch.equal(got, ref), (rep, (got - ref).abs().max().item())
