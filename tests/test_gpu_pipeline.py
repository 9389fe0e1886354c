"""GPU: the sequential calibration pipeline and its activation cache.

Checks: without error propagation the pipeline compresses exactly as one
calibration pass over the whole model (pipelines/basic), with it exactly as a
hand-run layer-by-layer loop (each layer calibrated on the compressed
predecessors' outputs); host offload and prefetch change nothing; the cache
round-trips nested values through pinned memory.
"""
import copy

import pytest
import torch

from llmcompressor_amd import GPTQModifier, SparseGPTModifier, workloads
from llmcompressor_amd.pipeline import IntermediatesCache, sequential_calibrate

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


class Block(torch.nn.Module):
    def __init__(self, d, f):
        super().__init__()
        self.q = torch.nn.Linear(d, d, bias=False)
        self.o = torch.nn.Linear(d, d, bias=False)
        self.up = torch.nn.Linear(d, f, bias=False)
        self.gate = torch.nn.Linear(d, f, bias=False)
        self.down = torch.nn.Linear(f, d, bias=False)

    def forward(self, x, scale=None):
        h = x + self.o(torch.tanh(self.q(x)) * scale)
        return h + self.down(torch.nn.functional.silu(self.gate(h)) * self.up(h))


class Toy(torch.nn.Module):
    def __init__(self, d=256, f=512, n=3):
        super().__init__()
        self.layers = torch.nn.ModuleList(Block(d, f) for _ in range(n))

    def forward(self, x):
        scale = torch.full((x.shape[-1],), 0.5, device=x.device, dtype=x.dtype)
        for layer in self.layers:
            x = layer(x, scale=scale)
        return x


def _setup(dev, n_batches=3):
    torch.manual_seed(0)
    model = Toy().to(dev).to(torch.bfloat16)
    for p in model.parameters():
        p.data.mul_(0.5)
    batches = [workloads.heavy_tailed_activations((2, 64, 256), seed=s).to(dev) for s in range(n_batches)]
    return model, batches


def _gptq():
    return GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=())


def _weights(model):
    return {k: v.detach().clone() for k, v in model.state_dict().items() if k.endswith("weight")}


def _assert_same(a, b):
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_pipeline_without_propagation_equals_one_pass(dev):
    say("pipeline propagate_error=False vs one calibration pass")
    model, batches = _setup(dev)
    ref = copy.deepcopy(model)
    _gptq().apply(ref, batches)
    sequential_calibrate(model, model.layers, batches, _gptq(), propagate_error=False)
    _assert_same(_weights(model), _weights(ref))


def test_pipeline_with_propagation_equals_layer_loop(dev):
    say("pipeline propagate_error=True vs hand-run layer loop")
    model, batches = _setup(dev)
    ref = copy.deepcopy(model)
    xs = [b.clone() for b in batches]
    scale = torch.full((256,), 0.5, device=dev, dtype=torch.bfloat16)
    for layer in ref.layers:
        wrapper = torch.nn.Module()
        wrapper.layer = layer
        wrapper.forward = lambda x, _l=layer: _l(x, scale=scale)
        _gptq().apply(wrapper, xs)
        with torch.no_grad():
            xs = [layer(x, scale=scale) for x in xs]
    cache = sequential_calibrate(model, model.layers, batches, _gptq(), propagate_error=True)
    _assert_same(_weights(model), _weights(ref))
    outs = [d["args"][0] for d in cache.iter()]
    for o, x in zip(outs, xs):
        assert torch.equal(o, x)


@pytest.mark.parametrize("offload,prefetch", [(None, False), ("cpu", False), ("cpu", True)])
def test_offload_and_prefetch_change_nothing(dev, offload, prefetch):
    say(f"pipeline offload={offload} prefetch={prefetch}")
    model, batches = _setup(dev, n_batches=4)
    ref = copy.deepcopy(model)
    sequential_calibrate(ref, ref.layers, batches, _gptq(), offload_device=None, prefetch=False)
    cache = sequential_calibrate(model, model.layers, batches, _gptq(), offload_device=offload, prefetch=prefetch)
    _assert_same(_weights(model), _weights(ref))
    sizes = cache.size()
    assert ("cpu" in sizes) == (offload == "cpu")


def test_cache_round_trip(dev):
    say("intermediates cache")
    cache = IntermediatesCache(2, offload_device="cpu")
    a = torch.randn(5, 7, device=dev)
    vals = {"args": (a, 3), "kwargs": {"pos": (a * 2, a * 3), "flag": True}}
    cache.update(0, vals)
    cache.update(1, {"args": (a + 1,)})
    assert cache.size()["cpu"] == 4 * a.numel() * 4
    got = cache.fetch(0)
    assert got["args"][1] == 3 and got["kwargs"]["flag"] is True
    assert torch.equal(got["args"][0], a) and torch.equal(got["kwargs"]["pos"][1], a * 3)
    assert got["args"][0].device == a.device
    seen = [d["args"][0] for d in cache.iter_prefetch(["args"])]
    assert torch.equal(seen[0], a) and torch.equal(seen[1], a + 1)
    cache.delete(0, ["kwargs"])
    assert list(cache.batches[0]) == ["args"]


def test_sparsegpt_through_the_pipeline(dev):
    say("SparseGPT through the pipeline")
    model, batches = _setup(dev)
    mod = SparseGPTModifier(sparsity=0.5, mask_structure="2:4", targets=["Linear"])
    sequential_calibrate(model, model.layers, batches, mod)
    for name, p in model.named_parameters():
        z = (p.reshape(p.shape[0], -1, 4) == 0).sum(-1)
        assert torch.all(z >= 2), name


def test_sparsegpt_shared_hessians_change_nothing(dev):
    say("SparseGPT: shared Hessians vs separate, through the pipeline")
    model, batches = _setup(dev)
    ref = copy.deepcopy(model)
    sequential_calibrate(ref, ref.layers, batches,
                         SparseGPTModifier(sparsity=0.5, targets=["Linear"], share_hessians=False))
    sequential_calibrate(model, model.layers, batches, SparseGPTModifier(sparsity=0.5, targets=["Linear"]))
    _assert_same(_weights(model), _weights(ref))


def test_shared_hessians_change_nothing(dev):
    """gate and up read the same tensor: one Hessian and one Cholesky chain
    for both give exactly the weights of separate ones."""
    say("shared Hessians vs separate")
    model, batches = _setup(dev)
    ref = copy.deepcopy(model)
    GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=(), share_hessians=False).apply(ref, batches)
    mod = _gptq()
    mod.apply(model, batches)
    _assert_same(_weights(model), _weights(ref))


class _TwoReaders(torch.nn.Module):
    """a and b read the same tensor in the first forward only."""

    def __init__(self):
        super().__init__()
        self.a = torch.nn.Linear(256, 256, bias=False)
        self.b = torch.nn.Linear(256, 256, bias=False)
        self.calls = 0

    def forward(self, x):
        y = self.a(x) + self.b(x if self.calls == 0 else x.clone())
        self.calls += 1
        return y


class _Skipper(torch.nn.Module):
    """a and b read the same tensor; b is skipped in forward number `skip`."""

    def __init__(self, skip):
        super().__init__()
        self.a = torch.nn.Linear(256, 256, bias=False)
        self.b = torch.nn.Linear(256, 256, bias=False)
        self.calls, self.skip = 0, skip

    def forward(self, x):
        y = self.a(x) if self.calls == self.skip else self.a(x) + self.b(x)
        self.calls += 1
        return y


@pytest.mark.parametrize("skip", [1, 2], ids=["middle", "last"])
def test_shared_hessians_member_skipping_a_forward_raises(dev, skip):
    say(f"shared Hessians: a member that misses forward {skip} of 3")
    batches = [workloads.heavy_tailed_activations((2, 64, 256), seed=50 + s).to(dev) for s in range(3)]
    model = _Skipper(skip).to(dev).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="share_hessians=False"):
        _gptq().apply(model, batches)


def test_shared_hessians_divergence_raises(dev):
    say("shared Hessians: inputs that stop being shared")
    torch.manual_seed(1)
    batches = [workloads.heavy_tailed_activations((2, 64, 256), seed=40 + s).to(dev) for s in range(2)]
    model = _TwoReaders().to(dev).to(torch.bfloat16)
    ref = copy.deepcopy(model)
    with pytest.raises(RuntimeError, match="share_hessians=False"):
        _gptq().apply(model, batches)
    GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=(), share_hessians=False).apply(ref, batches)


def test_pipeline_with_propagation_vs_oracle_loop(dev):
    """pipelines/sequential/pipeline.py:136-178 against an oracle loop: per
    layer the oracle runs the layer's forward on the CPU with its original
    weights and accumulates every module's Hessian from the inputs that
    forward gives it (calibration pass), solves each module with the
    oracle's GPTQ (compression), then runs the layer again with the
    compressed weights to make the next layer's inputs (propagation).  The
    propagation uses the GPU's compressed weights, whose codes pass the bar
    against the oracle's (so later layers compare the pipeline's order, not
    the cascades of a few flipped codes); the model is fp32 so that the
    CPU's forward and the GPU's agree to fp32 rounding.  Every module of both
    layers: the Hessian the pipeline's modifier solved is within 1e-5 of the
    oracle's, the codes pass the bar and the scales are equal.  Layer 2's
    inputs are the compressed layer 1's outputs, not the original layer's."""
    from oracle import gptq as og
    from oracle.qargs import OArgs
    from parity_util import code_agreement, code_bar

    say("pipeline propagate_error=True vs an oracle calibrate / compress / propagate loop")
    torch.manual_seed(0)
    model = Toy(n=2).to(dev)
    for p in model.parameters():
        p.data.mul_(0.5)
    batches = [workloads.heavy_tailed_activations((2, 128, 256), seed=60 + s).float().to(dev) for s in range(4)]
    cpu_layers = [copy.deepcopy(l).cpu() for l in model.layers]
    mod = _gptq()
    solved = {}
    compress_one = mod._compress_one

    def spy(module, H, n, prepared):
        solved[module] = (torch.triu(H).cpu(), float(n))
        return compress_one(module, H, n, prepared)

    mod._compress_one = spy
    sequential_calibrate(model, model.layers, batches, mod, propagate_error=True)

    oa = OArgs(num_bits=4, strategy="group", group_size=128, actorder="weight")
    scale = torch.full((256,), 0.5)
    xs = [b.cpu() for b in batches]
    names = ("q", "o", "up", "gate", "down")
    for li, (layer, ref) in enumerate(zip(model.layers, cpu_layers)):
        seen = {n: [] for n in names}
        hooks = [getattr(ref, n).register_forward_pre_hook(
            lambda m, a, _n=n: seen[_n].append(a[0].detach().clone())) for n in names]
        with torch.no_grad():
            for x in xs:                              # calibration pass, original weights
                ref(x, scale=scale)
        for h in hooks:
            h.remove()
        for n in names:
            m = getattr(layer, n)
            Ho, no = og.make_empty_hessian(m.weight.shape[1]), torch.zeros(())
            for x in seen[n]:
                Ho, no = og.accumulate_hessian(x, Ho, no)
            Hg, ng = solved[m]
            assert ng == float(no) == 8.0
            r = ((Hg.double() - torch.triu(Ho).double()).norm() / torch.triu(Ho).double().norm()).item()
            W0 = getattr(ref, n).weight.detach()
            _, out_o, ex = og.quantize_weight(W0, oa, og.normalise_hessian(Ho, no), return_codes=True)
            st = code_agreement(m.gptq_codes.cpu().to(torch.int32), ex["codes"])
            Xf = torch.cat([x.reshape(-1, x.shape[-1]) for x in seen[n]])[:512]
            e_gpu = (Xf @ (W0 - m.weight.detach().cpu()).t()).norm().item()
            e_ora = (Xf @ (W0 - out_o["weight"]).t()).norm().item()
            say(f"  layer {li} {n}: H rel {r:.2e} {st} err {e_gpu:.6g} vs {e_ora:.6g}")
            assert r <= 1e-5, (li, n, r)
            assert torch.equal(m.weight_scale.detach().cpu(), out_o["weight_scale"]), (li, n)
            assert code_bar(st, W0.shape[0]), (li, n)
            assert abs(e_gpu - e_ora) <= 0.005 * e_ora, (li, n)
        with torch.no_grad():
            plain = [ref(x, scale=scale) for x in xs]
            for n in names:                           # propagation pass, compressed weights
                getattr(ref, n).weight.copy_(getattr(layer, n).weight.detach().cpu())
            xs_next = [ref(x, scale=scale) for x in xs]
        d_q = max(((a - b).norm() / b.norm()).item() for a, b in zip(plain, xs_next))
        say(f"  layer {li}: compressed vs original outputs differ by {d_q:.3e} (relative)")
        assert d_q > 1e-3   # the next layer's Hessians tell the two apart by far more than 1e-5
        xs = xs_next


def test_offload_hessians_equals_on_device(dev):
    """offload_hessians=True (modifiers/gptq/base.py:664-674): the Hessians
    wait in host memory between calls and are moved to the device for each
    accumulation and for the solve; the weights equal those of on-device
    accumulation of the same calls (hessian_batch_tokens=0: one syrk per
    call, as the offloaded path runs)."""
    say("offload_hessians=True vs on-device accumulation")
    model, batches = _setup(dev)
    ref = copy.deepcopy(model)
    GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=(), hessian_batch_tokens=0).apply(ref, batches)
    mod = GPTQModifier(scheme="W4A16", targets=("Linear",), ignore=(), offload_hessians=True)
    where = set()
    epoch_end = mod.on_sequential_epoch_end

    def check(modules):
        where.update(str(h.device) for h in mod._hessians.values())
        return epoch_end(modules)

    mod.on_sequential_epoch_end = check
    mod.apply(model, batches)
    assert where == {"cpu"}
    _assert_same(_weights(model), _weights(ref))
