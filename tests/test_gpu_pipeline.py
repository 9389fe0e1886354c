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
