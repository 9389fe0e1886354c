"""Host-side logic of the drop-in API (CPU only, no kernel launches)."""
import pytest
import torch

from llmcompressor_amd import GPTQModifier, Observer, QuantizationArgs, preset_name_to_scheme
from llmcompressor_amd.calibration import initialize_module_for_quantization, initialize_observer
from llmcompressor_amd.quant_args import ActivationOrdering, QuantizationScheme, QuantizationStrategy


def test_quantization_args_defaults_follow_compressed_tensors():
    assert QuantizationArgs().strategy == QuantizationStrategy.TENSOR
    assert QuantizationArgs(group_size=128).strategy == QuantizationStrategy.GROUP
    assert QuantizationArgs(group_size=-1).strategy == QuantizationStrategy.CHANNEL
    assert QuantizationArgs().zp_dtype == torch.int8
    assert QuantizationArgs(num_bits=4).q_range() == (-8.0, 7.0)
    assert QuantizationArgs(num_bits=8, type="float").q_range() == (-448.0, 448.0)
    assert QuantizationArgs(actorder="static").actorder == ActivationOrdering.WEIGHT
    assert QuantizationArgs(actorder="dynamic").actorder == ActivationOrdering.GROUP
    assert QuantizationArgs(actorder=True).actorder == ActivationOrdering.GROUP
    with pytest.raises(ValueError):
        QuantizationArgs(strategy="block")


def test_presets():
    w4 = preset_name_to_scheme("W4A16", ["Linear"])
    assert w4.weights.num_bits == 4 and w4.weights.group_size == 128 and w4.input_activations is None
    w8 = preset_name_to_scheme("W8A8", ["Linear"])
    assert w8.weights.strategy == QuantizationStrategy.CHANNEL
    assert w8.input_activations.strategy == QuantizationStrategy.TOKEN and w8.input_activations.dynamic
    mx = preset_name_to_scheme("MXFP4", ["Linear"])
    assert mx.weights.is_mx and mx.input_activations.dynamic
    with pytest.raises(KeyError):
        preset_name_to_scheme("NOPE", ["Linear"])


def test_observer_registry_names():
    args = QuantizationArgs()
    for name in ("memoryless_minmax", "static_minmax", "minmax", "strict_symmetric_minmax"):
        assert isinstance(Observer.load_from_registry(name, base_name="weight", args=args), Observer)
    with pytest.raises(ValueError):
        Observer.load_from_registry("nope", base_name="weight", args=args)


def test_initialize_observer_overrides_weight_minmax():
    """calibration.py:64-71: weight minmax -> memoryless; dynamic args get none (:80)."""
    lin = torch.nn.Linear(16, 8, bias=False)
    initialize_module_for_quantization(lin, preset_name_to_scheme("W8A8", ["Linear"]))
    initialize_observer(lin, "weight")
    initialize_observer(lin, "input")
    assert type(lin.weight_observer).__name__ == "MemorylessMinMaxObserver"
    assert not hasattr(lin, "input_observer")
    assert lin.weight_scale.shape == (8, 1) and lin.weight_zero_point.dtype == torch.int8


def test_qparam_shapes_per_strategy():
    lin = torch.nn.Linear(64, 6, bias=False)
    initialize_module_for_quantization(lin, QuantizationScheme(weights=QuantizationArgs(num_bits=4, group_size=16)))
    assert lin.weight_scale.shape == (6, 4)
    lin2 = torch.nn.Linear(7, 5, bias=False)
    initialize_module_for_quantization(lin2, QuantizationScheme(
        weights=QuantizationArgs(num_bits=8, strategy="block", block_structure=[2, 4])))
    assert lin2.weight_scale.shape == (3, 2)


@pytest.mark.parametrize("modifier_actorder,scheme_actorder,expected", [
    ("static", None, ActivationOrdering.WEIGHT),
    ("static", "group", ActivationOrdering.GROUP),
    ("group", None, ActivationOrdering.GROUP),
    (None, None, None),
    ("weight", "weight", ActivationOrdering.WEIGHT),
])
def test_actorder_resolution(modifier_actorder, scheme_actorder, expected):
    """modifiers/gptq/base.py:137-193 truth table."""
    m = GPTQModifier(actorder=modifier_actorder)
    s = QuantizationScheme(weights=QuantizationArgs(num_bits=4, group_size=128, actorder=scheme_actorder))
    m._resolve_actorder(s)
    assert s.weights.actorder == expected


def test_actorder_conflict_raises():
    m = GPTQModifier(actorder="group")
    s = QuantizationScheme(weights=QuantizationArgs(num_bits=4, group_size=128, actorder="weight"))
    with pytest.raises(ValueError, match="Cannot resolve activation ordering"):
        m._resolve_actorder(s)


def test_actorder_group_on_channel_falls_back():
    m = GPTQModifier(actorder="group")
    s = QuantizationScheme(weights=QuantizationArgs(num_bits=8, strategy="channel"))
    m._resolve_actorder(s)
    assert s.weights.actorder is None


def test_cpu_tensors_are_refused():
    from llmcompressor_amd import ops
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.observe_minmax(torch.zeros(4, 4), "tensor")


def test_sparsegpt_host_checks_raise_as_reference():
    """sgpt_sparsify.py:160,185,181-182: the sort index past the block
    (IndexError), a topk wider than its group (RuntimeError), a preserved-mask
    window of another width (RuntimeError) - raised before any kernel runs."""
    from llmcompressor_amd.sparsegpt import _check_blocks
    with pytest.raises(IndexError):
        _check_blocks(8, 64, 1.0, 0, 0, 32, False)
    _check_blocks(8, 64, 0.999, 0, 0, 32, False)
    with pytest.raises(RuntimeError):
        _check_blocks(8, 64, 0.5, 3, 2, 32, False)
    with pytest.raises(RuntimeError):
        _check_blocks(8, 62, 0.5, 3, 4, 32, False)          # last group 2 wide, n = 3
    _check_blocks(8, 62, 0.5, 2, 4, 32, False)
    with pytest.raises(RuntimeError):
        _check_blocks(8, 64, 0.5, 1, 3, 32, True)           # block 32 ends in a 2-wide group, mask window 3
    with pytest.raises(NotImplementedError):
        _check_blocks(8, 512, 0.5, 0, 0, 256, False)


def test_sparsegpt_modifier_validation():
    from llmcompressor_amd import SparseGPTModifier
    m = SparseGPTModifier(sparsity=0.5, mask_structure="2:4")
    assert (m._prune_n, m._prune_m) == (2, 4)
    assert (SparseGPTModifier(sparsity=0.5)._prune_n, SparseGPTModifier(sparsity=0.5)._prune_m) == (0, 0)
    with pytest.raises(ValueError):
        SparseGPTModifier(sparsity=0.5, owl_m=5)
    with pytest.raises(ValueError):
        SparseGPTModifier(sparsity=0.5, sparsity_profile="bad")
    model = torch.nn.Sequential(torch.nn.Linear(8, 8), torch.nn.ReLU(), torch.nn.Linear(8, 8))
    for sp, targets in (([0.5, 0.2], "__ALL__"), ([0.2, 0.1, 0.3], ["0", "2"]), ([0.3, 0.4], ["re:.*1$"])):
        with pytest.raises(ValueError):
            SparseGPTModifier(sparsity=sp, targets=targets).on_initialize(model)
    assert SparseGPTModifier(sparsity=[0.5, 0.2], targets=["0", "2"]).on_initialize(model)


def _hook_sequence(events):
    """Drives the shared-Hessian bookkeeping of GPTQModifier as its forward
    hook does (no kernel launches): events are (module, input) in forward order."""
    from llmcompressor_amd.modifiers import _SharedHessians

    class Book(_SharedHessians):
        def __init__(self):
            self._num_samples = {}
            self._init_sharing(True)

    book = Book()
    name = {m: m for m in "abc"}.get
    for module, inp in events:
        if book._shared(module, inp, name):
            continue
        book._num_samples.setdefault(module, 0)
        book._note_accumulated(module, inp, name)
    return book, name


def test_shared_hessian_member_missing_the_last_forward_raises():
    """a and b read the same tensor; b misses the last batch: its Hessian
    would hold a batch it never saw, so compression raises."""
    x = [torch.randn(4, 8) for _ in range(3)]
    ok, name = _hook_sequence([("a", x[0]), ("b", x[0]), ("a", x[1]), ("b", x[1]), ("a", x[2]), ("b", x[2])])
    assert ok._take_groups(name) == {"a": ["a", "b"]}
    book, name = _hook_sequence([("a", x[0]), ("b", x[0]), ("a", x[1]), ("b", x[1]), ("a", x[2])])
    with pytest.raises(RuntimeError, match="share_hessians=False"):
        book._take_groups(name)
    with pytest.raises(RuntimeError, match="share_hessians=False"):   # a middle batch missed
        _hook_sequence([("a", x[0]), ("b", x[0]), ("a", x[1]), ("a", x[2]), ("b", x[2])])


def test_resolve_args_reads_compressed_tensors_fields_only():
    """A caller's arguments object (compressed-tensors' QuantizationArgs at
    modifiers/gptq/base.py:591-597) is read through CT's field names only,
    enum members by value, aliases and defaults as compressed-tensors has
    them; the caller's object is not modified."""
    from enum import Enum
    from types import SimpleNamespace

    from llmcompressor_amd import CT_ARG_FIELDS, resolve_args

    class S(str, Enum):
        GROUP = "group"
        CHANNEL = "channel"

    class A(str, Enum):
        STATIC = "static"
        DYNAMIC = "dynamic"

    class T(str, Enum):
        INT = "int"
        FLOAT = "float"

    read = []

    class Recording(SimpleNamespace):
        def __getattribute__(self, name):
            if not name.startswith("__"):
                read.append(name)
            return object.__getattribute__(self, name)

    ns = Recording(num_bits=4, type=T.INT, symmetric=True, group_size=128, strategy=S.GROUP,
                   block_structure=None, dynamic=False, actorder=A.STATIC, scale_dtype=None, zp_dtype=None,
                   observer="minmax", observer_kwargs={"maxshrink": 0.3}, unrelated_member=1)
    a = resolve_args(ns)
    assert set(read) <= set(CT_ARG_FIELDS) and "unrelated_member" not in read
    assert a.strategy == QuantizationStrategy.GROUP and a.actorder == ActivationOrdering.WEIGHT
    assert a.q_range() == (-8.0, 7.0) and a.zp_dtype == torch.int8 and not a.is_mx
    assert a.observer_kwargs == {"maxshrink": 0.3} and a.observer_kwargs is not ns.observer_kwargs
    assert ns.actorder is A.STATIC and ns.zp_dtype is None
    assert resolve_args(SimpleNamespace(num_bits=8, group_size=-1)).strategy == QuantizationStrategy.CHANNEL
    assert resolve_args(SimpleNamespace(num_bits=8, actorder=A.DYNAMIC, group_size=64)).actorder == \
        ActivationOrdering.GROUP
    assert resolve_args(SimpleNamespace(num_bits=8, actorder=True, group_size=64)).actorder == \
        ActivationOrdering.GROUP
    mx = resolve_args(SimpleNamespace(num_bits=4, type=T.FLOAT, strategy=S.GROUP, group_size=32,
                                      scale_dtype=torch.uint8, zp_dtype=torch.uint8))
    assert mx.is_mx and mx.q_range() == (-6.0, 6.0)
    fp8 = resolve_args(SimpleNamespace(num_bits=8, type="float", strategy="channel"))
    assert fp8.q_range() == (-448.0, 448.0) and fp8.zp_dtype == torch.float8_e4m3fn
    own = QuantizationArgs(num_bits=4, group_size=128)
    assert resolve_args(own) is own


def test_fused_observers_release_statistics_together():
    """observers/helpers.py:177-215 + fusion.py:82-105: q/k/v and gate/up
    NVFP4 weight observers are linked; each member's statistics stay until
    every member has asked for its qparams.  Non-tensor-group schemes are
    not linked; a set mixing tensor-group with other observers fails the
    reference's assertion."""
    from llmcompressor_amd import fuse_weight_observers

    def block(scheme_qkv, scheme_o="NVFP4A16"):
        attn = torch.nn.Module()
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            lin = torch.nn.Linear(32, 16, bias=False)
            initialize_module_for_quantization(lin, preset_name_to_scheme(
                scheme_qkv if n != "o_proj" else scheme_o, ["Linear"]))
            initialize_observer(lin, "weight")
            setattr(attn, n, lin)
        return attn

    attn = block("NVFP4A16")
    fuse_weight_observers(attn)
    obs = [getattr(attn, n).weight_observer for n in ("q_proj", "k_proj", "v_proj")]
    assert all(o.is_fused for o in obs) and not attn.o_proj.weight_observer.is_fused
    for o in obs:
        o.min_vals, o.max_vals = torch.zeros(16, 2), torch.ones(16, 2)
    obs[0].delete_statistics()
    obs[1].delete_statistics()
    assert all(o.has_statistics for o in obs)
    obs[2].delete_statistics()
    assert not any(o.has_statistics for o in obs)
    obs[0].min_vals, obs[0].max_vals = torch.zeros(16, 2), torch.ones(16, 2)
    obs[0].delete_statistics(check_fused=False)
    assert not obs[0].has_statistics

    w4 = block("W4A16", "W4A16")
    fuse_weight_observers(w4)
    assert not w4.q_proj.weight_observer.is_fused

    mixed = block("NVFP4A16")
    initialize_module_for_quantization(mixed.k_proj, preset_name_to_scheme("W4A16", ["Linear"]))
    initialize_observer(mixed.k_proj, "weight")
    with pytest.raises(AssertionError, match="non-TENSOR_GROUP"):
        fuse_weight_observers(mixed)


def test_expert_families_group_expert_lists_only():
    """Projections of an expert list (a container with num_experts, or named
    ...experts) form families by relative name; decoder-layer lists do not;
    members with different quantization arguments are left alone."""
    from llmcompressor_amd.moe import LinearExperts, expert_families
    from llmcompressor_amd.quant_args import resolve_args

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.experts = LinearExperts(4, 16, 8)
            self.layers = torch.nn.ModuleList(torch.nn.Linear(16, 16) for _ in range(3))

    blk = Block()
    for m in blk.modules():
        if isinstance(m, torch.nn.Linear):
            initialize_module_for_quantization(m, preset_name_to_scheme("W4A16", ["Linear"]))
    targets = {m for m in blk.modules() if isinstance(m, torch.nn.Linear)}
    args_of = lambda m: resolve_args(m.quantization_scheme.weights)  # noqa: E731
    fams = expert_families(blk.named_modules(), targets, args_of, 1 << 20)
    keys = sorted({f.key for f in fams.values()})
    assert keys == ["experts.*.down_proj", "experts.*.gate_proj", "experts.*.up_proj"]
    f = fams[blk.experts[2].up_proj]
    assert f.members == [blk.experts[e].up_proj for e in range(4)] and f.slot[blk.experts[2].up_proj] == 2
    assert not any(l in fams for l in blk.layers)
    initialize_module_for_quantization(blk.experts[1].down_proj, preset_name_to_scheme("W8A16", ["Linear"]))
    fams = expert_families(blk.named_modules(), targets, args_of, 1 << 20)
    assert blk.experts[0].down_proj not in fams and blk.experts[0].gate_proj in fams


def test_expert_families_of_a_bare_expert_list():
    """The expert list itself as the model: members named <e>.gate_proj."""
    from llmcompressor_amd.moe import LinearExperts, expert_families
    from llmcompressor_amd.quant_args import resolve_args

    ex = LinearExperts(3, 16, 8)
    for m in ex.modules():
        if isinstance(m, torch.nn.Linear):
            initialize_module_for_quantization(m, preset_name_to_scheme("W4A16", ["Linear"]))
    fams = expert_families(ex.named_modules(), {m for m in ex.modules() if isinstance(m, torch.nn.Linear)},
                           lambda m: resolve_args(m.quantization_scheme.weights), 1 << 20)
    assert sorted({f.key for f in fams.values()}) == ["*.down_proj", "*.gate_proj", "*.up_proj"]
