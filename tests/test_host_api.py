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
