"""Min-max and MSE observers backed by the gfx950 kernels.

Mirrors ``observers/base.py:29-206`` and ``observers/min_max.py:16-110``:
the same registry names (``memoryless_minmax``, ``static_minmax``,
``minmax``, ``strict_symmetric_minmax``), the same statistics
(``min_vals`` / ``max_vals`` shaped per strategy as
``observers/helpers.py:63-131`` flattens), weight observers that keep their
first statistics until ``get_qparams`` deletes them, and ``get_qparams``
returning ``{"scale", "zero_point", "global_scale"}`` with the scale in the
observed dtype (bf16 for a bf16 weight).  ``memoryless_mse`` / ``mse``
(``observers/mse.py:12-98``) shrink those min / max by the grid search of
``observers/mse_quant.py:19-273`` in one kernel pass over the values;
``imatrix_mse`` (``observers/imatrix.py:23-283``) weights that search by the
per-input-channel E[x^2] its forward pre-hook collects.
"""
from __future__ import annotations

import torch

import logging
import math
import weakref

from . import ops
from .quant_args import QuantizationArgs, QuantizationStrategy, QuantizationType, resolve_args

ACTIVATION_OBS = ("input", "output", "q", "k", "v")

# Layer names whose weight observers share one NVFP4 global scale
# (``observers/helpers.py:161-174``): the modules a runtime fuses into one
# GEMM (gate / up, q / k / v, DeepSeek's fused q_a / kv_a, w1 / w3 experts).
FUSED_LAYER_NAMES = [
    ("gate_proj", "up_proj"),
    ("q_proj", "k_proj", "v_proj"),
    ("q_a_proj", "kv_a_proj_with_mqa"),
    ("w1", "w3"),
]


class _FusionGroup:
    """Weight observers of one fused layer set (``observers/fusion.py:17-105``
    behaviour): each member's NVFP4 global scale comes from the statistics of
    every member, a member without statistics observes its module's weight
    first (modules held by weak reference), and statistics are deleted only
    once every member has asked for its qparams."""

    def __init__(self, pairs):
        self.members = [(obs, weakref.ref(mod)) for obs, mod in pairs]
        self.done: set[int] = set()

    def statistics(self, first):
        """[first's (min, max)] + the other members' (min, max), observing
        each member that holds none."""
        order = [first] + [o for o, _ in self.members if o is not first]
        refs = {id(o): r for o, r in self.members}
        for obs in order:
            if not obs.has_statistics:
                mod = refs[id(obs)]()
                assert mod is not None, "Fused module has been garbage collected before its weight was observed"
                obs(mod.weight)
        return [(o.min_vals, o.max_vals) for o in order]

    def release(self, obs) -> None:
        self.done.add(id(obs))
        if len(self.done) == len(self.members):
            self.done.clear()
            for o, _ in self.members:
                o.delete_statistics(check_fused=False)


class Observer(torch.nn.Module):
    _registry: dict[str, type] = {}
    _stats_attrs = ("min_vals", "max_vals")

    def __init__(self, base_name: str, args: QuantizationArgs, **observer_kwargs):
        super().__init__()
        self.base_name = base_name
        self.args = resolve_args(args)
        self.args.observer_kwargs = dict(self.args.observer_kwargs or {})
        self.args.observer_kwargs.update(observer_kwargs)
        self._observed_dtype: torch.dtype | None = None
        self._fusion: _FusionGroup | None = None

    # -- registry (compressed-tensors RegistryMixin semantics)
    @classmethod
    def register(cls, name: str):
        def deco(sub):
            cls._registry[name] = sub
            return sub
        return deco

    @classmethod
    def load_from_registry(cls, name: str, **kwargs) -> "Observer":
        try:
            sub = cls._registry[name]
        except KeyError:
            raise ValueError(f"Unknown observer {name}; registered: {sorted(cls._registry)}") from None
        return sub(**kwargs)

    @property
    def has_statistics(self) -> bool:
        return all(getattr(self, a, None) is not None for a in self._stats_attrs)

    @property
    def is_weight_obs(self) -> bool:
        return self.base_name == "weight"

    @property
    def is_fused(self) -> bool:
        return self._fusion is not None

    def delete_statistics(self, check_fused: bool = True) -> None:
        """Drop the statistics; with ``check_fused`` a fused member's are kept
        until every member of its group has asked (``fusion.py:82-105``)."""
        if check_fused and self._fusion is not None:
            self._fusion.release(self)
            return
        for a in self._stats_attrs:
            if hasattr(self, a):
                delattr(self, a)

    def get_statistics(self) -> dict:
        assert self.has_statistics, "No statistics available. Call observer(value) first."
        return {a: getattr(self, a) for a in self._stats_attrs}

    # -- observation
    def _min_max(self, observed: torch.Tensor):
        a = self.args
        s = a.strategy
        if self.is_weight_obs:
            if s == QuantizationStrategy.TOKEN:
                raise ValueError("Token quantization cannot be applied to weights")
            return ops.observe_minmax(observed, s.value, a.group_size, a.block_structure)
        # activations: (batch, seq, hidden) -> rows = tokens
        x2 = observed.reshape(-1, observed.shape[-1])
        if s == QuantizationStrategy.TENSOR:
            return ops.observe_minmax(x2, "tensor")
        if s in (QuantizationStrategy.GROUP, QuantizationStrategy.TENSOR_GROUP):
            mn, mx = ops.observe_minmax(x2, "group", a.group_size)
            return mn.amin(dim=0), mx.amax(dim=0)
        raise ValueError(f"{s.value} quantization cannot be observed for activations here")

    def update_statistics_from_observed(self, mn: torch.Tensor, mx: torch.Tensor) -> None:
        raise NotImplementedError

    @torch.no_grad()
    def forward(self, observed: torch.Tensor) -> "Observer":
        if observed.numel() == 0:
            return self
        if self.is_weight_obs and self.has_statistics:
            return self
        if not observed.is_floating_point():
            observed = observed.to(torch.float32)  # integer observations compute in fp32
        elif observed.dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"observer supports bf16 / fp32 values, got {observed.dtype}")
        self._observed_dtype = observed.dtype
        mn, mx = self._min_max(observed)
        # statistics live in the observed dtype, as torch.amin/amax return them
        self.update_statistics_from_observed(mn.to(observed.dtype), mx.to(observed.dtype))
        return self

    # -- qparams
    def _stats_dtype(self) -> torch.dtype:
        return self._observed_dtype if self._observed_dtype == torch.bfloat16 else torch.float32

    @torch.no_grad()
    def get_qparams(self) -> dict:
        assert self.has_statistics, "No statistics available. Call observer(value) first."
        a = self.args
        dt = self._stats_dtype()
        if a.is_mx:
            _, scale = ops.mx_scales(self.min_vals, self.max_vals, a.observer_kwargs.get("mx_rule", "ct"))
            zp = torch.zeros(scale.shape, dtype=a.zp_dtype, device=scale.device)
            out = {"scale": scale.to(torch.bfloat16), "zero_point": zp, "global_scale": None}
        elif a.strategy == QuantizationStrategy.TENSOR_GROUP:
            # NVFP4: the global scale from the absmax over this observer's and
            # its fused members' statistics, fp8 group scales
            # (observers/base.py:78-123)
            if a.type != QuantizationType.FLOAT or a.num_bits != 4 or not a.symmetric:
                raise NotImplementedError("tensor_group quantization is symmetric fp4 (NVFP4)")
            stats = self._fusion.statistics(self) if self._fusion is not None else [(self.min_vals, self.max_vals)]
            n_own = self.min_vals.numel()
            mn = torch.cat([m.reshape(-1).to(self.min_vals.dtype) for m, _ in stats])
            mx = torch.cat([m.reshape(-1).to(self.max_vals.dtype) for _, m in stats])
            gs, scale = ops.nvfp4_qparams(mn, mx, dt)
            scale = scale[:n_own].reshape(self.min_vals.shape)
            zp = torch.zeros(scale.shape, dtype=a.zp_dtype, device=scale.device)
            out = {"scale": scale, "zero_point": zp, "global_scale": gs}
        else:
            qmin, qmax = a.q_range()
            scale, zp = ops.calculate_qparams(self.min_vals, self.max_vals, qmin, qmax, a.symmetric, dt)
            if a.type == QuantizationType.FLOAT and not a.symmetric:
                raise NotImplementedError("asymmetric float quantization")
            scale = scale.to(a.scale_dtype if a.scale_dtype is not None else dt)
            out = {"scale": scale, "zero_point": zp.to(a.zp_dtype), "global_scale": None}
        self.delete_statistics()
        return out


@Observer.register("memoryless_minmax")
class MemorylessMinMaxObserver(Observer):
    def update_statistics_from_observed(self, mn, mx):
        self.min_vals, self.max_vals = mn, mx


@Observer.register("strict_symmetric_minmax")
class StrictSymmetricMinMaxObserver(MemorylessMinMaxObserver):
    """Symmetric int range [-(2^(b-1)-1), 2^(b-1)-1], fp32 scale (``min_max.py:28-55``)."""

    @torch.no_grad()
    def get_qparams(self):
        a = self.args
        if a.type != QuantizationType.INT or not a.symmetric:
            raise ValueError("strict_symmetric_minmax requires symmetric integer quantization")
        qmax = 2.0 ** (a.num_bits - 1) - 1
        sdt = a.scale_dtype if a.scale_dtype is not None else torch.float32
        scale, _ = ops.calculate_qparams(self.min_vals, self.max_vals, -qmax - 1, qmax, True,
                                         torch.bfloat16 if sdt == torch.bfloat16 else torch.float32, strict=True)
        scale = scale.to(sdt)
        self.delete_statistics()
        return {"scale": scale, "zero_point": torch.zeros_like(scale, dtype=a.zp_dtype), "global_scale": None}


@Observer.register("static_minmax")
class StaticMinMaxObserver(MemorylessMinMaxObserver):
    def update_statistics_from_observed(self, mn, mx):
        if self.has_statistics:
            mn, mx = torch.min(mn, self.min_vals), torch.max(mx, self.max_vals)
        self.min_vals, self.max_vals = mn, mx


@Observer.register("minmax")
class MinMaxObserver(Observer):
    """Moving average of min/max with ``averaging_constant`` (default 0.01)."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.avg_constant = self.args.observer_kwargs.get("averaging_constant", 0.01)

    def update_statistics_from_observed(self, mn, mx):
        if self.has_statistics and self.avg_constant != 1.0:
            c = self.avg_constant
            mn = self.min_vals * (1.0 - c) + mn * c
            mx = self.max_vals * (1.0 - c) + mx * c
        self.min_vals, self.max_vals = mn, mx


class _MSEObserver(Observer):
    """Grid-searched min / max (``observers/mse.py:12-49``): ``maxshrink``
    (0.20), ``patience`` (5), ``grid`` (100), ``norm`` (2.4) and ``chunk_size``
    (5; only validated: the search is one kernel pass) from observer_kwargs."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        kw = self.args.observer_kwargs
        self.maxshrink = kw.get("maxshrink", 0.20)
        self.patience = kw.get("patience", 5)
        self.grid = kw.get("grid", 100.0)
        self.norm = kw.get("norm", 2.4)
        self.chunk_size = kw.get("chunk_size", 5)
        if self.chunk_size <= 0:
            raise ValueError(f"chunk_size must be positive, got {self.chunk_size}")

    def _cells(self, observed: torch.Tensor):
        """(2-D values, cell rows, cell cols) of the strategy's groups."""
        a, s = self.args, self.args.strategy
        if self.is_weight_obs:
            rows, cols = observed.shape
            cell = {QuantizationStrategy.TENSOR: (rows, cols), QuantizationStrategy.CHANNEL: (1, cols),
                    QuantizationStrategy.GROUP: (1, a.group_size),
                    QuantizationStrategy.TENSOR_GROUP: (1, a.group_size)}.get(s)
            if s == QuantizationStrategy.BLOCK:
                cell = tuple(a.block_structure)
            if cell is None:
                raise ValueError(f"{s.value} quantization cannot be observed for weights here")
            return observed, cell[0], cell[1]
        x2 = observed.reshape(-1, observed.shape[-1])
        if s == QuantizationStrategy.TENSOR:
            return x2, x2.shape[0], x2.shape[1]
        if s == QuantizationStrategy.GROUP:
            return x2, x2.shape[0], a.group_size
        raise ValueError(f"{s.value} quantization cannot be observed for activations here")

    def _grid(self) -> str:
        """The value grid of the search: integers, fp8 e4m3, fp4 e2m1 or MXFP4
        (symmetric; the candidates' scales as calculate_qparams gives them
        without a global scale, mse_quant.py:255-262 - for NVFP4 the global
        scale then comes from the searched statistics, observers/base.py:78-96)."""
        a = self.args
        if a.type == QuantizationType.INT and not a.is_mx:
            return "int"
        if a.is_mx:
            # candidates' scales: the power of two of the e8m0 exponent of
            # their shrunk absmax, by the observer's MX rule
            return "mxfp4_" + a.observer_kwargs.get("mx_rule", "ct")
        if a.type == QuantizationType.FLOAT and a.symmetric:
            if a.num_bits == 8 and a.strategy != QuantizationStrategy.TENSOR_GROUP:
                return "fp8"
            # with fp8 scales (the NVFP4 preset) each candidate's scale would
            # be cast to float8 and the bf16 / fp32 value divided by it, a
            # promotion torch refuses: the reference's search there is not
            # pinned, so only searches without a scale dtype are provided
            if a.num_bits == 4 and a.scale_dtype is None:
                return "fp4"
        raise NotImplementedError("MSE observers for fp4 with fp8 scales and asymmetric float types are not "
                                  "provided by this build")

    def _min_max(self, observed: torch.Tensor):
        a = self.args
        qtype = self._grid()
        mn, mx = super()._min_max(observed)
        x2, ch, cw = self._cells(observed)
        qmin, qmax = a.q_range()
        mn2, mx2 = ops.observe_mse(x2, ch, cw, mn.reshape(-1), mx.reshape(-1), qmin, qmax, a.symmetric,
                                   int(self.maxshrink * self.grid), self.patience, self.grid, self.norm, qtype=qtype)
        return mn2.reshape(mn.shape), mx2.reshape(mx.shape)


@Observer.register("memoryless_mse")
class MemorylessMSEObserver(_MSEObserver):
    def update_statistics_from_observed(self, mn, mx):
        self.min_vals, self.max_vals = mn, mx


@Observer.register("mse")
class MovingAverageMSEObserver(_MSEObserver):
    """The grid search's min / max, interpolated into the running statistics
    with ``averaging_constant`` (0.01) after the first observation
    (``observers/mse.py:51-98``, ``helpers.py:219-221``)."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.avg_constant = self.args.observer_kwargs.get("averaging_constant", 0.01)

    def update_statistics_from_observed(self, mn, mx):
        if self.has_statistics and self.avg_constant != 1.0:
            c = self.avg_constant
            mn = (self.min_vals * (1.0 - c)) + (mn * c)
            mx = (self.max_vals * (1.0 - c)) + (mx * c)
        self.min_vals, self.max_vals = mn, mx


_logger = logging.getLogger("llmcompressor_amd")
_logged_once: set[str] = set()


def _warn_once(msg: str) -> None:
    if msg not in _logged_once:
        _logged_once.add(msg)
        _logger.warning(msg)


@Observer.register("imatrix_mse")
class IMatrixMSEObserver(_MSEObserver):
    """MSE observer weighted by per-input-channel importance E[x^2]
    (``observers/imatrix.py:23-283``): ``attach(module)`` installs a forward
    pre-hook accumulating sum x^2 and the token count on the module (or takes
    accumulators a previous pass left there), ``detach`` removes it.  Defaults
    maxshrink 0.95, patience 5 (0: no early stop), grid 20, norm 3; ``strict``
    raises where the reference would otherwise fall back to uniform MSE."""

    def __init__(self, *args, **kwargs):
        Observer.__init__(self, *args, **kwargs)
        kw = self.args.observer_kwargs
        self.maxshrink = kw.get("maxshrink", 0.95)
        self.patience = kw.get("patience", 5)
        self.grid = kw.get("grid", 20)
        self.norm = kw.get("norm", 3.0)
        self.strict = kw.get("strict", False)
        self.chunk_size = kw.get("chunk_size", 0)
        self._imatrix_sum = None
        self._imatrix_count = torch.tensor(0, dtype=torch.int64)
        if self.grid <= 0:
            raise ValueError(f"grid must be > 0, got {self.grid}")
        if self.patience < 0:
            raise ValueError(f"patience must be >= 0, got {self.patience}")
        if self.chunk_size < 0:
            raise ValueError(f"chunk_size must be >= 0, got {self.chunk_size}")
        if not (0 <= self.maxshrink <= 1):
            raise ValueError(f"maxshrink must be in [0, 1], got {self.maxshrink}")
        if not isinstance(self.norm, (int, float)) or not math.isfinite(self.norm) or self.norm <= 0:
            raise ValueError(f"norm must be a finite positive number, got {self.norm}")

    # -- hook lifecycle (imatrix.py:68-138)
    def attach(self, module: torch.nn.Module) -> None:
        if hasattr(module, "_imatrix_sum"):
            self._imatrix_sum, self._imatrix_count = module._imatrix_sum, module._imatrix_count
            del module._imatrix_sum
            del module._imatrix_count
            return
        if not hasattr(module, "in_features"):
            return
        module._imatrix_sum = torch.zeros(module.in_features, dtype=torch.float32)
        module._imatrix_count = torch.tensor(0, dtype=torch.int64)

        def _hook(mod, args):
            if isinstance(args, tuple):
                if len(args) == 0:
                    return
                x = args[0]
            else:
                x = args
            if isinstance(x, tuple):
                x = x[0]
            if x is None or not isinstance(x, torch.Tensor):
                return
            x = x.detach()
            mod._imatrix_sum = mod._imatrix_sum.to(x.device)
            mod._imatrix_count = mod._imatrix_count.to(x.device)
            ops.column_sumsq_(x.reshape(-1, x.shape[-1]), mod._imatrix_sum)
            mod._imatrix_count += math.prod(x.shape[:-1])

        module._imatrix_hook = module.register_forward_pre_hook(_hook)

    def detach(self, module: torch.nn.Module) -> None:
        if hasattr(module, "_imatrix_hook"):
            module._imatrix_hook.remove()
            del module._imatrix_hook

    # -- importance (imatrix.py:157-283)
    def _fallback(self, msg: str, exc=ValueError):
        if self.strict:
            raise exc(f"imatrix_mse: {msg}")
        _warn_once(f"imatrix_mse: {msg}. Falling back to uniform MSE.")
        return None

    def _importance(self, observed: torch.Tensor):
        a = self.args
        if not self.is_weight_obs:
            return self._fallback("only supported for weight observers", NotImplementedError)
        if a.strategy == QuantizationStrategy.TENSOR:
            return self._fallback("TENSOR strategy not supported", NotImplementedError)
        if self._imatrix_sum is None or int(self._imatrix_count) == 0:
            return self._fallback("no importance data available")
        imp = self._imatrix_sum.to(observed.device) / self._imatrix_count.to(observed.device).float()
        if not torch.isfinite(imp).all():
            return self._fallback("contains non-finite values")
        if (imp < 0).any():
            return self._fallback("contains negative values")
        if torch.all(imp == 0):
            return self._fallback("all zeros")
        if a.strategy not in (QuantizationStrategy.CHANNEL, QuantizationStrategy.GROUP,
                              QuantizationStrategy.TENSOR_GROUP):
            return self._fallback(f"unsupported strategy {a.strategy}", NotImplementedError)
        expected = observed.shape[-1]
        if imp.numel() != expected:
            return self._fallback(f"size mismatch: expected {expected}, got {imp.numel()}")
        imp = imp.to(torch.float32)
        return imp / (imp.mean() + torch.finfo(torch.float32).tiny)

    def _min_max(self, observed: torch.Tensor):
        a = self.args
        qtype = self._grid()
        imp = self._importance(observed)
        mn, mx = Observer._min_max(self, observed)
        x2, ch, cw = self._cells(observed)
        qmin, qmax = a.q_range()
        steps = max(1, int(self.maxshrink * self.grid)) + 1
        mn2, mx2 = ops.observe_mse(x2, ch, cw, mn.reshape(-1), mx.reshape(-1), qmin, qmax, a.symmetric, steps,
                                   self.patience, self.grid, self.norm, importance=imp, imatrix=True, qtype=qtype)
        return mn2.reshape(mn.shape), mx2.reshape(mx.shape)

    def update_statistics_from_observed(self, mn, mx):
        self.min_vals, self.max_vals = mn, mx


def fuse_weight_observers(model: torch.nn.Module) -> None:
    """Link the tensor-group (NVFP4) weight observers of each fused layer set
    in ``FUSED_LAYER_NAMES`` so that they share one global scale
    (``observers/helpers.py:177-215``).  A set is linked when a submodule
    holds all of its names; members that are None are skipped, and a set
    mixing tensor-group observers with missing or other observers fails the
    same assertions as the reference."""
    for sub in model.modules():
        for names in FUSED_LAYER_NAMES:
            if not all(hasattr(sub, n) for n in names):
                continue
            only_obs = only_tensor_group = True
            pairs = []
            for layer in (getattr(sub, n) for n in names):
                if layer is None:
                    continue
                obs = getattr(layer, "weight_observer", None)
                if obs is None:
                    only_obs = False
                    continue
                if obs.args.strategy != QuantizationStrategy.TENSOR_GROUP:
                    only_tensor_group = False
                    continue
                pairs.append((obs, layer))
            if not pairs:
                continue
            start = f"Some layers in fused group: {names} have"
            end = ", need all fused layers to have same quantization"
            assert only_obs, f"{start} no weight observer{end}"
            assert only_tensor_group, f"{start} non-TENSOR_GROUP quantization{end}"
            group = _FusionGroup(pairs)
            for obs, _ in pairs:
                obs._fusion = group
