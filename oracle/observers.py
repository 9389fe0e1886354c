"""Min-max observers and qparam calculation, restated for the CPU oracle.

Follows ``observers/min_max.py:16-110`` (memoryless, static, moving-average
and strict-symmetric min-max), ``observers/helpers.py:28-131`` (flattening
per strategy), ``observers/base.py:78-123`` (global scale + get_qparams) and
compressed-tensors ``calculate_qparams`` / ``generate_gparam`` as the
reference's tests pin them:

* ``tests/llmcompressor/observers/test_min_max.py:8-86``: int8 symmetric
  scale = 1/127.5, asymmetric scale = 1/255 with zp = -128, EMA updates.
* ``tests/llmcompressor/modifiers/calibration/test_observers.py:66-123``:
  min/max statistics of memoryless / static / moving-average observers.
* ``tests/llmcompressor/modifiers/calibration/test_lifecycle.py:16-165``:
  scale computed in the weight dtype (bf16), min/max widened to include 0.
* ``tests/llmcompressor/entrypoints/model_free/test_strict_symmetric.py:13-71``:
  fp32 scale = absmax / 127 clamped at 1e-8.

Zero scales are replaced by the scale dtype's epsilon (CT ``_get_dtype_eps``);
only exact zeros are affected, which the tests above do not reach: parity
unpinned for that corner.

MSE observers (``mse_grid_search``, ``observers/mse_quant.py:19-130,244-273``,
eager path, and ``observers/mse.py:12-98``) are pinned by the known-answer table
of ``tests/llmcompressor/observers/test_mse.py:9-43`` (eight strategy /
symmetry cases, loss to 1e-10) and by the brute-force argmin over the same
candidates.

MXFP4 shared scale (``mx_scale_exponent``) is parity unpinned: no reference
test covers it and CT is absent.  Two rules are provided:

* ``"ct"`` (default) - CT's ``generate_mx_scales`` as recalled from its
  published source (derived from vLLM's reference MXFP4 code): round the
  bf16 group absmax to a power of two by adding 1<<5 to the bf16 bit pattern
  and masking off the mantissa (so amax >= 1.75*2^e rounds up to 2^(e+1)),
  then e8m0 = 127 + log2(that power) - 2, clamped to [0, 254];
* ``"ocp"`` - OCP MX v1.0: e8m0 = 127 + floor(log2(amax)) - 2, clamped.
A zero group gets e8m0 = 0 under both rules.
"""
from __future__ import annotations

import torch

from .qargs import OArgs

FP8_MAX = 448.0
FP4_MAX = 6.0


# ---------------------------------------------------------------- flattening
def flatten_weight(value: torch.Tensor, args: OArgs) -> torch.Tensor:
    """``observers/helpers.py:63-101`` -> (1, *qparam_shape, group)."""
    if args.strategy == "tensor":
        return value.reshape((1, 1, -1))
    if args.strategy == "channel":
        return value.unsqueeze(-2).unsqueeze(0)
    if args.strategy in ("group", "tensor_group"):
        return value.unflatten(-1, (-1, args.group_size)).unsqueeze(0)
    if args.strategy == "block":
        bh, bw = args.block_structure
        rows, cols = value.shape
        pr, pc = (-rows) % bh, (-cols) % bw
        if pr or pc:
            value = torch.nn.functional.pad(value, (0, pc, 0, pr))
            rows, cols = value.shape
        return (value.reshape(rows // bh, bh, cols // bw, bw)
                .transpose(1, 2).flatten(-2, -1).unsqueeze(0))
    raise ValueError(f"strategy {args.strategy} not valid for weights")


def flatten_activation(value: torch.Tensor, args: OArgs) -> torch.Tensor:
    """``observers/helpers.py:105-131``."""
    if args.strategy == "tensor":
        return value.reshape((-1, 1, value.size(-1)))
    if args.strategy == "token":
        return value
    if args.strategy in ("group", "tensor_group"):
        return value.flatten(0, 1).unflatten(-1, (-1, args.group_size))
    raise ValueError(f"strategy {args.strategy} not valid for activations")


def get_min_max(observed: torch.Tensor):
    """``observers/min_max.py:106-110``."""
    return torch.amin(observed, dim=(0, -1)), torch.amax(observed, dim=(0, -1))


# ---------------------------------------------------------------- observers
class OMinMax:
    """One observer object; ``kind`` in memoryless_minmax|static_minmax|minmax|
    strict_symmetric_minmax (``observers/min_max.py:16-103``)."""

    def __init__(self, kind: str, base_name: str, args: OArgs, averaging_constant=0.01):
        self.kind, self.base_name, self.args = kind, base_name, args
        self.avg = args.observer_kwargs.get("averaging_constant", averaging_constant)
        self.min_vals = self.max_vals = None
        # (min, max) statistics of the other members of a fused layer set
        # (q/k/v, gate/up): the tensor-group global scale is taken over all
        # of them (observers/base.py:78-96, observers/fusion.py:58-80)
        self.fused_stats: list = []

    @property
    def has_statistics(self):
        return self.min_vals is not None

    def __call__(self, observed: torch.Tensor):
        if observed.numel() == 0:
            return self
        if self.base_name == "weight" and self.has_statistics:
            return self
        if self.base_name == "weight":
            flat = flatten_weight(observed, self.args)
        else:
            flat = flatten_activation(observed, self.args)
        mn, mx = get_min_max(flat)
        if self.kind == "static_minmax" and self.has_statistics:
            mn, mx = torch.min(mn, self.min_vals), torch.max(mx, self.max_vals)
        elif self.kind == "minmax" and self.has_statistics and self.avg != 1.0:
            mn = self.min_vals * (1.0 - self.avg) + mn * self.avg
            mx = self.max_vals * (1.0 - self.avg) + mx * self.avg
        self.min_vals, self.max_vals = mn, mx
        return self

    def get_qparams(self, mx_rule="ct"):
        assert self.has_statistics, "No statistics available. Call observer(value) first."
        if self.kind == "strict_symmetric_minmax":
            out = strict_symmetric_qparams(self.min_vals, self.max_vals, self.args)
        else:
            gs = None
            if self.args.strategy == "tensor_group" and not self.args.is_mx:
                gs = global_scale_from_stats([(self.min_vals, self.max_vals)] + list(self.fused_stats))
            s, z = calculate_qparams(self.min_vals, self.max_vals, self.args, gs, mx_rule)
            out = {"scale": s, "zero_point": z, "global_scale": gs}
        self.min_vals = self.max_vals = None
        return out


# ---------------------------------------------------------------- qparams
def _dtype_eps(dtype: torch.dtype) -> float:
    if dtype == torch.float8_e4m3fn:
        return 0.125
    if dtype.is_floating_point:
        return torch.finfo(dtype).eps
    return 1.0


def mx_scale_exponent(amax: torch.Tensor, rule: str = "ct") -> torch.Tensor:
    """e8m0 exponent byte (as int32) of the group shared scale; ``amax`` >= 0."""
    a = amax.to(torch.bfloat16) if rule == "ct" else amax.to(torch.float32)
    if rule == "ct":
        bits = a.view(torch.int16).to(torch.int32) & 0xFFFF
        bits = (bits + (1 << 5)) & 0xFF80
        e = ((bits >> 7) & 0xFF) - 127
        zero = bits == 0
    elif rule == "ocp":
        bits = a.view(torch.int32)
        e = ((bits >> 23) & 0xFF) - 127
        # fp32 subnormals: floor(log2) from the mantissa
        sub = ((bits >> 23) & 0xFF) == 0
        if bool(sub.any()):
            m = (bits & 0x7FFFFF).to(torch.float64)
            e = torch.where(sub, (torch.floor(torch.log2(m.clamp(min=1))) - 149).to(torch.int32), e)
        zero = a == 0
    else:
        raise ValueError(rule)
    e8 = torch.clamp(e + 127 - 2, 0, 254)
    return torch.where(zero, torch.zeros_like(e8), e8).to(torch.int32)


def e8m0_to_float(e8: torch.Tensor) -> torch.Tensor:
    return torch.pow(2.0, e8.to(torch.float64) - 127.0).to(torch.float32)


def calculate_qparams(min_vals, max_vals, args: OArgs, global_scale=None, mx_rule="ct"):
    """CT ``calculate_qparams`` as the reference's tests pin it."""
    min_vals = torch.min(min_vals, torch.zeros_like(min_vals))
    max_vals = torch.max(max_vals, torch.zeros_like(max_vals))
    q_min, q_max = args.q_range()
    bit_range = q_max - q_min
    if args.is_mx:
        amax = torch.max(torch.abs(min_vals), torch.abs(max_vals))
        scales = e8m0_to_float(mx_scale_exponent(amax, mx_rule))
        return scales, torch.zeros(scales.shape, dtype=torch.int8)
    if args.symmetric:
        max_val_pos = torch.max(torch.abs(min_vals), torch.abs(max_vals))
        if args.type == "float" and args.num_bits == 4 and global_scale is not None:
            scales = global_scale * (max_val_pos / FP4_MAX)
            scales = torch.clamp(scales, -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
        else:
            scales = max_val_pos / (float(bit_range) / 2)
        zero_points = torch.zeros(scales.shape, dtype=min_vals.dtype)
    else:
        if args.type == "float":
            raise NotImplementedError("asymmetric float quantization")
        scales = (max_vals - min_vals) / float(bit_range)
        zero_points = q_min - (min_vals / scales)
        zero_points = torch.clamp(zero_points, q_min, q_max)
    if args.type == "int":
        zero_points = torch.round(zero_points)
    if args.scale_dtype is not None and scales.dtype != args.scale_dtype:
        scales = scales.to(args.scale_dtype)
    eps = _dtype_eps(scales.dtype)
    if scales.dtype == torch.float8_e4m3fn:
        sf = scales.float()
        scales = torch.where(sf == 0, torch.full_like(sf, eps), sf).to(scales.dtype)
    else:
        scales = torch.where(scales == 0, torch.full_like(scales, eps), scales)
    zero_points = zero_points.to(args.zp_dtype)
    if scales.ndim == 0:
        scales, zero_points = scales.reshape(1), zero_points.reshape(1)
    return scales, zero_points


def strict_symmetric_qparams(min_vals, max_vals, args: OArgs):
    """``observers/min_max.py:33-55``."""
    if args.type != "int" or not args.symmetric:
        raise ValueError("strict_symmetric_minmax requires symmetric integer quantization")
    mvp = torch.max(torch.abs(min_vals.to(torch.float32)), torch.abs(max_vals.to(torch.float32)))
    qmax = 2.0 ** (args.num_bits - 1) - 1
    scales = torch.clamp(mvp / qmax, min=1e-8)
    if args.scale_dtype is not None:
        scales = scales.to(args.scale_dtype)
    return {"scale": scales, "zero_point": torch.zeros_like(scales, dtype=args.zp_dtype),
            "global_scale": None}


def generate_gparam(min_v, max_v):
    """CT ``generate_gparam``: fp8_max * fp4_max / absmax, in the stats dtype.

    A Python scalar over a tensor is ``Tensor.__rtruediv__``, which torch
    evaluates as ``reciprocal(absmax) * scalar`` with both results rounded to
    the tensor's dtype (bf16 for bf16 statistics), not as one division."""
    mn = torch.min(min_v, torch.zeros_like(min_v))
    mx = torch.max(max_v, torch.zeros_like(max_v))
    mvp = torch.max(torch.abs(mn), torch.abs(mx))
    return (FP8_MAX * FP4_MAX / mvp).to(torch.float32).reshape([1])


def global_scale_from_stats(stats):
    """``observers/base.py:78-96`` over a fusion group's (min, max) statistics."""
    gabs = stats[0][1].max()
    for mn, mx in stats:
        gabs = torch.max(gabs, -mn.min())
        gabs = torch.max(gabs, mx.max())
    return generate_gparam(-gabs.reshape(1), gabs.reshape(1))


# ---------------------------------------------------------------- MSE observers
def mse_grid_search(observed: torch.Tensor, args: OArgs, maxshrink: float = 0.20, patience: int = 5,
                    grid: float = 100.0, norm: float = 2.4, return_steps: bool = False):
    """``observers/mse_quant.py:48-130`` (eager): min / max of each group (dims
    0 and -1 reduced) shrunk by p = 1 - i / grid for i < int(maxshrink * grid);
    per group the first pair with the smallest error sum |q - x|^norm (in the
    observed dtype), stopping once ``patience`` consecutive steps improve no
    group.  ``return_steps`` also returns the number of steps evaluated."""
    from dataclasses import replace

    from .fake_quant import fake_quantize

    min_val = torch.amin(observed, dim=(0, -1))
    max_val = torch.amax(observed, dim=(0, -1))
    best_error = torch.full_like(min_val, torch.finfo(min_val.dtype).max)
    best_min, best_max = min_val.clone(), max_val.clone()
    total_steps = int(maxshrink * grid)
    token_args = replace(args, strategy="token")
    no_improve, steps = 0, 0
    for i in range(total_steps):
        steps += 1
        p = 1 - i / grid
        smin, smax = min_val * p, max_val * p
        scale, zp = calculate_qparams(smin, smax, args)
        q = fake_quantize(observed, scale.unsqueeze(-1), zp.unsqueeze(-1), token_args).to(observed.dtype)
        err = torch.sum((q - observed).abs().pow(norm), dim=(0, -1))
        improved = err < best_error
        if torch.any(improved):
            best_error[improved] = err[improved]
            best_min[improved] = smin[improved]
            best_max[improved] = smax[improved]
            no_improve = 0
        else:
            no_improve += 1
            if no_improve >= patience:
                break
    return (best_min, best_max, steps) if return_steps else (best_min, best_max)


class OMSE(OMinMax):
    """``memoryless_mse`` / ``mse`` (``observers/mse.py:12-98``): the grid
    search's min / max as statistics; ``mse`` interpolates later observations
    into them (``helpers.py:219-221``, ``averaging_constant``)."""

    def __init__(self, kind: str, base_name: str, args: OArgs):
        super().__init__(kind, base_name, args)
        kw = args.observer_kwargs or {}
        self.maxshrink, self.patience = kw.get("maxshrink", 0.20), kw.get("patience", 5)
        self.grid, self.norm = kw.get("grid", 100.0), kw.get("norm", 2.4)

    def __call__(self, observed: torch.Tensor):
        if observed.numel() == 0 or (self.base_name == "weight" and self.has_statistics):
            return self
        flat = flatten_weight(observed, self.args) if self.base_name == "weight" else \
            flatten_activation(observed, self.args)
        mn, mx = mse_grid_search(flat, self.args, self.maxshrink, self.patience, self.grid, self.norm)
        if self.kind == "mse" and self.has_statistics and self.avg != 1.0:
            mn = self.min_vals * (1.0 - self.avg) + mn * self.avg
            mx = self.max_vals * (1.0 - self.avg) + mx * self.avg
        self.min_vals, self.max_vals = mn, mx
        return self


# ---------------------------------------------------------------- imatrix MSE observer
def imatrix_grid_search(observed: torch.Tensor, args: OArgs, maxshrink: float = 0.95, patience: int = 5,
                        grid: float = 20, norm: float = 3.0, importance: torch.Tensor | None = None):
    """``observers/imatrix.py:289-440`` (unchunked): as ``mse_grid_search``
    but max(1, int(maxshrink * grid)) + 1 steps, the error |q - x|^norm in
    fp32 (q fake-quantised in the observed dtype) weighted by ``importance``
    (broadcast like ``observed``), summed in fp32, and no early stop when
    patience is 0."""
    from dataclasses import replace

    from .fake_quant import fake_quantize

    min_val = torch.amin(observed, dim=(0, -1))
    max_val = torch.amax(observed, dim=(0, -1))
    best_error = torch.full(min_val.shape, torch.finfo(torch.float32).max, dtype=torch.float32)
    best_min, best_max = min_val.clone(), max_val.clone()
    observed_f = observed.float()
    token_args = replace(args, strategy="token")
    no_improve = 0
    for i in range(max(1, int(maxshrink * grid)) + 1):
        p = 1 - i / grid
        smin, smax = p * min_val, p * max_val
        scale, zp = calculate_qparams(smin, smax, args)
        q = fake_quantize(observed, scale.unsqueeze(-1), zp.unsqueeze(-1), token_args).float()
        q = (q - observed_f).abs().pow(norm)
        if importance is not None:
            q = q * importance.to(torch.float32)
        err = q.sum(dim=(0, -1), dtype=torch.float32)
        improved = err < best_error
        if torch.any(improved):
            best_error[improved] = err[improved]
            best_min[improved] = smin[improved]
            best_max[improved] = smax[improved]
            no_improve = 0
        else:
            no_improve += 1
            if patience > 0 and no_improve >= patience:
                break
    return best_min, best_max


def imatrix_importance(imatrix_sum: torch.Tensor, count: int, observed: torch.Tensor, args: OArgs,
                       base_name: str = "weight"):
    """``observers/imatrix.py:157-283`` (non-strict): E[x^2] = sum / count,
    normalised by its mean, broadcast over the weight's rows and flattened
    like the weight; None (uniform MSE) for non-weight observers, TENSOR and
    unsupported strategies, missing, non-finite, negative, all-zero or
    mis-sized data."""
    if base_name != "weight" or args.strategy == "tensor" or imatrix_sum is None or count == 0:
        return None
    imp = imatrix_sum / torch.tensor(count).float()
    if not torch.isfinite(imp).all() or (imp < 0).any() or torch.all(imp == 0):
        return None
    if args.strategy == "channel":
        expected = observed.shape[-1]
    elif args.strategy in ("group", "tensor_group"):
        expected = observed.shape[2] * observed.shape[3]
    else:
        return None
    if imp.numel() != expected:
        return None
    imp = imp.to(torch.float32)
    imp = imp / (imp.mean() + torch.finfo(torch.float32).tiny)
    return flatten_weight(imp.unsqueeze(0).expand(observed.shape[1], -1), args)
