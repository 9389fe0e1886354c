"""GPTQ Hessian accumulation and solve on the GPU (drop-in functions).

Same names, signatures, return values and error behaviour as
``modifiers/gptq/gptq_quantize.py``:

* ``make_empty_hessian(module, device=None)``                 (``:54-60``)
* ``accumulate_hessian(inp, module, H, num_samples)``          (``:63-97``)
* ``quantize_weight(module, quant_args, hessian, blocksize=128, percdamp=0.01)``
                                                              (``:100-296``)

One documented difference: ``accumulate_hessian`` maintains the upper
triangle of H (diagonal included) and leaves the strictly-lower part as it
was (zero for a matrix from ``make_empty_hessian``).  ``quantize_weight``
reads only the upper triangle, and ``symmetrize_hessian`` restores the full
symmetric matrix when a caller needs it.
"""
from __future__ import annotations

import logging
from dataclasses import dataclass

import torch

from . import _lib, ops
from .quant_args import ActivationOrdering, QuantizationArgs, QuantizationStrategy, QuantizationType, resolve_args

logger = logging.getLogger("llmcompressor_amd")

GPTQ_PRECISION = torch.float32

__all__ = ["make_empty_hessian", "accumulate_hessian", "quantize_weight", "symmetrize_hessian",
           "GPTQResult", "GPTQBatch", "gptq_quantize", "gptq_quantize_batched", "PreparedHessian", "prepare_hessian",
           "prepare_hessians_batched"]


def make_empty_hessian(module: torch.nn.Module, device: torch.device | None = None) -> torch.Tensor:
    weight = module.weight
    num_columns = weight.shape[1]
    device = device if device is not None else weight.device
    return torch.zeros((num_columns, num_columns), device=device, dtype=GPTQ_PRECISION)


def _is_linear_like(module) -> bool:
    if isinstance(module, torch.nn.Linear):
        return True
    return type(module).__name__ == "Conv1D"  # transformers.Conv1D


def conv2d_rows(inp: torch.Tensor, module: torch.nn.Conv2d) -> torch.Tensor:
    """The patches a Conv2d sees, one row each: [batch * positions,
    in_channels * kh * kw] in the order of ``gptq_quantize.py:80-89``'s
    unfold, permute and flatten (the transpose of its columns)."""
    cols = torch.nn.functional.unfold(inp, module.kernel_size, dilation=module.dilation, padding=module.padding,
                                      stride=module.stride)
    return cols.transpose(1, 2).reshape(-1, cols.shape[1])


def hessian_rows(inp: torch.Tensor, module: torch.nn.Module, device) -> tuple[torch.Tensor, int]:
    """The 2-D rows of one accumulation call on ``device`` and the
    reference's sample count for it: the leading dimension after a 2-D input
    is unsqueezed to 3-D (``gptq_quantize.py:72-80``); a Conv2d's input
    becomes its unfolded patches (``:80-89``; its Hessian has in_channels *
    kh * kw columns, which ``make_empty_hessian``'s weight.shape[1] matches
    for 1 x 1 kernels only, as in the reference)."""
    if inp.device != device:
        inp = inp.to(device=device)
    if inp.dim() == 2:
        inp = inp.unsqueeze(0)
    if isinstance(module, torch.nn.Conv2d):
        return conv2d_rows(inp, module), inp.shape[0]
    if not _is_linear_like(module):
        raise NotImplementedError(f"GPTQ Hessian for {type(module).__name__} is not provided by this build")
    return inp.reshape(-1, inp.shape[-1]), inp.shape[0]


def accumulate_hessian(inp: torch.Tensor, module: torch.nn.Module, H: torch.Tensor,
                       num_samples: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """H += 2 * X^T X over the rows of ``inp`` (upper triangle, in place).

    ``num_samples`` grows by the leading dimension after a 2-D input is
    unsqueezed to 3-D, exactly as the reference counts it.
    """
    x, num_added = hessian_rows(inp, module, H.device)
    num_samples += num_added
    if x.shape[0] > 0:
        ops.hessian_syrk_(H, x, alpha=2.0)
    return H, num_samples


def symmetrize_hessian(H: torch.Tensor) -> torch.Tensor:
    """Mirror the upper triangle onto the lower one (in place)."""
    return ops.symmetrize_upper_(H)


@dataclass
class GPTQResult:
    loss: float
    weight: torch.Tensor            # fake-quantised, original dtype, original column order
    scale: torch.Tensor             # as the observer produced it
    zero_point: torch.Tensor
    g_idx: torch.Tensor | None      # reference g_idx in working order (None if no groups)
    perm: torch.Tensor | None
    codes: torch.Tensor             # int8, original column order: integer codes, or the
                                    # float8_e4m3fn bits / e2m1 codes (sign << 3 | grid index)
    hinv_ok: bool
    global_scale: torch.Tensor | None = None   # tensor-group (NVFP4) global scale, fp32 [1]


_SWEEP_STRATEGIES = (QuantizationStrategy.TENSOR, QuantizationStrategy.CHANNEL, QuantizationStrategy.GROUP,
                     QuantizationStrategy.TENSOR_GROUP, QuantizationStrategy.BLOCK)
_GROUPED = (QuantizationStrategy.GROUP, QuantizationStrategy.TENSOR_GROUP)


def _value_type(quant_args: QuantizationArgs) -> str:
    """The sweep's value type: integers, or CT's float8_e4m3fn / fp4 e2m1 grids."""
    if quant_args.strategy not in _SWEEP_STRATEGIES:
        raise ValueError(f"Quantization strategy is not supported for GPTQ: {quant_args.strategy}")
    if quant_args.type == QuantizationType.INT:
        return "int"
    if not quant_args.symmetric:
        raise NotImplementedError("asymmetric float quantization")
    if quant_args.num_bits == 8:
        return "fp8"
    if quant_args.num_bits == 4:
        return "fp4"
    raise NotImplementedError(f"float weights of {quant_args.num_bits} bits")


def _qparams_for_sweep(scale: torch.Tensor, zero_point: torch.Tensor, strategy: QuantizationStrategy,
                       symmetric: bool = False):
    """fp32 scales and zero points shaped for the sweep; symmetric: no zero
    points (the sweep's variant without them)."""
    s = scale.to(torch.float32)
    z = None if symmetric else zero_point.to(torch.float32)
    if strategy == QuantizationStrategy.TENSOR:
        s = s.reshape(1, 1)
        z = None if z is None else z.reshape(1, 1)
    elif s.dim() == 1:
        s = s.reshape(-1, 1)
        z = None if z is None else z.reshape(-1, 1)
    return s.contiguous(), None if z is None else z.contiguous()


@dataclass
class PreparedHessian:
    """The weight-independent part of the solve for one Hessian (or a stack):
    activation-order permutation, dead columns and the upper Cholesky factor of
    the damped inverse, with the RTN fallback already applied on the device
    (hinv = identity where the Hessian is not positive definite).  ``status``
    is the device flag (int32 [1] or [B], 0 = positive definite); it is read
    on the host only after the solve's final synchronisation.  Modules whose
    inputs are the same tensor (q/k/v, gate/up) share it."""
    actorder: ActivationOrdering | None
    perm: torch.Tensor | None
    invperm: torch.Tensor | None
    hinv: torch.Tensor
    dead: torch.Tensor
    status: torch.Tensor

    @property
    def ok(self):
        """Positive definite: a bool (single) or a host bool tensor [B]
        (synchronises)."""
        st = self.status.cpu()
        _lib.check_hinv_status(st.tolist())
        ok = st == 0
        return bool(ok[0]) if ok.numel() == 1 and self.hinv.dim() == 2 else ok


def _effective_actorder(quant_args: QuantizationArgs):
    quant_args = resolve_args(quant_args)
    actorder = quant_args.actorder
    if actorder == ActivationOrdering.GROUP and quant_args.strategy not in (QuantizationStrategy.GROUP,
                                                                            QuantizationStrategy.TENSOR_GROUP):
        logger.warning("ActivationOrdering.GROUP requires a grouped quantization strategy; "
                       "falling back to actorder=None for this module.")
        actorder = None
    return actorder


def _hinv_fallback_warning():
    logger.warning("Failed to invert hessian due to numerical instability. Consider increasing "
                   "GPTQModifier.dampening_frac, increasing the number of calibration samples, or "
                   "shuffling the calibration dataset. Falling back to round-to-nearest for this module.")


def prepare_hessian(hessian: torch.Tensor, quant_args: QuantizationArgs, num_samples: float = 1.0,
                    percdamp: float = 0.01) -> PreparedHessian:
    """Permutation, dead columns and Hinv for one upper-triangle Hessian
    (``gptq_quantize.py:130-196``)."""
    quant_args = resolve_args(quant_args)
    actorder = _effective_actorder(quant_args)
    perm = invperm = None
    if actorder:
        perm = torch.argsort(torch.diagonal(hessian), descending=True, stable=True)
        invperm = torch.argsort(perm)
    hinv, dead, status = ops.gptq_hinv_rtn(hessian, perm, float(num_samples), percdamp)
    return PreparedHessian(actorder, perm, invperm, hinv, dead, status)


def prepare_hessians_batched(hessians: torch.Tensor, quant_args: QuantizationArgs, num_samples=1.0,
                             percdamp: float = 0.01) -> PreparedHessian:
    """``prepare_hessian`` for a stack [B, d, d] (one launch per step)."""
    quant_args = resolve_args(quant_args)
    actorder = _effective_actorder(quant_args)
    B, d, _ = hessians.shape
    ns = torch.as_tensor(num_samples, dtype=torch.float32, device=hessians.device).expand(B).contiguous()
    perm = invperm = None
    if actorder:
        perm = torch.argsort(torch.diagonal(hessians, dim1=1, dim2=2), dim=1, descending=True, stable=True)
        invperm = torch.argsort(perm, dim=1)
    hinv, dead, status = ops.gptq_hinv_batched(hessians, perm, ns, percdamp, sync=False)
    return PreparedHessian(actorder, perm, invperm, hinv, dead, status)


def gptq_quantize(weight: torch.Tensor, quant_args: QuantizationArgs, hessian: torch.Tensor, observer,
                  blocksize: int = 128, percdamp: float = 0.01, num_samples: float = 1.0,
                  prepared: PreparedHessian | None = None) -> GPTQResult:
    """The GPTQ solve of ``gptq_quantize.py:100-296`` on the GPU.

    ``hessian`` is the accumulated upper-triangle Hessian; ``num_samples``
    is divided out inside the kernels (the reference divides before the call,
    ``modifiers/gptq/base.py:594``).  ``observer`` must already hold the
    weight statistics (``observe``), as in the reference.  ``prepared`` (from
    ``prepare_hessian`` on the same Hessian and quantization args) skips the
    Cholesky chain for modules that share their input.  ``quant_args`` is
    this package's ``QuantizationArgs`` or any object with compressed-tensors'
    field names (``resolve_args``).
    """
    quant_args = resolve_args(quant_args)
    strategy = quant_args.strategy
    qtype = _value_type(quant_args)
    W = weight
    rows, cols = W.shape
    prep = prepared if prepared is not None else prepare_hessian(hessian, quant_args, num_samples, percdamp)
    actorder, perm, invperm = prep.actorder, prep.perm, prep.invperm
    if actorder == ActivationOrdering.GROUP:
        observer.delete_statistics(check_fused=False)
        observer(ops.gptq_load_weight(W, perm))   # permuted fp32 weight

    g_idx = None
    if strategy in _GROUPED + (QuantizationStrategy.BLOCK,):
        divisor = quant_args.group_size if strategy != QuantizationStrategy.BLOCK else quant_args.block_structure[1]
        g_idx = torch.arange(cols, device=W.device, dtype=torch.int) // divisor
        if actorder == ActivationOrdering.WEIGHT:
            g_idx = g_idx[perm]

    qp = observer.get_qparams()
    scale, zero_point, global_scale = qp["scale"], qp["zero_point"], qp.get("global_scale")

    hinv, dead = prep.hinv, prep.dead
    w_work = ops.gptq_load_weight(W, perm, dead)
    s, z = _qparams_for_sweep(scale, zero_point, strategy, quant_args.symmetric)
    qmin, qmax = quant_args.q_range()
    bh = quant_args.block_structure[0] if strategy == QuantizationStrategy.BLOCK else 1
    codes, losses = ops.gptq_sweep_(w_work, hinv, s, z, strategy.value, g_idx, qmin, qmax,
                                    dequant_bf16=scale.dtype == torch.bfloat16, blocksize=blocksize, block_h=bh,
                                    qtype=qtype, global_scale=global_scale)
    w_out, codes_out = ops.gptq_store_weight(w_work, invperm, W.dtype, codes)
    loss_st = torch.stack([torch.sum(losses), prep.status[0].float()]).cpu()  # the one sync
    _lib.check_hinv_status([loss_st[1]])
    loss_ok = torch.stack([loss_st[0], (loss_st[1] == 0).float()])
    ok = bool(loss_ok[1])
    if not ok:
        _hinv_fallback_warning()
    return GPTQResult(loss=float(loss_ok[0]), weight=w_out, scale=scale, zero_point=zero_point, g_idx=g_idx,
                      perm=perm, codes=codes_out, hinv_ok=ok, global_scale=global_scale)


@dataclass
class GPTQBatch:
    """The results of a batched solve as stacked tensors (member b at [b]):
    loss and hinv_ok on the host [B], weight [B, rows, cols], scale and
    zero_point [B, rows, groups] (TENSOR: [B, 1, 1]), codes [B, rows, cols],
    g_idx [B, cols] or [cols] or None, perm [B, cols] or None, global_scale
    [B] or None."""
    loss: torch.Tensor
    weight: torch.Tensor
    scale: torch.Tensor
    zero_point: torch.Tensor
    g_idx: torch.Tensor | None
    perm: torch.Tensor | None
    codes: torch.Tensor
    hinv_ok: torch.Tensor
    global_scale: torch.Tensor | None = None


def gptq_quantize_batched(weights: torch.Tensor, quant_args: QuantizationArgs, hessians: torch.Tensor,
                          num_samples=1.0, blocksize: int = 128, percdamp: float = 0.01,
                          observer: str = "memoryless_minmax",
                          prepared: PreparedHessian | None = None, stacked: bool = False):
    """``gptq_quantize`` for B same-shaped modules at once (the experts of an
    MoE layer): weights [B, rows, cols], hessians [B, cols, cols] (upper
    triangles), num_samples a number or [B].  Each module gets the result of
    its own ``gptq_quantize`` call (one launch per step for the whole batch,
    one host synchronisation for the status flags and one for the losses):
    bit for bit while the batch's lazy-update products take the same GEMM
    tile kernel as a single module's, which depends on the total row count;
    otherwise they differ by fp32 summation order.  The weight observer named ``observer`` is run
    here on the stacked weights (its statistics are per row for channel and
    group strategies).  ``prepared`` (``prepare_hessians_batched`` on the same
    stack and args) is shared by projections with the same input (gate, up).
    ``stacked`` returns one ``GPTQBatch`` of stacked tensors instead of the
    list (no per-member Python objects).
    """
    from .observers import Observer

    quant_args = resolve_args(quant_args)
    strategy = quant_args.strategy
    qtype = _value_type(quant_args)
    B, rows, cols = weights.shape
    if hessians.shape != (B, cols, cols):
        raise ValueError(f"hessians must be [{B}, {cols}, {cols}], got {tuple(hessians.shape)}")
    dev = weights.device
    prep = prepared if prepared is not None else prepare_hessians_batched(hessians, quant_args, num_samples,
                                                                          percdamp)
    actorder, perm, invperm = prep.actorder, prep.perm, prep.invperm
    src = ops.gptq_load_weight_batched(weights, perm) if actorder == ActivationOrdering.GROUP else weights

    def observe(x):
        obs = Observer.load_from_registry(observer, base_name="weight", args=quant_args)
        obs(x)
        qp = obs.get_qparams()
        return qp["scale"], qp["zero_point"], qp.get("global_scale")

    # per-row statistics observe the stacked weights at once; tensor-wide
    # ones (tensor scales, tensor-group global scales) member by member
    stackable = strategy in (QuantizationStrategy.CHANNEL, QuantizationStrategy.GROUP) or (
        strategy == QuantizationStrategy.BLOCK and rows % quant_args.block_structure[0] == 0)
    global_scale = None
    if stackable:
        sc, zp, _ = observe(src.reshape(B * rows, cols))
        scale, zero_point = sc.reshape(B, -1, sc.shape[-1]), zp.reshape(B, -1, zp.shape[-1])
    else:
        qps = [observe(src[b]) for b in range(B)]
        scale = torch.stack([q[0] for q in qps]).reshape(B, 1, 1) if strategy == QuantizationStrategy.TENSOR \
            else torch.stack([q[0] for q in qps])
        zero_point = torch.stack([q[1] for q in qps]).reshape(scale.shape)
        if qps[0][2] is not None:
            global_scale = torch.cat([q[2].reshape(1) for q in qps])

    g_idx = None
    if strategy in _GROUPED + (QuantizationStrategy.BLOCK,):
        divisor = quant_args.group_size if strategy != QuantizationStrategy.BLOCK else quant_args.block_structure[1]
        g_idx = torch.arange(cols, device=dev, dtype=torch.int) // divisor
        if actorder == ActivationOrdering.WEIGHT:
            g_idx = g_idx[perm]

    hinv, dead = prep.hinv, prep.dead
    w_work = ops.gptq_load_weight_batched(weights, perm, dead)
    qmin, qmax = quant_args.q_range()
    bh = quant_args.block_structure[0] if strategy == QuantizationStrategy.BLOCK else 1
    codes, losses = ops.gptq_sweep_batched_(w_work, hinv, scale.to(torch.float32),
                                            None if quant_args.symmetric else zero_point.to(torch.float32),
                                            strategy.value, g_idx, qmin, qmax,
                                            dequant_bf16=scale.dtype == torch.bfloat16, blocksize=blocksize,
                                            block_h=bh, qtype=qtype, global_scale=global_scale)
    w_out, codes_out = ops.gptq_store_weight_batched(w_work, invperm, weights.dtype, codes)
    loss_st = torch.stack([torch.sum(losses, dim=1), prep.status.float()]).cpu()  # the one sync
    _lib.check_hinv_status(loss_st[1].tolist())
    loss, ok = loss_st[0], loss_st[1] == 0
    for _ in range(int((~ok).sum())):
        _hinv_fallback_warning()
    if stacked:
        return GPTQBatch(loss=loss, weight=w_out, scale=scale, zero_point=zero_point, g_idx=g_idx, perm=perm,
                         codes=codes_out, hinv_ok=ok, global_scale=global_scale)
    out = []
    for b in range(B):
        sb, zb = scale[b], zero_point[b]
        if strategy == QuantizationStrategy.TENSOR:
            sb, zb = sb.reshape(-1), zb.reshape(-1)
        out.append(GPTQResult(loss=float(loss[b]), weight=w_out[b], scale=sb, zero_point=zb,
                              g_idx=None if g_idx is None else (g_idx[b] if g_idx.dim() == 2 else g_idx),
                              perm=None if perm is None else perm[b], codes=codes_out[b], hinv_ok=bool(ok[b]),
                              global_scale=None if global_scale is None else global_scale[b:b + 1]))
    return out


def quantize_weight(module: torch.nn.Module, quant_args: QuantizationArgs, hessian: torch.Tensor,
                    blocksize: int = 128, percdamp: float = 0.01):
    """Drop-in for ``gptq_quantize.quantize_weight``: returns ``(loss, q_param_dict)``.

    ``quant_args`` may be compressed-tensors' ``QuantizationArgs`` (as
    ``modifiers/gptq/base.py:591-597`` passes it) or any object with its
    field names; only ``CT_ARG_FIELDS`` are read.  ``module.weight_observer``
    is used through ``__call__``, ``get_qparams()`` and
    ``delete_statistics(check_fused=False)`` only, as ``gptq_quantize.py:145-172``
    uses it."""
    zp_dtype = getattr(quant_args, "zp_dtype", None)
    qa = resolve_args(quant_args)
    res = gptq_quantize(module.weight, qa, hessian, module.weight_observer, blocksize, percdamp)
    final_dtype = module.weight.dtype
    q = {
        "weight": res.weight.reshape(module.weight.shape),
        "weight_scale": res.scale.to(dtype=final_dtype),
        "weight_zero_point": res.zero_point.to(dtype=zp_dtype if zp_dtype is not None else qa.zp_dtype),
    }
    if res.global_scale is not None:
        q["weight_global_scale"] = res.global_scale.to(dtype=final_dtype)
    if qa.actorder == ActivationOrdering.GROUP and qa.strategy in _GROUPED:
        q["weight_g_idx"] = res.g_idx[torch.argsort(res.perm)]
    return res.loss, q
