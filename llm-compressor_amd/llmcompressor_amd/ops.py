"""Tensor-level wrappers of the libmi355q kernels.

Each function validates shapes, allocates outputs and workspaces with the
torch caching allocator on the inputs' device, and launches on torch's
current stream.  All tensors must live on a ROCm GPU; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib as L


def _dt(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return L.BF16
    if t.dtype == torch.float32:
        return L.F32
    raise TypeError(f"unsupported dtype {t.dtype} (bf16 or fp32)")


def _ws(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


# ---------------------------------------------------------------- Hessian
_HESS_DT = {torch.bfloat16: L.BF16, torch.float16: L.F16, torch.float32: L.F32}


def _hessian_input(x: torch.Tensor) -> torch.Tensor:
    """x as a row-major 2-D matrix of a type the Hessian kernels take: bf16 and
    fp16 as they are (16-byte aligned rows, a multiple of 8 features), any
    other floating type - and 16-bit inputs whose width is not a multiple
    of 8 - converted to fp32, as the reference converts every input
    (gptq_quantize.py:93)."""
    if not x.dtype.is_floating_point:
        raise TypeError(f"hessian input must be a floating-point tensor, got {x.dtype}")
    if x.dim() != 2 or x.stride(1) != 1:
        x = x.reshape(-1, x.shape[-1]).contiguous()
    if x.dtype not in _HESS_DT or (x.dtype != torch.float32 and x.shape[1] % 8):
        x = x.to(torch.float32)
    if x.dtype != torch.float32 and (x.data_ptr() % 16 or x.stride(0) % 8):
        x = x.contiguous()
    return x


def hessian_syrk_(H: torch.Tensor, x: torch.Tensor, alpha: float = 2.0, beta: float = 1.0) -> torch.Tensor:
    """H[i, j] = beta * H[i, j] + alpha * sum_t x[t, i] x[t, j] for i <= j, in
    place (beta == 1: H += ...).

    ``x`` is [tokens, d] (row stride may exceed d) bf16 or fp16 (16-bit MFMA,
    exact products) or fp32 (fp32 MFMA); other floating types are converted
    to fp32.  H is fp32 [d, d].
    """
    L.require_gpu(H, x)
    x = _hessian_input(x)
    n, d = x.shape
    if H.dtype != torch.float32 or H.shape != (d, d) or H.stride(1) != 1:
        raise ValueError(f"H must be fp32 [{d}, {d}] row-major, got {tuple(H.shape)} {H.dtype}")
    lib = L.lib()
    dt = _HESS_DT[x.dtype]
    ws = _ws(lib.mi355q_hessian_syrk_workspace_size(n, d, dt), x.device)
    L.check(lib.mi355q_hessian_syrk(x.data_ptr(), dt, n, d, x.stride(0), H.data_ptr(), H.stride(0), C.c_float(alpha),
                                    C.c_float(beta), L.ptr(ws), 0 if ws is None else ws.numel(), L.stream_of(x)))
    return H


def hessian_syrk_segments_(H: torch.Tensor, xs, alpha: float = 2.0, beta: float = 1.0) -> torch.Tensor:
    """``hessian_syrk_`` over the rows of several [n_k, d] tensors at once:
    H = beta * H + alpha * sum_k X_k^T X_k (upper triangle, in place), the
    sum a single call over their concatenation forms (segments of
    multiples of 32 rows: bit for bit) without the concatenation.  16-bit
    segments sharing one dtype and row stride run in one launch per 64
    segments; others take one ``hessian_syrk_`` per segment."""
    xs = [_hessian_input(x) for x in xs]
    if len(xs) == 1:
        return hessian_syrk_(H, xs[0], alpha=alpha, beta=beta)
    L.require_gpu(H, *xs)
    d = H.shape[-1]
    if any(x.shape[1] != d for x in xs):
        raise ValueError(f"every segment needs {d} columns, got {[tuple(x.shape) for x in xs]}")
    if H.dtype != torch.float32 or H.shape != (d, d) or H.stride(1) != 1:
        raise ValueError(f"H must be fp32 [{d}, {d}] row-major, got {tuple(H.shape)} {H.dtype}")
    dts = {x.dtype for x in xs}
    ldx = {x.stride(0) for x in xs if x.shape[0] > 0}
    if len(dts) != 1 or len(ldx) > 1 or xs[0].dtype == torch.float32 or any(x.device != H.device for x in xs):
        b = beta
        for x in xs:
            if x.shape[0] > 0 or x is xs[-1]:
                hessian_syrk_(H, x, alpha=alpha, beta=b)
                b = 1.0
        return H
    lib = L.lib()
    dt = _HESS_DT[xs[0].dtype]
    n = len(xs)
    ptrs = (C.c_void_p * n)(*[x.data_ptr() for x in xs])
    rows = (C.c_int64 * n)(*[x.shape[0] for x in xs])
    ws = _ws(lib.mi355q_hessian_syrk_segments_workspace_size(rows, n, d, dt), H.device)
    L.check(lib.mi355q_hessian_syrk_segments(ptrs, rows, n, dt, d, ldx.pop() if ldx else d, H.data_ptr(), H.stride(0),
                                             C.c_float(alpha), C.c_float(beta), L.ptr(ws),
                                             0 if ws is None else ws.numel(), L.stream_of(xs[0])))
    return H


def hessian_grouped_syrk_(H: torch.Tensor, x: torch.Tensor, rows: torch.Tensor | None, offsets,
                          alpha: float = 2.0, beta: float = 1.0) -> torch.Tensor:
    """Per-group upper-triangle syrk: H[e] = beta * H[e] + alpha * X_e^T X_e
    where X_e are the rows ``x[rows[offsets[e]:offsets[e+1]]]`` (``rows``
    None: the rows ``x[offsets[e]:offsets[e+1]]``).  H is [E, d, d] fp32;
    ``offsets`` a list or an int64 tensor of E + 1 non-decreasing entries.
    ``beta`` is 1 (add) or 0: H's upper triangle is written without being
    read (a freshly allocated H need not be zeroed; groups without rows get
    zeros).  bf16 and fp16 ``x`` take one grouped launch whose work table is
    built on the device; other types are converted to fp32 and each group's
    rows take the dense fp32 product."""
    if beta not in (0.0, 1.0):
        raise ValueError("beta must be 0 or 1")
    L.require_gpu(H, x)
    if isinstance(offsets, torch.Tensor):
        off_dev = offsets.to(device=x.device, dtype=torch.int64).contiguous()
        E = off_dev.numel() - 1
        off_list = None
    else:
        off_list = [int(o) for o in offsets]
        E = len(off_list) - 1
        if any(b < a for a, b in zip(off_list, off_list[1:])) or (off_list and off_list[0] < 0):
            raise ValueError("offsets must be non-negative and non-decreasing")
        off_dev = None
    x = _hessian_input(x)
    n_x, d = x.shape
    n_rows = n_x if rows is None else rows.numel()
    if off_list is not None and off_list[-1] > n_rows:
        raise ValueError(f"offsets end at {off_list[-1]} > {n_rows} rows")
    if H.shape != (E, d, d) or H.dtype != torch.float32 or not H.is_contiguous():
        raise ValueError(f"H must be contiguous fp32 [{E}, {d}, {d}]")
    if x.dtype == torch.float32:
        offs = off_list if off_list is not None else off_dev.tolist()
        for e in range(E):
            if offs[e + 1] > offs[e]:
                xe = x[offs[e]:offs[e + 1]] if rows is None else x[rows[offs[e]:offs[e + 1]].long()]
                if beta == 0.0:
                    H[e].zero_()
                hessian_syrk_(H[e], xe, alpha=alpha)
            elif beta == 0.0:
                H[e].zero_()
        return H
    if rows is not None:
        L.require_gpu(rows)
        rows = rows.to(torch.int32).contiguous()
    if off_dev is None:
        off_dev = torch.tensor(off_list, dtype=torch.int64).to(x.device, non_blocking=True)
    lib = L.lib()
    ws = _ws(lib.mi355q_hessian_grouped_syrk_workspace_size(n_rows, E, d), x.device)
    L.check(lib.mi355q_hessian_grouped_syrk(x.data_ptr(), _HESS_DT[x.dtype], n_x, x.stride(0), d,
                                            None if rows is None else rows.data_ptr(), n_rows, off_dev.data_ptr(),
                                            E, H.data_ptr(), d * d, C.c_float(alpha), C.c_float(beta), L.ptr(ws),
                                            0 if ws is None else ws.numel(), L.stream_of(x)))
    return H


def symmetrize_upper_(H: torch.Tensor) -> torch.Tensor:
    """Copy the upper triangle onto the lower one, in place."""
    L.require_gpu(H)
    d = H.shape[0]
    L.call("mi355q_symmetrize_upper", H.data_ptr(), d, H.stride(0), L.stream_of(H))
    return H


# ---------------------------------------------------------------- GPTQ pieces
def _row_major_square(H: torch.Tensor) -> torch.Tensor:
    """H as a row-major fp32 square matrix (rows may be padded): the kernels
    read H[i][j] at i * ldh + j."""
    if H.dim() != 2 or H.shape[0] != H.shape[1] or H.dtype != torch.float32:
        raise ValueError(f"H must be a square fp32 matrix, got {tuple(H.shape)} {H.dtype}")
    return H if H.stride(1) == 1 and H.stride(0) >= H.shape[1] else H.contiguous()


def gptq_hinv(H: torch.Tensor, perm: torch.Tensor | None, num_samples: float, percdamp: float):
    """Upper Cholesky factor of inverse(damped H / num_samples).

    Returns (hinv [d, d] fp32, dead [d] int32, positive_definite: bool).
    Synchronises once to read the status flag.
    """
    L.require_gpu(H)
    H = _row_major_square(H)
    d = H.shape[0]
    dev = H.device
    hinv = torch.empty((d, d), dtype=torch.float32, device=dev)
    dead = torch.empty(d, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    lib = L.lib()
    ws = _ws(lib.mi355q_gptq_hinv_workspace_size(d), dev)
    p = None if perm is None else perm.to(torch.int32).contiguous()
    L.check(lib.mi355q_gptq_hinv(H.data_ptr(), H.stride(0), d, L.ptr(p), C.c_float(num_samples),
                                 C.c_float(percdamp), hinv.data_ptr(), dead.data_ptr(), status.data_ptr(),
                                 ws.data_ptr(), ws.numel(), L.stream_of(H)))
    st = int(status.item())
    L.check_hinv_status([st])
    return hinv, dead, st == 0


def gptq_hinv_rtn(H: torch.Tensor, perm: torch.Tensor | None, num_samples: float, percdamp: float):
    """``gptq_hinv`` without a host synchronisation: a Hessian that is not
    positive definite gets hinv = identity on the device (the reference's
    round-to-nearest fallback).  Returns (hinv, dead, status [1] int32 on the
    device, 0 = positive definite)."""
    L.require_gpu(H)
    H = _row_major_square(H)
    d = H.shape[0]
    dev = H.device
    hinv = torch.empty((d, d), dtype=torch.float32, device=dev)
    dead = torch.empty(d, dtype=torch.int32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    lib = L.lib()
    ws = _ws(lib.mi355q_gptq_hinv_workspace_size(d), dev)
    p = None if perm is None else perm.to(torch.int32).contiguous()
    L.check(lib.mi355q_gptq_hinv(H.data_ptr(), H.stride(0), d, L.ptr(p), C.c_float(num_samples),
                                 C.c_float(percdamp), hinv.data_ptr(), dead.data_ptr(), status.data_ptr(),
                                 ws.data_ptr(), ws.numel(), L.stream_of(H)))
    L.call("mi355q_gptq_hinv_fallback", hinv.data_ptr(), d, d * d, 1, status.data_ptr(), L.stream_of(H))
    return hinv, dead, status


def gptq_load_weight(w: torch.Tensor, perm=None, dead=None) -> torch.Tensor:
    L.require_gpu(w)
    rows, cols = w.shape
    out = torch.empty((rows, cols), dtype=torch.float32, device=w.device)
    p = None if perm is None else perm.to(torch.int32).contiguous()
    dd = None if dead is None else dead.to(torch.int32).contiguous()
    L.call("mi355q_gptq_load_weight", w.data_ptr(), _dt(w), rows, cols, w.stride(0), L.ptr(p), L.ptr(dd),
           out.data_ptr(), L.stream_of(w))
    return out


STRATEGY_CODE = {"tensor": L.TENSOR, "channel": L.CHANNEL, "group": L.GROUP, "tensor_group": L.GROUP,
                 "block": L.BLOCK, "token": L.TOKEN}


QTYPE = {"int": L.QTYPE_INT, "fp8": L.QTYPE_FP8_E4M3, "fp4": L.QTYPE_FP4_E2M1, "mxfp4_ct": L.QTYPE_MXFP4_CT,
         "mxfp4_ocp": L.QTYPE_MXFP4_OCP}


def gptq_sweep_(w_work: torch.Tensor, hinv: torch.Tensor, scale: torch.Tensor, zero_point, strategy: str,
                g_idx: torch.Tensor | None, qmin: float, qmax: float, dequant_bf16: bool,
                blocksize: int = 128, block_h: int = 1, qtype: str = "int",
                global_scale: torch.Tensor | None = None):
    """In-place GPTQ column sweep.  Returns (codes int8 [rows, cols], losses
    fp32 [rows]); ``qtype`` int / fp8 / fp4 (codes: integers, e4m3 bits, e2m1
    codes), ``global_scale`` (fp32 [1]) divides the scales (tensor groups)."""
    L.require_gpu(w_work, hinv, scale)
    rows, cols = w_work.shape
    if hinv.shape != (cols, cols) or hinv.dtype != torch.float32:
        raise ValueError(f"hinv must be fp32 [{cols}, {cols}], got {tuple(hinv.shape)} {hinv.dtype}")
    s = scale.to(torch.float32).contiguous()
    if s.dim() == 1:
        s = s.reshape(-1, 1)
    z = None if zero_point is None else \
        zero_point.to(device=w_work.device, dtype=torch.float32).reshape(s.shape).contiguous()
    return gptq_sweep_batched_(w_work.unsqueeze(0), hinv.unsqueeze(0), s.unsqueeze(0),
                               None if z is None else z.unsqueeze(0), strategy, g_idx, qmin, qmax, dequant_bf16,
                               blocksize, block_h, qtype, global_scale, _unbatch=True)


def gptq_store_weight(w_work: torch.Tensor, invperm, out_dtype: torch.dtype, codes=None):
    rows, cols = w_work.shape
    out = torch.empty((rows, cols), dtype=out_dtype, device=w_work.device)
    ip = None if invperm is None else invperm.to(torch.int32).contiguous()
    cout = None if codes is None else torch.empty_like(codes)
    L.call("mi355q_gptq_store_weight", w_work.data_ptr(), rows, cols, L.ptr(ip), out.data_ptr(), _dt(out),
           out.stride(0), L.ptr(codes), L.ptr(cout), L.stream_of(w_work))
    return out, cout


# ---------------------------------------------------------------- batched GPTQ
def gptq_hinv_batched(H: torch.Tensor, perm: torch.Tensor | None, num_samples: torch.Tensor, percdamp: float,
                      sync: bool = True):
    """``gptq_hinv`` for a stack H [B, d, d] of same-order Hessians (perm [B, d]
    or None, num_samples [B]).  Returns (hinv [B, d, d], dead [B, d], ok
    [B] bool tensor on the host); synchronises once.  With ``sync=False``:
    no synchronisation, members that are not positive definite get
    hinv = identity on the device, and the third value is the status [B]
    int32 device tensor (0 = positive definite)."""
    L.require_gpu(H)
    if H.dim() != 3 or H.shape[1] != H.shape[2] or H.dtype != torch.float32:
        raise ValueError(f"H must be a stack of square fp32 matrices, got {tuple(H.shape)} {H.dtype}")
    if H.stride(2) != 1 or H.stride(1) < H.shape[2] or H.stride(0) < H.stride(1) * H.shape[1]:
        H = H.contiguous()
    B, d, _ = H.shape
    dev = H.device
    hinv = torch.empty((B, d, d), dtype=torch.float32, device=dev)
    dead = torch.empty((B, d), dtype=torch.int32, device=dev)
    status = torch.zeros(B, dtype=torch.int32, device=dev)
    ns = num_samples.to(device=dev, dtype=torch.float32).reshape(B).contiguous()
    lib = L.lib()
    ws = _ws(lib.mi355q_gptq_hinv_workspace_size(d) * B, dev)
    p = None if perm is None else perm.to(torch.int32).reshape(B, d).contiguous()
    L.check(lib.mi355q_gptq_hinv_batched(H.data_ptr(), H.stride(1), H.stride(0), d, B, L.ptr(p),
                                         0 if p is None else d, ns.data_ptr(), C.c_float(percdamp),
                                         hinv.data_ptr(), d * d, dead.data_ptr(), status.data_ptr(),
                                         ws.data_ptr(), ws.numel(), L.stream_of(H)))
    if not sync:
        L.call("mi355q_gptq_hinv_fallback", hinv.data_ptr(), d, d * d, B, status.data_ptr(), L.stream_of(H))
        return hinv, dead, status
    st = status.cpu()
    L.check_hinv_status(st.tolist())
    return hinv, dead, st == 0


def gptq_load_weight_batched(w: torch.Tensor, perm=None, dead=None) -> torch.Tensor:
    L.require_gpu(w)
    B, rows, cols = w.shape
    out = torch.empty((B, rows, cols), dtype=torch.float32, device=w.device)
    p = None if perm is None else perm.to(torch.int32).reshape(B, cols).contiguous()
    dd = None if dead is None else dead.to(torch.int32).reshape(B, cols).contiguous()
    L.call("mi355q_gptq_load_weight_batched", w.data_ptr(), _dt(w), rows, cols, w.stride(1), w.stride(0), B,
           L.ptr(p), 0 if p is None else cols, L.ptr(dd), out.data_ptr(), L.stream_of(w))
    return out


def gptq_sweep_batched_(w_work: torch.Tensor, hinv: torch.Tensor, scale: torch.Tensor, zero_point, strategy: str,
                        g_idx: torch.Tensor | None, qmin: float, qmax: float, dequant_bf16: bool,
                        blocksize: int = 128, block_h: int = 1, qtype: str = "int",
                        global_scale: torch.Tensor | None = None, _unbatch: bool = False):
    """``gptq_sweep_`` over a batch: w_work [B, rows, cols], hinv [B, cols, cols],
    scale / zero_point [B, rows or 1, groups], g_idx [B, cols] or [cols] (shared),
    global_scale [B] (or one value for all)."""
    L.require_gpu(w_work, hinv, scale)
    B, rows, cols = w_work.shape
    dev = w_work.device
    if hinv.shape != (B, cols, cols) or hinv.dtype != torch.float32:
        raise ValueError(f"hinv must be fp32 [{B}, {cols}, {cols}], got {tuple(hinv.shape)} {hinv.dtype}")
    if hinv.stride(2) != 1 or hinv.stride(1) != cols:
        hinv = hinv.contiguous()   # row-major matrices, any batch stride
    s = scale.to(torch.float32).reshape(B, -1, scale.shape[-1] if scale.dim() == 3 else 1).contiguous()
    z = None if zero_point is None else zero_point.to(device=dev, dtype=torch.float32).reshape(s.shape).contiguous()
    gi = None if g_idx is None else g_idx.to(device=dev, dtype=torch.int32).contiguous()
    gs = None
    if global_scale is not None:
        gs = global_scale.to(device=dev, dtype=torch.float32).reshape(-1)
        gs = (gs.expand(B) if gs.numel() == 1 else gs).contiguous()
    codes = torch.empty((B, rows, cols), dtype=torch.int8, device=dev)
    losses = torch.zeros((B, rows), dtype=torch.float32, device=dev)
    lib = L.lib()
    ws = _ws(lib.mi355q_gptq_sweep_workspace_size(rows, cols, blocksize) * B, dev)
    L.check(lib.mi355q_gptq_sweep_typed_batched(
        w_work.data_ptr(), rows, cols, B, hinv.data_ptr(), hinv.stride(0), s.data_ptr(), L.ptr(z), s.stride(1),
        s.stride(0), L.ptr(gi), 0 if gi is None or gi.dim() == 1 else gi.stride(0), STRATEGY_CODE[strategy],
        block_h, QTYPE[qtype], C.c_float(qmin), C.c_float(qmax), L.ptr(gs), 1 if dequant_bf16 else 0, blocksize,
        codes.data_ptr(), losses.data_ptr(), ws.data_ptr(), ws.numel(), L.stream_of(w_work)))
    if _unbatch:
        return codes[0], losses[0]
    return codes, losses


def gptq_store_weight_batched(w_work: torch.Tensor, invperm, out_dtype: torch.dtype, codes=None):
    B, rows, cols = w_work.shape
    out = torch.empty((B, rows, cols), dtype=out_dtype, device=w_work.device)
    ip = None if invperm is None else invperm.to(torch.int32).reshape(B, cols).contiguous()
    cout = None if codes is None else torch.empty_like(codes)
    L.call("mi355q_gptq_store_weight_batched", w_work.data_ptr(), rows, cols, B, L.ptr(ip),
           0 if ip is None else cols, out.data_ptr(), _dt(out), out.stride(1), out.stride(0), L.ptr(codes),
           L.ptr(cout), L.stream_of(w_work))
    return out, cout


# ---------------------------------------------------------------- observers
def observe_minmax(x: torch.Tensor, strategy: str, group_size: int | None = None,
                   block_structure=None):
    """Min/max statistics of a 2-D tensor per strategy, as fp32 tensors.

    Shapes: tensor -> [1]; channel/token -> [rows, 1]; group ->
    [rows, cols / group]; block -> [ceil(rows/bh), ceil(cols/bw)].
    """
    L.require_gpu(x)
    if x.dim() != 2:
        raise ValueError("observe_minmax expects a 2-D tensor")
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, cols = x.shape
    bh = bw = 1
    if strategy == "tensor":
        shape = (1,)
    elif strategy in ("channel", "token"):
        shape = (rows, 1)
    elif strategy in ("group", "tensor_group"):
        if not group_size or cols % group_size:
            raise ValueError(f"columns ({cols}) must be divisible by group_size ({group_size})")
        shape = (rows, cols // group_size)
    elif strategy == "block":
        bh, bw = block_structure
        shape = (-(-rows // bh), -(-cols // bw))
    else:
        raise ValueError(f"unknown strategy {strategy}")
    mn = torch.empty(shape, dtype=torch.float32, device=x.device)
    mx = torch.empty(shape, dtype=torch.float32, device=x.device)
    L.call("mi355q_observe_minmax", x.data_ptr(), _dt(x), rows, cols, x.stride(0), STRATEGY_CODE[strategy],
           group_size or 0, bh, bw, mn.data_ptr(), mx.data_ptr(), L.stream_of(x))
    return mn, mx


def calculate_qparams(mn: torch.Tensor, mx: torch.Tensor, qmin: float, qmax: float, symmetric: bool,
                      scale_dtype: torch.dtype, strict: bool = False):
    """Scale / zero-point from min/max statistics (fp32 outputs holding
    ``scale_dtype`` values and integer zero-points)."""
    L.require_gpu(mn, mx)
    mn = mn.to(torch.float32).contiguous()
    mx = mx.to(torch.float32).contiguous()
    scale = torch.empty_like(mn)
    zp = torch.empty_like(mn)
    L.call("mi355q_calculate_qparams", mn.data_ptr(), mx.data_ptr(), mn.numel(), C.c_float(qmin),
           C.c_float(qmax), 1 if symmetric else 0, 1 if strict else 0,
           L.BF16 if scale_dtype == torch.bfloat16 else L.F32, scale.data_ptr(), zp.data_ptr(), L.stream_of(mn))
    return scale, zp


MX_RULES = {"ct": L.MX_RULE_CT, "ocp": L.MX_RULE_OCP}


def mx_scales(mn: torch.Tensor, mx: torch.Tensor, rule: str = "ct"):
    """(e8m0 uint8, 2^(e-127) fp32) per group from min/max statistics."""
    L.require_gpu(mn, mx)
    mn = mn.to(torch.float32).contiguous()
    mx = mx.to(torch.float32).contiguous()
    e8 = torch.empty(mn.shape, dtype=torch.uint8, device=mn.device)
    sc = torch.empty_like(mn)
    L.call("mi355q_mx_scales", mn.data_ptr(), mx.data_ptr(), mn.numel(), MX_RULES[rule], e8.data_ptr(),
           sc.data_ptr(), L.stream_of(mn))
    return e8, sc


def nvfp4_qparams(mn: torch.Tensor, mx: torch.Tensor, stats_dtype: torch.dtype):
    """NVFP4 tensor-group qparams from group min / max statistics: (global
    scale fp32 [1], group scales as float8_e4m3fn shaped like ``mn``)."""
    L.require_gpu(mn, mx)
    mn = mn.to(torch.float32).contiguous()
    mx = mx.to(torch.float32).contiguous()
    gs = torch.empty(1, dtype=torch.float32, device=mn.device)
    bits = torch.empty(mn.shape, dtype=torch.uint8, device=mn.device)
    L.call("mi355q_nvfp4_qparams", mn.data_ptr(), mx.data_ptr(), mn.numel(),
           L.BF16 if stats_dtype == torch.bfloat16 else L.F32, gs.data_ptr(), None, bits.data_ptr(), L.stream_of(mn))
    return gs, bits.view(torch.float8_e4m3fn)


# ---------------------------------------------------------------- quantize / pack
def quantize_int(x: torch.Tensor, scale: torch.Tensor, zero_point, strategy: str, num_bits: int,
                 group_size: int | None = None, g_idx=None, block_structure=None,
                 div_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Integer codes (int8) of ``x`` with CT quantize arithmetic."""
    L.require_gpu(x, scale)
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, cols = x.shape
    s = scale.to(torch.float32).contiguous()
    s2 = s.reshape(-1, 1) if s.dim() < 2 else s
    z = None if zero_point is None else \
        zero_point.to(device=x.device, dtype=torch.float32).reshape(s2.shape).contiguous()
    gi = None if g_idx is None else g_idx.to(device=x.device, dtype=torch.int32).contiguous()
    bh, bw = block_structure if block_structure else (1, 1)
    if div_dtype is None:
        div_dtype = torch.promote_types(x.dtype, scale.dtype)
    out = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    L.call("mi355q_quantize_int", x.data_ptr(), _dt(x), rows, cols, x.stride(0), s2.data_ptr(), L.ptr(z),
           s2.stride(0), L.ptr(gi), STRATEGY_CODE[strategy], group_size or 0, bh, bw, num_bits,
           L.BF16 if div_dtype == torch.bfloat16 else L.F32, out.data_ptr(), L.stream_of(x))
    return out


def pack_int4_int32(codes: torch.Tensor) -> torch.Tensor:
    L.require_gpu(codes)
    codes = codes.contiguous()
    rows, cols = codes.shape
    out = torch.empty((rows, cols // 8), dtype=torch.int32, device=codes.device)
    L.call("mi355q_pack_int4_int32", codes.data_ptr(), rows, cols, out.data_ptr(), L.stream_of(codes))
    return out


def observe_mse(x: torch.Tensor, cell_rows: int, cell_cols: int, mn: torch.Tensor, mx: torch.Tensor, qmin: float,
                qmax: float, symmetric: bool, total_steps: int, patience: int, grid: float, norm: float,
                importance: torch.Tensor | None = None, imatrix: bool = False, qtype: str = "int"):
    """MSE grid search over the cells of x (``mi355q_observe_mse``, or with
    ``imatrix`` ``mi355q_observe_imatrix_mse`` weighted by ``importance``
    [cols]) on the integer grid or, with ``qtype="fp8"``, the fp8 e4m3 grid:
    returns the chosen (min, max) per cell as fp32 tensors shaped like
    ``mn``."""
    L.require_gpu(x, mn, mx, importance)
    if x.dim() != 2 or x.stride(1) != 1:
        x = x.reshape(-1, x.shape[-1]).contiguous()
    rows, cols = x.shape
    mn32, mx32 = mn.to(torch.float32).contiguous(), mx.to(torch.float32).contiguous()
    out_mn, out_mx = torch.empty_like(mn32), torch.empty_like(mx32)
    lib = L.lib()
    ws = _ws(lib.mi355q_observe_mse_workspace_size(rows, cols, cell_rows, cell_cols, total_steps), x.device)
    common = (x.data_ptr(), _dt(x), rows, cols, x.stride(0), cell_rows, cell_cols, C.c_float(qmin), C.c_float(qmax),
              1 if symmetric else 0, QTYPE[qtype], int(total_steps), int(patience), C.c_double(grid), C.c_float(norm))
    tail = (mn32.data_ptr(), mx32.data_ptr(), out_mn.data_ptr(), out_mx.data_ptr(), L.ptr(ws),
            0 if ws is None else ws.numel(), L.stream_of(x))
    if imatrix:
        imp = None if importance is None else importance.to(torch.float32).contiguous()
        if imp is not None and imp.numel() != cols:
            raise ValueError(f"importance must have {cols} entries, got {imp.numel()}")
        L.check(lib.mi355q_observe_imatrix_mse(*common, L.ptr(imp), *tail))
    else:
        L.check(lib.mi355q_observe_mse(*common, *tail))
    return out_mn, out_mx


def column_sumsq_(x: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out[c] += sum over rows of x[:, c]^2 (fp32 accumulation), in place."""
    L.require_gpu(x, out)
    if x.dim() != 2 or x.stride(1) != 1:
        x = x.reshape(-1, x.shape[-1]).contiguous()
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.to(torch.float32)
    rows, cols = x.shape
    if out.dtype != torch.float32 or out.numel() != cols or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 vector of {cols}")
    lib = L.lib()
    ws = _ws(lib.mi355q_column_sumsq_workspace_size(rows, cols), x.device)
    L.check(lib.mi355q_column_sumsq(x.data_ptr() if rows else None, _dt(x), rows, cols, x.stride(0), out.data_ptr(),
                                    L.ptr(ws), 0 if ws is None else ws.numel(), L.stream_of(x)))
    return out


def pack_int32(codes: torch.Tensor, num_bits: int) -> torch.Tensor:
    """CT pack_to_int32 layout for 2-, 4- or 8-bit codes (rows padded with 0)."""
    L.require_gpu(codes)
    codes = codes.contiguous()
    rows, cols = codes.shape
    pf = 32 // num_bits
    out = torch.empty((rows, -(-cols // pf)), dtype=torch.int32, device=codes.device)
    L.call("mi355q_pack_int32", codes.data_ptr(), rows, cols, int(num_bits), out.data_ptr(), L.stream_of(codes))
    return out


def pack_int4_int8(codes: torch.Tensor) -> torch.Tensor:
    L.require_gpu(codes)
    if codes.dim() != 2:
        raise ValueError(f"Expected 2D tensor, but got {codes.dim()}D")
    rows, cols = codes.shape
    if cols % 2:
        raise ValueError(f"Expected even number of columns for int4 packing, but got shape {tuple(codes.shape)}")
    codes = codes.contiguous()
    out = torch.empty((rows, cols // 2), dtype=torch.int8, device=codes.device)
    L.call("mi355q_pack_int4_int8", codes.data_ptr(), rows, cols, out.data_ptr(), L.stream_of(codes))
    return out


def mxfp4_quantize_pack(x: torch.Tensor, rule: str = "ct", out=None):
    """bf16 [rows, cols] -> (codes uint8 [rows, cols/2], e8m0 uint8 [rows, cols/32])."""
    L.require_gpu(x)
    if x.dtype != torch.bfloat16:
        raise TypeError("MXFP4 quantize expects bf16 input")
    if x.dim() != 2:
        x = x.reshape(-1, x.shape[-1])
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    rows, cols = x.shape
    if cols % 32:
        raise ValueError(f"MXFP4 needs the last dim divisible by 32, got {cols}")
    if out is None:
        codes = torch.empty((rows, cols // 2), dtype=torch.uint8, device=x.device)
        scales = torch.empty((rows, cols // 32), dtype=torch.uint8, device=x.device)
    else:
        codes, scales = out
    L.call("mi355q_mxfp4_quantize_pack", x.data_ptr(), rows, cols, x.stride(0), MX_RULES[rule],
           codes.data_ptr(), scales.data_ptr(), L.stream_of(x))
    return codes, scales


def mxfp4_dequantize(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    L.require_gpu(codes, scales)
    rows, half = codes.shape
    out = torch.empty((rows, half * 2), dtype=torch.bfloat16, device=codes.device)
    L.call("mi355q_mxfp4_dequantize", codes.contiguous().data_ptr(), scales.contiguous().data_ptr(), rows,
           half * 2, out.data_ptr(), L.stream_of(codes))
    return out


def quantize_fp8(x: torch.Tensor, scale: torch.Tensor, strategy: str, group_size: int | None = None,
                 div_dtype: torch.dtype | None = None) -> torch.Tensor:
    """float8_e4m3fn codes (as a float8 tensor) with CT quantize arithmetic."""
    L.require_gpu(x, scale)
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, cols = x.shape
    s = scale.to(torch.float32).contiguous()
    s2 = s.reshape(-1, 1) if s.dim() < 2 else s
    if div_dtype is None:
        div_dtype = torch.promote_types(x.dtype, scale.dtype)
    out = torch.empty((rows, cols), dtype=torch.uint8, device=x.device)
    L.call("mi355q_quantize_fp8", x.data_ptr(), _dt(x), rows, cols, x.stride(0), s2.data_ptr(), s2.stride(0),
           STRATEGY_CODE[strategy], group_size or 0, L.BF16 if div_dtype == torch.bfloat16 else L.F32,
           out.data_ptr(), L.stream_of(x))
    return out.view(torch.float8_e4m3fn)


def fp4_quantize_pack(x: torch.Tensor, scale: torch.Tensor, group_size: int,
                      global_scale: torch.Tensor | None = None) -> torch.Tensor:
    """e2m1 codes of x / (scale / global_scale) per column group, two per byte
    (even column in the low nibble): uint8 [rows, cols / 2] (the NVFP4
    ``weight_packed`` tensor)."""
    L.require_gpu(x, scale)
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.float()
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, cols = x.shape
    s = scale.to(torch.float32).reshape(rows, -1).contiguous()
    gs = None if global_scale is None else \
        global_scale.to(device=x.device, dtype=torch.float32).reshape(1).contiguous()
    out = torch.empty((rows, cols // 2), dtype=torch.uint8, device=x.device)
    L.call("mi355q_fp4_quantize_pack", x.data_ptr(), _dt(x), rows, cols, x.stride(0), s.data_ptr(), s.stride(0),
           group_size, L.ptr(gs), out.data_ptr(), L.stream_of(x))
    return out


def quantize_int8_per_token(x: torch.Tensor):
    """Dynamic per-token int8: (codes int8 [rows, cols], scale bf16 [rows, 1])."""
    L.require_gpu(x)
    if x.dtype != torch.bfloat16:
        raise TypeError("per-token int8 expects bf16 activations")
    if x.dim() != 2:
        x = x.reshape(-1, x.shape[-1])
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, cols = x.shape
    codes = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    scale = torch.empty((rows, 1), dtype=torch.bfloat16, device=x.device)
    L.call("mi355q_quantize_int8_per_token", x.data_ptr(), rows, cols, x.stride(0), codes.data_ptr(),
           scale.data_ptr(), L.stream_of(x))
    return codes, scale


# ---------------------------------------------------------------- SparseGPT
def sparsegpt_base_mask(w_work: torch.Tensor):
    """(mask uint8 [rows, cols] = w_work == 0, count int32 [1] on the device)."""
    L.require_gpu(w_work)
    rows, cols = w_work.shape
    mask = torch.empty((rows, cols), dtype=torch.uint8, device=w_work.device)
    count = torch.empty(1, dtype=torch.int32, device=w_work.device)
    L.call("mi355q_sparsegpt_base_mask", w_work.data_ptr(), rows, cols, mask.data_ptr(), count.data_ptr(),
           L.stream_of(w_work))
    return mask, count


def sparsegpt_sweep_(w_work: torch.Tensor, hinv: torch.Tensor, sparsity: float, prune_n: int, prune_m: int,
                     blocksize: int = 128, mask: torch.Tensor | None = None) -> torch.Tensor:
    """In-place SparseGPT sweep of w_work (fp32 [rows, cols]) with the upper
    factor hinv.  ``mask`` (uint8, from ``sparsegpt_base_mask``) preserves the
    entries it holds.  Returns the per-row losses fp32 [rows]."""
    L.require_gpu(w_work, hinv, mask)
    rows, cols = w_work.shape
    if hinv.shape != (cols, cols) or hinv.dtype != torch.float32 or not hinv.is_contiguous():
        raise ValueError(f"hinv must be a contiguous fp32 [{cols}, {cols}] matrix")
    if mask is not None and (mask.shape != (rows, cols) or mask.dtype != torch.uint8 or not mask.is_contiguous()):
        raise ValueError("mask must be a contiguous uint8 matrix shaped like w_work")
    losses = torch.zeros(rows, dtype=torch.float32, device=w_work.device)
    lib = L.lib()
    ws = _ws(lib.mi355q_sparsegpt_workspace_size(rows, cols, blocksize), w_work.device)
    L.check(lib.mi355q_sparsegpt_sweep(w_work.data_ptr(), rows, cols, hinv.data_ptr(), C.c_double(sparsity),
                                       int(prune_n), int(prune_m), blocksize, L.ptr(mask), losses.data_ptr(),
                                       ws.data_ptr(), ws.numel(), L.stream_of(w_work)))
    return losses
