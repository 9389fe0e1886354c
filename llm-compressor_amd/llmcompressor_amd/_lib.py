"""ctypes binding of ``libmi355q.so`` (the C ABI in ``include/mi355q.h``).

The library is loaded lazily on first use.  There is no CPU fallback: if
the library is missing or no GPU is present, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import threading

import torch

from ._build import LIB_PATH

OK, INVALID_ARGUMENT, UNSUPPORTED, NOT_POSITIVE_DEFINITE, HIP_ERROR, TIMEOUT = 0, 1, 2, 3, 4, 5
BF16, F32, F16 = 0, 1, 2
TENSOR, CHANNEL, GROUP, BLOCK, TOKEN = 0, 1, 2, 3, 4
MX_RULE_CT, MX_RULE_OCP = 0, 1
QTYPE_INT, QTYPE_FP8_E4M3, QTYPE_FP4_E2M1, QTYPE_MXFP4_CT, QTYPE_MXFP4_OCP = 0, 1, 2, 3, 4

_vp, _i64, _i32, _f32, _f64, _sz = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_double, C.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "mi355q_last_error": (C.c_char_p, []),
    "mi355q_version": (_i32, []),
    "mi355q_hessian_workspace_size": (_sz, [_i64, _i64]),
    "mi355q_hessian_syrk_bf16": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _f32, _vp, _sz, _vp]),
    "mi355q_hessian_syrk_scaled_bf16": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _f32, _f32, _vp, _sz, _vp]),
    "mi355q_hessian_syrk_workspace_size": (_sz, [_i64, _i64, _i32]),
    "mi355q_hessian_syrk": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _f32, _f32, _vp, _sz, _vp]),
    "mi355q_hessian_syrk_segments_workspace_size": (_sz, [_vp, _i32, _i64, _i32]),
    "mi355q_hessian_syrk_segments": (_i32, [_vp, _vp, _i32, _i32, _i64, _i64, _vp, _i64, _f32, _f32, _vp, _sz, _vp]),
    "mi355q_hessian_grouped_syrk_workspace_size": (_sz, [_i64, _i32, _i64]),
    "mi355q_hessian_grouped_syrk": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _vp, _i64, _f32, _f32, _vp,
                                           _sz, _vp]),
    "mi355q_symmetrize_upper": (_i32, [_vp, _i64, _i64, _vp]),
    "mi355q_gptq_hinv_workspace_size": (_sz, [_i64]),
    "mi355q_gptq_hinv": (_i32, [_vp, _i64, _i64, _vp, _f32, _f32, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mi355q_gptq_load_weight": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "mi355q_gptq_sweep_workspace_size": (_sz, [_i64, _i64, _i64]),
    "mi355q_gptq_sweep": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i32, _f32, _f32, _i32,
                                 _i64, _vp, _vp, _vp, _sz, _vp]),
    "mi355q_gptq_store_weight": (_i32, [_vp, _i64, _i64, _vp, _vp, _i32, _i64, _vp, _vp, _vp]),
    "mi355q_gptq_sweep_noalloc_max_bytes": (_sz, []),
    "mi355q_gptq_sweep_noalloc": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _i32, _i32, _f32, _f32, _i32,
                                         _i64, _vp, _vp, _vp]),
    "mi355q_gptq_hinv_batched": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _f32, _vp, _i64, _vp, _vp,
                                        _vp, _sz, _vp]),
    "mi355q_gptq_hinv_fallback": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "mi355q_gptq_load_weight_batched": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp,
                                               _vp]),
    "mi355q_gptq_sweep_batched": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _i64, _i32,
                                         _i32, _f32, _f32, _i32, _i64, _vp, _vp, _vp, _sz, _vp]),
    "mi355q_gptq_sweep_typed_batched": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _i64,
                                               _i32, _i32, _i32, _f32, _f32, _vp, _i32, _i64, _vp, _vp, _vp, _sz,
                                               _vp]),
    "mi355q_gptq_store_weight_batched": (_i32, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i32, _i64, _i64, _vp,
                                                _vp, _vp]),
    "mi355q_sparsegpt_base_mask": (_i32, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "mi355q_sparsegpt_workspace_size": (_sz, [_i64, _i64, _i64]),
    "mi355q_sparsegpt_sweep": (_i32, [_vp, _i64, _i64, _vp, _f64, _i32, _i32, _i64, _vp, _vp, _vp, _sz, _vp]),
    "mi355q_observe_minmax": (_i32, [_vp, _i32, _i64, _i64, _i64, _i32, _i64, _i32, _i32, _vp, _vp, _vp]),
    "mi355q_calculate_qparams": (_i32, [_vp, _vp, _i64, _f32, _f32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "mi355q_observe_mse_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i32]),
    "mi355q_observe_mse": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32, _i32, _i32, _i32,
                                  _f64, _f32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mi355q_observe_imatrix_mse": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32, _i32, _i32,
                                          _i32, _f64, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mi355q_column_sumsq_workspace_size": (_sz, [_i64, _i64]),
    "mi355q_column_sumsq": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    "mi355q_mx_scales": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _vp]),
    "mi355q_nvfp4_qparams": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp]),
    "mi355q_quantize_int": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i32, _i64, _i32, _i32,
                                   _i32, _i32, _vp, _vp]),
    "mi355q_pack_int4_int32": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "mi355q_pack_int4_int8": (_i32, [_vp, _i64, _i64, _vp, _vp]),
    "mi355q_pack_int32": (_i32, [_vp, _i64, _i64, _i32, _vp, _vp]),
    "mi355q_mxfp4_quantize_pack": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp]),
    "mi355q_mxfp4_dequantize": (_i32, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "mi355q_quantize_fp8": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _i32, _i64, _i32, _vp, _vp]),
    "mi355q_fp4_quantize_pack": (_i32, [_vp, _i32, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp]),
    "mi355q_quantize_int8_per_token": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp]),
}

_lock = threading.Lock()
_lib = None


class Mi355qError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"mi355q status {status}: {msg}")
        self.status = status


def load_library(path=None) -> C.CDLL:
    """Load and declare the library (no GPU needed)."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not p.exists():
            raise RuntimeError(f"{p} is not built; run __graft_entry__.build() (hipcc, gfx950) first")
        lib = C.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def lib() -> C.CDLL:
    return _lib if _lib is not None else load_library()


def check(status: int) -> None:
    if status != OK:
        raise Mi355qError(status, lib().mi355q_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def check_hinv_status(values) -> None:
    """Raise if a per-matrix hinv status (host values) reports that the
    factorisation's workgroups stopped waiting for each other: its results
    are invalid, unlike a Hessian that is not positive definite."""
    if any(int(v) == TIMEOUT for v in values):
        raise Mi355qError(TIMEOUT, "hinv: the dataflow factorisation timed out waiting between workgroups")


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of an optional operand (None: a null pointer); a
    tensor on the host is refused, as the kernels would read it as device
    memory."""
    if t is None:
        return None
    require_gpu(t)
    return t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "llmcompressor_amd runs on the GPU only (HIP kernels); got a tensor on "
                f"{t.device}. Move inputs to a ROCm device.")
