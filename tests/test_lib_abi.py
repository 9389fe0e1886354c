"""The C-ABI library loads, exports every declared symbol, and validates
arguments on the host (CPU only: no kernel launches)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from llmcompressor_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mi355q.h"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mi355q_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load_library()
    names = declared_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_version_and_workspace_queries():
    lib = _lib.load_library()
    assert lib.mi355q_version() == 1
    assert lib.mi355q_hessian_workspace_size(2048, 4096) == 0            # single split, direct update
    # d = 4096: 136 tiles, 8 splits; the last 8 tiles run as 4 parts per split
    # (128 * 8 split slots + 8 * 8 * 4 part slots, summed by the reduction)
    assert lib.mi355q_hessian_workspace_size(131072, 4096) == (128 * 8 + 8 * 8 * 4) * 256 * 256 * 4
    assert lib.mi355q_hessian_workspace_size(131072, 384) == 8 * 6 * 128 * 128 * 4
    assert lib.mi355q_gptq_sweep_workspace_size(4096, 4096, 128) == 4096 * 1024 * 4   # errors of one 1024-column super-block
    assert lib.mi355q_gptq_sweep_workspace_size(768, 768, 128) == 768 * 768 * 4       # fewer columns than a super-block
    assert lib.mi355q_gptq_hinv_workspace_size(4096) >= 2 * 4096 * 4096 * 4
    # SparseGPT: the super-block error buffer plus the radix-select words
    assert lib.mi355q_sparsegpt_workspace_size(4096, 4096, 128) == 4096 * 1024 * 4 + 2 * (256 + 2048 + 4096 + 64) * 4


@pytest.mark.parametrize("call,needle", [
    (lambda l: l.mi355q_hessian_syrk_bf16(None, 10, 7, 7, None, 7, C.c_float(2.0), None, 0, None), "multiple of 8"),
    (lambda l: l.mi355q_pack_int4_int8(None, 2, 3, None, None), "null pointer"),
    (lambda l: l.mi355q_mxfp4_quantize_pack(C.c_void_p(16), 4, 30, 32, 0, C.c_void_p(16), C.c_void_p(16), None),
     "multiple of 32"),
    (lambda l: l.mi355q_gptq_sweep(C.c_void_p(16), 4, 4, C.c_void_p(16), C.c_void_p(16), None, 1, None, 7, 1,
                                   C.c_float(-8), C.c_float(7), 1, 128, C.c_void_p(16), C.c_void_p(16),
                                   C.c_void_p(16), 1 << 20, None), "not supported for GPTQ"),
    (lambda l: l.mi355q_calculate_qparams(C.c_void_p(16), C.c_void_p(16), 4, C.c_float(0), C.c_float(7), 1, 0, 0,
                                          C.c_void_p(16), C.c_void_p(16), None), "straddle zero"),
    (lambda l: l.mi355q_sparsegpt_sweep(C.c_void_p(16), 4, 64, C.c_void_p(16), C.c_double(1.0), 0, 0, 32, None,
                                        C.c_void_p(16), C.c_void_p(16), 1 << 20, None), "out of bounds"),
    (lambda l: l.mi355q_sparsegpt_sweep(C.c_void_p(16), 4, 64, C.c_void_p(16), C.c_double(0.5), 3, 2, 32, None,
                                        C.c_void_p(16), C.c_void_p(16), 1 << 20, None), "out of range"),
    (lambda l: l.mi355q_sparsegpt_sweep(C.c_void_p(16), 4, 64, C.c_void_p(16), C.c_double(0.5), 1, 3, 32,
                                        C.c_void_p(16), C.c_void_p(16), C.c_void_p(16), 1 << 20, None),
     "broadcast"),
])
def test_invalid_arguments_are_rejected_on_the_host(call, needle):
    lib = _lib.load_library()
    assert call(lib) == _lib.INVALID_ARGUMENT
    assert needle in lib.mi355q_last_error().decode()


def test_hessian_grouped_host_checks():
    """Argument checks of the grouped Hessian that need no device: H stride,
    an ungathered call with more rows than x, and the workspace bound."""
    lib = _lib.load_library()
    rc = lib.mi355q_hessian_grouped_syrk(C.c_void_p(16), _lib.BF16, 100, 8, 8, None, 100, C.c_void_p(16), 2,
                                         C.c_void_p(16), 63, C.c_float(2.0), C.c_float(1.0), None, 0, None)
    assert rc == _lib.INVALID_ARGUMENT and "stride" in lib.mi355q_last_error().decode()
    rc = lib.mi355q_hessian_grouped_syrk(C.c_void_p(16), _lib.BF16, 100, 8, 8, None, 101, C.c_void_p(16), 2,
                                         C.c_void_p(16), 64, C.c_float(2.0), C.c_float(1.0), None, 0, None)
    assert rc == _lib.INVALID_ARGUMENT and "n_rows > n_x" in lib.mi355q_last_error().decode()
    need = lib.mi355q_hessian_grouped_syrk_workspace_size(100, 2, 8)
    rc = lib.mi355q_hessian_grouped_syrk(C.c_void_p(16), _lib.BF16, 100, 8, 8, None, 100, C.c_void_p(16), 2,
                                         C.c_void_p(16), 64, C.c_float(2.0), C.c_float(1.0), C.c_void_p(16), need - 1, None)
    assert rc == _lib.INVALID_ARGUMENT and "workspace too small" in lib.mi355q_last_error().decode()
    rc = lib.mi355q_hessian_grouped_syrk(C.c_void_p(16), _lib.BF16, 100, 8, 8, None, 100, C.c_void_p(16), 2,
                                         C.c_void_p(16), 64, C.c_float(2.0), C.c_float(0.5), C.c_void_p(16), need, None)
    assert rc == _lib.INVALID_ARGUMENT and "beta must be 0" in lib.mi355q_last_error().decode()
    # slots: one per later chunk of 4096 rows and upper 256-tile
    big = lib.mi355q_hessian_grouped_syrk_workspace_size(3 * 4096, 2, 512)
    assert big >= 3 * 3 * 256 * 256 * 4


def test_sparsegpt_limits_are_reported_unsupported():
    lib = _lib.load_library()
    rc = lib.mi355q_sparsegpt_sweep(C.c_void_p(16), 4, 512, C.c_void_p(16), C.c_double(0.5), 0, 0, 256, None,
                                    C.c_void_p(16), C.c_void_p(16), 1 << 24, None)
    assert rc == _lib.UNSUPPORTED and "block sizes" in lib.mi355q_last_error().decode()
    rc = lib.mi355q_sparsegpt_sweep(C.c_void_p(16), 4, 512, C.c_void_p(16), C.c_double(0.5), 16, 32, 128, None,
                                    C.c_void_p(16), C.c_void_p(16), 1 << 24, None)
    assert rc == _lib.UNSUPPORTED and "wider than 16" in lib.mi355q_last_error().decode()


def test_host_tensors_are_refused_as_device_operands():
    """An optional operand left on the host would be read as device memory;
    the pointer helper refuses it before any call."""
    import torch
    assert _lib.ptr(None) is None
    with pytest.raises(RuntimeError, match="GPU only"):
        _lib.ptr(torch.zeros(4))
