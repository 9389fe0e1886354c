"""MI355X (gfx950) calibration-time quantization for llm-compressor's hot path.

The public functions keep the reference's names and signatures
(``make_empty_hessian``, ``accumulate_hessian``, ``quantize_weight``, the
observer registry, ``observe`` / ``update_qparams``); the arithmetic runs in
hand-written HIP kernels (``libmi355q.so``, C ABI in ``include/mi355q.h``).
"""
from .calibration import initialize_module_for_quantization, initialize_observer, observe, update_qparams
from .gptq import GPTQResult, PreparedHessian, accumulate_hessian, gptq_quantize, gptq_quantize_batched, \
    make_empty_hessian, prepare_hessian, prepare_hessians_batched, quantize_weight, symmetrize_hessian
from . import pipeline, save, sparsegpt
from .modifiers import GPTQModifier, QuantizationModifier, SparseGPTModifier
from .observers import FUSED_LAYER_NAMES, Observer, fuse_weight_observers
from .quant_args import (CT_ARG_FIELDS, ActivationOrdering, QuantizationArgs, QuantizationScheme,
                         QuantizationStrategy, QuantizationType, preset_name_to_scheme, resolve_args)

__all__ = [
    "CT_ARG_FIELDS", "FUSED_LAYER_NAMES", "fuse_weight_observers", "resolve_args", "ActivationOrdering", "GPTQModifier", "GPTQResult", "Observer", "QuantizationArgs", "QuantizationModifier",
    "QuantizationScheme", "QuantizationStrategy", "QuantizationType", "SparseGPTModifier", "pipeline", "save", "sparsegpt", "accumulate_hessian", "gptq_quantize",
    "gptq_quantize_batched", "initialize_module_for_quantization", "initialize_observer", "make_empty_hessian",
    "observe", "prepare_hessian", "prepare_hessians_batched", "PreparedHessian", "preset_name_to_scheme",
    "quantize_weight", "symmetrize_hessian", "update_qparams",
]
