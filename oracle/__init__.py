"""CPU oracle for the calibration-time quantization path.

TEST INFRASTRUCTURE ONLY.  This package is a CPU restatement of the
reference's algorithm (llm-compressor's GPTQ Hessian/solve, min-max
observers and the compressed-tensors quantize/pack arithmetic it calls).
It is imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and there only as the reference the GPU
results are compared with, never as the thing measured.  The
product path (``llmcompressor_amd``) never imports it and fails loudly when
its HIP library is missing.

Modules and the reference code each one restates:

* ``qargs``      - the subset of compressed-tensors ``QuantizationArgs`` used.
* ``observers``  - ``observers/min_max.py:16-110``, ``observers/base.py:99-145``,
                   ``observers/helpers.py:28-131`` and compressed-tensors
                   ``calculate_qparams`` (restated from its call sites and the
                   reference's known-answer tests).
* ``fake_quant`` - compressed-tensors ``fake_quantize`` / ``quantize`` as
                   called at ``modifiers/gptq/gptq_quantize.py:215-257``.
* ``gptq``       - ``modifiers/gptq/gptq_quantize.py:15-310`` and the
                   normalisation at ``modifiers/gptq/base.py:594``.
* ``pack``       - ``utils/pack_int4_to_int8.py:13-28`` and the
                   compressed-tensors packers (int32 nibble pack, MXFP4
                   e2m1 + e8m0, fp8 e4m3) in numpy.
* ``moe``        - ``modeling/moe/linear_experts.py:244-277`` token routing.

Pinning status of each function is stated in its module header.
"""
