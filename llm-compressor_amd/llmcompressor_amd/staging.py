"""Calibration rows of one Hessian gathered on the device between syrk calls.

The reference's hooks (``modifiers/gptq/base.py:255-289``,
``modifiers/pruning/sparsegpt/base.py``) accumulate every forward pass into
the Hessian at once; with its default of one 2048-token sample per batch
(``args/dataset_arguments.py:72-73``) each call has 2048 rows.  A syrk over
so few rows runs only the 136 upper 256 x 256 tiles of a d = 4096 Hessian on
the 256 CUs, each with a full read-modify-write of its H tile, at half the
rate of a long call.  ``HessianStage`` copies the rows of small calls into a
[tokens, d] buffer of the input dtype and hands them to the syrk when the
buffer is full or when the Hessian is read, so the same sum is formed in
fewer, longer calls (another order of fp32 additions; the sample count is
the reference's).  A stage holds up to 65536 rows and at most 512 MiB
(18432 rows of a 14336-wide bf16 input), so that each syrk call runs the
eight token splits of 8192 rows a one-call Hessian of a 4096-wide layer
runs.
"""
from __future__ import annotations

import torch

DEFAULT_TOKENS = 65536
DEFAULT_BUDGET = 2 << 30   # bytes of stage buffers one modifier holds at a time
STAGE_BYTES_MAX = 512 << 20


def stage_tokens(tokens: int, d: int, element_size: int) -> int:
    """Rows of one stage for a [*, d] input: ``tokens``, lowered to a
    multiple of 2048 that fits in ``STAGE_BYTES_MAX`` (at least 2048)."""
    fit = STAGE_BYTES_MAX // max(1, d * element_size) // 2048 * 2048
    return min(tokens, max(2048, fit))


class HessianStage:
    """Rows waiting for one Hessian.  ``add(x, samples, flush)`` stages the
    2-D rows x (on the Hessian's device) and the reference's sample count of
    their call; ``flush(rows, samples)`` is the accumulation the caller
    would have run on them, called with every staged row exactly once, in
    call order.  Calls of more than ``tokens / 2`` rows go through at once
    (after the staged ones)."""

    def __init__(self, tokens: int = DEFAULT_TOKENS):
        if tokens <= 0:
            raise ValueError("staging needs a positive row count")
        self.tokens = tokens
        self.buf: torch.Tensor | None = None
        self._key = None
        self.fill = 0
        self.samples = 0

    def add(self, x: torch.Tensor, samples, flush) -> None:
        n, d = x.shape
        key = (x.dtype, d, x.device)
        if self.buf is not None and key != self._key:
            self.flush(flush)
            self.buf = None
        if 2 * n > self.tokens:
            self.flush(flush)
            flush(x, samples)
            return
        if self.fill + n > self.tokens:
            self.flush(flush)
        if self.buf is None:
            self.buf = torch.empty((self.tokens, d), dtype=x.dtype, device=x.device)
            self._key = key
        self.buf.narrow(0, self.fill, n).copy_(x)
        self.fill += n
        self.samples += samples
        if self.fill == self.tokens:
            self.flush(flush)

    def flush(self, flush) -> None:
        if self.fill:
            flush(self.buf[:self.fill], self.samples)
            self.fill = 0
            self.samples = 0

    def release(self) -> None:
        self.buf = None
        self.fill = 0
        self.samples = 0
