"""Calibration rows of one Hessian gathered on the device between syrk calls.

The reference's hooks (``modifiers/gptq/base.py:255-289``,
``modifiers/pruning/sparsegpt/base.py``) accumulate every forward pass into
the Hessian at once; with its default of one 2048-token sample per batch
(``args/dataset_arguments.py:72-73``) each call has 2048 rows.  A syrk over
so few rows runs only the 136 upper 256 x 256 tiles of a d = 4096 Hessian on
the 256 CUs, each with a full read-modify-write of its H tile, at half the
rate of a long call.  ``HessianStage`` holds the rows of small calls and
hands them to the syrk when it holds ``tokens`` rows or when the Hessian is
read, so the same sum is formed in fewer, longer calls (another order of
fp32 additions; the sample count is the reference's).

16-bit rows at least 512 wide (the segmented syrk's inputs) are held by
reference: the hook's own tensor, no copy, summed in place by one
``ops.hessian_syrk_segments_`` launch.  A held tensor modified in place
before the flush (torch's version counter moved) makes the flush raise
rather than sum rows the hook never saw.  Tensors that cannot be held
(inference tensors, another row stride, storage much larger than the rows)
are held as a copy; calls under 256 rows (each segment starts a new 32-row
stage) are copied into a buffer of ``tokens / 8`` rows; other dtypes and
narrower rows into a buffer of ``tokens`` rows, as one segment.  A stage
holds up to 131072 rows and at most 1 GiB (36864 rows of a 14336-wide
bf16 input): 64 held calls of 2048 rows of a 4096-wide layer fill one stage
and one segmented syrk, which then runs the eight token splits of 16384
rows the one-call Hessian of those rows runs (two stages of 65536 rows took
2.37-2.41 ms against 1.92-2.02 for one call, the second launch's rounds and
reduction).
"""
from __future__ import annotations

import torch

DEFAULT_TOKENS = 131072
DEFAULT_BUDGET = 4 << 30   # bytes of staged rows one modifier holds at a time
STAGE_BYTES_MAX = 1 << 30
MAX_SEGMENTS = 64          # segments of one segmented syrk launch
SMALL_ROWS = 256           # calls below this are copied, not held
_SEG_DTYPES = (torch.bfloat16, torch.float16)


def stage_tokens(tokens: int, d: int, element_size: int) -> int:
    """Rows of one stage for a [*, d] input: ``tokens``, lowered to a
    multiple of 2048 that fits in ``STAGE_BYTES_MAX`` (at least 2048)."""
    fit = STAGE_BYTES_MAX // max(1, d * element_size) // 2048 * 2048
    return min(tokens, max(2048, fit))


def hold(x: torch.Tensor):
    """(x, its version) for a tensor kept until a later flush; an inference
    tensor (no version counter) is copied instead (version None)."""
    if x.is_inference():
        return x.clone(), None
    return x, x._version


def held(x: torch.Tensor, version) -> torch.Tensor:
    """A tensor kept by ``hold``, unless it was modified in place since."""
    if version is not None and x._version != version:
        raise RuntimeError(
            "a calibration input held for a Hessian was modified in place after its forward hook ran; "
            "its rows are no longer the ones the hook saw.  Turn staging off for this model "
            "(hessian_batch_tokens=0) so that each call is accumulated at once.")
    return x


def _holdable(x: torch.Tensor) -> bool:
    n, d = x.shape
    return (x.stride(1) == 1 and x.stride(0) == d and x.data_ptr() % 16 == 0 and not x.is_inference()
            and x.untyped_storage().nbytes() <= 2 * n * d * x.element_size())


class HessianStage:
    """Rows waiting for one Hessian.  ``add(x, samples, flush)`` stages the
    2-D rows x (on the Hessian's device) and the reference's sample count of
    their call; ``flush(segments, samples)`` is the accumulation the caller
    would have run on them: ``segments`` a list of 2-D row tensors, every
    staged row in exactly one of them, once (held calls in call order, then
    the copied rows in call order).  Calls of more than ``tokens / 2`` rows
    go through at once (after the staged ones)."""

    def __init__(self, tokens: int = DEFAULT_TOKENS):
        if tokens <= 0:
            raise ValueError("staging needs a positive row count")
        self.tokens = tokens
        self.buf: torch.Tensor | None = None
        self._key = None
        self._refs = False       # this key's rows are held by reference
        self._segs: list = []    # (tensor, version) of the held calls
        self.buf_fill = 0
        self.fill = 0            # staged rows, held and copied
        self.samples = 0

    def add(self, x: torch.Tensor, samples, flush) -> None:
        n, d = x.shape
        key = (x.dtype, d, x.device)
        if key != self._key:
            self.flush(flush)
            self.buf = None
            self._key = key
            self._refs = x.dtype in _SEG_DTYPES and d >= 512 and d % 8 == 0
        if 2 * n > self.tokens:
            self.flush(flush)
            flush([x], samples)
            return
        if self.fill + n > self.tokens:
            self.flush(flush)
        if self._refs and n >= SMALL_ROWS:
            if len(self._segs) == MAX_SEGMENTS:
                self.flush(flush)
            self._segs.append(hold(x) if _holdable(x) else (x.clone(memory_format=torch.contiguous_format), None))
        else:
            cap = min(self.tokens, max(SMALL_ROWS, self.tokens // 8)) if self._refs else self.tokens
            if self.buf_fill + n > cap:
                self.flush(flush)
            if self.buf is None:
                self.buf = torch.empty((cap, d), dtype=x.dtype, device=x.device)
            self.buf.narrow(0, self.buf_fill, n).copy_(x)
            self.buf_fill += n
        self.fill += n
        self.samples += samples
        if self.fill == self.tokens:
            self.flush(flush)

    def flush(self, flush) -> None:
        if not self.fill:
            return
        segs = [held(x, v) for x, v in self._segs]
        if self.buf_fill:
            segs.append(self.buf[:self.buf_fill])
        samples = self.samples
        self._segs, self.buf_fill, self.fill, self.samples = [], 0, 0, 0
        flush(segs, samples)

    def release(self) -> None:
        self.buf = None
        self._key = None
        self._segs = []
        self.buf_fill = 0
        self.fill = 0
        self.samples = 0
