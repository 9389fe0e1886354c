"""Sequential calibration: layer-by-layer calibration with an activation cache.

Replaces ``pipelines/sequential/pipeline.py:51-178`` (calibrate a subgraph on
every batch with the modifier hooks live, compress it, then run it again with
the hooks off so that the next subgraph sees the compressed layer's outputs)
and ``pipelines/cache.py:37-330`` (the per-batch intermediates, offloaded to
host memory between uses and prefetched back).  Instead of tracing the model
into subgraphs, the runner takes the model's list of decoder layers: the
inputs of the first layer are captured by a pre-hook that stops the model's
forward there, and every later layer consumes its predecessor's output in
place of its first argument, with the same keyword arguments (attention
masks, position embeddings) for all layers, as decoder stacks call them.

Offloading copies tensors into pinned host memory on a copy stream of its own
(default priority) once their producer has run; fetching copies them back on
a second copy stream (so a fetch never queues behind unrelated offloads, and
the two directions of the link run at once), and the consumer's stream waits
on an event, so the prefetch of
batch b + 1 overlaps the layer's work on batch b, and the first batch of a
pass is fetched while the previous step (the layer's compression, or the end
of the previous pass) still runs.
"""
from __future__ import annotations

import contextlib
from typing import Any, Iterator

import torch

__all__ = ["IntermediatesCache", "sequential_calibrate"]


class _Offloaded:
    """A host copy of a device tensor, ready once ``event`` has completed."""

    __slots__ = ("host", "event", "device")

    def __init__(self, host: torch.Tensor, event, device: torch.device):
        self.host, self.event, self.device = host, event, device


class IntermediatesCache:
    """Per-batch dictionaries of intermediate values (``pipelines/cache.py``).
    ``offload_device`` "cpu": tensors are kept in pinned host memory between
    uses; None: they stay where they are."""

    def __init__(self, num_batches: int, offload_device: str | None = "cpu"):
        self.batches: list[dict[str, Any]] = [{} for _ in range(num_batches)]
        self.offload_device = offload_device
        self._streams = {}

    def _stream(self, device, direction: str):
        """The copy stream for "d2h" (offload) or "h2d" (fetch)."""
        if direction not in self._streams:
            self._streams[direction] = torch.cuda.Stream(device=device)
        return self._streams[direction]

    # -- offload / onload of nested values
    def _offload(self, v):
        if isinstance(v, torch.Tensor):
            if self.offload_device is None or v.device.type != "cuda":
                return v
            cs = self._stream(v.device, "d2h")
            cs.wait_stream(torch.cuda.current_stream(v.device))
            host = torch.empty(v.shape, dtype=v.dtype, pin_memory=True)
            with torch.cuda.stream(cs):
                host.copy_(v, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(cs)
            v.record_stream(cs)
            return _Offloaded(host, ev, v.device)
        if isinstance(v, tuple):
            return tuple(self._offload(x) for x in v)
        if isinstance(v, list):
            return [self._offload(x) for x in v]
        if isinstance(v, dict):
            return {k: self._offload(x) for k, x in v.items()}
        return v

    def _onload_async(self, v):
        """Start the copies back; returns the value with _Pending leaves."""
        if isinstance(v, _Offloaded):
            cs = self._stream(v.device, "h2d")
            with torch.cuda.stream(cs):
                cs.wait_event(v.event)
                dev = torch.empty(v.host.shape, dtype=v.host.dtype, device=v.device)
                dev.copy_(v.host, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(cs)
            return _Pending(dev, ev)
        if isinstance(v, tuple):
            return tuple(self._onload_async(x) for x in v)
        if isinstance(v, list):
            return [self._onload_async(x) for x in v]
        if isinstance(v, dict):
            return {k: self._onload_async(x) for k, x in v.items()}
        return v

    @staticmethod
    def _ready(v):
        """Make the current stream wait for pending copies; plain values."""
        if isinstance(v, _Pending):
            cur = torch.cuda.current_stream(v.tensor.device)
            cur.wait_event(v.event)
            v.tensor.record_stream(cur)
            return v.tensor
        if isinstance(v, tuple):
            return tuple(IntermediatesCache._ready(x) for x in v)
        if isinstance(v, list):
            return [IntermediatesCache._ready(x) for x in v]
        if isinstance(v, dict):
            return {k: IntermediatesCache._ready(x) for k, x in v.items()}
        return v

    # -- the reference's interface
    def update(self, batch_index: int, values: dict[str, Any]) -> None:
        self.batches[batch_index].update({k: self._offload(v) for k, v in values.items()})

    def delete(self, batch_index: int, consumed_names: list[str] | None = None) -> None:
        names = list(self.batches[batch_index]) if consumed_names is None else consumed_names
        for k in names:
            self.batches[batch_index].pop(k, None)

    def fetch(self, batch_index: int, input_names: list[str] | None = None) -> dict[str, Any]:
        d = self.batches[batch_index]
        names = list(d) if input_names is None else input_names
        return self._ready({k: self._onload_async(d[k]) for k in names})

    def iter(self, input_names=None) -> Iterator[dict[str, Any]]:
        for b in range(len(self.batches)):
            yield self.fetch(b, input_names)

    def iter_prefetch(self, input_names=None, first=None) -> Iterator[dict[str, Any]]:
        """As ``iter``, with batch b + 1's copies issued before batch b is used;
        ``first``: batch 0 as already started by ``prefetch(0)``."""
        n = len(self.batches)
        nxt = first
        for b in range(n):
            cur = nxt if nxt is not None else self._start(b, input_names)
            nxt = self._start(b + 1, input_names) if b + 1 < n else None
            yield self._ready(cur)

    def prefetch(self, batch_index: int, input_names=None):
        """Starts the copies of one batch back to the device (for a later
        ``iter_prefetch(first=...)``); the batch must not be updated before
        it is consumed."""
        return self._start(batch_index, input_names)

    def _start(self, b, input_names):
        d = self.batches[b]
        names = list(d) if input_names is None else input_names
        return {k: self._onload_async(d[k]) for k in names}

    def size(self) -> dict[str, int]:
        """Bytes held, per device ("cpu" for offloaded values)."""
        out: dict[str, int] = {}

        def walk(v):
            if isinstance(v, _Offloaded):
                out["cpu"] = out.get("cpu", 0) + v.host.numel() * v.host.element_size()
            elif isinstance(v, torch.Tensor):
                out[str(v.device)] = out.get(str(v.device), 0) + v.numel() * v.element_size()
            elif isinstance(v, (tuple, list)):
                for x in v:
                    walk(x)
            elif isinstance(v, dict):
                for x in v.values():
                    walk(x)
        for d in self.batches:
            walk(d)
        return out

    def __len__(self):
        return len(self.batches)


class _Pending:
    __slots__ = ("tensor", "event")

    def __init__(self, tensor, event):
        self.tensor, self.event = tensor, event


class _StopForward(Exception):
    pass


def _first_output(out):
    return out[0] if isinstance(out, (tuple, list)) else out


@torch.no_grad()
def sequential_calibrate(model: torch.nn.Module, layers, batches, modifier, propagate_error: bool = True,
                         offload_device: str | None = "cpu", prefetch: bool = True) -> IntermediatesCache:
    """Calibrate and compress ``layers`` (the model's decoder layers, in
    order) one at a time over ``batches`` with ``modifier`` (a GPTQModifier or
    SparseGPTModifier of this package), as ``SequentialPipeline.__call__``
    does: capture the first layer's inputs, then per layer a calibration pass
    (hooks live), the layer's compression, and — with ``propagate_error`` — a
    second pass with the hooks off whose outputs feed the next layer (without
    it, the calibration pass's outputs do).  Returns the cache holding the
    last layer's outputs."""
    layers = list(layers)
    cache = IntermediatesCache(len(batches), offload_device)

    def catch(mod, args, kwargs):
        catch.inputs = (args, kwargs)
        raise _StopForward

    if not layers:
        raise ValueError("sequential_calibrate needs at least one layer")
    h = layers[0].register_forward_pre_hook(catch, with_kwargs=True)
    try:
        for b, x in enumerate(batches):
            catch.inputs = None
            try:
                model(x) if not isinstance(x, dict) else model(**x)
            except _StopForward:
                pass
            if catch.inputs is None:
                raise RuntimeError("the model's forward did not reach the first of the given layers")
            args, kwargs = catch.inputs
            cache.update(b, {"args": args, "kwargs": kwargs})
    finally:
        h.remove()

    modifier.on_initialize(model)
    modifier.on_calibration_start(model)

    def batches_of(first):
        return cache.iter_prefetch(first=first) if prefetch else cache.iter()

    def run(layer, b, inputs):
        out = layer(*inputs["args"], **inputs["kwargs"])
        return _first_output(out)

    # With prefetch, the first batch of each pass is copied back while the
    # previous step still runs: the propagation pass's (unchanged inputs)
    # during the layer's compression, the next layer's as soon as this pass
    # has replaced it.
    pending = None
    for li, layer in enumerate(layers):
        ahead = prefetch and li + 1 < len(layers) and len(cache) > 0  # a next layer to prefetch for
        nxt = None
        # each batch's entry is replaced as soon as it has been consumed (the
        # prefetch has already issued the next batch's copies)
        for b, inputs in enumerate(batches_of(pending)):
            out = run(layer, b, inputs)
            if not propagate_error:
                cache.update(b, {"args": (out,) + tuple(inputs["args"][1:])})
                if b == 0 and ahead:
                    nxt = cache.prefetch(0)
        if propagate_error:
            pending = cache.prefetch(0) if prefetch and len(cache) > 0 else None
            _compress(modifier, layer)
            with _hooks_disabled(modifier):
                for b, inputs in enumerate(batches_of(pending)):
                    cache.update(b, {"args": (run(layer, b, inputs),) + tuple(inputs["args"][1:])})
                    if b == 0 and ahead:
                        nxt = cache.prefetch(0)
        else:
            _compress(modifier, layer)
        pending = nxt
    modifier.on_calibration_end()
    modifier.on_finalize()
    return cache


def _compress(modifier, layer):
    """The modifier's epoch end for the modules of ``layer`` (the only ones
    whose hooks ran since the last compression)."""
    from .modifiers import GPTQModifier

    if isinstance(modifier, GPTQModifier):
        modifier.on_sequential_epoch_end([m for m in layer.modules() if m in modifier._modules])
    else:
        modifier.on_sequential_epoch_end()


@contextlib.contextmanager
def _hooks_disabled(modifier):
    prev = getattr(modifier, "_hooks_disabled", False)
    modifier._hooks_disabled = True
    try:
        yield
    finally:
        modifier._hooks_disabled = prev
