"""The decode step as a HIP graph, and the emit ring of the generate loop.

``capture_decode(step, reset)`` returns a :class:`StepGraph`: one decode
step recorded by stream capture, replayed with one launch per step
(litemoe/execution.py:48-64 is the reference's counterpart).

``OutputRing(emit, consume, asynchronous=False, depth=4)`` hands the
per-step snapshots of ``emit [B, 3] = (token, index, valid)`` to
``consume`` in step order, each exactly once (litemoe/execution.py:6-45 is
the reference's counterpart; its contract is kept, its mechanism is not):

* synchronous: a blocking copy after every step;
* asynchronous: ``depth`` slots of pinned host memory. A slot is filled in
  one of two ways. With a device view (:meth:`OutputRing.device_target`)
  the step's greedy epilogue kernel stores the rows into the slot itself,
  so the device-to-host transfer is part of the captured step and needs no
  copy, stream or cross-stream wait of its own; otherwise a copy is queued
  behind the step on the compute stream. Either way an event recorded
  behind step n tells when slot ``n % depth`` holds step n. Slot reuse is
  safe because ``publish(n)`` consumes step ``n + 1 - depth`` before it
  returns, i.e. before the step that writes that slot again is queued; the
  host runs at most ``depth - 1`` steps ahead of the device.
"""
import contextlib
import ctypes
import gc
from collections import deque

import torch

from . import _lib


# Pinned host buffers and events of output rings that were dropped while a
# stream capture was running: freeing them then makes runtime calls that a
# capture forbids (the process aborts), so they are kept here and released
# at the next point known to be outside a capture.
_PARKED = []


def _capturing():
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def release_parked():
    """Free the ring buffers parked during a capture (no-op inside one)."""
    if _PARKED and not _capturing():
        _PARKED.clear()


class StepGraph:
    """One recorded decode step; :meth:`replay` launches it on the current stream."""

    def __init__(self, graph, stream, pool):
        self.graph, self.stream, self.pool = graph, stream, pool

    def replay(self):
        self.graph.replay()


@contextlib.contextmanager
def no_collection_while_recording():
    """Around a HIP graph recording: dead Python cycles (a finished engine's
    pinned output ring and its events, say) are freed before it, and no
    automatic collection runs inside it. Their destructors make runtime calls
    that a global-mode capture forbids, and an error raised there aborts the
    process. (This torch build collects before a capture only when asked to.)"""
    gc.collect()
    enabled = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if enabled:
            gc.enable()


def capture_decode(step, reset, warmups=2, pool=None):
    """Record ``step`` into a HIP graph.

    ``step`` runs ``warmups`` times first, each after ``reset``, on the
    capture stream, so that lazy set-up (library handles, workspaces, cached
    buffers) happens outside the recording; the recording itself also
    advances the state, so ``reset`` runs once more before returning. A
    ``pool`` (``torch.cuda.graph_pool_handle()``) lets several step graphs
    share their private memory. Stream priorities stay at the default."""
    if warmups < 1:
        raise ValueError("capture needs at least one warm-up step")
    caller = torch.cuda.current_stream()
    stream = torch.cuda.Stream(device=caller.device)
    stream.wait_stream(caller)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        for _ in range(warmups):
            reset()
            step()
        reset()
        stream.synchronize()
        with no_collection_while_recording():
            with torch.cuda.graph(graph, pool=pool, stream=stream):
                step()
    caller.wait_stream(stream)
    reset()
    torch.cuda.synchronize(caller.device)
    release_parked()
    return StepGraph(graph, stream, graph.pool() if pool is None else pool)


class OutputRing:
    """Ordered, exactly-once delivery of the per-step emit snapshots."""

    def __init__(self, emit, consume, asynchronous=False, depth=4):
        if depth < 2:
            raise ValueError("an asynchronous ring needs at least two slots")
        self.emit, self.consume = emit, consume
        self.asynchronous = asynchronous
        self.depth = depth
        self.pending = deque()        # published steps not yet consumed, ascending
        self.device_writes = False    # set once a step's epilogue writes the slots
        self._device_ptr = None
        self.counter = None
        if asynchronous:
            release_parked()
            self.host = torch.empty((depth, *emit.shape), dtype=emit.dtype, pin_memory=True)
            self.events = [torch.cuda.Event() for _ in range(depth)]

    def __del__(self):
        # Dropped during a capture (e.g. a finished engine collected while a
        # caller records its own graph): keep the pinned slots and events
        # alive until release_parked() runs outside the capture.
        if getattr(self, "asynchronous", False) and hasattr(self, "host") and _capturing():
            _PARKED.append((self.host, self.events))

    # -- device view -----------------------------------------------------
    def device_target(self, rows):
        """``(device address of the slots, depth, step counter)`` for the
        greedy epilogue to write into, and the counter the decode prologue
        increments. After this call :meth:`publish` copies nothing."""
        if not self.asynchronous:
            raise ValueError("only an asynchronous ring has host slots to write")
        if rows != self.emit.shape[0]:
            raise ValueError("emit rows do not match the ring")
        if self._device_ptr is None:
            address = ctypes.c_void_p()
            _lib.call("lm_host_device_pointer", self.host.data_ptr(), ctypes.byref(address))
            self._device_ptr = address.value
            self.counter = torch.zeros(1, dtype=torch.int64, device=self.emit.device)
        self.device_writes = True
        return self._device_ptr, self.depth, self.counter

    def start(self):
        """Begin a run of steps numbered from 0 (clears the step counter;
        captured warm-ups advance it too)."""
        if self.pending:
            raise RuntimeError("start() with snapshots still pending")
        if self.counter is not None:
            self.counter.zero_()

    # -- delivery ----------------------------------------------------------
    def _deliver(self, n):
        slot = n % self.depth
        self.events[slot].synchronize()
        self.consume(self.host[slot].tolist())

    def publish(self, n):
        """Step ``n`` (0, 1, 2, ... in order) has been queued."""
        if not self.asynchronous:
            self.consume(self.emit.cpu().tolist())
            return
        if self.pending and n != self.pending[-1] + 1:
            raise RuntimeError("steps must be published in order")
        slot = n % self.depth
        if not self.device_writes:
            self.host[slot].copy_(self.emit, non_blocking=True)
        self.events[slot].record()
        self.pending.append(n)
        # Step n + 1 writes slot (n + 1) % depth: deliver its previous
        # occupant now, then whatever else has already landed.
        while self.pending and (self.pending[0] <= n + 1 - self.depth
                                or self.events[self.pending[0] % self.depth].query()):
            self._deliver(self.pending.popleft())

    def drain(self):
        while self.pending:
            self._deliver(self.pending.popleft())
