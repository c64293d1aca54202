"""Deferred writeback of recurrent-state pages under graph capture.

The role of the reference's kernels/writeback.py:13-141 (public names
``attention_window``, ``defer_writeback``, ``CapturedWrites``,
``WritebackChunk`` and ``WritebackGraph`` are kept, so the serving adapter
binds unchanged), built on this package's writer kernel (``sq_writeback``)
and on ``GraphEvent`` nodes.

While a forward pass is captured inside ``defer_writeback``, every layer's
step queues its writer as chunks of ``writeback_chunk`` requests instead of
launching it.  Chunks leave the queue at release points: a GDN layer (or a
KDA layer with early writeback) releases right after its readout, other
layers at the next ``attention_window()``.  How many chunks a release point
takes is the reference's rule, which its schedule tests pin: with attention
windows a layer releases all its chunks at once, an early-writeback KDA
layer ``max(min(n, 3), ceil(n / 2))`` per point; without windows,
``ceil(n / 2)`` per point.  Whatever is still queued leaves when the
deferral ends.

Two ways to run the released writers:

* joined (the serving path): a released chunk's writer is forked onto the
  writeback stream inside the captured graph, at its release point, and the
  branch rejoins the capturing stream when the deferral ends.  Layer L's
  writer runs beside layers L+1... of the same replay; a replay ends with
  its last writer.
* paired: each release point records a ``GraphEvent`` node in the forward
  graph.  ``WritebackGraph`` captures the writers into a second graph on
  the writeback stream whose chunks wait on those nodes, and launches it
  right behind the forward graph: the forward graph finishes without
  waiting for the writers of its last layers, and the next forward waits on
  each layer's own writer (through the pool's ``graph_ready``).
"""
from __future__ import annotations

import math
from collections import deque
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass

import torch

from .events import GraphEvent, wait_for

_active = ContextVar("stepquant_deferred_writes", default=None)


@dataclass
class WritebackChunk:
    """One released writer chunk: ``tensors`` are the pool's scratch views of
    the chunk's requests; ``ready`` is the release point's event (paired
    mode) or None; ``final`` marks the pool's last chunk."""
    pool: object
    ready: object
    tensors: tuple
    final: bool


def _release_quota(pool, chunks, attention_windows):
    """Chunks a release point takes for a layer of ``chunks`` chunks."""
    if not attention_windows:
        return math.ceil(chunks / 2)
    if _early_kda(pool):
        return max(min(chunks, 3), math.ceil(chunks / 2))
    return chunks


def _early_kda(pool):
    return pool.plan.architecture == "kda" and (pool.storage == "byte" or getattr(pool, "early_writeback", False))


class CapturedWrites(list):
    """The chunks of one captured forward, in release order."""

    def __init__(self, attention_windows=False, joined=False):
        super().__init__()
        self.attention_windows = attention_windows
        self.joined = joined
        self.window_count = 0
        self.pending = deque()   # (pool, tensors, final) not yet released
        self.quota = 0
        self.layers = set()
        self._forked = set()     # writeback streams with a captured branch to join

    # -- called by PackedStatePool._schedule_writeback -------------------
    def append(self, task):
        pool, *tensors = task
        if id(pool) in self.layers:
            raise ValueError("a layer may write its state only once per forward graph")
        self.layers.add(id(pool))
        batch = tensors[-1].numel()
        size = pool.writeback_chunk or batch
        starts = range(0, batch, size)
        for start in starts:
            stop = min(start + size, batch)
            self.pending.append((pool, tuple(t[start:stop] for t in tensors), stop == batch))
        self.quota = _release_quota(pool, len(starts), self.attention_windows)
        if not self.attention_windows or pool.plan.architecture == "gdn" or _early_kda(pool):
            self.release_window()

    # -- release points -------------------------------------------------------
    def release_window(self, count=None):
        """Release up to ``count`` (default: the quota) queued chunks here.

        Capture-time only: it adds graph nodes, it never waits on the host."""
        count = self.quota if count is None else count
        count = min(count, len(self.pending))
        if count <= 0:
            return
        here = torch.cuda.current_stream()
        gate = None
        if not self.joined:
            gate = GraphEvent()
            gate.record(here)
        released = []
        for _ in range(count):
            pool, tensors, final = self.pending.popleft()
            super().append(WritebackChunk(pool, gate, tensors, final))
            released.append((pool, tensors))
        if self.joined:
            self._fork(here, released)

    def _fork(self, here, released):
        """Fork the released writers onto their writeback stream(s): one
        dependency edge from the capturing stream per release point, then
        the chunks as a chain on the writeback stream.  (A captured node
        whose dependents fan out to many nodes of another stream broke the
        ordering of queued replays against the work queued between them on
        ROCm; one edge per release point keeps the ordering.)"""
        forked = set()
        for pool, tensors in released:
            side = pool.writeback_stream
            if side not in forked:
                side.wait_stream(here)
                forked.add(side)
            with torch.cuda.stream(side):
                pool._finish_update(*tensors)
        self._forked |= forked

    def close(self):
        """End of the deferral: release the rest, rejoin forked writers."""
        self.release_window(len(self.pending))
        here = torch.cuda.current_stream()
        for side in self._forked:
            here.wait_stream(side)
        self._forked.clear()


def attention_window():
    """Release point placed before attention work (full attention included)."""
    tasks = _active.get()
    if tasks is not None and tasks.attention_windows:
        tasks.window_count += 1
        tasks.release_window()


@contextmanager
def defer_writeback(pools, *, attention_windows=False, joined=False):
    """Defer the writers of ``pools`` while a forward pass is captured."""
    pools = tuple(pools)
    if any(pool.deferred is not None for pool in pools):
        raise RuntimeError("nested writeback capture is unsupported")
    tasks = CapturedWrites(attention_windows, joined)
    for pool in pools:
        pool.deferred = tasks
    token = _active.set(tasks)
    try:
        yield tasks
        if attention_windows and tasks.layers and not tasks.window_count:
            raise RuntimeError("no attention release hooks executed during graph capture")
    finally:
        _active.reset(token)
        tasks.close()
        for pool in pools:
            pool.deferred = None


class WritebackGraph:
    """A captured forward graph with its deferred writers.

    Joined: the writers are inside ``forward``.  Paired: a writer graph on the
    writeback stream, captured here, waits on the forward graph's release
    nodes.  ``replay()`` leaves every pool pending on ``completion``."""

    def __init__(self, forward, tasks, joined=False):
        self.forward = forward
        self.tasks = tasks   # the captured scratch views stay alive with the graph
        self.pools = tuple(dict.fromkeys(chunk.pool for chunk in tasks))
        self.stream = tasks[0].pool.writeback_stream
        if any(pool.writeback_stream != self.stream for pool in self.pools):
            raise ValueError("captured layers must share one writeback stream")
        self.joined = joined
        self.completion = GraphEvent()
        self.writers = None
        if joined:
            return
        self.writers = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.writers, stream=self.stream):
            gate = None
            for chunk in tasks:
                if chunk.ready is not gate:   # one wait node per release point
                    gate = chunk.ready
                    gate.wait(self.stream)
                chunk.pool._finish_update(*chunk.tensors)
                if chunk.final:
                    chunk.pool.graph_ready.record(self.stream)
        for chunk in tasks:
            for tensor in chunk.tensors:
                tensor.record_stream(self.stream)

    def replay(self):
        here = torch.cuda.current_stream()
        # Writers launched outside this graph (eager steps, another graph)
        # finish before it reads their pages.
        done = set()
        for pool in self.pools:
            if pool.pending and id(pool.completion) not in done:
                wait_for(here, pool.completion)
                done.add(id(pool.completion))
        self.forward.replay()
        if self.writers is not None:
            with torch.cuda.stream(self.stream):
                self.writers.replay()
                self.completion.record(self.stream)
        else:
            self.completion.record(here)
            for pool in self.pools:
                if pool.captured_consumers:
                    # consumers captured elsewhere wait on graph_ready
                    pool.graph_ready.record(here)
        for pool in self.pools:
            pool.completion = self.completion
            pool.pending = True
