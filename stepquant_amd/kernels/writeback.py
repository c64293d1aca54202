"""Deferred, graph-captured writeback of packed states (reference writeback.py:13-141).

During graph capture a forward pass can defer each layer's writer (the
``sq_writeback`` kernel) into chunks of ``writeback_chunk`` requests.  Chunks
are released at attention windows so the writer of layer L overlaps the
foreground work of later layers; a ``WritebackGraph`` then replays the
foreground graph and, unless the writers were joined into it, a separate
writer graph on the writeback stream, recording one completion event that
every pool's ``wait()`` orders against.  The release schedule (quotas per
window, early release for GDN and KDA early writeback) is the reference's.
"""
from collections import deque
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass
import math

import torch

_captured = ContextVar("stepquant_captured_writes", default=None)


def attention_window():
    """Release gate placed before attention work (including full attention)."""
    tasks = _captured.get()
    if tasks is not None and tasks.attention_windows:
        tasks.window_count += 1
        tasks.release_window()


@dataclass
class WritebackChunk:
    pool: object
    ready: object
    tensors: tuple
    final: bool


class CapturedWrites(list):
    """Released writer chunks, in release order; pending ones wait in a queue."""

    def __init__(self, attention_windows=False, joined=False):
        super().__init__()
        self.attention_windows = attention_windows
        self.joined = joined
        self.window_count = 0
        self.pending = deque()
        self.quota = 0
        self.layers = set()

    def release_window(self, count=None):
        # A capture-time GPU gate (an event), never a host-side wait.
        count = self.quota if count is None else count
        if not self.pending or not count:
            return
        ready = torch.cuda.Event()
        ready.record()
        for _ in range(min(count, len(self.pending))):
            pool, tensors, final = self.pending.popleft()
            super().append(WritebackChunk(pool, ready, tensors, final))
            if self.joined:
                # Joined writers run on the capturing stream itself: a graph
                # whose writer branch is forked to another stream and joined
                # at the end was observed to let queued replays overlap that
                # branch with the next replay on ROCm.
                pool._finish_update(*tensors)

    def append(self, task):
        pool, *tensors = task
        if id(pool) in self.layers:
            raise ValueError("a layer may write its state only once per forward graph")
        self.layers.add(id(pool))
        batch = tensors[-1].numel()
        chunk = pool.writeback_chunk or batch
        for start in range(0, batch, chunk):
            end = min(start + chunk, batch)
            self.pending.append((pool, tuple(t[start:end] for t in tensors), end == batch))
        chunks = math.ceil(batch / chunk)
        early_kda = pool.plan.architecture == "kda" and (pool.storage == "byte" or getattr(pool, "early_writeback", False))
        # Two release points per recurrent layer: releasing fewer than half
        # of its chunks at each would leave a tail at the end of the forward.
        early_quota = max(min(chunks, 3), math.ceil(chunks / 2))
        if self.attention_windows:
            self.quota = early_quota if early_kda else chunks
        else:
            self.quota = math.ceil(chunks / 2)
        if not self.attention_windows or pool.plan.architecture == "gdn" or early_kda:
            self.release_window()


@contextmanager
def defer_writeback(pools, *, attention_windows=False, joined=False):
    pools = tuple(pools)
    tasks = CapturedWrites(attention_windows, joined)
    if any(pool.deferred is not None for pool in pools):
        raise RuntimeError("nested writeback capture is unsupported")
    for pool in pools:
        pool.deferred = tasks
    token = _captured.set(tasks)
    try:
        yield tasks
        if attention_windows and tasks.layers and not tasks.window_count:
            raise RuntimeError("no attention release hooks executed during graph capture")
    finally:
        _captured.reset(token)
        tasks.release_window(len(tasks.pending))
        for pool in pools:
            pool.deferred = None


class WritebackGraph:
    """Foreground graph plus (unless joined) a writer graph on the writeback stream."""

    def __init__(self, forward, tasks, joined=False):
        self.forward = forward
        self.tasks = tasks  # keeps captured inputs and their views alive across replays
        self.stream = tasks[0].pool.writeback_stream
        self.pools = tuple(dict.fromkeys(task.pool for task in tasks))
        if any(pool.writeback_stream != self.stream for pool in self.pools):
            raise ValueError("captured layers must share one writeback stream")
        self.completion = torch.cuda.Event()
        self.background = None
        if joined:
            return
        # Without external events the writer graph cannot wait on release
        # events of the forward graph; replay() starts it after the forward.
        self.background = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.background, stream=self.stream):
            for task in tasks:
                task.pool._finish_update(*task.tensors)
                if task.final:
                    task.pool.graph_ready.record()
        for task in tasks:
            for tensor in task.tensors:
                tensor.record_stream(self.stream)

    def replay(self):
        seen = set()
        for pool in self.pools:
            if pool.pending and pool.completion not in seen:
                torch.cuda.current_stream().wait_event(pool.completion)
                seen.add(pool.completion)
        self.forward.replay()
        main = torch.cuda.current_stream()
        stream = self.stream if self.background is not None else main
        with torch.cuda.stream(stream):
            if self.background is not None:
                self.stream.wait_stream(main)
                self.background.replay()
            # a submitted (not captured) event also orders eager consumers
            self.completion.record()
            if self.background is None:
                for pool in self.pools:
                    if pool.captured_consumers:
                        pool.graph_ready.record()
        for pool in self.pools:
            pool.completion = self.completion
            pool.pending = True
