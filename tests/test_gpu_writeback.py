"""Ordering contract of the deferred writer on an MI355X, with a writer
slowed by a bounded spin (``torch.cuda._sleep``) so that missing
dependencies show up as wrong pages or wrong event states.

The behaviour follows the reference's tests/test_writeback_graph.py:91-236
(forward ends before a paired writer; several consumer streams; graph
allocations never alias writer inputs; a joined writer protects a consumer
captured in another graph, whatever produces next), checked here against
twin pools stepped eagerly.
"""
import numpy as np
import pytest
import torch

from tests.helpers import dev, device_plan, make_plan

pytestmark = pytest.mark.gpu

SPIN = 50_000_000   # cycles of torch.cuda._sleep: tens of milliseconds


def _pool(arch, slots, V=32, storage="packed", stream=None):
    from stepquant_amd.kernels.pool import PackedStatePool
    oplan = make_plan(arch, np.full((1, 32), 4), impact=np.ones((1, 32)))
    return PackedStatePool(device_plan(oplan), slots, V, writeback_stream=stream or torch.cuda.Stream(),
                           storage=storage)


def _slow_writer(monkeypatch, pool):
    original = pool._finish_update

    def slow(*tensors):
        torch.cuda._sleep(SPIN)
        return original(*tensors)

    monkeypatch.setattr(pool, "_finish_update", slow)


def _inputs(B, arch, seed=0):
    g = torch.Generator(device=dev()).manual_seed(seed)
    q = torch.randn(B, 1, 32, device=dev(), generator=g)
    k = torch.nn.functional.normalize(torch.randn(B, 1, 32, device=dev(), generator=g), dim=-1)
    v = torch.randn(B, 1, 32, device=dev(), generator=g)
    gate = -torch.rand(B, 1, 32, device=dev(), generator=g) * .1 if arch == "kda" else \
        -torch.rand(B, 1, device=dev(), generator=g) * .1
    beta = torch.rand(B, 1, device=dev(), generator=g) * .5 + .25
    return q, k, v, gate, beta


def test_forward_completes_before_its_paired_writer(monkeypatch):
    """The foreground and the writer run on two streams created one after the
    other: streams share the device's few hardware queues round-robin (two
    streams on one queue run in submission order), and work on the legacy
    default stream waits for blocking streams, so neither is used here."""
    from stepquant_amd.kernels.writeback import WritebackGraph, defer_writeback
    print("case paired writer after forward", flush=True)
    foreground, side = torch.cuda.Stream(), torch.cuda.Stream()
    pool = _pool("gdn", 2, stream=side)
    slots = torch.ones(1, device=dev(), dtype=torch.long)
    args = (*_inputs(1, "gdn"), slots)
    with torch.cuda.stream(foreground):
        pool.step(*args)
        torch.cuda.synchronize()
        forward = torch.cuda.CUDAGraph()
        with torch.cuda.graph(forward):
            with defer_writeback([pool]) as tasks:
                pool.step(*args)
        _slow_writer(monkeypatch, pool)
        graph = WritebackGraph(forward, tasks)
        graph.replay()
        done = torch.cuda.Event()
        done.record(foreground)
        done.synchronize()
        assert not pool.graph_ready.query(), "the forward graph waited for its writer"
        assert not graph.completion.query()
        pool.wait()
    torch.cuda.synchronize()
    assert pool.graph_ready.query() and graph.completion.query()


def test_every_consumer_stream_keeps_its_dependency(monkeypatch):
    print("case two consumer streams", flush=True)
    pool = _pool("kda", 2)
    slots = torch.ones(1, device=dev(), dtype=torch.long)
    args = (*_inputs(1, "kda"), slots)
    pool.step(*args)
    torch.cuda.synchronize()
    _slow_writer(monkeypatch, pool)
    pool.step(*args)
    first, second = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(first):
        pool.wait()
    with torch.cuda.stream(second):
        pool.wait()
        consumed = torch.cuda.Event()
        consumed.record()
    consumed.synchronize()
    assert pool.completion.query(), "the second stream did not wait for the writer"


def test_graph_allocations_do_not_alias_writer_inputs(monkeypatch):
    from stepquant_amd.kernels.writeback import WritebackGraph, defer_writeback
    print("case graph prefix allocation vs writer inputs", flush=True)
    pool = _pool("kda", 5)
    ref = _pool("kda", 5)
    slots = torch.arange(1, 5, device=dev())
    args = (*_inputs(4, "kda", 7), slots)
    state = torch.randn(4, 1, 32, 32, device=dev()) * .1
    pool.step(*args)
    torch.cuda.synchronize()
    forward = torch.cuda.CUDAGraph()
    with torch.cuda.graph(forward):
        prefix = torch.empty_like(args[0])   # freed before the layer: the pool may reuse it
        prefix.fill_(1000.)
        del prefix
        with defer_writeback([pool]) as tasks:
            out = pool.step(*args)
    _slow_writer(monkeypatch, pool)
    graph = WritebackGraph(forward, tasks)
    pool.encode(state, slots)
    ref.encode(state, slots)
    graph.replay()
    graph.replay()
    ref.step(*args)
    expected = ref.step(*args)
    ref.wait()
    torch.testing.assert_close(out, expected, atol=0, rtol=0)
    assert torch.equal(pool.decode(slots), ref.decode(slots))


@pytest.mark.parametrize("next_producer", ["same", "joined", "paired", "eager"])
def test_consumer_captured_elsewhere_waits_for_the_writer(monkeypatch, next_producer):
    from stepquant_amd.kernels.writeback import WritebackGraph, defer_writeback
    print(f"case captured consumer, next producer {next_producer}", flush=True)
    pool = _pool("kda", 2, storage="byte")
    slots = torch.ones(1, device=dev(), dtype=torch.long)
    q, k, v, gate, beta = _inputs(1, "kda", 3)
    v.fill_(1.)
    args = (q, k, v, gate, beta, slots)
    for _ in range(2):
        pool.step(*args)
    torch.cuda.synchronize()
    _slow_writer(monkeypatch, pool)
    forward = torch.cuda.CUDAGraph()
    with torch.cuda.graph(forward):
        with defer_writeback([pool], joined=True) as tasks:
            pool.step(*args)
    graph = WritebackGraph(forward, tasks, joined=True)
    graph.replay()
    torch.cuda.synchronize()
    consumer = torch.cuda.CUDAGraph()
    with torch.cuda.graph(consumer):
        observed = pool.decode(slots)
    if next_producer in ("joined", "paired"):
        other = torch.cuda.CUDAGraph()
        joined = next_producer == "joined"
        with torch.cuda.graph(other):
            with defer_writeback([pool], joined=joined) as tasks:
                pool.step(*args)
        graph = WritebackGraph(other, tasks, joined=joined)
    v.fill_(7.)
    producer = torch.cuda.Stream()
    producer.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(producer):
        if next_producer == "eager":
            pool.step(*args)
        else:
            graph.replay()
    consumer.replay()
    done = torch.cuda.Event()
    done.record()
    done.synchronize()
    assert pool.completion.query(), "the captured consumer ran before the producer's writer"
    torch.testing.assert_close(observed, pool.decode(slots), atol=0, rtol=0)
