"""Serving-path behaviour on an MI355X: raw gates, GQA, strided q/k/v views,
bf16 inputs, padding slots, HIP-graph capture and deferred writeback graphs.

Mirrors the reference's tests/test_fused_cuda.py:58-153 and
tests/test_writeback_graph.py, with the CPU oracle as the numerical check.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import dev, device_plan, make_plan

pytestmark = pytest.mark.gpu


def _pool(oplan, slots, V, **kw):
    from stepquant_amd.kernels.pool import PackedStatePool
    return PackedStatePool(device_plan(oplan), slots, V, **kw)


@pytest.mark.parametrize("arch", ["gdn", "kda"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("batch", [3, 16])
@pytest.mark.parametrize("asynchronous", [False, True])
def test_raw_gates_gqa_strides_padding_and_graph(arch, dtype, batch, asynchronous):
    print(f"case {arch} {dtype} B={batch} async={asynchronous}", flush=True)
    torch.manual_seed(8)
    h, hq, k, v = 4, 2, 32, 32
    oplan = make_plan(arch, np.full((h, k), 6), impact=np.ones((h, k)))
    pool = _pool(oplan, batch + 1, v, writeback_stream=torch.cuda.Stream() if asynchronous else None)
    d = dev()
    slots = torch.arange(batch - 1, -1, -1, device=d)  # last request is padding (slot 0)
    mixed = torch.randn(batch, 2 * hq * k + h * v, device=d, dtype=dtype)
    q, key, val = mixed.split([hq * k, hq * k, h * v], -1)
    a = torch.randn(batch, h, k, device=d) if arch == "kda" else torch.randn(batch, h, device=d)
    bias = torch.randn(h * k if arch == "kda" else h, device=d)
    a_log = torch.randn(h, device=d)
    beta = torch.randn(batch, h, device=d)
    pool.encode(torch.randn(batch, h, k, v, device=d) * .1, slots)

    def call():
        return pool.step(q, key, val, a, beta, slots, normalize=True, scale=k ** -.5, a_log=a_log, dt_bias=bias)

    call()
    pool.wait()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
        pool.wait()
    lay = O.layout(oplan, v)
    for _ in range(3):
        torch.cuda.synchronize()
        state = O.decode_page(pool.data.cpu().numpy(), slots.cpu().numpy(), oplan, lay, v)
        qp, kp, ld, bt = O.prepare(q.float().cpu().numpy(), key.float().cpu().numpy(), a.cpu().numpy(),
                                   beta.cpu().numpy(), h, k, arch == "kda", True, k ** -.5,
                                   a_log.cpu().numpy(), bias.cpu().numpy())
        expected, _ = O.delta_step(state, qp, kp, val.float().cpu().numpy().reshape(batch, h, v), ld, bt)
        graph.replay()
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        if dtype == torch.float32:
            np.testing.assert_allclose(got[:-1], expected[:-1], rtol=1e-3, atol=1e-4)
        else:
            np.testing.assert_allclose(got[:-1], expected[:-1].astype(np.float32), rtol=.008, atol=.002)
        assert not got[-1].any()
        assert pool.data[0].count_nonzero() == 0


@pytest.mark.parametrize("arch", ["gdn", "kda"])
def test_multilayer_graph_replay_and_slot_reuse(arch):
    """Reference tests/test_fused_cuda.py:120-153 (graph vs eager twins)."""
    torch.manual_seed(51)
    bits = np.repeat(np.array([2, 4, 6, 16])[:, None], 32, 1)
    if arch == "kda":
        bits[:, ::3] = 16
    oplan = make_plan(arch, bits, seed=4)
    stream = torch.cuda.Stream()
    pools = [_pool(oplan, 6, 32, writeback_stream=stream) for _ in range(3)]
    refs = [_pool(oplan, 6, 32) for _ in pools]
    d = dev()
    slots = torch.tensor([3, 1, 0], device=d)
    q = torch.randn(3, 4, 32, device=d)
    k = torch.nn.functional.normalize(torch.randn_like(q), dim=-1)
    v = torch.randn_like(q)
    g = -torch.rand_like(q) if arch == "kda" else -torch.rand(3, 4, device=d)
    beta = torch.rand(3, 4, device=d)

    def forward():
        outs = [pool.step(q, k, v, g, beta, slots) for pool in pools]
        for pool in pools:
            pool.wait()
        return outs

    for _ in range(3):
        forward()
    for pool in pools:
        pool.clear(slots)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outputs = forward()
    for step in range(8):
        if step == 4:
            src, dst = torch.tensor([3], device=d), torch.tensor([4], device=d)
            for pool in pools + refs:
                pool.copy(src, dst)
            slots.copy_(torch.tensor([4, 1, 0], device=d))
        graph.replay()
        for pool, ref, output in zip(pools, refs, outputs):
            expected = ref.step(q, k, v, g, beta, slots)
            torch.testing.assert_close(output, expected, atol=0, rtol=0)
            assert torch.equal(pool.decode(slots), ref.decode(slots))
            assert pool.data[0].count_nonzero() == 0


@pytest.mark.parametrize("arch", ["gdn", "kda"])
@pytest.mark.parametrize("attention_windows", [False, True])
@pytest.mark.parametrize("joined", [False, True])
@pytest.mark.parametrize("large_batch", [16, 64])
def test_split_graph_queued_replays_and_batch_switch(arch, attention_windows, joined, large_batch):
    """Reference tests/test_writeback_graph.py:11-90 on deferred writer chunks."""
    from stepquant_amd.kernels.writeback import WritebackGraph, attention_window, defer_writeback
    print(f"case {arch} windows={attention_windows} joined={joined} B={large_batch}", flush=True)
    torch.manual_seed(92)
    size = 32
    bits = np.repeat(np.array([2, 4, 6, 16])[:, None], size, 1)
    if arch == "kda":
        bits[:, ::5] = 16
    oplan = make_plan(arch, bits, seed=9)
    from stepquant_amd.kernels.resources import writeback_resources
    resources = writeback_resources("cuda:0", 32)
    assert 0 < resources.actual_sms <= resources.total_sms
    stream = resources.stream
    capacity = max(20, large_batch + 1)
    workspace = {}
    pools = [_pool(oplan, capacity, size, writeback_stream=stream, writeback_workspace=workspace,
                   writeback_chunk=5) for _ in range(3)]
    assert len({pool.coefficients.data_ptr() for pool in pools}) == 1
    ref_stream = torch.cuda.Stream()
    refs = [_pool(oplan, capacity, size, writeback_stream=ref_stream) for _ in pools]
    graphs, inputs, outputs = {}, {}, {}
    shared = torch.cuda.graph_pool_handle()
    d = dev()
    for batch in (large_batch, 3):
        slots = torch.arange(batch, 0, -1, device=d)
        slots[-1] = 0
        q = torch.randn(batch, 4, size, device=d)
        k = torch.nn.functional.normalize(torch.randn_like(q), dim=-1)
        v = torch.randn_like(q)
        g = -torch.rand_like(q) if arch == "kda" else -torch.rand(batch, 4, device=d)
        beta = torch.rand(batch, 4, device=d)
        inputs[batch] = (q, k, v, g, beta, slots)
        for _ in range(2):
            for pool in pools:
                pool.step(*inputs[batch])
        torch.cuda.synchronize()
        fg = torch.cuda.CUDAGraph()
        with torch.cuda.graph(fg, pool=shared):
            with defer_writeback(pools, attention_windows=attention_windows,
                                 joined=joined and batch == large_batch) as tasks:
                outputs[batch] = []
                for pool in pools:
                    attention_window()
                    outputs[batch].append(pool.step(*inputs[batch]))
                    attention_window()
        graphs[batch] = WritebackGraph(fg, tasks, joined=joined and batch == large_batch)
    all_slots = torch.arange(capacity, device=d)
    for pool in pools:
        pool.clear(all_slots)
    sequence = [large_batch, 3, large_batch, large_batch, 3, 3] * 3
    actual = []
    for index, batch in enumerate(sequence):
        if index == 7:
            for pool in pools:
                pool.copy(all_slots[1:2], all_slots[2:3])
                pool.clear(all_slots[3:4])
        graphs[batch].replay()
        actual.append([x.clone() for x in outputs[batch]])
    actual_eager = [pool.step(*inputs[3]).clone() for pool in pools]
    graphs[large_batch].replay()
    actual_last = [x.clone() for x in outputs[large_batch]]
    for index, batch in enumerate(sequence):
        if index == 7:
            for pool in refs:
                pool.copy(all_slots[1:2], all_slots[2:3])
                pool.clear(all_slots[3:4])
        for ref, result in zip(refs, actual[index]):
            torch.testing.assert_close(result, ref.step(*inputs[batch]), atol=0, rtol=0)
    for ref, result in zip(refs, actual_eager):
        torch.testing.assert_close(result, ref.step(*inputs[3]), atol=0, rtol=0)
    for ref, result in zip(refs, actual_last):
        torch.testing.assert_close(result, ref.step(*inputs[large_batch]), atol=0, rtol=0)
    for pool, ref in zip(pools, refs):
        assert torch.equal(pool.decode(all_slots), ref.decode(all_slots))
        assert pool.data[0].count_nonzero() == 0


@pytest.mark.parametrize("arch", ["gdn", "kda"])
def test_queued_replays_of_captured_async_steps(arch):
    """Graph replays queued back to back (no host sync) match eager twins.

    Regression test: a writer forked to the writeback stream inside a capture
    overlapped the next queued replay; captured writers now stay on the
    capturing stream.
    """
    bits = np.repeat(np.array([6, 4, 8, 16])[:, None], 128, 1) if arch == "gdn" else \
        np.where(np.random.default_rng(1).random((4, 128)) < .05, 16, np.random.default_rng(2).choice([4, 6, 8], (4, 128)))
    oplan = make_plan(arch, bits, seed=12)
    d = dev()
    B = 32
    pools = [_pool(oplan, B + 1, 128, writeback_stream=torch.cuda.Stream()) for _ in range(2)]
    refs = [_pool(oplan, B + 1, 128) for _ in pools]
    slots = torch.arange(1, B + 1, device=d)
    x = torch.randn(B, 4, 128, 128, device=d) * .1
    for p in pools + refs:
        p.encode(x, slots)
    g = torch.Generator(device=d).manual_seed(3)
    q = torch.randn(B, 4, 128, device=d, generator=g)
    k = torch.nn.functional.normalize(torch.randn(B, 4, 128, device=d, generator=g), dim=-1)
    v = torch.randn(B, 4, 128, device=d, generator=g)
    gate = -torch.rand(B, 4, 128, device=d, generator=g) if arch == "kda" else -torch.rand(B, 4, device=d, generator=g)
    beta = torch.rand(B, 4, device=d, generator=g)

    def forward():
        outs = [p.step(q, k, v, gate, beta, slots) for p in pools]
        for p in pools:
            p.wait()
        return outs

    forward()
    for p, r in zip(pools, refs):
        r.step(q, k, v, gate, beta, slots)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = forward()
    got = []
    for _ in range(6):
        graph.replay()
        got.append([o.clone() for o in outs])
    torch.cuda.synchronize()
    for step in range(6):
        for r, o in zip(refs, got[step]):
            torch.testing.assert_close(o, r.step(q, k, v, gate, beta, slots), atol=0, rtol=0)
    for p, r in zip(pools, refs):
        assert torch.equal(p.data, r.data)
