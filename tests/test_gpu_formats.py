"""Baseline-format pages (FormatStatePool, reference kernels/format_pool.py)
on an MI355X, against the CPU oracle.

Bars: encode and decode bit-identical to the oracle's group_fit / dual_fit
page for the same input; a decode step's readout within the reference's own
bar (atol 1e-5, rtol 1e-4, tests/test_formats_cuda.py:37) of delta_step on the
decoded state; the re-encoded page equal to the oracle's encoding of the
oracle's updated state except for codes one level apart on at most 0.5% of
values (the two fp32 updates differ in summation order), every decoded value
within the reference's 5e-3 and at most 0.1% outside rtol 1e-3 / atol 1e-4.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import dev

pytestmark = pytest.mark.gpu

NAMES = ["fp32", "sym_int4_g128", "sym_int6_g128", "sym_int8_g128", "dsq_int4", "dsq_int6"]


def _pool(name, arch, H, K, V, slots):
    from stepquant_amd.formats import FormatPlan, get_format
    from stepquant_amd.kernels.format_pool import FormatStatePool
    spec = get_format(name)
    bits = torch.full((H, K), spec.bits, device=dev(), dtype=torch.int32)
    plan = FormatPlan(arch, bits, torch.ones((H, K), device=dev()))
    return FormatStatePool(plan, slots, V, spec)


def _codes(pages, slots, name, lay, H, K, V):
    kind, b, _ = O.format_spec(name)
    out = np.zeros((len(slots), H, K, V), np.int64)
    for n, s in enumerate(slots):
        if s <= 0:
            continue
        for r in range(H * K):
            off = int(lay.offsets[r])
            out[n, r // K, r % K] = O.unpack(pages[s, off:off + V * b // 8], b, V)
    return out


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("arch", ["gdn", "kda"])
def test_format_encode_step_against_oracle(name, arch):
    print(f"case {name} {arch}", flush=True)
    kind = O.format_spec(name)[0]
    H, K, V = 2, 32, 128
    pool = _pool(name, arch, H, K, V, 4)
    lay = O.format_layout(np.full((H, K), O.format_spec(name)[1]), V, kind, O.format_spec(name)[2])
    assert pool.page_bytes == lay.page_bytes
    g = torch.Generator().manual_seed(42)
    slots = torch.tensor([1, 2], device=dev())
    sl = slots.cpu().numpy()
    x = torch.randn(2, H, K, V, generator=g) * .3
    pool.encode(x.to(dev()), slots)
    ref = np.zeros((4, lay.page_bytes), np.uint8)
    O.format_encode_page(x.numpy(), sl, name, lay, ref)
    got = pool.data.cpu().numpy()
    assert (got != ref).sum() == 0, f"encode: {(got != ref).sum()} bytes differ"
    np.testing.assert_array_equal(pool.decode(slots).cpu().numpy(),
                                  O.format_decode_page(ref, sl, name, lay, H, K, V))
    for it in range(3):
        initial = pool.decode(slots).cpu().numpy()
        q = torch.nn.functional.normalize(torch.randn(2, H, K, generator=g), dim=-1)
        key = torch.nn.functional.normalize(torch.randn(2, H, K, generator=g), dim=-1)
        val = torch.randn(2, H, V, generator=g)
        gate = -torch.rand((2, H, K) if arch == "kda" else (2, H), generator=g)
        beta = torch.rand(2, H, generator=g)
        expected, updated = O.delta_step(initial, q.numpy(), key.numpy(), val.numpy(), gate.numpy(), beta.numpy())
        out = pool.step(q.to(dev()), key.to(dev()), val.to(dev()), gate.to(dev()), beta.to(dev()), slots)
        torch.testing.assert_close(out.cpu(), torch.from_numpy(expected), atol=1e-5, rtol=1e-4)
        got = pool.data.cpu().numpy()
        ref = np.zeros_like(got)
        O.format_encode_page(updated, sl, name, lay, ref)
        actual = O.format_decode_page(got, sl, name, lay, H, K, V)
        oracle = O.format_decode_page(ref, sl, name, lay, H, K, V)
        np.testing.assert_allclose(actual, oracle, atol=5e-3, rtol=5e-3)
        assert (~np.isclose(actual, oracle, rtol=1e-3, atol=1e-4)).mean() <= 1e-3
        if kind != "fp32":
            diff = np.abs(_codes(got, sl, name, lay, H, K, V) - _codes(ref, sl, name, lay, H, K, V))
            assert diff.max() <= 1 and (diff > 0).mean() <= 5e-3, f"step {it}: {(diff > 0).mean():.2e} codes differ"
    # slot operations and masking (tests/test_formats_cuda.py:41-49)
    pool.copy(slots[:1], slots[1:])
    d = pool.decode(slots)
    assert torch.equal(d[0], d[1])
    pool.clear(slots)
    assert pool.decode(slots).count_nonzero() == 0
    padded = torch.tensor([0, -1], device=dev())
    saved = pool.data.clone()
    assert pool.step(q.to(dev()), key.to(dev()), val.to(dev()), gate.to(dev()), beta.to(dev()),
                     padded).count_nonzero() == 0
    assert torch.equal(pool.data, saved)


@pytest.mark.parametrize("name", NAMES)
def test_format_full_heads_raw_gates(name):
    """K = V = 128, GQA, bf16 inputs, raw gates with A_log / dt_bias, normalize."""
    print(f"case {name}", flush=True)
    kind, b, group = O.format_spec(name)
    H, HK, K, V, B = 4, 2, 128, 128, 6
    pool = _pool(name, "gdn", H, K, V, B + 2)
    lay = O.format_layout(np.full((H, K), b), V, kind, group)
    g = torch.Generator().manual_seed(5)
    slots_np = np.array([3, 1, 0, 7, 2, 5])
    slots = torch.from_numpy(slots_np).to(dev())
    x = torch.randn(B, H, K, V, generator=g) * torch.exp(torch.randn(B, H, K, 1, generator=g) * .5) * .1
    pool.encode(x.to(dev()), slots)
    ref = np.zeros((B + 2, lay.page_bytes), np.uint8)
    O.format_encode_page(x.numpy(), slots_np, name, lay, ref)
    assert (pool.data.cpu().numpy() != ref).sum() == 0
    q = torch.randn(B, HK * K, generator=g).to(torch.bfloat16)
    k = torch.randn(B, HK * K, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H * V, generator=g).to(torch.bfloat16)
    a = torch.randn(B, H, generator=g)
    bl = torch.randn(B, H, generator=g)
    a_log = torch.randn(H, generator=g) * .3
    dt_bias = torch.randn(H, generator=g) * .3
    state = O.format_decode_page(ref, slots_np, name, lay, H, K, V)
    qp, kp, ld, bo = O.prepare(q.float().numpy(), k.float().numpy(), a.numpy(), bl.numpy(), H, K, False, True,
                               K ** -.5, a_log.numpy(), dt_bias.numpy())
    expected, _ = O.delta_step(state, qp, kp, v.float().numpy().reshape(B, H, V), ld, bo)
    out = pool.step(q.to(dev()), k.to(dev()), v.to(dev()), a.to(dev()), bl.to(dev()), slots, normalize=True,
                    scale=K ** -.5, a_log=a_log.to(dev()), dt_bias=dt_bias.to(dev()))
    assert out.dtype == torch.bfloat16
    live = slots_np > 0
    o = out.float().cpu().numpy()
    np.testing.assert_allclose(o[live], expected[live], rtol=2 ** -8, atol=1e-4)
    assert not o[~live].any()


@pytest.mark.parametrize("name", ["fp32", "sym_int6_g128", "dsq_int4"])
@pytest.mark.parametrize("arch", ["gdn", "kda"])
@pytest.mark.parametrize("batch", [2, 64, 512])
def test_format_graph_replay_matches_eager(name, arch, batch):
    """tests/test_formats_cuda.py:52-75: a captured step equals the eager one."""
    print(f"case {name} {arch} {batch}", flush=True)
    torch.manual_seed(11)
    H, K, V = 2, 128, 128
    pool = _pool(name, arch, H, K, V, batch + 1)
    slots = torch.arange(1, batch + 1, device=dev())
    q, key = [torch.nn.functional.normalize(torch.randn(batch, H, K, device=dev()), dim=-1) for _ in range(2)]
    val = torch.randn(batch, H, V, device=dev())
    gate = -torch.rand_like(q) if arch == "kda" else -torch.rand(batch, H, device=dev())
    beta = torch.rand(batch, H, device=dev())
    for _ in range(3):
        pool.step(q, key, val, gate, beta, slots)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pool.step(q, key, val, gate, beta, slots)
    for rep in range(3):
        pool.clear(slots)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        actual, packed = out.clone(), pool.data.clone()
        pool.clear(slots)
        expected = pool.step(q, key, val, gate, beta, slots)
        torch.cuda.synchronize()
        assert torch.equal(actual, expected), f"replay {rep}"
        assert torch.equal(pool.data, packed), f"replay {rep}"
