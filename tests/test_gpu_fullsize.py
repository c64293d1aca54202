"""The benchmark shapes themselves (MI355X): G6 and K6 decode steps over
B=256 requests x 32 heads, the G4 step over B=512 requests (per-head widths
{2,4,6,8}, log-normal row and column scales), and the P6 prefill (8 sequences
of 2048 tokens, 32 value heads over 16 key heads, 5 prefix slots per
sequence).  The whole problem runs on the GPU; the float oracle checks eight
requests spread over the batch (tiles are independent) and, for prefill,
eight heads over all sequences, and the properties that need no oracle are
checked everywhere: the fused step equals the split readout + writer bit for
bit, every output is finite, the sentinel page stays zero, every prefix page
is the oracle encoding of the kernel's state.
"""
import numpy as np
import pytest
import torch

import bench
from oracle import oracle as O
from tests.helpers import PREFILL_REFIT_BUDGET, check_prefill, check_requant, check_states, dev, make_plan, sub_pages
from tests.test_gpu_pool import _check_requant

pytestmark = pytest.mark.gpu

SAMPLE = 8


def _oracle_plan(arch, bits, impact):
    return make_plan(arch, bits.numpy(), impact=impact.numpy())


def _spread(B, n=SAMPLE):
    return np.unique(np.linspace(0, B - 1, n).round().astype(np.int64))


SHAPES = {
    # name: arch, B, HK, nominal width, log-normal row/column scales
    "G6": ("gdn", 256, 16, 6, False),
    "K6": ("kda", 256, 32, 6, False),
    "G4": ("gdn", 512, 16, 4, True),
}


@pytest.mark.parametrize("name", list(SHAPES))
def test_decode_step_at_bench_shape(name):
    arch, B, HK, nominal, lognormal = SHAPES[name]
    print(f"case {name}: {arch} B={B} H=32 HK={HK} @{nominal}", flush=True)
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    H, K, V = 32, 128, 128
    bits, impact = bench.make_plan(torch, arch, H, K, nominal)
    plan = QuantizationPlan(arch, bits.to(dev()), impact.to(dev()))
    oplan = _oracle_plan(arch, bits, impact)
    fused = PackedStatePool(plan, B + 1, V)
    split = PackedStatePool(plan, B + 1, V, writeback_stream=torch.cuda.Stream())
    g = torch.Generator(device=dev()).manual_seed(5)
    slots = torch.arange(1, B + 1, device=dev())
    if lognormal:
        r = torch.exp(torch.randn(B, H, K, 1, device=dev(), generator=g) * .5)
        c = torch.exp(torch.randn(B, H, 1, V, device=dev(), generator=g) * .5)
        x0 = r * torch.randn(B, H, K, V, device=dev(), generator=g) * c
    else:
        x0 = torch.randn(B, H, K, V, device=dev(), generator=g) * .05
    fused.encode(x0, slots)
    split.encode(x0, slots)
    del x0
    mixed = torch.randn(B, 2 * HK * K + H * V, device=dev(), generator=g).to(torch.bfloat16)
    q, k, v = mixed.split([HK * K, HK * K, H * V], -1)  # column views with the row stride of mixed
    gate = torch.randn(B, H * K if arch == "kda" else H, device=dev(), generator=g)
    beta = torch.randn(B, H, device=dev(), generator=g)
    a_log = torch.randn(H, device=dev(), generator=g) * .3  # per head; dt_bias per channel for KDA
    dt_bias = torch.randn(H * K if arch == "kda" else H, device=dev(), generator=g) * .3
    kw = dict(normalize=True, scale=K ** -.5, a_log=a_log, dt_bias=dt_bias)
    pick = _spread(B)
    lay = O.layout(oplan, V)
    for it in range(2):
        pages0 = fused.data.cpu().numpy()
        out = fused.step(q, k, v, gate, beta, slots, **kw)
        out_split = split.step(q, k, v, gate, beta, slots, **kw)
        split.wait()
        torch.cuda.synchronize()
        assert torch.equal(out, out_split), "fused and split readouts differ"
        assert torch.equal(fused.data, split.data), "fused and split pages differ"
        assert torch.isfinite(out.float()).all()
        assert not fused.data[0].any(), "slot 0 (sentinel) stays zero"
        state = O.decode_page(pages0, pick + 1, oplan, lay, V)
        qp, kp, ld, bo = O.prepare(q.float().cpu().numpy()[pick], k.float().cpu().numpy()[pick],
                                   gate.cpu().numpy()[pick], beta.cpu().numpy()[pick], H, K, arch == "kda",
                                   normalize=True, scale=K ** -.5, a_log=a_log.cpu().numpy(),
                                   dt_bias=dt_bias.cpu().numpy())
        vs = v.float().cpu().numpy()[pick].reshape(len(pick), H, V)
        ref_out, upd = O.delta_step(state, qp, kp, vs, ld, bo)
        # the readout is stored in bf16 (q's dtype): one bf16 rounding
        np.testing.assert_allclose(out.float().cpu().numpy()[pick], ref_out, rtol=2 ** -8, atol=1e-4)
        _check_requant(fused.data.cpu().numpy(), pick + 1, oplan, lay, V, upd)
        mixed.copy_(torch.randn(mixed.shape, device=dev(), generator=g).to(torch.bfloat16))


def test_prefill_at_bench_heads():
    """Two 2048-token sequences over all 32 heads, checkpoints inside and at
    the end; value heads 0, 1 (key head 0) and 30, 31 (key head 15) against
    the float64 recurrence."""
    print("case prefill B=2 T=2048 H=32 HK=16", flush=True)
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    H, HK, K, V, T = 32, 16, 128, 128, 2048
    bits, impact = bench.make_plan(torch, "gdn", H, K, 6)
    oplan = _oracle_plan("gdn", bits, impact)
    pool = PackedStatePool(QuantizationPlan("gdn", bits.to(dev()), impact.to(dev())), 8, V)
    g = torch.Generator().manual_seed(9)
    init = torch.tensor([1, 2])
    pool.encode((torch.randn(2, H, K, V, generator=g) * .05).to(dev()), init.to(dev()))
    lay = O.layout(oplan, V)
    pages0 = pool.data.cpu().numpy()
    S0 = O.decode_page(pages0, init.numpy(), oplan, lay, V).astype(np.float64)
    q = torch.randn(2 * T, HK, K, generator=g).to(torch.bfloat16)
    k = torch.randn(2 * T, HK, K, generator=g).to(torch.bfloat16)
    v = torch.randn(2 * T, H, V, generator=g).to(torch.bfloat16)
    gate = torch.randn(2 * T, H, generator=g)
    beta = torch.randn(2 * T, H, generator=g)
    a_log = torch.zeros(H)
    dt_bias = torch.zeros(H)
    cu = np.array([0, T, 2 * T])
    ck = np.array([[1000, T], [640, T]])
    ck_slots = torch.tensor([[3, 4], [5, 6]])
    pool.keep_prefill_states = True
    out = pool.extend(q.to(dev()), k.to(dev()), v.to(dev()), gate.to(dev()), beta.to(dev()), init,
                      torch.from_numpy(cu), checkpoints=torch.from_numpy(ck), checkpoint_slots=ck_slots,
                      init_slots=init, normalize=True, scale=K ** -.5, a_log=a_log.to(dev()),
                      dt_bias=dt_bias.to(dev()))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    states = pool.last_prefill[-1].cpu().numpy().reshape(2, 2, H, K, V)
    assert np.isfinite(got).all()
    heads = [0, 1, 30, 31]
    ref_out, ref_states, _ = O.prefill(q.float().numpy()[:, [0, 15]], k.float().numpy()[:, [0, 15]],
                                       v.float().numpy()[:, heads], gate.numpy()[:, heads],
                                       beta.numpy()[:, heads], S0[:, heads], cu, ck, normalize=True,
                                       scale=K ** -.5, a_log=a_log.numpy()[heads], dt_bias=dt_bias.numpy()[heads])
    check_prefill(out[:, heads], ref_out, "bf16 outputs")
    check_states(states[:, :, heads], ref_states)
    pages = _check_prefix_pages(pool, states, ref_states, ck_slots.numpy(), oplan, lay, pages0, heads)
    assert not pages[7].any(), "unused slot stays empty"


def _check_prefix_pages(pool, states, ref_states, ck_slots, oplan, lay, pages0, heads):
    """Prefix pages: every one the oracle encoding of the kernel's states, bit
    for bit; on the heads the oracle recurrence ran for, within the
    requantisation bar of the oracle's encoding of its own states."""
    B, NC = ck_slots.shape
    H, K = oplan.bits.shape
    V = states.shape[-1]
    live = ck_slots.reshape(-1)
    ref_pages = pages0.copy()
    O.encode_page(states.reshape(B * NC, H, K, V), live, oplan, lay, ref_pages)
    pages = pool.data.cpu().numpy()
    bad = [int(s) for s in live if not np.array_equal(pages[s], ref_pages[s])]
    assert not bad, f"prefix pages differ from the oracle encoding of the kernel's states: slots {bad}"
    sub, sl, sp = sub_pages(pages, oplan, lay, heads, V)
    check_requant(sp, live, sub, sl, V, ref_states.reshape(B * NC, len(heads), K, V),
                  refit_budget=PREFILL_REFIT_BUDGET)
    return pages


def test_prefill_at_bench_shape():
    """P6 itself: 8 sequences of 2048 tokens over 32 value heads and 16 key
    heads, prefix states at bench.py's five positions per sequence written
    into 40 slots.  Eight value heads (four GQA pairs spread over the key
    heads) against the float64 recurrence for every sequence; every prefix
    page against the oracle encoding of the kernel's state."""
    print("case prefill P6 B=8 T=2048 H=32 HK=16 NC=5", flush=True)
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    B, H, HK, K, V, T, NC = 8, 32, 16, 128, 128, 2048, 5
    bits, impact = bench.make_plan(torch, "gdn", H, K, 6)
    oplan = _oracle_plan("gdn", bits, impact)
    pool = PackedStatePool(QuantizationPlan("gdn", bits.to(dev()), impact.to(dev())), B * (NC + 1) + 1, V)
    g = torch.Generator().manual_seed(21)
    init = torch.arange(1, B + 1)
    pool.encode((torch.randn(B, H, K, V, generator=g) * .05).to(dev()), init.to(dev()))
    lay = O.layout(oplan, V)
    pages0 = pool.data.cpu().numpy()
    S0 = O.decode_page(pages0, init.numpy(), oplan, lay, V).astype(np.float64)
    tot = B * T
    q = torch.randn(tot, HK, K, generator=g).to(torch.bfloat16)
    k = torch.randn(tot, HK, K, generator=g).to(torch.bfloat16)
    v = torch.randn(tot, H, V, generator=g).to(torch.bfloat16)
    gate = torch.randn(tot, H, generator=g)
    beta = torch.randn(tot, H, generator=g)
    a_log = torch.randn(H, generator=g) * .3
    dt_bias = torch.randn(H, generator=g) * .3
    cu = np.arange(0, tot + 1, T)
    pos = [((T * (c + 1)) // NC + 63) // 64 * 64 for c in range(NC)]
    pos[-1] = T
    ck = np.tile(np.array(pos), (B, 1))
    ck_slots = torch.arange(B + 1, B + 1 + B * NC).reshape(B, NC)
    pool.keep_prefill_states = True
    out = pool.extend(q.to(dev()), k.to(dev()), v.to(dev()), gate.to(dev()), beta.to(dev()), init,
                      torch.from_numpy(cu), checkpoints=torch.from_numpy(ck), checkpoint_slots=ck_slots,
                      init_slots=init, normalize=True, scale=K ** -.5, a_log=a_log.to(dev()),
                      dt_bias=dt_bias.to(dev()))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    states = pool.last_prefill[-1].cpu().numpy().reshape(B, NC, H, K, V)
    assert np.isfinite(got).all() and np.isfinite(states).all()
    heads = [0, 1, 10, 11, 20, 21, 30, 31]
    kheads = [h // 2 for h in heads[::2]]
    ref_out, ref_states, _ = O.prefill(q.float().numpy()[:, kheads], k.float().numpy()[:, kheads],
                                       v.float().numpy()[:, heads], gate.numpy()[:, heads],
                                       beta.numpy()[:, heads], S0[:, heads], cu, ck, normalize=True,
                                       scale=K ** -.5, a_log=a_log.numpy()[heads],
                                       dt_bias=dt_bias.numpy()[heads])
    check_prefill(out[:, heads], ref_out, "bf16 outputs")
    check_states(states[:, :, heads], ref_states)
    pages = _check_prefix_pages(pool, states, ref_states, ck_slots.numpy(), oplan, lay, pages0, heads)
    # the initial slots are not overwritten (the final state goes to the last prefix slot)
    assert np.array_equal(pages[1:B + 1], pages0[1:B + 1])


def test_kda_prefill_at_bench_shape():
    """The KDA prefill at the P6 shape (8 sequences of 2048 tokens, 32 value
    heads, one key head each, per-channel decays as bench.py draws them, five
    prefix slots per sequence): four heads against the float64 recurrence
    for every sequence; every prefix page against the oracle encoding of
    the kernel's state."""
    print("case KDA prefill B=8 T=2048 H=HK=32 NC=5", flush=True)
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    B, H, K, V, T, NC = 8, 32, 128, 128, 2048, 5
    bits, impact = bench.make_plan(torch, "kda", H, K, 6)
    oplan = _oracle_plan("kda", bits, impact)
    pool = PackedStatePool(QuantizationPlan("kda", bits.to(dev()), impact.to(dev())), B * (NC + 1) + 1, V)
    g = torch.Generator().manual_seed(23)
    init = torch.arange(1, B + 1)
    pool.encode((torch.randn(B, H, K, V, generator=g) * .05).to(dev()), init.to(dev()))
    lay = O.layout(oplan, V)
    pages0 = pool.data.cpu().numpy()
    S0 = O.decode_page(pages0, init.numpy(), oplan, lay, V).astype(np.float64)
    tot = B * T
    q = torch.randn(tot, H, K, generator=g).to(torch.bfloat16)
    k = torch.randn(tot, H, K, generator=g).to(torch.bfloat16)
    v = torch.randn(tot, H, V, generator=g).to(torch.bfloat16)
    gate = torch.randn(tot, H, K, generator=g) * .5
    beta = torch.randn(tot, H, generator=g)
    a_log = torch.zeros(H)
    dt_bias = torch.zeros(H * K)
    cu = np.arange(0, tot + 1, T)
    pos = [((T * (c + 1)) // NC + 63) // 64 * 64 for c in range(NC)]
    pos[-1] = T
    ck = np.tile(np.array(pos), (B, 1))
    ck_slots = torch.arange(B + 1, B + 1 + B * NC).reshape(B, NC)
    pool.keep_prefill_states = True
    out = pool.extend(q.to(dev()), k.to(dev()), v.to(dev()), gate.to(dev()), beta.to(dev()), init,
                      torch.from_numpy(cu), checkpoints=torch.from_numpy(ck), checkpoint_slots=ck_slots,
                      init_slots=init, normalize=True, scale=K ** -.5, a_log=a_log.to(dev()),
                      dt_bias=dt_bias.to(dev()))
    torch.cuda.synchronize()
    states = pool.last_prefill[-1].cpu().numpy().reshape(B, NC, H, K, V)
    assert np.isfinite(out.float().cpu().numpy()).all() and np.isfinite(states).all()
    heads = [0, 9, 22, 31]
    hb = np.concatenate([np.arange(h * K, (h + 1) * K) for h in heads])
    ref_out, ref_states, _ = O.prefill(q.float().numpy()[:, heads], k.float().numpy()[:, heads],
                                       v.float().numpy()[:, heads], gate.numpy()[:, heads],
                                       beta.numpy()[:, heads], S0[:, heads], cu, ck, normalize=True,
                                       scale=K ** -.5, a_log=a_log.numpy()[heads], dt_bias=dt_bias.numpy()[hb])
    check_prefill(out[:, heads], ref_out, "bf16 outputs")
    check_states(states[:, :, heads], ref_states)
    _check_prefix_pages(pool, states, ref_states, ck_slots.numpy(), oplan, lay, pages0, heads)
