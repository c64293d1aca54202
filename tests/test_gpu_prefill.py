"""Chunked MFMA prefill against the token-sequential oracle (MI355X).

Bars (elementwise): checkpoint states within rtol 1e-3 / atol 1e-4 of the
float64 recurrence, outputs within rtol 1e-3 (fp32) or 2^-8 (bf16) / atol
1e-4; checkpoint pages bit-identical to the oracle's fit_state + page layout
of the kernel's own fp32 states, and within the requantisation bar (codes at
most one level off on at most 0.1%, scales within one fp16 ulp) of the
oracle's encoding of the recurrence's own states.  The chunk products carry
~2^-17 relative error from hi/lo bf16 operands.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import PREFILL_REFIT_BUDGET, check_prefill, check_requant, check_states, dev, device_plan, make_plan

pytestmark = pytest.mark.gpu


def _check_pages(pool, ck_state, ref_states, ck_slots, oplan, lay, pages0, storage="packed"):
    """Checkpoint pages: the oracle encoding of the kernel's states, bit for
    bit, and within the requantisation bar of the oracle's own states."""
    B, NC = ck_slots.shape
    H, K = oplan.bits.shape
    V = ck_state.shape[-1]
    pages = pool.data.cpu().numpy()
    live = ck_slots.reshape(-1)
    ref_pages = pages0.copy()
    O.encode_page(ck_state.reshape(B * NC, H, K, V), live, oplan, lay, ref_pages, storage)
    for s in live[live > 0]:
        assert np.array_equal(pages[s], ref_pages[s]), f"slot {s} page differs"
    used = np.where(live[:, None, None, None] > 0, ref_states.reshape(B * NC, H, K, V), 0)
    check_requant(pages, live, oplan, lay, V, used, storage=storage, refit_budget=PREFILL_REFIT_BUDGET)
    return pages


@pytest.mark.parametrize("raw,normalize", [(False, True), (True, True), (False, False)])
def test_prefill_against_sequential_oracle(raw, normalize):
    print(f"case raw={raw} normalize={normalize}", flush=True)
    _prefill_case(raw, normalize, [130, 37, 64], [[50, 130], [37, 0], [10, 64]], [[6, 7], [8, 0], [9, 10]],
                  [3, 0, 5], [3, 4, 5], (1, 2, 11))


def test_prefill_key_head_pairs_on_one_xcd():
    """4 sequences x 4 value heads over 2 key heads: the grid (16 workgroups)
    divides into groups of 8 x 2, so the two value heads of a key head run as
    workgroups x and x + 8; ragged lengths, a one-token sequence and
    checkpoints inside and at the end of chunks."""
    print("case grouped heads", flush=True)
    _prefill_case(False, True, [100, 64, 1, 150], [[64, 100], [30, 64], [1, 0], [70, 128]],
                  [[6, 7], [8, 9], [10, 0], [11, 13]], [3, 0, 5, 12], [3, 4, 5, 12], (1, 2, 14, 15))


def _prefill_case(raw, normalize, lens, ck, ck_slots, init, slots, untouched):
    from stepquant_amd.kernels.pool import PackedStatePool
    H, HK, K, V = 4, 2, 128, 128
    B = len(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    oplan = make_plan("gdn", np.repeat(np.array([6, 4, 8, 6])[:, None], K, 1), seed=3)
    pool = PackedStatePool(device_plan(oplan), 16, V)
    rng = np.random.default_rng(7 + raw + 2 * normalize)
    g = torch.Generator().manual_seed(11)
    scale = K ** -.5 if normalize else .05
    qf = torch.randn(T, HK, K, generator=g)
    kf = torch.randn(T, HK, K, generator=g)
    if not normalize:
        kf = torch.nn.functional.normalize(kf, dim=-1)
    q = qf.to(torch.bfloat16)
    k = kf.to(torch.bfloat16)
    v = torch.randn(T, H, V, generator=g).to(torch.bfloat16)
    if raw:
        gate = torch.randn(T, H, generator=g)
        beta = torch.randn(T, H, generator=g)
        a_log = torch.randn(H, generator=g) * .3
        dt_bias = torch.randn(H, generator=g) * .3
    else:
        gate = -torch.nn.functional.softplus(torch.randn(T, H, generator=g))
        beta = torch.sigmoid(torch.randn(T, H, generator=g))
        a_log = dt_bias = None
    init = torch.tensor(init)  # slot 0: the sequence starts from zero
    x0 = torch.randn(B, H, K, V, generator=g) * .1
    pool.encode(x0.to(dev()), init.to(dev()))
    lay = O.layout(oplan, V)
    pages0 = pool.data.cpu().numpy()
    S0 = O.decode_page(pages0, init.numpy(), oplan, lay, V).astype(np.float64)
    ck = np.array(ck)
    ck_slots = torch.tensor(ck_slots)
    pool.keep_prefill_states = True
    # q as float32 holding bf16 values: the kernel reads the same bf16 inputs and
    # the outputs come back in float32, so their error is the kernel's own
    out = pool.extend(q.float().to(dev()), k.to(dev()), v.to(dev()), gate.to(dev()), beta.to(dev()),
                      torch.tensor(slots), torch.from_numpy(cu), checkpoints=torch.from_numpy(ck),
                      checkpoint_slots=ck_slots, init_slots=init, normalize=normalize, scale=scale,
                      a_log=None if a_log is None else a_log.to(dev()),
                      dt_bias=None if dt_bias is None else dt_bias.to(dev()))
    torch.cuda.synchronize()
    ref_out, ref_states, _ = O.prefill(q.float().numpy(), k.float().numpy(), v.float().numpy(), gate.numpy(),
                                       beta.numpy(), S0, cu, ck, normalize=normalize, scale=scale,
                                       a_log=None if a_log is None else a_log.numpy(),
                                       dt_bias=None if dt_bias is None else dt_bias.numpy())
    ck_state = pool.last_prefill[-1].cpu().numpy().reshape(B, 2, H, K, V)
    for b in range(B):
        for c in range(2):
            if ck_slots[b, c] > 0:
                check_states(ck_state[b, c], ref_states[b, c], f"state b={b} c={c}")
    assert out.dtype == torch.float32
    check_prefill(out, ref_out)
    pages = _check_pages(pool, ck_state, ref_states, ck_slots.numpy(), oplan, lay, pages0)
    for s in untouched:
        assert not pages[s].any(), "untouched slots stay empty"


def test_extend_defaults_write_final_state_back_to_the_slots():
    from stepquant_amd.kernels.pool import PackedStatePool
    H, K, V = 2, 128, 128
    oplan = make_plan("gdn", np.full((H, K), 6), seed=1)
    pool = PackedStatePool(device_plan(oplan), 4, V)
    g = torch.Generator().manual_seed(2)
    lens = [70, 5]
    cu = torch.tensor([0, 70, 75])
    q = torch.randn(75, H * K, generator=g).to(torch.bfloat16)
    k = torch.randn(75, H * K, generator=g).to(torch.bfloat16)
    v = torch.randn(75, H * V, generator=g).to(torch.bfloat16)
    gate = -torch.nn.functional.softplus(torch.randn(75, H, generator=g))
    beta = torch.sigmoid(torch.randn(75, H, generator=g))
    slots = torch.tensor([2, 1])
    pool.encode((torch.randn(2, H, K, V, generator=g) * .1).to(dev()), slots.to(dev()))
    lay = O.layout(oplan, V)
    S0 = O.decode_page(pool.data.cpu().numpy(), slots.numpy(), oplan, lay, V).astype(np.float64)
    pool.keep_prefill_states = True
    out = pool.extend(q.to(dev()), k.to(dev()), v.to(dev()), gate.to(dev()), beta.to(dev()), slots, cu,
                      normalize=True, scale=K ** -.5)
    torch.cuda.synchronize()
    ref_out, _, final = O.prefill(q.float().numpy().reshape(75, H, K), k.float().numpy().reshape(75, H, K),
                                  v.float().numpy().reshape(75, H, V), gate.numpy(), beta.numpy(), S0,
                                  cu.numpy(), normalize=True, scale=K ** -.5)
    dense = pool.last_prefill[-1].cpu().numpy()
    check_states(dense, final, "final states")
    assert out.dtype == torch.bfloat16
    check_prefill(out, ref_out, "bf16 outputs")
    ref_pages = np.zeros_like(pool.data.cpu().numpy())
    O.encode_page(dense, slots.numpy(), oplan, lay, ref_pages)
    got = pool.data.cpu().numpy()
    assert np.array_equal(got[slots.numpy()], ref_pages[slots.numpy()])
    check_requant(got, slots.numpy(), oplan, lay, V, final, refit_budget=PREFILL_REFIT_BUDGET)
    assert len(lens) == 2


def test_prefill_rows_far_apart_match_contiguous_rows():
    """Row strides of 2^23 elements or more (views into wide buffers) give the
    same outputs and pages as contiguous rows."""
    from stepquant_amd.kernels.pool import PackedStatePool
    H, K, V, T = 2, 128, 128, 3
    oplan = make_plan("gdn", np.full((H, K), 6), seed=3)
    g = torch.Generator().manual_seed(4)
    q = torch.randn(T, H * K, generator=g).to(torch.bfloat16).to(dev())
    k = torch.randn(T, H * K, generator=g).to(torch.bfloat16).to(dev())
    v = torch.randn(T, H * V, generator=g).to(torch.bfloat16).to(dev())
    gate = -torch.nn.functional.softplus(torch.randn(T, H, generator=g)).to(dev())
    beta = torch.sigmoid(torch.randn(T, H, generator=g)).to(dev())
    init = (torch.randn(1, H, K, V, generator=g) * .1).to(dev())
    slots = torch.tensor([1])
    cu = torch.tensor([0, T])
    wide = torch.zeros(T, (1 << 23) + 256, dtype=torch.bfloat16, device=dev())
    outs, pages = [], []
    for spread in (False, True):
        pool = PackedStatePool(device_plan(oplan), 2, V)
        pool.encode(init, slots.to(dev()))
        qq = q
        if spread:
            wide[:, :H * K] = q
            qq = wide[:, :H * K]
            assert qq.stride(0) >= 1 << 23
        outs.append(pool.extend(qq, k, v, gate, beta, slots, cu, normalize=True, scale=K ** -.5))
        torch.cuda.synchronize()
        pages.append(pool.data.cpu())
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(pages[0], pages[1])


@pytest.mark.parametrize("arch,storage,raw", [("kda", "packed", False), ("kda", "packed", True),
                                              ("kda", "byte", True), ("gdn", "byte", False)])
def test_prefill_kda_and_byte_pages(arch, storage, raw):
    """KDA pools (per-channel decay, chunks of 16 tokens) and byte-carrier
    pages go through the same extend: outputs and checkpoint states against
    the float64 recurrence, checkpoint pages equal to the oracle encoding
    of the kernel's states."""
    print(f"case {arch} {storage} raw={raw}", flush=True)
    from stepquant_amd.kernels.pool import PackedStatePool
    H, HK, K, V = 4, 2 if arch == "gdn" else 4, 128, 128
    lens = [97, 40, 33]
    B = len(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    rng = np.random.default_rng(5)
    if arch == "kda":
        bits = np.where(rng.random((H, K)) < .03, 16, rng.choice([2, 4, 6, 8], (H, K)))
    else:
        bits = np.repeat(np.array([6, 2, 8, 16])[:, None], K, 1)
    oplan = make_plan(arch, bits, seed=3)
    stream = torch.cuda.Stream() if storage == "byte" else None
    pool = PackedStatePool(device_plan(oplan), 12, V, writeback_stream=stream, storage=storage)
    g = torch.Generator().manual_seed(17)
    q = torch.randn(T, HK, K, generator=g).to(torch.bfloat16)
    k = torch.randn(T, HK, K, generator=g).to(torch.bfloat16)
    v = torch.randn(T, H, V, generator=g).to(torch.bfloat16)
    gshape = (T, H, K) if arch == "kda" else (T, H)
    if raw:
        gate = torch.randn(gshape, generator=g) * .5
        beta = torch.randn(T, H, generator=g)
        a_log = torch.randn(H, generator=g) * .3
        dt_bias = torch.randn(H * K if arch == "kda" else H, generator=g) * .3
    else:
        gate = -torch.nn.functional.softplus(torch.randn(gshape, generator=g) * (.5 if arch == "kda" else 1.))
        beta = torch.sigmoid(torch.randn(T, H, generator=g))
        a_log = dt_bias = None
    init = torch.tensor([3, 0, 5])
    pool.encode((torch.randn(B, H, K, V, generator=g) * .1).to(dev()), init.to(dev()))
    pool.wait()
    lay = O.layout(oplan, V, storage)
    pages0 = pool.data.cpu().numpy()
    S0 = O.decode_page(pages0, init.numpy(), oplan, lay, V, storage).astype(np.float64)
    ck = np.array([[50, 97], [40, 0], [10, 33]])
    ck_slots = torch.tensor([[6, 7], [8, 0], [9, 10]])
    pool.keep_prefill_states = True
    out = pool.extend(q.to(dev()), k.to(dev()), v.to(dev()), gate.to(dev()), beta.to(dev()),
                      torch.tensor([3, 4, 5]), torch.from_numpy(cu), checkpoints=torch.from_numpy(ck),
                      checkpoint_slots=ck_slots, init_slots=init, normalize=True, scale=K ** -.5,
                      a_log=None if a_log is None else a_log.to(dev()),
                      dt_bias=None if dt_bias is None else dt_bias.to(dev()))
    torch.cuda.synchronize()
    ref_out, ref_states, _ = O.prefill(q.float().numpy(), k.float().numpy(), v.float().numpy(), gate.numpy(),
                                       beta.numpy(), S0, cu, ck, normalize=True, scale=K ** -.5,
                                       a_log=None if a_log is None else a_log.numpy(),
                                       dt_bias=None if dt_bias is None else dt_bias.numpy())
    ck_state = pool.last_prefill[-1].cpu().numpy().reshape(B, 2, H, K, V)
    for b in range(B):
        for c in range(2):
            if ck_slots[b, c] > 0:
                check_states(ck_state[b, c], ref_states[b, c], f"state b={b} c={c}")
    assert out.dtype == torch.bfloat16
    check_prefill(out, ref_out, "bf16 outputs")
    pages = _check_pages(pool, ck_state, ref_states, ck_slots.numpy(), oplan, lay, pages0, storage)
    for s in (1, 2, 11):
        assert not pages[s].any(), "untouched slots stay empty"


@pytest.mark.parametrize("arch", ["gdn", "kda"])
def test_prefill_reads_initial_pages_in_kernel(arch):
    """Packed pools that the K = V = 128 kernels take have their initial
    pages decoded inside the recurrence kernel; the same pages in a pool
    whose fast flags are cleared go through the dense decode (the general
    step kernel's decode mode) first.  Outputs, checkpoint states and pages
    agree bit for bit: GDN 2-bit (four value groups), 4-, 6-, 8-bit and FP16
    pivot heads; KDA rows of every width with FP16 pivot rows (odd tile
    offsets); a zero slot and ragged sequences."""
    print(f"case in-kernel initial pages {arch}", flush=True)
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd import _native as N
    H, HK, K, V = 5, 5, 128, 128
    lens = [70, 1, 129]
    B = len(lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]).astype(np.int64))
    T = int(cu[-1])
    if arch == "gdn":
        bits = np.repeat(np.array([2, 4, 6, 8, 16])[:, None], K, 1)
    else:
        rng = np.random.default_rng(8)
        bits = np.where(rng.random((H, K)) < .05, 16, rng.choice([2, 4, 6, 8], (H, K)))
        bits[4] = 16  # a head of pivot rows only
    oplan = make_plan(arch, bits, seed=4)
    pools = [PackedStatePool(device_plan(oplan), 12, V) for _ in range(2)]
    assert pools[0]._desc.flags & (N.POOL_FAST_GDN128 if arch == "gdn" else N.POOL_FAST_KDA128)
    pools[1]._desc.flags = 0  # the dense decode path
    g = torch.Generator().manual_seed(23)
    init = torch.tensor([3, 0, 5])
    pools[0].encode((torch.randn(B, H, K, V, generator=g) * .1).to(dev()), init.to(dev()))
    pools[1].data.copy_(pools[0].data)
    q = torch.randn(T, HK, K, generator=g).to(torch.bfloat16).to(dev())
    k = torch.randn(T, HK, K, generator=g).to(torch.bfloat16).to(dev())
    v = torch.randn(T, H, V, generator=g).to(torch.bfloat16).to(dev())
    gshape = (T, H, K) if arch == "kda" else (T, H)
    gate = (-torch.nn.functional.softplus(torch.randn(gshape, generator=g) * (.5 if arch == "kda" else 1.))).to(dev())
    beta = torch.sigmoid(torch.randn(T, H, generator=g)).to(dev())
    ck = torch.tensor([[64, 70], [1, 0], [100, 129]], dtype=torch.int32)
    ck_slots = torch.tensor([[6, 7], [8, 0], [9, 10]])
    outs, states = [], []
    for pool in pools:
        pool.keep_prefill_states = True
        outs.append(pool.extend(q, k, v, gate, beta, torch.tensor([3, 4, 5]), cu, checkpoints=ck,
                                checkpoint_slots=ck_slots, init_slots=init, normalize=True, scale=K ** -.5))
        states.append(pool.last_prefill[-1])
    torch.cuda.synchronize()
    assert pools[0].last_prefill[-2] is None and pools[1].last_prefill[-2] is not None
    used = (ck_slots.reshape(-1) > 0).to(dev())  # unused checkpoints leave their workspace entry unwritten
    assert torch.equal(states[0][used], states[1][used]), "checkpoint states differ between the two initial-state paths"
    assert torch.equal(outs[0], outs[1]), "outputs differ between the two initial-state paths"
    assert torch.equal(pools[0].data, pools[1].data), "pages differ between the two initial-state paths"


@pytest.mark.parametrize("arch", ["gdn", "kda"])
def test_prefill_timing_events_change_nothing(arch):
    """The benchmark's timing hook: the two events bracket the recurrence
    kernel (a positive interval no longer than the whole call's), and the
    outputs and pages equal those of a call without them."""
    from stepquant_amd.kernels.pool import PackedStatePool
    print(f"case timing events {arch}", flush=True)
    H, K, V, T = 2, 128, 128, 150
    oplan = make_plan(arch, np.full((H, K), 6), seed=3)
    pools = [PackedStatePool(device_plan(oplan), 4, V) for _ in range(2)]
    g = torch.Generator().manual_seed(4)
    q = torch.randn(T, H * K, generator=g).to(torch.bfloat16).to(dev())
    k = torch.randn(T, H * K, generator=g).to(torch.bfloat16).to(dev())
    v = torch.randn(T, H * V, generator=g).to(torch.bfloat16).to(dev())
    gshape = (T, H, K) if arch == "kda" else (T, H)
    gate = (-torch.nn.functional.softplus(torch.randn(gshape, generator=g))).to(dev())
    beta = torch.sigmoid(torch.randn(T, H, generator=g)).to(dev())
    slots = torch.tensor([2, 1])
    x = (torch.randn(2, H, K, V, generator=g) * .1).to(dev())
    for p in pools:
        p.encode(x, slots.to(dev()))
    cu = torch.tensor([0, 100, T])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with pytest.raises(ValueError):
        pools[0].extend(q, k, v, gate, beta, slots, cu, normalize=True, scale=K ** -.5, events=(e0, e1))
    e0.record()
    e1.record()
    outer0, outer1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    outer0.record()
    a = pools[0].extend(q, k, v, gate, beta, slots, cu, normalize=True, scale=K ** -.5, events=(e0, e1))
    outer1.record()
    b = pools[1].extend(q, k, v, gate, beta, slots, cu, normalize=True, scale=K ** -.5)
    torch.cuda.synchronize()
    assert 0 < e0.elapsed_time(e1) <= outer0.elapsed_time(outer1)
    assert torch.equal(a, b)
    assert torch.equal(pools[0].data, pools[1].data)
    # the pools keep no reference to the call's inputs and state workspaces
    assert not any(hasattr(p, "last_prefill") for p in pools)


@pytest.mark.parametrize("a_log", [3.0, -2.0])
def test_kda_prefill_with_extreme_decays(a_log):
    """KDA gates far outside the typical range: with A_log = 3 some
    channels forget ~20-60 nats per token (hundreds over a chunk) while others
    keep their state; with A_log = -2 every channel barely decays.  The
    chunked kernel forms the in-chunk decays pairwise, so nothing overflows:
    outputs and states against the float64 recurrence."""
    from stepquant_amd.kernels.pool import PackedStatePool
    print(f"case kda extreme decays a_log={a_log}", flush=True)
    H, K, V = 2, 128, 128
    lens = [75, 33]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    oplan = make_plan("kda", np.full((H, K), 8), seed=2)
    pool = PackedStatePool(device_plan(oplan), 6, V)
    g = torch.Generator().manual_seed(31)
    q = torch.randn(T, H, K, generator=g).to(torch.bfloat16)
    k = torch.randn(T, H, K, generator=g).to(torch.bfloat16)
    v = torch.randn(T, H, V, generator=g).to(torch.bfloat16)
    gate = torch.randn(T, H, K, generator=g) * 2.0
    gate[:, :, ::3] = -30.0  # a third of the channels: softplus ~ 0, almost no decay
    beta = torch.rand(T, H, generator=g)
    a_log_t = torch.full((H,), a_log)
    dt_bias = torch.randn(H * K, generator=g)
    init = torch.tensor([2, 4])
    pool.encode((torch.randn(2, H, K, V, generator=g) * .1).to(dev()), init.to(dev()))
    lay = O.layout(oplan, V)
    S0 = O.decode_page(pool.data.cpu().numpy(), init.numpy(), oplan, lay, V).astype(np.float64)
    ck = np.array([[16, 75], [20, 33]])
    ck_slots = torch.tensor([[1, 3], [5, 0]])
    pool.keep_prefill_states = True
    out = pool.extend(q.to(dev()), k.to(dev()), v.to(dev()), gate.to(dev()), beta.to(dev()), init,
                      torch.from_numpy(cu), checkpoints=torch.from_numpy(ck), checkpoint_slots=ck_slots,
                      init_slots=init, normalize=True, scale=K ** -.5, a_log=a_log_t.to(dev()),
                      dt_bias=dt_bias.to(dev()), beta_logits=False)
    torch.cuda.synchronize()
    ref_out, ref_states, _ = O.prefill(q.float().numpy(), k.float().numpy(), v.float().numpy(), gate.numpy(),
                                       beta.numpy(), S0, cu, ck, normalize=True, scale=K ** -.5,
                                       a_log=a_log_t.numpy(), dt_bias=dt_bias.numpy(), beta_logits=False)
    states = pool.last_prefill[-1].cpu().numpy().reshape(2, 2, H, K, V)
    assert np.isfinite(out.float().cpu().numpy()).all() and np.isfinite(states).all()
    check_prefill(out, ref_out, "bf16 outputs")
    for b in range(2):
        for c in range(2):
            if ck_slots[b, c] > 0:
                check_states(states[b, c], ref_states[b, c], f"state b={b} c={c}")
