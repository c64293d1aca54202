"""The pool-side calls of the reference's serving adapter on an MI355X.

The reference adapter (stepquant/sglang/runtime.py) runs unchanged over this
package's pools; SGLang is not installed here, so these tests make the calls
its hooks make, with the arguments they pass: slot allocation clears pages
(runtime.py:137-144), copy_from copies them (:147-151), CPU offload copies
the page bytes after a synchronisation and loads them back after ``wait()``
(:154-166), the temporal cache reports ``nbytes`` (TemporalPages).  The
extend hook is this package's own (``stepquant_amd.sglang.extend``): fused
prefill into the pages for GDN and KDA pools with K = V = 128 (packed or
byte pages), with the chunk kernels' argument conventions (KDA: raw gate
with ``A_log``/``dt_bias``, beta after the sigmoid); the reference's decode /
chunk kernel / encode round trip for the others.  prefill_reduce
runs on device tensors with a stand-in coordinator.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import oracle as O
from stepquant_amd.sglang import extend as E
from stepquant_amd.sglang import prefill_reduce as PR
from tests.helpers import PREFILL_REFIT_BUDGET, check_prefill, check_requant, check_states, dev

pytestmark = pytest.mark.gpu


def _pages(kind, size):
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    from stepquant_amd.formats import FormatPlan, get_format
    from stepquant_amd.kernels.format_pool import FormatStatePool
    H, K, V = 4, 128, 128
    if kind == "sym_int6_g128":
        spec = get_format(kind)
        plan = FormatPlan("kda", torch.full((H, K), spec.bits, device=dev()), torch.ones(H, K, device=dev()))
        return [FormatStatePool(plan, size + 1, V, spec) for _ in range(2)]
    plan = QuantizationPlan("kda", torch.full((H, K), 6, device=dev()), torch.ones(H, K, device=dev()))
    stream = torch.cuda.Stream() if kind == "byte" else None
    return [PackedStatePool(plan, size + 1, V, writeback_stream=stream, storage="packed" if kind != "byte" else "byte")
            for _ in range(2)]


@pytest.mark.parametrize("kind", ["packed", "byte", "sym_int6_g128"])
def test_pool_lifecycle_calls(kind):
    print(f"case {kind}", flush=True)
    size = 3
    pages = _pages(kind, size)
    free = torch.arange(1, size + 1, device=dev())
    # alloc: take slots, clear their pages
    slots, free = free[:3], free[3:]
    for p in pages:
        p.clear(slots)
    layer = pages[0]
    x = torch.randn(1, 4, 128, 128, device=dev()) * .1
    layer.encode(x, slots[:1])
    # copy_from
    for p in pages:
        p.copy(slots[:1], slots[1:2])
    assert torch.equal(layer.decode(slots[:1]), layer.decode(slots[1:2]))
    # CPU offload: page bytes after a synchronisation, loaded back after wait()
    torch.cuda.synchronize()
    saved = [p.data[slots[1:2]].cpu() for p in pages]
    assert saved[0].shape == (1, layer.page_bytes) and saved[0].device.type == "cpu"
    layer.clear(slots[1:2])
    assert layer.decode(slots[1:2]).count_nonzero() == 0
    for p, src in zip(pages, saved):
        p.wait()
        p.data[slots[1:2]] = src.to(p.data.device)
    assert torch.equal(layer.decode(slots[:1]), layer.decode(slots[1:2]))
    # free, reuse: the reused slot starts from a cleared page
    free = torch.cat([free, slots[1:2]])
    reused = free[:1]
    for p in pages:
        p.clear(reused)
    assert layer.decode(reused).count_nonzero() == 0
    assert torch.equal(layer.decode(slots[:1]), layer.decode(slots[:1]))
    assert sum(p.nbytes for p in pages) == 2 * (size + 1) * layer.page_bytes


def test_decode_calls_and_fused_extend_hook():
    """The adapter's decode hooks call step() on the column split of
    mixed_qkv with normalize=True and the scale (runtime.py:173-190); the
    extend hook runs the chunked prefill into the pages (GDN K = V = 128)."""
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    H, HK, K, V, B = 4, 2, 128, 128, 3
    plan = QuantizationPlan("gdn", torch.tensor([6, 4, 8, 6])[:, None].expand(H, K).contiguous().to(dev()),
                            torch.ones(H, K, device=dev()))
    pool_a = PackedStatePool(plan, B + 1, V)
    assert E.fused(pool_a)
    g = torch.Generator().manual_seed(1)
    slots = torch.tensor([3, 1, 2], device=dev())
    x = (torch.randn(B, H, K, V, generator=g) * .1).to(dev())
    pool_a.encode(x, slots)
    mixed = torch.randn(B, 2 * HK * K + H * V, generator=g).to(torch.bfloat16).to(dev())
    a = torch.randn(B, H, generator=g).to(dev())
    b = torch.randn(B, H, generator=g).to(dev())
    a_log = torch.randn(H, generator=g).to(dev()) * .3
    dt = torch.randn(H, generator=g).to(dev()) * .3
    q, k, v = mixed.split([HK * K, HK * K, H * V], -1)
    oplan = O.Plan("gdn", plan.bits.cpu().numpy(), np.ones((H, K), np.float32), 32)
    lay = O.layout(oplan, V)
    state = O.decode_page(pool_a.data.cpu().numpy(), slots.cpu().numpy(), oplan, lay, V)
    out = pool_a.step(q, k, v, a, b, slots, normalize=True, scale=K ** -.5, a_log=a_log, dt_bias=dt).unsqueeze(0)
    torch.cuda.synchronize()
    qp, kp, ld, bo = O.prepare(q.float().cpu().numpy(), k.float().cpu().numpy(), a.cpu().numpy(), b.cpu().numpy(),
                               H, K, False, True, K ** -.5, a_log.cpu().numpy(), dt.cpu().numpy())
    ref, _ = O.delta_step(state, qp, kp, v.float().cpu().numpy().reshape(B, H, V), ld, bo)
    assert out.shape == (1, B, H, V)
    np.testing.assert_allclose(out[0].float().cpu().numpy(), ref, rtol=2 ** -8, atol=1e-4)
    # extend: the hook against the float64 recurrence on the decoded states
    lens = [70, 5, 33]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T = int(cu[-1])
    qe = torch.randn(1, T, HK, K, generator=g).to(torch.bfloat16)
    ke = torch.randn(1, T, HK, K, generator=g).to(torch.bfloat16)
    ve = torch.randn(1, T, H, V, generator=g).to(torch.bfloat16)
    ge = -torch.nn.functional.softplus(torch.randn(1, T, H, generator=g))
    be = torch.sigmoid(torch.randn(1, T, H, generator=g))
    S0 = pool_a.decode(slots).cpu().numpy().astype(np.float64)
    pool_a.keep_prefill_states = True
    oe = E.kernel_extend(None, None, qe.to(dev()), ke.to(dev()), ve.to(dev()), ge.to(dev()), be.to(dev()),
                         ssm_states=pool_a, cache_indices=slots, query_start_loc=cu.to(dev()))
    torch.cuda.synchronize()
    ref_out, _, final = O.prefill(qe[0].float().numpy(), ke[0].float().numpy(), ve[0].float().numpy(),
                                  ge[0].numpy(), be[0].numpy(), S0, cu.numpy(), normalize=True, scale=K ** -.5)
    assert oe.shape == (1, T, H, V)
    check_prefill(oe[0], ref_out, "bf16 outputs")
    dense = pool_a.last_prefill[-1].cpu().numpy()  # the kernel's fp32 final states
    check_states(dense, final)
    ref = pool_a.data.cpu().numpy().copy()
    O.encode_page(dense, slots.cpu().numpy(), oplan, lay, ref)
    assert np.array_equal(pool_a.data.cpu().numpy(), ref), "final pages are the oracle encoding"
    check_requant(pool_a.data.cpu().numpy(), slots.cpu().numpy(), oplan, lay, V, final,
                  refit_budget=PREFILL_REFIT_BUDGET)


@pytest.mark.parametrize("storage", ["packed", "byte"])
def test_fused_extend_hook_kda_reference_call_shape(storage):
    """Kimi-Linear prefill through the hook exactly as the reference's KDA
    call passes it (tests/test_sglang_cuda.py:30-45): q, k, v [1, T, H, K]
    bf16, a raw per-channel gate g [1, T, H, K], beta [1, T, H] already in
    (0, 1), A_log [H] and dt_bias [H*K] as keyword arguments, int32 offsets
    on the device.  The log decay is -exp(A_log) softplus(g + dt_bias) and
    beta is used as given; outputs, final states and pages against the
    float64 recurrence."""
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    print(f"case kda extend hook {storage}", flush=True)
    h, K, V = 4, 128, 128
    rng = np.random.default_rng(54)
    bits = np.where(rng.random((h, K)) < .02, 16, rng.choice([4, 6, 8], (h, K)))
    oplan = O.Plan("kda", bits.astype(np.int32), np.ones((h, K), np.float32), 32)
    plan = QuantizationPlan("kda", torch.from_numpy(bits).to(dev()), torch.ones(h, K, device=dev()))
    stream = torch.cuda.Stream() if storage == "byte" else None
    pool = PackedStatePool(plan, 5, V, writeback_stream=stream, storage=storage)
    assert E.fused(pool)
    g = torch.Generator().manual_seed(54)
    slots = torch.tensor([3, 1], device=dev())
    pool.encode((torch.randn(2, h, K, V, generator=g) * .1).to(dev()), slots)
    pool.wait()
    lay = O.layout(oplan, V, storage)
    S0 = O.decode_page(pool.data.cpu().numpy(), slots.cpu().numpy(), oplan, lay, V, storage).astype(np.float64)
    cu = torch.tensor([0, 8, 24], device=dev(), dtype=torch.int32)
    q, key, val = [torch.randn(1, 24, h, K, generator=g).to(torch.bfloat16) for _ in range(3)]
    alog = torch.randn(h, generator=g) * .3
    bias = torch.randn(h * K, generator=g) * .3
    graw = torch.randn(1, 24, h, K, generator=g)
    beta = torch.rand(1, 24, h, generator=g)
    pool.keep_prefill_states = True
    out = E.kernel_extend(None, None, q.to(dev()), key.to(dev()), val.clone().to(dev()), graw.to(dev()),
                          beta.to(dev()), ssm_states=pool, cache_indices=slots, query_start_loc=cu,
                          A_log=alog.to(dev()), dt_bias=bias.to(dev()))
    torch.cuda.synchronize()
    ref_out, _, final = O.prefill(q[0].float().numpy(), key[0].float().numpy(), val[0].float().numpy(),
                                  graw[0].numpy(), beta[0].numpy(), S0, cu.cpu().numpy(), normalize=True,
                                  scale=K ** -.5, a_log=alog.numpy(), dt_bias=bias.numpy(), beta_logits=False)
    assert out.shape == (1, 24, h, V) and out.dtype == torch.bfloat16
    check_prefill(out[0], ref_out, "bf16 outputs")
    check_states(pool.last_prefill[-1].cpu().numpy(), final)
    pages = pool.data.cpu().numpy()
    check_requant(pages, slots.cpu().numpy(), oplan, lay, V, final, storage=storage,
                  refit_budget=PREFILL_REFIT_BUDGET)


def test_extend_round_trip_for_format_pools():
    """Pools without the fused prefill take the reference's round trip:
    decode to V-first fp32, run the wrapped kernel, encode back."""
    from stepquant_amd.formats import FormatPlan, get_format
    from stepquant_amd.kernels.format_pool import FormatStatePool
    H, K, V = 2, 128, 128
    spec = get_format("fp32")
    pool = FormatStatePool(FormatPlan("gdn", torch.full((H, K), 32, device=dev()), torch.ones(H, K, device=dev())),
                           4, V, spec)
    slots = torch.tensor([2, 3], device=dev())
    x = torch.randn(2, H, K, V, device=dev())
    pool.encode(x, slots)
    seen = {}

    def original(self, q, k, v, g, beta, *, ssm_states, cache_indices, query_start_loc):
        seen["shape"] = tuple(ssm_states.shape)
        seen["indices"] = cache_indices.tolist()
        ssm_states.mul_(2.0)  # a stand-in kernel: the states are updated in place
        return "out"

    assert not E.fused(pool)
    assert E.kernel_extend(original, None, None, None, None, None, None, ssm_states=pool, cache_indices=slots,
                           query_start_loc=None) == "out"
    assert seen == {"shape": (2, H, V, K), "indices": [0, 1]}
    torch.testing.assert_close(pool.decode(slots), 2 * x, atol=0, rtol=0)


def test_other_kernels_states_go_to_the_wrapped_kernel():
    seen = {}

    def original(self, q, k, v, g, beta, *, ssm_states, cache_indices, query_start_loc):
        seen["states"] = ssm_states
        return "upstream"

    dense = torch.zeros(2, 4, 32, 32, device=dev())
    assert E.kernel_extend(original, None, None, None, None, None, None, ssm_states=dense,
                           cache_indices=None, query_start_loc=None) == "upstream"
    assert seen["states"] is dense


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_reduce_on_device_tensors(dtype):
    parts = [torch.tensor([4096., -3.], dtype=dtype, device=dev()), torch.tensor([1., 1.], dtype=dtype, device=dev()),
             torch.tensor([-4096., 2.], dtype=dtype, device=dev()), torch.tensor([1., 1.], dtype=dtype, device=dev())]
    group = SimpleNamespace(world_size=4)
    seen = []

    def ring(group, x):
        seen.append((x.dtype, x.device.type))
        for part in parts[1:]:
            x = x + part.to(x.dtype)
        return x

    batch = SimpleNamespace(forward_mode=SimpleNamespace(is_extend=lambda: True))
    out = PR.forward(lambda self, fb: PR.all_reduce(ring, group, parts[0]), None, batch)
    assert seen == [(torch.float32, "cuda")]
    assert out.dtype == dtype and out.device.type == "cuda"
    torch.testing.assert_close(out.cpu(), sum(p.double().cpu() for p in parts).to(dtype), rtol=0, atol=0)
