"""Serving-adapter pool lifecycle on an MI355X (reference
tests/test_sglang_cuda.py:69-99, with a stand-in for SGLang's MambaPool,
which is not installed here): pool_init without a dense temporal cache, slot
allocation, copy, CPU offload copies of the page bytes, reuse of freed
slots, and the decode/extend hooks routed to the pools.
"""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import oracle as O
from stepquant_amd.sglang import runtime as R
from tests.helpers import dev

pytestmark = pytest.mark.gpu


@dataclasses.dataclass(frozen=True)
class Shape:
    conv: list
    temporal: tuple


@dataclasses.dataclass(frozen=True)
class Params:
    layers: list
    shape: Shape
    conv_dtype: torch.dtype = torch.bfloat16

    @property
    def mamba_cache_per_req(self):
        h, v, k = self.shape.temporal
        conv = sum(int(np.prod(s)) for s in self.shape.conv) * 2
        return len(self.layers) * (h * v * k * 4 + conv)


class MambaPool:
    """The parts of SGLang's MambaPool the hooks touch: per-conv-shape caches
    [layers, size + 1, ...], a temporal cache [layers, size + 1, H, V, K]
    (zero-sized when the hook passes an empty shape), free slot list."""

    @dataclasses.dataclass(frozen=True)
    class State:
        conv: list
        temporal: object

        def mem_usage_bytes(self):
            t = self.temporal
            return sum(c.numel() * c.element_size() for c in self.conv) + t.numel() * t.element_size()

    def __init__(self, *, size, cache_params, mamba_layer_ids, device, spec_state_size=0, **kw):
        n = len(mamba_layer_ids)
        conv = [torch.zeros((n, size + 1) + tuple(s), device=device, dtype=cache_params.conv_dtype)
                for s in cache_params.shape.conv]
        temporal = torch.zeros((n, size + 1) + tuple(cache_params.shape.temporal), device=device)
        self.mamba_cache = self.State(conv, temporal)
        self.free_slots = torch.arange(1, size + 1, device=device)
        self.layer_index = {layer: i for i, layer in enumerate(mamba_layer_ids)}

    def alloc(self, need_size):  # replaced by the hook
        raise AssertionError

    def free(self, slots):
        self.free_slots = torch.cat([self.free_slots, slots])

    def mamba2_layer_cache(self, layer):
        i = self.layer_index[layer]
        return types_ns(conv=[c[i] for c in self.mamba_cache.conv], temporal=self.mamba_cache.temporal[i])


def types_ns(**kw):
    import types
    return types.SimpleNamespace(**kw)


@pytest.mark.parametrize("fmt", ["stepquant", "sym_int6_g128"])
def test_pool_lifecycle(monkeypatch, fmt):
    print(f"case {fmt}", flush=True)
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    monkeypatch.setenv("STEPQUANT_STATE_FORMAT", fmt)
    monkeypatch.setenv("STEPQUANT_ASYNC_WRITEBACK", "0")
    monkeypatch.setenv("STEPQUANT_ARCHITECTURE", "kda")
    if fmt == "stepquant":
        plan = QuantizationPlan("kda", torch.full((4, 128), 6, device=dev()), torch.ones(4, 128, device=dev()))
        monkeypatch.setattr(R, "local_plans", lambda *args: [plan, plan])
    params = Params(layers=[0, 2], shape=Shape(conv=[(3, 512)], temporal=(4, 128, 128)))
    pool = object.__new__(MambaPool)
    R.pool_init(MambaPool.__init__, pool, size=3, spec_state_size=0, cache_params=params,
                mamba_layer_ids=[0, 2], device=dev())
    assert pool.mamba_cache.temporal.numel() == 2 * pool.mamba_cache.temporal.pages[0].page_bytes * 4
    slots = R.pool_alloc(MambaPool.alloc, pool, 3)
    assert R.pool_alloc(MambaPool.alloc, pool, 1) is None
    page = pool.mamba2_layer_cache(0).temporal
    assert isinstance(page, PackedStatePool)
    page.encode(torch.randn(1, 4, 128, 128, device=dev()) * .1, slots[:1])
    for conv in pool.mamba_cache.conv:
        conv[:, slots[:1]] = 1
    R.pool_copy_from(MambaPool.__init__, pool, slots[:1], slots[1:2])
    assert torch.equal(page.decode(slots[:1]), page.decode(slots[1:2]))
    saved = R.pool_get_cpu_copy(None, pool, slots[1:2])
    assert saved[1][0].device.type == "cpu" and saved[1][0].shape == (1, page.page_bytes)
    page.clear(slots[1:2])
    R.pool_load_cpu_copy(None, pool, saved, slots[1:2])
    assert torch.equal(page.decode(slots[:1]), page.decode(slots[1:2]))
    pool.free(slots[1:2])
    reused = R.pool_alloc(MambaPool.alloc, pool, 1)
    assert reused.item() == slots[1].item()
    assert page.decode(reused).count_nonzero() == 0
    assert all(conv[:, reused].count_nonzero() == 0 for conv in pool.mamba_cache.conv)
    assert pool.mamba_cache.mem_usage_bytes() < params.mamba_cache_per_req * 4
    with pytest.raises(NotImplementedError):
        R.pool_get_contiguous_buf_infos(None, pool)


def test_decode_and_extend_hooks():
    """kernel_decode / kernel_packed_decode reach the fused step; kernel_extend
    runs the chunked prefill into the pages (GDN K = V = 128)."""
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    H, HK, K, V, B = 4, 2, 128, 128, 3
    plan = QuantizationPlan("gdn", torch.tensor([6, 4, 8, 6])[:, None].expand(H, K).contiguous().to(dev()),
                            torch.ones(H, K, device=dev()))
    pool_a = PackedStatePool(plan, B + 1, V)
    pool_b = PackedStatePool(plan, B + 1, V)
    g = torch.Generator().manual_seed(1)
    slots = torch.tensor([3, 1, 2], device=dev())
    x = (torch.randn(B, H, K, V, generator=g) * .1).to(dev())
    pool_a.encode(x, slots)
    pool_b.encode(x, slots)
    mixed = torch.randn(B, 2 * HK * K + H * V, generator=g).to(torch.bfloat16).to(dev())
    a = torch.randn(B, H, generator=g).to(dev())
    b = torch.randn(B, H, generator=g).to(dev())
    a_log = torch.randn(H, generator=g).to(dev()) * .3
    dt = torch.randn(H, generator=g).to(dev()) * .3
    out = R.kernel_packed_decode(None, None, mixed, a, b, A_log=a_log, dt_bias=dt, scale=K ** -.5,
                                 ssm_states=pool_a, cache_indices=slots, num_v_heads=H, head_v_dim=V)
    q, k, v = mixed.split([HK * K, HK * K, H * V], -1)
    ref = pool_b.step(q, k, v, a, b, slots, normalize=True, scale=K ** -.5, a_log=a_log, dt_bias=dt)
    torch.cuda.synchronize()
    assert out.shape == (1, B, H, V) and torch.equal(out[0], ref)
    assert torch.equal(pool_a.data, pool_b.data)
    out2 = R.kernel_decode(None, None, q, k, v, a, b, A_log=a_log, dt_bias=dt, ssm_states=pool_a,
                           cache_indices=slots, query_start_loc=None)
    ref2 = pool_b.step(q, k, v, a, b, slots, normalize=True, scale=K ** -.5, a_log=a_log, dt_bias=dt)
    torch.cuda.synchronize()
    assert torch.equal(out2[0], ref2) and torch.equal(pool_a.data, pool_b.data)
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
    oe = R.kernel_extend(None, None, qe.to(dev()), ke.to(dev()), ve.to(dev()), ge.to(dev()), be.to(dev()),
                         ssm_states=pool_a, cache_indices=slots, query_start_loc=cu.to(dev()))
    torch.cuda.synchronize()
    ref_out, _, final = O.prefill(qe[0].float().numpy(), ke[0].float().numpy(), ve[0].float().numpy(),
                                  ge[0].numpy(), be[0].numpy(), S0, cu.numpy(), normalize=True, scale=K ** -.5)
    assert oe.shape == (1, T, H, V)
    err = np.abs(oe[0].float().cpu().numpy() - ref_out) / (np.abs(ref_out).max(-1, keepdims=True) + 1e-30)
    assert err.max() <= 2 ** -8 + 1e-3
    dense = pool_a._last_prefill[-1].cpu().numpy()  # the kernel's fp32 final states
    err = np.abs(dense - final) / (np.abs(final).max(-1, keepdims=True) + 1e-30)
    assert err.max() <= 1e-3
    oplan = O.Plan("gdn", plan.bits.cpu().numpy(), np.ones((H, K), np.float32), 32)
    lay = O.layout(oplan, V)
    ref = pool_a.data.cpu().numpy().copy()
    O.encode_page(dense, slots.cpu().numpy(), oplan, lay, ref)
    assert np.array_equal(pool_a.data.cpu().numpy(), ref), "final pages are the oracle encoding"


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

    assert R.kernel_extend(original, None, None, None, None, None, None, ssm_states=pool, cache_indices=slots,
                           query_start_loc=None) == "out"
    assert seen == {"shape": (2, H, V, K), "indices": [0, 1]}
    torch.testing.assert_close(pool.decode(slots), 2 * x, atol=0, rtol=0)
