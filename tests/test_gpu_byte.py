"""Byte-carrier pages (storage='byte', reference kernels/pool.py:29-43,
kernels/byte_codec.py, kernels/fit.py BYTE path) on an MI355X.

Bars as for packed pages: encode and decode bit-identical to the oracle; a
decode step (byte pages use the writeback stream, as in the reference) within
rtol 1e-3 / atol 1e-4 on the readout and at most one level per carrier on at
most 0.1% of the requantised values; row and column scales within one fp16
ulp of the oracle's.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import check_scales, dev, device_plan, make_plan
from tests.test_gpu_pool import SCALE_BUDGET

pytestmark = pytest.mark.gpu


def _pool(oplan, slots, V):
    from stepquant_amd.kernels.pool import PackedStatePool
    return PackedStatePool(device_plan(oplan), slots, V, writeback_stream=torch.cuda.Stream(), storage="byte")


def _carriers(pages, slots, oplan, lay, V):
    """int8 carriers [B, H, K, V] of integer rows (0 for pivot rows)."""
    H, K = oplan.bits.shape
    out = np.zeros((len(slots), H, K, V), np.int64)
    for b, s in enumerate(slots):
        if s <= 0:
            continue
        for h in range(H):
            base = int(lay.offsets[H * K + h])
            plane = pages[s, base:base + K * V].view(np.int8).reshape(V, K).T
            integer = oplan.bits[h] != 16
            out[b, h][integer] = plane[integer]
    return out


PLANS = {
    "gdn_mixed": ("gdn", lambda: np.repeat(np.array([6, 4, 8, 16, 2])[:, None], 128, 1), 128),
    "kda_mixed": ("kda", lambda: np.where(np.random.default_rng(4).random((4, 128)) < .03, 16,
                                          np.random.default_rng(5).choice([2, 4, 6, 8], (4, 128))), 128),
    "kda_small": ("kda", lambda: np.array([[2, 4, 8, 16, 6, 16, 2, 8]]), 32),
    "gdn_small": ("gdn", lambda: np.repeat(np.array([2, 6, 16])[:, None], 16, 1), 32),
}


@pytest.mark.parametrize("name", list(PLANS))
def test_byte_encode_and_decode_bit_exact(name):
    arch, mk, V = PLANS[name]
    print(f"case {name}", flush=True)
    oplan = make_plan(arch, mk(), seed=6)
    H, K = oplan.bits.shape
    B = 5
    rng = np.random.default_rng(1)
    r = np.exp(rng.normal(0, .5, (B, H, K, 1)))
    c = np.exp(rng.normal(0, .5, (B, H, 1, V)))
    x = (r * rng.standard_normal((B, H, K, V)) * c * .1).astype(np.float32)
    pool = _pool(oplan, B + 2, V)
    slots = torch.tensor([2, 6, 1, 4, 3], device=dev())
    pool.encode(torch.from_numpy(x).to(dev()), slots)
    lay = O.layout(oplan, V, "byte")
    assert pool.page_bytes == lay.page_bytes
    ref = np.zeros((B + 2, lay.page_bytes), np.uint8)
    O.encode_page(x, slots.cpu().numpy(), oplan, lay, ref, "byte")
    got = pool.data.cpu().numpy()
    assert (got != ref).sum() == 0, f"{(got != ref).sum()} bytes differ"
    dec = pool.decode(slots).cpu().numpy()
    np.testing.assert_array_equal(dec, O.decode_page(ref, slots.cpu().numpy(), oplan, lay, V, "byte"))


@pytest.mark.parametrize("name", list(PLANS))
def test_byte_decode_step_against_oracle(name):
    arch, mk, V = PLANS[name]
    print(f"case {name}", flush=True)
    oplan = make_plan(arch, mk(), seed=8)
    H, K = oplan.bits.shape
    kda = arch == "kda"
    B = 4
    pool = _pool(oplan, B + 2, V)
    slots_np = np.array([3, 0, 1, 5])
    slots = torch.from_numpy(slots_np).to(dev())
    g = torch.Generator().manual_seed(3)
    pool.encode((torch.randn(B, H, K, V, generator=g) * .1).to(dev()), slots)
    lay = O.layout(oplan, V, "byte")
    for it in range(3):
        state = O.decode_page(pool.data.cpu().numpy(), slots_np, oplan, lay, V, "byte")
        q = torch.randn(B, H, K, generator=g)
        k = torch.nn.functional.normalize(torch.randn(B, H, K, generator=g), dim=-1)
        v = torch.randn(B, H, V, generator=g)
        ld = -torch.nn.functional.softplus(torch.randn(B, H, K, generator=g) * .5) if kda else \
            -torch.nn.functional.softplus(torch.randn(B, H, generator=g))
        beta = torch.sigmoid(torch.randn(B, H, generator=g))
        out_ref, upd = O.delta_step(state, q.numpy(), k.numpy(), v.numpy(), ld.numpy(), beta.numpy())
        out = pool.step(q.to(dev()), k.to(dev()), v.to(dev()), ld.to(dev()), beta.to(dev()), slots)
        pool.wait()
        torch.cuda.synchronize()
        o = out.cpu().numpy()
        live = slots_np > 0
        np.testing.assert_allclose(o[live], out_ref[live], rtol=1e-3, atol=1e-4)
        assert not o[~live].any()
        got = pool.data.cpu().numpy()
        assert not got[0].any()
        ref = got.copy()
        O.encode_page(upd, slots_np, oplan, lay, ref, "byte")
        a = _carriers(got, slots_np, oplan, lay, V)[live]
        b = _carriers(ref, slots_np, oplan, lay, V)[live]
        step = np.ones_like(a)
        if kda:
            widths = np.minimum(oplan.bits, 8)[None, :, :, None]
            step = np.broadcast_to(1 << (8 - widths), a.shape)
        elif (oplan.bits == 2).any():
            step = np.broadcast_to(np.where(oplan.bits[None, :, :, None] == 2, 2, 1), a.shape)
        diff = np.abs(a - b)
        assert (diff <= step).all(), "carrier differs by more than one level"
        assert (diff > 0).mean() <= 1e-3, f"{(diff > 0).mean():.2e} of carriers differ"
        check_scales(got, ref, slots_np, oplan, lay, V, SCALE_BUDGET, upd)
        ga = O.decode_page(got, slots_np, oplan, lay, V, "byte")[live]
        gb = O.decode_page(ref, slots_np, oplan, lay, V, "byte")[live]
        assert (~np.isclose(ga, gb, rtol=1e-3, atol=1e-4)).mean() <= 1e-3
