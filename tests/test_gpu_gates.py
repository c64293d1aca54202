"""Gate inputs in 16 bits on the K = V = 128 decode kernels (runs on an MI355X).

The step reads the gate, beta, A_log and dt_bias in the dtype they share
(float32, bfloat16 or float16, stepquant_amd/kernels/pool.py) and converts
each to float32 exactly, so a step on 16-bit gates must match, bit for bit,
the same step on those values widened to float32 (the path the oracle tests
cover): readout and requantised pages alike, with and without A_log /
dt_bias, on GDN (GQA, mixed widths with 2-bit and pivot heads) and KDA
(per-row widths with pivot rows) pools.
"""
import numpy as np
import pytest
import torch

from tests.helpers import dev, device_plan, make_plan

pytestmark = pytest.mark.gpu

PLANS = {
    "gdn": lambda H, K: np.repeat(np.array([6, 2, 8, 16])[:, None], K, 1),
    "kda": lambda H, K: np.where(np.random.default_rng(4).random((H, K)) < .03, 16,
                                 np.random.default_rng(5).choice([4, 6, 8], (H, K))),
}


@pytest.mark.parametrize("arch", ["gdn", "kda"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("raw", [False, True])
def test_sixteen_bit_gates_match_widened_gates(arch, dtype, raw):
    from stepquant_amd.kernels.pool import PackedStatePool
    print(f"case {arch} {dtype} raw={raw}", flush=True)
    kda = arch == "kda"
    H, HK, K, V, B = 4, (4 if kda else 2), 128, 128, 5
    oplan = make_plan(arch, PLANS[arch](H, K), seed=9)
    pools = [PackedStatePool(device_plan(oplan), B + 2, V) for _ in range(2)]
    assert all(p._desc.flags & (1 if arch == "gdn" else 2) for p in pools)  # the K = V = 128 kernel
    g = torch.Generator().manual_seed(11)
    slots = torch.tensor([3, 1, 0, 6, 2], device=dev())
    x = (torch.randn(B, H, K, V, generator=g) * .1).to(dev())
    for p in pools:
        p.encode(x, slots)
    gate_shape = (B, H, K) if kda else (B, H)
    for it in range(2):
        q = torch.randn(B, HK * K, generator=g).to(torch.bfloat16).to(dev())
        k = torch.randn(B, HK * K, generator=g).to(torch.bfloat16).to(dev())
        v = torch.randn(B, H * V, generator=g).to(torch.bfloat16).to(dev())
        if raw:
            a = (torch.randn(gate_shape, generator=g) * .5).to(dtype)
            a_log = (torch.randn(H, generator=g) * .3).to(dtype)
            dt_bias = (torch.randn(H * K if kda else H, generator=g) * .3).to(dtype)
            kw16 = dict(a_log=a_log.to(dev()), dt_bias=dt_bias.to(dev()))
            kw32 = dict(a_log=a_log.float().to(dev()), dt_bias=dt_bias.float().to(dev()))
            beta = torch.randn(B, H, generator=g).to(dtype)
        else:
            a = (-torch.nn.functional.softplus(torch.randn(gate_shape, generator=g))).to(dtype)
            beta = torch.sigmoid(torch.randn(B, H, generator=g)).to(dtype)
            kw16 = kw32 = {}
        o16 = pools[0].step(q, k, v, a.to(dev()), beta.to(dev()), slots, normalize=True, scale=K ** -.5, **kw16)
        o32 = pools[1].step(q, k, v, a.float().to(dev()), beta.float().to(dev()), slots, normalize=True,
                            scale=K ** -.5, **kw32)
        torch.cuda.synchronize()
        assert torch.equal(o16, o32), f"step {it}: readout differs"
        assert torch.equal(pools[0].data, pools[1].data), f"step {it}: pages differ"
        assert torch.isfinite(o16.float()).all()
