"""sq_copy_slots_static (allocation-free copy through the library's static
device staging) against sq_copy_slots (caller-provided staging), through the
C ABI on an MI355X: two calls in a row, the second smaller, with
overlapping index sets and a skipped pair; oversize requests are refused
before any launch."""
import numpy as np
import pytest
import torch

from tests.helpers import dev, device_plan, make_plan

pytestmark = pytest.mark.gpu


def _pools(n_slots):
    from stepquant_amd.kernels.pool import PackedStatePool
    import bench
    bits, impact = bench.make_plan(torch, "gdn", 32, 128, 6)
    oplan = make_plan("gdn", bits.numpy(), impact=impact.numpy())
    a = PackedStatePool(device_plan(oplan), n_slots, 128)
    b = PackedStatePool(device_plan(oplan), n_slots, 128)
    g = torch.Generator(device=dev()).manual_seed(3)
    slots = torch.arange(1, n_slots, device=dev())
    x = torch.randn(n_slots - 1, 32, 128, 128, device=dev(), generator=g) * .05
    a.encode(x, slots)
    b.encode(x, slots)
    torch.cuda.synchronize()
    assert torch.equal(a.data, b.data)
    return a, b


def _copy(pool, src, dst, static):
    from stepquant_amd import _native as N
    src = torch.as_tensor(src, dtype=torch.int64, device=dev())
    dst = torch.as_tensor(dst, dtype=torch.int64, device=dev())
    if static:
        rc = N.lib().sq_copy_slots_static(pool._desc, N.ptr(src), N.ptr(dst), N.I64, src.numel(), N.stream_handle())
    else:
        temp = torch.empty((src.numel(), pool.page_bytes), device=dev(), dtype=torch.uint8)
        rc = N.lib().sq_copy_slots(pool._desc, N.ptr(src), N.ptr(dst), N.I64, src.numel(), N.ptr(temp),
                                   N.stream_handle())
    torch.cuda.synchronize()
    return rc


def test_static_copy_matches_copy_on_two_calls():
    from stepquant_amd import _native as N
    print("case static copy: 30 pages then 7 pages of 409,600 B", flush=True)
    a, b = _pools(48)
    assert 30 * a.page_bytes <= N.COPY_STATIC_BYTES
    # first call: 30 pages, destinations overlapping the sources
    src = list(range(1, 31))
    dst = list(range(11, 41))
    assert _copy(a, src, dst, False) == 0
    assert _copy(b, src, dst, True) == 0
    assert torch.equal(a.data, b.data), "first call: pools differ"
    # second, smaller call: 7 pages, one pair with a source outside the pool
    # (skipped: the staging still holds the first call's pages, which must
    # not reach its destination)
    src = [45, 3, 99, 40, 2, 7, -1]
    dst = [4, 46, 20, 1, 3, 8, 30]
    before = b.data.clone()
    assert _copy(a, src, dst, False) == 0
    assert _copy(b, src, dst, True) == 0
    assert torch.equal(a.data, b.data), "second call: pools differ"
    assert torch.equal(b.data[20], before[20]), "skipped pair wrote its destination"
    assert torch.equal(b.data[30], before[47])  # -1 wraps to the last slot
    assert not b.data[0].any()


def test_static_copy_refuses_more_than_its_staging():
    from stepquant_amd import _native as N
    a, b = _pools(48)
    n = N.COPY_STATIC_BYTES // a.page_bytes + 1
    before = b.data.clone()
    rc = _copy(b, list(range(1, n + 1)), list(range(1, n + 1)), True)
    assert rc == -22
    assert "exceed the static staging" in N.lib().sq_last_error().decode()
    assert torch.equal(b.data, before)
