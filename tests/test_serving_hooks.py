"""This build's serving hooks on the CPU: prefill_reduce's contract (the
reference's tests/test_prefill_reduce.py:11-45 behaviour with a stand-in
coordinator, and a real two-rank gloo all-reduce), the module alias the
reference adapter imports through, and cli.fingerprint."""
import hashlib
import os
import socket
import sys
from types import SimpleNamespace

import pytest
import torch

from stepquant_amd.sglang import prefill_reduce as PR


def _batch(extend):
    return SimpleNamespace(forward_mode=SimpleNamespace(is_extend=lambda: extend))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_sum_is_rounded_once(dtype):
    """4096 + 1 - 4096 + 1 in bf16/fp16 loses the ones when every partial sum
    rounds; summed in fp32 and rounded once it is exact."""
    parts = [torch.tensor([4096., -3.], dtype=dtype), torch.tensor([1., 1.], dtype=dtype),
             torch.tensor([-4096., 2.], dtype=dtype), torch.tensor([1., 1.], dtype=dtype)]
    group = SimpleNamespace(world_size=len(parts))
    seen = []

    def ring(group, x):          # stand-in collective: adds the other ranks' parts in x's dtype
        seen.append(x.dtype)
        for part in parts[1:]:
            x = x + part.to(x.dtype)
        return x

    def model(self, batch):
        return PR.all_reduce(ring, group, parts[0])

    out = PR.forward(model, None, _batch(True))
    assert seen == [torch.float32]
    assert out.dtype == dtype
    exact = sum(p.double() for p in parts).to(dtype)
    torch.testing.assert_close(out, exact, rtol=0, atol=0)
    # the same sum in the low dtype loses the small terms: the hook matters
    low = parts[0]
    for part in parts[1:]:
        low = low + part
    assert not torch.equal(low, exact)


@pytest.mark.parametrize("extend,world", [(False, 4), (True, 1)])
def test_decode_and_single_rank_pass_the_tensor_through(extend, world):
    x = torch.ones(3, dtype=torch.bfloat16)

    def ring(group, value):
        assert value is x
        return value

    def model(self, batch):
        return PR.all_reduce(ring, SimpleNamespace(world_size=world), x)

    assert PR.forward(model, None, _batch(extend)) is x


def test_fp32_inputs_are_not_touched():
    x = torch.ones(2)
    out = PR.forward(lambda self, b: PR.all_reduce(lambda g, v: v, SimpleNamespace(world_size=2), x),
                     None, _batch(True))
    assert out is x


def test_prefill_mark_is_cleared_when_the_forward_raises():
    def broken(self, batch):
        raise RuntimeError("forward failed")

    with pytest.raises(RuntimeError, match="forward failed"):
        PR.forward(broken, None, _batch(True))
    x = torch.ones(2, dtype=torch.float16)
    assert PR.all_reduce(lambda g, v: v, SimpleNamespace(world_size=4), x) is x


def _rank(rank, world, port, out):
    import torch.distributed as dist
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        group = SimpleNamespace(world_size=world)

        def collective(group, x):
            x = x.clone()
            dist.all_reduce(x)
            return x

        big = torch.tensor([4096., 4096.], dtype=torch.bfloat16)
        one = torch.tensor([1., 1.], dtype=torch.bfloat16)
        mine = [big, one, -big, one][rank]
        out[rank] = PR.forward(lambda self, b: PR.all_reduce(collective, group, mine), None, _batch(True))
    finally:
        dist.destroy_process_group()


def test_prefill_reduce_over_four_gloo_ranks():
    import torch.multiprocessing as mp
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    out = mp.Manager().dict()
    mp.spawn(_rank, args=(4, port, out), nprocs=4, join=True)
    for rank in range(4):
        assert out[rank].dtype == torch.bfloat16
        torch.testing.assert_close(out[rank], torch.tensor([2., 2.], dtype=torch.bfloat16), rtol=0, atol=0)


def test_alias_binds_the_reference_module_names():
    import stepquant_amd
    saved = {k: v for k, v in sys.modules.items() if k == "stepquant" or k.startswith("stepquant.")}
    try:
        stepquant_amd.install_alias("stepquant")
        from stepquant.kernels.pool import PackedStatePool, packed_layout  # noqa: F401
        from stepquant.kernels.writeback import defer_writeback, WritebackGraph, attention_window  # noqa: F401
        from stepquant.formats import get_format, FormatPlan  # noqa: F401
        from stepquant.quantization import QuantizationPlan  # noqa: F401
        from stepquant.sglang import prefill_reduce
        from stepquant.cli import fingerprint  # noqa: F401
        assert prefill_reduce is PR
        assert get_format("stepquant6").bits == 6
    finally:
        for k in [k for k in sys.modules if k == "stepquant" or k.startswith("stepquant.")]:
            del sys.modules[k]
        sys.modules.update(saved)


def test_fingerprint(tmp_path):
    from stepquant_amd.cli import fingerprint
    assert fingerprint(tmp_path) == hashlib.sha256().hexdigest()
    (tmp_path / "config.json").write_text('{"a": 1}')
    (tmp_path / "model.safetensors.index.json").write_text('{"w": 2}')
    assert fingerprint(tmp_path) == hashlib.sha256(b'{"a": 1}{"w": 2}').hexdigest()


def _registry(patched_all):
    from stepquant_amd.sglang import extend as E
    hooks = {"a.TritonGDNKernel.extend": [("around", E.kernel_extend, None)],
             "b.GroupCoordinator.all_reduce": [("around", PR.all_reduce, None)],
             "c.Unrelated.forward": [("around", len, None)]}
    patched = set(hooks) if patched_all else {"c.Unrelated.forward", "b.GroupCoordinator.all_reduce"}
    return SimpleNamespace(_hooks=hooks, _patched=patched)


def test_verify_hooks_counts_this_package_hooks():
    """The reference plugin's verify_hooks only sees hooks of its own
    stepquant.sglang modules; this package's extend and prefill_reduce hooks
    are counted here, and an unpatched one refuses to serve."""
    from stepquant_amd.sglang import verify_hooks
    assert verify_hooks(_registry(True)) == ["a.TritonGDNKernel.extend", "b.GroupCoordinator.all_reduce"]
    with pytest.raises(RuntimeError, match="TritonGDNKernel.extend"):
        verify_hooks(_registry(False))
    with pytest.raises(RuntimeError, match="incomplete"):
        verify_hooks(SimpleNamespace(_hooks={}, _patched=set()))


def test_fused_extend_rejects_keyword_arguments_it_would_drop():
    """The fused branch consumes A_log and dt_bias (KDA's raw gate) and
    nothing else: any other keyword argument is an error, not dropped.  The
    checks run before any device work, so a host stand-in of the pool is
    enough."""
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.sglang import extend as E
    pool = object.__new__(PackedStatePool)
    pool.keys = pool.values = 128
    assert E.fused(pool)
    call = dict(ssm_states=pool, cache_indices=None, query_start_loc=None)
    with pytest.raises(TypeError, match="layer_id"):
        E.kernel_extend(None, None, None, None, None, None, None, layer_id=3, **call)
    with pytest.raises(TypeError, match="together"):
        E.kernel_extend(None, None, None, None, None, None, None, A_log=torch.zeros(2), **call)
