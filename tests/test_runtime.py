"""Plan artifacts, per-rank plans and pool sizing of the serving adapter (CPU).

Follows reference sglang/runtime.py:24-80, 297-324 and cli.py:12-18; the
tensor-parallel slot agreement runs over two gloo ranks.
"""
import hashlib
import os
import types

import pytest
import torch

from stepquant_amd.sglang import runtime as R


def _plan_file(tmp_path, *, layers=(0, 2), heads=8, keys=16, nominal=6, fmt=None, version=2, name="plan.pt"):
    g = torch.Generator().manual_seed(0)
    plans = {}
    for layer in layers:
        bits = torch.tensor([4, 6, 8, 6, 6, 8, 4, 6][:heads] * (heads // 8 or 1))[:heads, None].expand(heads, keys)
        plans[f"model.layers.{layer}.linear_attn"] = dict(
            architecture="gdn", bits=bits.clone(), impact=torch.rand(heads, keys, generator=g) + .5,
            value_group_size=32)
    value = dict(format_version=version, plans=plans, settings=dict(nominal_bits=nominal))
    if fmt is not None:
        value["state_format"] = fmt
    path = tmp_path / name
    torch.save(value, path)
    return path, value


@pytest.fixture
def env(monkeypatch):
    R.artifact.cache_clear()
    for k in ("STEPQUANT_PLAN", "STEPQUANT_STATE_FORMAT", "STEPQUANT_ARCHITECTURE", "STEPQUANT_STATE_STORAGE",
              "STEPQUANT_WRITEBACK_SMS", "STEPQUANT_WRITEBACK_CHUNK"):
        monkeypatch.delenv(k, raising=False)
    yield monkeypatch
    R.artifact.cache_clear()


def test_artifact_loads_plans_without_running_code(env, tmp_path):
    path, value = _plan_file(tmp_path)
    env.setenv("STEPQUANT_PLAN", str(path))
    got = R.artifact()
    assert got["format_version"] == 2 and set(got["plans"]) == set(value["plans"])
    assert R.artifact() is got  # cached
    bad, _ = _plan_file(tmp_path, version=1, name="old.pt")
    R.artifact.cache_clear()
    env.setenv("STEPQUANT_PLAN", str(bad))
    with pytest.raises(ValueError, match="unsupported STEPQuant plan format"):
        R.artifact()
    # a file that would need unpickling of arbitrary objects is refused
    evil = tmp_path / "evil.pt"
    torch.save({"format_version": 2, "plans": {}, "x": types.SimpleNamespace(a=1)}, evil)
    R.artifact.cache_clear()
    env.setenv("STEPQUANT_PLAN", str(evil))
    with pytest.raises(Exception, match="(?i)weights_only|unpickl"):
        R.artifact()


@pytest.mark.parametrize("rank", [0, 1])
def test_local_plans_slice_the_rank_heads(env, tmp_path, rank):
    path, value = _plan_file(tmp_path, heads=8)
    env.setenv("STEPQUANT_PLAN", str(path))
    env.setenv("STEPQUANT_STATE_FORMAT", "stepquant6")
    env.setattr(R, "tensor_parallel", lambda: (rank, 2))
    plans = R.local_plans([2, 0], 4, "cpu", 16)
    assert [type(p).__name__ for p in plans] == ["QuantizationPlan"] * 2
    for layer, plan in zip([2, 0], plans):
        full = value["plans"][f"model.layers.{layer}.linear_attn"]
        assert torch.equal(plan.bits, full["bits"][4 * rank:4 * rank + 4])
        assert torch.equal(plan.impact, full["impact"][4 * rank:4 * rank + 4])
        assert plan.bits.is_contiguous() and plan.value_group_size == 32


def test_local_plans_reject_mismatches(env, tmp_path):
    path, _ = _plan_file(tmp_path, heads=8, nominal=4)
    env.setenv("STEPQUANT_PLAN", str(path))
    env.setenv("STEPQUANT_STATE_FORMAT", "stepquant6")
    with pytest.raises(ValueError, match="nominal bits"):
        R.local_plans([0], 8, "cpu", 16)
    env.setenv("STEPQUANT_STATE_FORMAT", "stepquant")
    with pytest.raises(ValueError, match="does not match tensor-parallel shard"):
        R.local_plans([0], 4, "cpu", 16)  # 8 calibrated heads, one rank of 4
    R.artifact.cache_clear()
    path, _ = _plan_file(tmp_path, fmt="sym_int6_g128", name="sym.pt")
    env.setenv("STEPQUANT_PLAN", str(path))
    with pytest.raises(ValueError, match="requires its matching --state-format"):
        R.local_plans([0], 8, "cpu", 16)
    R.artifact.cache_clear()
    torch.save(dict(format_version=2, plans={"model.linear_attn": {}}, settings={}), tmp_path / "odd.pt")
    env.setenv("STEPQUANT_PLAN", str(tmp_path / "odd.pt"))
    with pytest.raises(ValueError, match="cannot map layer name"):
        R.local_plans([0], 8, "cpu", 16)


def test_uncalibrated_formats_need_no_artifact(env):
    env.setenv("STEPQUANT_STATE_FORMAT", "dsq_int4")
    env.setenv("STEPQUANT_ARCHITECTURE", "kda")
    plans = R.local_plans([0, 1, 5], 2, "cpu", 128)
    assert len(plans) == 3
    assert all(p.architecture == "kda" and p.bits.shape == (2, 128) and (p.bits == 4).all() for p in plans)


def test_writeback_settings(env):
    env.setenv("STEPQUANT_STATE_FORMAT", "sym_int8_g128")
    assert R.writeback_settings("gdn", 256) == (32, 64)
    env.setenv("STEPQUANT_STATE_FORMAT", "stepquant6")
    from stepquant_amd.kernels.profiles import stepquant6_profile
    prof = stepquant6_profile("gdn", 256)
    assert R.writeback_settings("gdn", 256) == (prof.sms, prof.chunk)
    env.setenv("STEPQUANT_WRITEBACK_SMS", "40")
    env.setenv("STEPQUANT_WRITEBACK_CHUNK", "16")
    assert R.writeback_settings("kda", 64) == (40, 16)


def test_fingerprint(tmp_path):
    from stepquant_amd.cli import fingerprint
    assert fingerprint(tmp_path) == hashlib.sha256().hexdigest()
    (tmp_path / "config.json").write_text('{"a": 1}')
    (tmp_path / "model.safetensors.index.json").write_text('{"w": 2}')
    assert fingerprint(tmp_path) == hashlib.sha256(b'{"a": 1}{"w": 2}').hexdigest()


def test_temporal_pages_report_page_bytes():
    pages = R.TemporalPages([types.SimpleNamespace(nbytes=100), types.SimpleNamespace(nbytes=28)])
    assert pages.numel() == 128 and pages.shape == (128,) and pages.element_size() == 1
    assert pages.dtype == torch.uint8 and pages[1].nbytes == 28
    with pytest.raises(NotImplementedError):
        pages[0:1]


def _sizing_runner(plans_heads=8, values=128, keys=128, layers=(0, 1, 2), server=None):
    shape = types.SimpleNamespace(temporal=(plans_heads, values, keys), conv=[(3, 2048), (3, 1024)])
    params = types.SimpleNamespace(shape=shape, layers=list(layers), dtype=types.SimpleNamespace(conv=torch.bfloat16),
                                   mamba_cache_per_req=len(layers) * plans_heads * values * keys * 4 + 9216 * 2 * 3)
    server = server or types.SimpleNamespace(max_mamba_cache_size=None, disable_radix_cache=True,
                                             max_running_requests=None, mamba_full_memory_ratio=0.9,
                                             dp_size=1, enable_dp_attention=False)
    return types.SimpleNamespace(mambaish_config=types.SimpleNamespace(mamba2_cache_params=params),
                                 server_args=server)


def test_size_pool_counts_compressed_pages(env, tmp_path):
    path, _ = _plan_file(tmp_path, layers=(0, 1, 2), heads=8, keys=128)
    env.setenv("STEPQUANT_PLAN", str(path))
    runner = _sizing_runner()
    from stepquant_amd.kernels.pool import packed_layout
    plans = R.local_plans([0, 1, 2], 8, "cpu", 128)
    compact = (3 * 2048 + 3 * 1024) * 2 * 3 + sum(packed_layout(p, 128)[-1] for p in plans)
    rest = 40.0
    seen = {}

    def original(self, total):
        seen["cap"] = self.server_args.max_mamba_cache_size
        return 7.0

    got = R.size_pool(original, runner, rest)
    budget = rest * .9 / 1.9
    count = int(budget * (1 << 30) // compact) - 1
    assert seen["cap"] == count == runner.server_args.max_mamba_cache_size
    dense = runner.mambaish_config.mamba2_cache_params.mamba_cache_per_req
    assert got == pytest.approx(7.0 + (count * (dense - compact) - compact) / (1 << 30))
    # an explicit capacity is kept
    runner2 = _sizing_runner()
    runner2.server_args.max_mamba_cache_size = 5
    R.size_pool(original, runner2, rest)
    assert runner2.server_args.max_mamba_cache_size == 5
    with pytest.raises(ValueError, match="insufficient memory"):
        R.size_pool(original, _sizing_runner(), 1e-6)


def _rank_sizes(rank, world, port, tmp, out):
    import torch.distributed as dist
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port), STEPQUANT_PLAN=tmp,
                      STEPQUANT_STATE_FORMAT="stepquant")
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        R.artifact.cache_clear()
        runner = _sizing_runner(plans_heads=4)
        R.size_pool(lambda self, total: 0.0, runner, 2.0)
        out[rank] = (runner.server_args.max_mamba_cache_size,
                     sum(R.packed_layout(p, 128)[-1] for p in R.local_plans([0, 1, 2], 4, "cpu", 128)))
    finally:
        dist.destroy_process_group()


def test_size_pool_agrees_across_tensor_parallel_ranks(tmp_path):
    """Mixed plans give the two ranks different page sizes; both expose the
    smaller slot count (MIN all-reduce over gloo)."""
    import socket
    import torch.multiprocessing as mp
    path, _ = _plan_file(tmp_path, layers=(0, 1, 2), heads=8, keys=128)
    value = torch.load(path, weights_only=True)
    for entry in value["plans"].values():  # rank 1's heads are all 8-bit
        entry["bits"][4:] = 8
    torch.save(value, path)
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    out = mp.Manager().dict()
    mp.spawn(_rank_sizes, args=(2, port, str(path), out), nprocs=2, join=True)
    (c0, p0), (c1, p1) = out[0], out[1]
    assert p1 > p0, "rank 1 holds the larger pages"
    assert c0 == c1
