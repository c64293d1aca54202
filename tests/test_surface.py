"""Host-side surface on the CPU: the C ABI exports, layout, plans, schedules."""
import ctypes
import os
import re
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import oracle as O

ROOT = __import__("os").path.dirname(__import__("os").path.dirname(__import__("os").path.abspath(__file__)))


def _declared_symbols():
    text = open(f"{ROOT}/include/stepquant_hip.h").read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(sq_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from stepquant_amd import _native as N
    lib = ctypes.CDLL(N.library_path())
    declared = _declared_symbols()
    assert len(declared) >= 11
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(N.EXPORTS)
    assert N.lib().sq_abi_version() == N.ABI_VERSION


def test_structs_match_header_layout(tmp_path):
    """Every ctypes field sits at the offset gcc gives the header's struct."""
    import subprocess
    from stepquant_amd import _native as N
    structs = {"sq_pool": N.Pool, "sq_step_args": N.StepArgs, "sq_writeback_scratch": N.Scratch,
               "sq_prefill_args": N.PrefillArgs, "sq_format_pool": N.FormatPool}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "stepquant_hip.h"', "int main(void) {"]
    for name, cls in structs.items():
        lines.append(f'  printf("{name} size %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", f"{ROOT}/include", "-o", str(exe), str(src)], check=True)
    seen = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        name, field, value = line.split()
        seen[name, field] = int(value)
    for name, cls in structs.items():
        assert seen[name, "size"] == ctypes.sizeof(cls), name
        for field, _ in cls._fields_:
            assert seen[name, field] == getattr(cls, field).offset, (name, field)


def test_invalid_arguments_are_reported_without_a_device():
    from stepquant_amd import _native as N
    lib = N.lib()
    rc = lib.sq_encode(None, None, None, 4, 1, None)
    assert rc == -22 and b"pool" in lib.sq_last_error()
    with pytest.raises(ValueError):
        N.check(rc, "encode")
    rc = lib.sq_format_step(None, None, None)
    assert rc == -22 and b"format pool" in lib.sq_last_error()
    # a DSQ pool wider than 128 values is rejected before any device access
    fmt = N.FormatPool(data=1, page_bytes=1024, num_slots=2, offsets=1, rows=1, columns=1, heads=1, keys=32,
                       values=256, kind=N.FMT_DSQ, bits=4, group=128, kda=0, flags=0)
    assert lib.sq_format_encode(fmt, None, None, 4, 0, None) == -23
    # a negative row stride would address rows before q/k/v: refused before any launch
    pool = N.Pool(data=1, page_bytes=1024, num_slots=2, bits=1, offsets=1, rows=1, columns=1, impact=1,
                  head_meta=1, heads=1, keys=128, values=128, group=32)
    args = N.StepArgs(q=1, k=1, v=1, g=1, beta=1, out=1, slots=1, batch=1, q_stride=-128, k_stride=128,
                      v_stride=128, key_heads=1, slots_dtype=N.I32)
    rc = lib.sq_decode_step(ctypes.byref(pool), ctypes.byref(args), None)
    assert rc == -22 and b"stride" in lib.sq_last_error()


@pytest.mark.parametrize("arch,bits,V,group", [
    ("gdn", [[6] * 8, [4] * 8, [16] * 8, [2] * 8], 32, 8),
    ("kda", [[2, 4, 6, 8, 16, 6, 16, 2]], 8, 32),
    ("kda", [[2, 4, 8, 16], [16, 16, 16, 16]], 32, 32),
    ("gdn", [[6] * 128] * 32, 128, 32),
])
@pytest.mark.parametrize("storage", ["packed", "byte"])
def test_product_layout_equals_oracle(arch, bits, V, group, storage):
    from stepquant_amd.kernels.pool import packed_layout
    from stepquant_amd.quantization import QuantizationPlan
    b = torch.tensor(bits)
    plan = QuantizationPlan(arch, b, torch.ones_like(b, dtype=torch.float32), group)
    offsets, rows, columns, total = packed_layout(plan, V, storage)
    lay = O.layout(O.Plan(arch, np.array(bits), np.ones(b.shape), group), V, storage)
    assert offsets == lay.offsets.tolist() and rows == lay.rows.tolist()
    assert columns == lay.columns.tolist() and total == lay.page_bytes


def test_plan_validation_messages():
    from stepquant_amd.quantization import QuantizationPlan
    ones = torch.ones(2, 4)
    with pytest.raises(ValueError, match="architecture"):
        QuantizationPlan("mamba", torch.full((2, 4), 6), ones)
    with pytest.raises(ValueError, match="precision"):
        QuantizationPlan("kda", torch.full((2, 4), 3), ones)
    with pytest.raises(ValueError, match="per whole head"):
        QuantizationPlan("gdn", torch.tensor([[6, 4, 6, 6], [6, 6, 6, 6]]), ones)
    with pytest.raises(ValueError, match="positive"):
        QuantizationPlan("kda", torch.full((2, 4), 6), -ones)
    with pytest.raises(ValueError, match="shape"):
        QuantizationPlan("kda", torch.full((2, 4), 6), torch.ones(4, 2))


def test_pool_requires_a_gpu_plan():
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    plan = QuantizationPlan("gdn", torch.full((2, 8), 6), torch.ones(2, 8))
    with pytest.raises(ValueError):
        PackedStatePool(plan, 4, 8)


def test_profiles_tiers():
    from stepquant_amd.kernels.profiles import stepquant6_profile
    for arch in ("gdn", "kda"):
        for batch in (1, 17, 32, 33, 64, 65, 128, 129, 256, 257, 512):
            p = stepquant6_profile(arch, batch)
            assert 0 < p.sms <= 256 and p.chunk % 32 == 0
        assert stepquant6_profile(arch, 33) == stepquant6_profile(arch, 64)
    for batch in (0, 513, True, 32.5):
        with pytest.raises(ValueError):
            stepquant6_profile("gdn", batch)
    with pytest.raises(ValueError):
        stepquant6_profile("mamba", 32)


@pytest.mark.parametrize("chunk", [32, 64, 128, 256, 512])
def test_release_schedule_keeps_tail_bounded(monkeypatch, chunk):
    """Reference tests/test_writeback_schedule.py:8-23 on the same schedule."""
    from stepquant_amd.kernels import writeback
    from stepquant_amd.kernels.writeback import CapturedWrites
    # release points record a gate event on the capturing stream: stubbed on the CPU
    monkeypatch.setattr(writeback, "GraphEvent", lambda: SimpleNamespace(record=lambda stream: None))
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a: None)
    tasks = CapturedWrites(attention_windows=True)
    slots = torch.arange(512)
    recurrent = [True, True, True, False] * 6 + [True, True, False]
    chunks = (len(slots) + chunk - 1) // chunk
    for is_recurrent in recurrent:
        tasks.release_window()
        if is_recurrent:
            pool = SimpleNamespace(plan=SimpleNamespace(architecture="kda"), storage="byte", writeback_chunk=chunk)
            tasks.append((pool, slots))
        assert len(tasks.pending) <= chunks
    assert not tasks.pending
    assert len(tasks) == sum(recurrent) * chunks
    assert sum(task.final for task in tasks) == sum(recurrent)


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
@pytest.mark.parametrize("n", [0, 1, 7, 128, 513])
def test_packing_matches_oracle(bits, n):
    from stepquant_amd.packing import pack, unpack
    x = torch.randint(2 ** bits, (n,), generator=torch.Generator().manual_seed(n))
    p = pack(x, bits)
    assert p.dtype == torch.uint8
    np.testing.assert_array_equal(p.numpy(), O.pack(x.numpy(), bits))
    torch.testing.assert_close(unpack(p, bits, n).long(), x)


def _bare_gdn_pool():
    from stepquant_amd.kernels.pool import PackedStatePool
    pool = object.__new__(PackedStatePool)
    pool.plan = SimpleNamespace(architecture="gdn")
    pool.keys = pool.values = 128
    pool.device = torch.device("cpu")
    pool.deferred = None
    pool.pending = False
    return pool


@pytest.mark.parametrize("cu", [[1, 4, 9], [0, 9, 4], [0, 4, 2, 9]])
def test_prefill_rejects_offsets_outside_the_rows(cu):
    """Offsets that start past row 0 or decrease would send a sequence's
    rows outside q/k/v/out: refused on the host before any launch."""
    pool = _bare_gdn_pool()
    x = torch.zeros(9, 128)
    with pytest.raises(ValueError, match="cu_seqlens must start at 0 and never decrease"):
        pool.extend(x, x, x, torch.zeros(9, 1), torch.zeros(9, 1), [1] * (len(cu) - 1), torch.tensor(cu))


def test_constructor_signature_matches_the_reference_order():
    """PackedStatePool(plan, slots, value_dim=128, writeback_stream=None,
    writeback_workspace=None, writeback_chunk=64, storage='packed')
    (reference kernels/pool.py:70), as INTEGRATION.md documents it."""
    import inspect
    import re
    from stepquant_amd.kernels.pool import PackedStatePool
    params = list(inspect.signature(PackedStatePool.__init__).parameters.values())[1:]
    got = [(p.name, p.default) for p in params]
    assert got == [("plan", inspect.Parameter.empty), ("slots", inspect.Parameter.empty), ("value_dim", 128),
                   ("writeback_stream", None), ("writeback_workspace", None), ("writeback_chunk", 64),
                   ("storage", "packed")]
    doc = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")).read()
    sig = re.search(r"PackedStatePool\(plan, slots, value_dim=128,\s+writeback_stream=None,\s+"
                    r"writeback_workspace=None,\s+writeback_chunk=64,\s+storage=\"packed\"\)", doc)
    assert sig, "INTEGRATION.md documents the constructor in this order"
