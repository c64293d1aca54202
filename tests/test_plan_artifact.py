"""Plan artifacts (format_version 2) on the CPU: a plan file of the shape the
reference's calibration writes (calibration.py:130-143: per layer name the
``asdict`` of a QuantizationPlan) and its own tests save
(tests/test_benchmark_protocol.py:15-24), loaded the way the serving adapter
loads it (sglang/runtime.py:24-29 ``weights_only=True``; runtime.py:62-77:
layer index from the name, the plan keys, the tensor-parallel head slice),
builds this package's plans and page layouts."""
import dataclasses
import re

import numpy as np
import pytest
import torch

from oracle import oracle as O
from stepquant_amd.formats import FormatPlan, get_format
from stepquant_amd.kernels.format_pool import format_layout
from stepquant_amd.kernels.pool import packed_layout
from stepquant_amd.quantization import QuantizationPlan

PLAN_KEYS = ("architecture", "bits", "impact", "value_group_size")


def _entry(architecture):
    # the reference's fixture: widths 4/6/8/16 over four heads of 128 key rows
    if architecture == "gdn":
        bits = torch.tensor([4, 6, 8, 16])[:, None].expand(4, 128).clone()
    else:
        bits = torch.tensor([4, 6, 8, 16]).repeat(4, 32)
    return dict(architecture=architecture, bits=bits, impact=torch.linspace(.2, 2., 512).reshape(4, 128),
                value_group_size=32)


def _save(tmp_path, plans, bits=6, state_format="stepquant"):
    path = tmp_path / "plan.pt"
    torch.save(dict(format_version=2, state_format=state_format, settings={"nominal_bits": bits},
                    plans=plans, checkpoint_fingerprint="0" * 64), path)
    return path


def _load(path, layer_ids, heads, rank, world, cls):
    artifact = torch.load(path, map_location="cpu", weights_only=True)
    assert artifact["format_version"] == 2
    mapping = {}
    for name, entry in artifact["plans"].items():
        mapping[int(re.search(r"\.layers\.(\d+)\.", name)[1])] = entry
    plans = []
    for layer in layer_ids:
        p = cls(**{k: v for k, v in mapping[layer].items() if k in PLAN_KEYS})
        assert p.bits.shape[0] == heads * world
        sl = slice(rank * heads, (rank + 1) * heads)
        plans.append(cls(p.architecture, p.bits[sl].contiguous(), p.impact[sl].contiguous(), p.value_group_size))
    return plans


@pytest.mark.parametrize("architecture", ["gdn", "kda"])
@pytest.mark.parametrize("storage", ["packed", "byte"])
def test_artifact_round_trip_builds_pools_layouts(tmp_path, architecture, storage):
    entry = _entry(architecture)
    path = _save(tmp_path, {"model.layers.0.linear_attn": entry, "model.layers.3.linear_attn": _entry(architecture)})
    for rank, world, heads in ((0, 1, 4), (1, 2, 2)):
        plans = _load(path, [0, 3], heads, rank, world, QuantizationPlan)
        for plan in plans:
            sl = slice(rank * heads, (rank + 1) * heads)
            assert torch.equal(plan.bits, entry["bits"][sl]) and torch.equal(plan.impact, entry["impact"][sl])
            assert plan.bits.dtype == torch.int64 and plan.value_group_size == 32
            offsets, rows, columns, total = packed_layout(plan, 128, storage)
            lay = O.layout(O.Plan(architecture, plan.bits.numpy(), plan.impact.numpy(), 32), 128, storage)
            assert offsets == list(lay.offsets) and rows == list(lay.rows) and columns == list(lay.columns)
            assert total == lay.page_bytes
    # whole plan, packed GDN: codes K*V*b/8 per head, 2 bytes per integer row,
    # 2*V bytes of column scales per head with integer rows
    if architecture == "gdn" and storage == "packed":
        plan = _load(path, [0], 4, 0, 1, QuantizationPlan)[0]
        expect = sum(128 * 128 * b // 8 for b in (4, 6, 8, 16)) + 3 * 128 * 2 + 3 * 2 * 128
        assert packed_layout(plan, 128)[3] == expect


def test_calibration_entries_are_dataclass_dicts(tmp_path):
    """calibration.py:134 stores ``asdict(QuantizationPlan(...))``: this
    package's plan round-trips through the same dict."""
    plan = QuantizationPlan("kda", _entry("kda")["bits"], _entry("kda")["impact"], 32)
    path = _save(tmp_path, {"model.layers.2.self_attn": dataclasses.asdict(plan)})
    again = _load(path, [2], 4, 0, 1, QuantizationPlan)[0]
    assert again.architecture == "kda" and again.value_group_size == 32
    assert torch.equal(again.bits, plan.bits) and torch.equal(again.impact, plan.impact)


@pytest.mark.parametrize("name", ["sym_int6_g128", "dsq_int4", "fp32"])
def test_artifact_builds_baseline_format_layouts(tmp_path, name):
    spec = get_format(name)
    entry = _entry("gdn")
    entry["bits"] = torch.full((4, 128), spec.bits, dtype=torch.long)
    path = _save(tmp_path, {"model.layers.1.linear_attn": entry}, state_format=name)
    plan = _load(path, [1], 4, 0, 1, FormatPlan)[0]
    offsets, rows, columns, total = format_layout(plan, 128, spec)
    code_bytes = 4 * 128 * 128 * spec.bits // 8
    assert offsets[:2] == [0, 128 * spec.bits // 8] and total >= code_bytes
    if spec.kind == "fp32":
        assert total == code_bytes and all(r == -1 for r in rows)
    layout = O.format_layout(np.full((4, 128), spec.bits), 128, spec.kind, spec.group_size)
    assert offsets == list(layout.offsets) and rows == list(layout.rows) and total == layout.page_bytes


def test_artifact_rejects_plans_the_reference_rejects(tmp_path):
    entry = _entry("gdn")
    entry["bits"] = entry["bits"].clone()
    entry["bits"][0, 5] = 6  # GDN widths are per whole head
    path = _save(tmp_path, {"model.layers.0.linear_attn": entry})
    with pytest.raises(ValueError, match="per whole head"):
        _load(path, [0], 4, 0, 1, QuantizationPlan)
    entry = _entry("kda")
    entry["bits"] = entry["bits"].clone()
    entry["bits"][1, 1] = 3  # no 3-bit codes
    path = _save(tmp_path, {"model.layers.0.linear_attn": entry})
    with pytest.raises(ValueError, match="2, 4, 6, 8 or 16"):
        _load(path, [0], 4, 0, 1, QuantizationPlan)
