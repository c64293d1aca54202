"""State-format registry (stepquant/formats.py:12-101).

Keeps the names, ``get_format``, ``half_scale`` and ``FormatPlan`` that the
serving adapter imports.  The paper's baseline formats (fp32, sym_int*,
dsq_int*) are named here so plans and configs validate, but their fitting
routines belong to the baseline pool, which this build does not provide.
"""
from dataclasses import asdict, dataclass
import re

import torch


@dataclass(frozen=True)
class StateFormat:
    name: str
    kind: str
    bits: int = 8
    group_size: int = 32
    group_axis: str = "v"

    @property
    def calibrated(self):
        return self.kind == "stepquant"

    def to_dict(self):
        return asdict(self)


def get_format(name):
    if name in ("stepquant", "stepquant4", "stepquant6"):
        return StateFormat(name, "stepquant", 4 if name.endswith("4") else 6, 32)
    if name == "fp32":
        return StateFormat(name, "fp32", 32, 32)
    match = re.fullmatch(r"sym_int([468])_g128", name)
    if match:
        return StateFormat(name, "symmetric", int(match[1]), 128)
    match = re.fullmatch(r"dsq_int([46])", name)
    if match:
        return StateFormat(name, "dsq", int(match[1]), 128, group_axis="k")
    raise ValueError(f"unknown state format: {name}")


BASELINE_NAMES = ["fp32", "sym_int4_g128", "sym_int6_g128", "sym_int8_g128", "dsq_int4", "dsq_int6"]
FORMAT_NAMES = BASELINE_NAMES + ["stepquant4", "stepquant6"]


def half_scale(x):
    """Scales stored as FP16: clamp to [2^-24, 65504], round to half, back to float."""
    return x.clamp(2 ** -24, 65504).half().float()


def group_fit(x, spec):
    raise NotImplementedError("baseline format fits (formats.py:51-70) are outside this build")


def dual_fit(x, bits, impact):
    raise NotImplementedError("baseline format fits (formats.py:71-82) are outside this build")


@dataclass
class FormatPlan:
    architecture: str
    bits: torch.Tensor
    impact: torch.Tensor
    value_group_size: int = 32

    def __post_init__(self):
        if self.architecture not in ("gdn", "kda") or self.bits.ndim != 2 or self.bits.shape != self.impact.shape:
            raise ValueError("invalid format plan shape/architecture")
        if not torch.isin(self.bits, torch.tensor([2, 4, 6, 8, 16, 32], device=self.bits.device)).all():
            raise ValueError("invalid state precision")
        if not torch.isfinite(self.impact).all() or (self.impact <= 0).any():
            raise ValueError("impact must be finite and positive")

    def to(self, device):
        return FormatPlan(self.architecture, self.bits.to(device), self.impact.to(device), self.value_group_size)
