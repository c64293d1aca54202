"""State-format registry (stepquant/formats.py:12-101).

Keeps the names, ``get_format``, ``half_scale`` and ``FormatPlan`` that the
serving adapter imports, and the dense fits of the paper's baseline formats
(``group_fit``: fp32 and symmetric per-group absmax; ``dual_fit``: DSQ
row/column scales) as device-agnostic torch functions.  The pages of these
formats live in ``kernels.format_pool.FormatStatePool`` (HIP kernels).
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
    """Symmetric absmax codes per value group (formats.py:53-70).

    Returns ``(codes, scale, zero_point, reconstruction)``: per group of
    ``spec.group_size`` values along the last axis, s = fp16(max|x| / L) and
    z = L with L = 2^(b-1) - 1; codes rint(x / s) clamped to [-L, L] plus z.
    FP32 returns the input with no scales.
    """
    x = x.float()
    if spec.kind == "fp32":
        return x, None, None, x
    if spec.kind != "symmetric":
        raise ValueError("group_fit requires FP32 or symmetric rowwise absmax")
    n = spec.group_size
    if x.shape[-1] % n:
        raise ValueError("value dimension must be divisible by group size")
    levels = float(2 ** (spec.bits - 1) - 1)
    grouped = x.unflatten(-1, (x.shape[-1] // n, n))
    scale = half_scale(grouped.abs().amax(-1, keepdim=True) / levels)
    zero = torch.full_like(scale, levels)
    codes = torch.clamp(torch.round(grouped / scale), -levels, levels) + zero
    return codes.flatten(-2), scale, zero, ((codes - zero) * scale).flatten(-2)


def dual_fit(x, bits, impact):
    """DSQ dual-axis codes (formats.py:73-86): fp16 row scale
    r = fp16(sqrt(max(mean|x|, 1e-20))), fp16 column scale
    c = fp16(max over keys of |x / r| / L), codes clamp(rint((x / r) / c)) + L.
    FP16 rows (width 16) keep ``x.half()``.  ``impact`` is not used (DSQ fits
    no weights).  Returns ``(codes, r, c, zero_points, reconstruction)``."""
    x = x.float()
    if x.shape[-2] > 128:
        raise ValueError("dual-axis g128 currently requires key_dim <= 128")
    width = bits.to(x.device)[None, :, :, None]
    integer = width != 16
    levels = 2 ** (width.clamp_max(8) - 1) - 1
    r = half_scale(x.abs().mean(-1, keepdim=True).clamp_min(1e-20).sqrt())
    y = x / r
    c = half_scale(torch.where(integer, y.abs() / levels, 0).amax(-2, keepdim=True))
    q = torch.round(y / c).maximum(-levels).minimum(levels)
    recon = torch.where(integer, r * c * q, x.half().float())
    return q + levels, r, c, torch.zeros_like(c), recon


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
