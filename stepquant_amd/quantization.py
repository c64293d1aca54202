"""Quantisation plan of the packed state (stepquant/quantization.py:7-30).

A plan holds, per value head and key row, the code width (2, 4, 6, 8 or 16
for an FP16 pivot row) and the fit weight ``impact``.  GDN plans use one
width per whole head; KDA plans may mix widths across rows.  The same
checks and error messages as the reference apply.
"""
from dataclasses import dataclass

import torch


@dataclass
class QuantizationPlan:
    architecture: str
    bits: torch.Tensor  # [H,K], 16 denotes pivots
    impact: torch.Tensor  # [H,K], normalized w
    value_group_size: int = 32  # GDN INT2 row-scale group along the value axis

    def __post_init__(self):
        if self.architecture not in ("gdn", "kda"):
            raise ValueError("architecture must be gdn or kda")
        if self.bits.ndim != 2 or self.bits.shape != self.impact.shape:
            raise ValueError("bits and impact must have shape [heads, key_dim]")
        allowed = torch.tensor([2, 4, 6, 8, 16], device=self.bits.device)
        if not torch.isin(self.bits, allowed).all():
            raise ValueError("precision must be 2, 4, 6, 8 or 16")
        if self.architecture == "gdn" and not (self.bits == self.bits[:, :1]).all():
            raise ValueError("GDN allocation is per whole head")
        if not torch.isfinite(self.impact).all() or (self.impact <= 0).any():
            raise ValueError("impact factors must be finite and positive")
        if self.value_group_size < 1:
            raise ValueError("value_group_size must be positive")

    def to(self, device):
        return QuantizationPlan(self.architecture, self.bits.to(device), self.impact.to(device),
                                self.value_group_size)
