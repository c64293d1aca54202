"""Writer budgets per captured batch for STEPQuant@6 (reference profiles.py:16-28).

``sms`` is the compute-unit budget of the writeback stream on MI355X (256
CUs in 8 XCDs); the tiers are the reference's A800 budgets scaled by the CU
count (x256/108, rounded to multiples of 8).  ``chunk`` is the number of
requests per deferred writer launch.  Stream priorities are not used on this
platform, so ``foreground_priority`` is False.
"""
from dataclasses import dataclass


@dataclass(frozen=True)
class WritebackProfile:
    sms: int
    chunk: int
    foreground_priority: bool = False


def stepquant6_profile(architecture, batch):
    if architecture not in ("gdn", "kda"):
        raise ValueError("architecture must be gdn or kda")
    if not isinstance(batch, int) or isinstance(batch, bool) or not 1 <= batch <= 512:
        raise ValueError("batch must be an integer in 1..512")
    tier = next(n for n in (32, 64, 128, 256, 512) if batch <= n)
    if architecture == "gdn":
        cus = {32: 72, 64: 56, 128: 152, 256: 192, 512: 192}[tier]
        chunk = {32: 64, 64: 64, 128: 128, 256: 256, 512: 64}[tier]
    else:
        cus = 112 if tier == 512 else 72
        chunk = {32: 64, 64: 64, 128: 128, 256: 256, 512: 128}[tier]
    return WritebackProfile(cus, chunk)
