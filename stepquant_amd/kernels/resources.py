"""A compute-unit-bounded writeback stream (reference resources.py:19-53).

The reference carves an SM partition with a CUDA Green Context.  On MI355X
the writer gets a stream restricted to ``sm_budget`` compute units spread
over all eight XCDs (``hipExtStreamCreateWithCUMask`` through
``sq_create_cu_stream``), at default priority.  A budget of 0 means an
unrestricted stream.  Streams are cached per (device, budget) and live for
the process, since captured graphs refer to them.

Two scheduling facts of this platform matter to a caller.  A CU-masked
stream is a blocking stream (the call takes no flags): work on the legacy
default stream waits for it, so the foreground should run on a stream of its
own.  And streams share the device's hardware queues (``GPU_MAX_HW_QUEUES``,
4 here) round-robin in creation order: two streams on one queue run in
submission order, so streams created one after the other are the ones that
can run side by side.
"""
from dataclasses import dataclass

import torch

from .. import _native as N


@dataclass
class WritebackResources:
    stream: torch.cuda.Stream
    requested_sms: int
    actual_sms: int
    total_sms: int
    context: object = None
    descriptor: object = None


_resources = {}


def writeback_resources(device, sm_budget=32):
    device = torch.device(device)
    ordinal = torch.cuda.current_device() if device.index is None else device.index
    key = (ordinal, sm_budget)
    if key in _resources:
        return _resources[key]
    with torch.cuda.device(ordinal):
        total = torch.cuda.get_device_properties(ordinal).multi_processor_count
        if not 0 <= sm_budget <= total:
            raise ValueError(f"writeback CU budget must be between 0 and {total}")
        if not sm_budget:
            result = WritebackResources(torch.cuda.Stream(device=ordinal), 0, total, total)
        else:
            raw, actual, total = N.create_cu_stream(ordinal, sm_budget)
            stream = torch.cuda.ExternalStream(raw, device=ordinal)
            result = WritebackResources(stream, sm_budget, actual, total)
        _resources[key] = result
        return result
