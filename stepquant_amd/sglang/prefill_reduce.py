"""Tensor-parallel sums of prefill activations accumulated in fp32.

Contract of the reference's sglang/prefill_reduce.py:13-25 (module and hook
names kept: the adapter's plugin registers ``forward`` around
``ModelRunner.forward`` and ``all_reduce`` around
``GroupCoordinator.all_reduce``): while an extend (prefill) batch runs, a
bf16 or fp16 all-reduce over more than one rank sums in fp32 and rounds to
the input dtype once, so that identical prompt rows split differently over
ranks reach the recurrent-state quantiser with identical values.  Decode
batches and single-rank groups pass the input through untouched.

On MI355X the wrapped collective is RCCL's all-reduce over xGMI; the upcast
doubles its bytes only during prefill, where the reduce is a small share of
the step.
"""
from contextvars import ContextVar

import torch

_in_prefill = ContextVar("stepquant_prefill_reduce", default=False)

_LOW = (torch.bfloat16, torch.float16)


def forward(original, self, forward_batch, *args, **kwargs):
    """Mark the batch as prefill (extend) or not for the duration of the call."""
    token = _in_prefill.set(bool(forward_batch.forward_mode.is_extend()))
    try:
        return original(self, forward_batch, *args, **kwargs)
    finally:
        _in_prefill.reset(token)


def all_reduce(original, self, input_, *args, **kwargs):
    """Sum over the group in fp32 during prefill; otherwise unchanged."""
    if not (_in_prefill.get() and self.world_size > 1 and input_.dtype in _LOW):
        return original(self, input_, *args, **kwargs)
    return original(self, input_.float(), *args, **kwargs).to(input_.dtype)
