"""Prefill (extend) hook of the linear-attention kernels, fused into the pool.

The reference adapter's ``kernel_extend`` (sglang/runtime.py:193-202) decodes
the active slots into a V-first fp32 state, runs SGLang's chunk kernel on it
and encodes the states back.  For pools whose prefill this package runs
natively (``PackedStatePool.extend``: GDN and KDA pools with K = V = 128,
packed or byte pages) this hook replaces that round trip with one
chunked-prefill call that reads the initial states from the pages and writes
the final states into them; other pools (other shapes, the baseline formats)
keep the round trip.  Registering it in place of the reference's
``runtime.kernel_extend`` is the only change to the adapter.

The chunk kernels' call conventions (reference tests/test_sglang_cuda.py:
36-43) hold: ``beta`` is the write strength after the sigmoid; q and k are
L2-normalised in the kernel and q is scaled by K^-0.5; ``query_start_loc``
holds the sequence offsets.  GDN passes ``g`` as the log decay ``[1, T, H]``.
KDA passes a raw per-channel gate ``[1, T, H, K]`` with ``A_log`` ``[H]``
and ``dt_bias`` ``[H*K]`` keyword arguments, and the log decay is
``-exp(A_log) * softplus(g + dt_bias)``; the fused call computes it inside
the prefill kernel.  Keyword arguments the fused call does not consume raise
``TypeError`` rather than being dropped.
"""
from __future__ import annotations

import torch

from ..kernels.pool import PackedStatePool

# keyword arguments of the chunk kernels' extend that the fused call consumes
_GATE_KWARGS = ("A_log", "dt_bias")


def fused(pool) -> bool:
    """Whether ``pool``'s prefill runs in ``PackedStatePool.extend``."""
    return type(pool) is PackedStatePool and pool.keys == 128 and pool.values == 128


def kernel_extend(original, self, q, k, v, g, beta, *, ssm_states, cache_indices, query_start_loc, **kwargs):
    if fused(ssm_states):
        extra = sorted(set(kwargs) - set(_GATE_KWARGS))
        if extra:
            raise TypeError(f"fused extend does not take keyword arguments {extra}")
        a_log, dt_bias = kwargs.get("A_log"), kwargs.get("dt_bias")
        if (a_log is None) != (dt_bias is None):
            raise TypeError("fused extend takes A_log and dt_bias together")
        out = ssm_states.extend(q, k, v, g, beta, cache_indices, query_start_loc, normalize=True,
                                scale=ssm_states.keys ** -.5, a_log=a_log, dt_bias=dt_bias, beta_logits=False)
        return out.unsqueeze(0)
    if not isinstance(ssm_states, PackedStatePool):
        return original(self, q, k, v, g, beta, ssm_states=ssm_states, cache_indices=cache_indices,
                        query_start_loc=query_start_loc, **kwargs)
    # the wrapped kernel updates V-first fp32 states in place, indexed 0..n-1
    states = ssm_states.decode(cache_indices).transpose(-1, -2).contiguous()
    local = torch.arange(cache_indices.numel(), device=cache_indices.device, dtype=cache_indices.dtype)
    out = original(self, q, k, v, g, beta, ssm_states=states, cache_indices=local,
                   query_start_loc=query_start_loc, **kwargs)
    ssm_states.encode(states.transpose(-1, -2), cache_indices)
    return out
