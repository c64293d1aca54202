"""Plan artifacts and the mamba-pool lifecycle of the serving adapter.

Mirrors reference sglang/runtime.py (24-202, 297-324) over this build's
pools: ``artifact`` loads the calibrated plan file, ``local_plans`` slices it
per tensor-parallel rank, and the ``pool_*`` / ``kernel_*`` / ``size_pool``
functions are AROUND hooks of SGLang's ``MambaPool``, linear-attention
kernels and memory sizing: each takes the wrapped function ``original`` and
its ``self`` first, as SGLang's hook registry calls them.  SGLang itself is
imported lazily and only where a hook needs its internals; without it the
tensor-parallel rank and world come from ``torch.distributed`` (or are 0, 1).

Environment (as the reference): ``STEPQUANT_PLAN`` (plan file),
``STEPQUANT_STATE_FORMAT`` (default ``stepquant``), ``STEPQUANT_ARCHITECTURE``
(uncalibrated formats), ``STEPQUANT_STATE_STORAGE`` (``packed``/``byte``),
``STEPQUANT_ASYNC_WRITEBACK``, ``STEPQUANT_WRITEBACK_SMS``,
``STEPQUANT_WRITEBACK_CHUNK``.
"""
from __future__ import annotations

import dataclasses
import functools
import logging
import math
import os
import re
import weakref

import torch

from ..formats import FormatPlan, get_format
from ..kernels.format_pool import FormatStatePool, format_layout
from ..kernels.pool import PackedStatePool, packed_layout
from ..quantization import QuantizationPlan

log = logging.getLogger(__name__)
_temporal_pools = weakref.WeakSet()
_writeback_profiles = {}

_PLAN_FIELDS = ("architecture", "bits", "impact", "value_group_size")


@functools.lru_cache(maxsize=1)
def artifact():
    """The calibrated plan file named by ``STEPQUANT_PLAN`` (runtime.py:24-29).

    A ``torch.save``'d dict: ``format_version`` (must be 2), ``plans`` (layer
    module name -> QuantizationPlan fields), ``settings`` (``nominal_bits``,
    ...), optionally ``state_format`` and ``checkpoint_fingerprint``.  Loaded
    with ``weights_only=True``: nothing in the file is executed.
    """
    value = torch.load(os.environ["STEPQUANT_PLAN"], map_location="cpu", weights_only=True)
    if not isinstance(value, dict) or value.get("format_version") != 2:
        raise ValueError("unsupported STEPQuant plan format")
    return value


def state_format():
    return get_format(os.environ.get("STEPQUANT_STATE_FORMAT", "stepquant"))


def writeback_settings(architecture, batch):
    """(compute units, chunk) of the writeback stream (runtime.py:38-47):
    STEPQuant@6 defaults from ``stepquant6_profile``, else 32 and 64; the
    environment overrides either ('auto' keeps the profile's value)."""
    from ..kernels.profiles import stepquant6_profile
    six = state_format().name == "stepquant6"
    profile = stepquant6_profile(architecture, batch) if six else None
    sms = os.environ.get("STEPQUANT_WRITEBACK_SMS", "auto" if six else "32")
    chunk = os.environ.get("STEPQUANT_WRITEBACK_CHUNK", "auto" if six else "64")
    return (profile.sms if sms == "auto" else int(sms), profile.chunk if chunk == "auto" else int(chunk))


def tensor_parallel():
    """(rank, world size) of this tensor-parallel worker."""
    try:
        from sglang.srt.distributed import (get_tensor_model_parallel_rank,
                                            get_tensor_model_parallel_world_size)
    except ImportError:
        if torch.distributed.is_available() and torch.distributed.is_initialized():
            return torch.distributed.get_rank(), torch.distributed.get_world_size()
        return 0, 1
    return get_tensor_model_parallel_rank(), get_tensor_model_parallel_world_size()


def local_plans(layer_ids, heads, device, keys=128):
    """This rank's plan of every layer in ``layer_ids`` (runtime.py:50-80).

    Uncalibrated formats (fp32, sym_int*, dsq_int*) get a uniform-width
    FormatPlan from ``STEPQUANT_ARCHITECTURE``.  Calibrated formats read the
    artifact, check that its nominal width and state format match the
    requested one, map module names ``...layers.<i>...`` to layer ids and
    keep the rank's ``heads`` rows of each plan.
    """
    rank, world = tensor_parallel()
    spec = state_format()
    if not spec.calibrated:
        architecture = os.environ["STEPQUANT_ARCHITECTURE"]
        return [FormatPlan(architecture, torch.full((heads, keys), spec.bits, dtype=torch.long),
                           torch.ones(heads, keys)).to(device) for _ in layer_ids]
    plan_file = artifact()
    expected = plan_file.get("state_format", "stepquant")
    if spec.name in ("stepquant4", "stepquant6") and plan_file.get("settings", {}).get("nominal_bits") != spec.bits:
        raise ValueError("plan nominal bits do not match the requested STEPQuant format")
    if spec.kind == "stepquant" and expected != "stepquant":
        raise ValueError(f"{expected} plan requires its matching --state-format")
    if spec.kind != "stepquant" and expected != spec.name:
        raise ValueError(f"plan format {expected} does not match {spec.name}")
    kind = QuantizationPlan if spec.kind == "stepquant" else FormatPlan
    by_layer = {}
    for name, entry in plan_file["plans"].items():
        found = re.search(r"\.layers\.(\d+)\.", name)
        if not found:
            raise ValueError(f"cannot map layer name {name}")
        by_layer[int(found[1])] = entry
    plans = []
    for layer in layer_ids:
        full = kind(**{k: v for k, v in by_layer[layer].items() if k in _PLAN_FIELDS})
        if full.bits.shape[0] != heads * world:
            raise ValueError("calibration head count does not match tensor-parallel shard")
        rows = slice(rank * heads, (rank + 1) * heads)
        plans.append(kind(full.architecture, full.bits[rows].contiguous(), full.impact[rows].contiguous(),
                          full.value_group_size).to(device))
    return plans


class TemporalPages:
    """The per-layer pools in the place of SGLang's dense temporal cache
    (runtime.py:83-99): integer indexing gives a layer's pool, sizes are the
    pools' page bytes."""

    dtype = torch.uint8

    def __init__(self, pages):
        self.pages = pages
        _temporal_pools.add(self)

    def __getitem__(self, index):
        if not isinstance(index, int):
            raise NotImplementedError("use packed pool slot operations")
        return self.pages[index]

    def numel(self):
        return sum(p.nbytes for p in self.pages)

    def element_size(self):
        return 1

    @property
    def shape(self):
        return (self.numel(),)


def pool_init(original, self, **kwargs):
    """MambaPool.__init__ around hook (runtime.py:102-135): the upstream
    constructor runs with an empty temporal shape (so no dense recurrent pool
    is ever allocated), then every layer gets a page pool of ``size + 1``
    slots (slot 0 is the all-zero sentinel)."""
    if kwargs.get("speculative_num_draft_tokens") is not None:
        raise ValueError("STEPQuant currently does not support speculative decoding")
    params = kwargs["cache_params"]
    heads, values, keys = params.shape.temporal  # SGLang orders the temporal shape [H, V, K]
    plans = local_plans(kwargs["mamba_layer_ids"], heads, kwargs["device"], keys)
    if any(p.bits.shape[1] != keys for p in plans):
        raise ValueError("calibration key dimension mismatch")
    empty = dataclasses.replace(params, shape=dataclasses.replace(params.shape, temporal=(heads, 0, 0)))
    original(self, **dict(kwargs, cache_params=empty))
    stream = None
    architecture = plans[0].architecture if plans else os.environ.get("STEPQUANT_ARCHITECTURE", "gdn")
    sms, chunk = writeback_settings(architecture, min(512, max(1, kwargs["size"])))
    if os.environ.get("STEPQUANT_ASYNC_WRITEBACK") == "1":
        from ..kernels.resources import writeback_resources
        resources = writeback_resources(kwargs["device"], sms)
        stream = resources.stream
        log.warning("STEPQuant background CUs: requested=%d actual=%d total=%d", resources.requested_sms,
                    resources.actual_sms, resources.total_sms)
        os.environ["STEPQUANT_WRITEBACK_ACTUAL_SMS"] = str(resources.actual_sms)
    spec = state_format()
    storage = os.environ.get("STEPQUANT_STATE_STORAGE", "packed")
    workspace = {}
    slots = kwargs["size"] + 1
    if spec.kind == "stepquant":
        pools = [PackedStatePool(p, slots, values, writeback_stream=stream, writeback_workspace=workspace,
                                 writeback_chunk=chunk, storage=storage) for p in plans]
    else:
        pools = [FormatStatePool(p, slots, values, spec, writeback_stream=stream) for p in plans]
    pages = TemporalPages(pools)
    self.mamba_cache = dataclasses.replace(self.mamba_cache, temporal=pages)
    self.mem_usage = self.mamba_cache.mem_usage_bytes() / 1024 ** 3
    dense = len(plans) * slots * heads * values * keys * 4
    log.warning("STEPQuant state pool (%s): %d bytes (FP32 %d bytes), %d layers, slots=%d", storage,
                pages.numel(), dense, len(plans), slots)


def pool_alloc(original, self, need_size):
    """MambaPool.alloc (runtime.py:138-147): hand out free slots with their
    convolution state and pages cleared; None when too few are free."""
    if need_size > len(self.free_slots):
        return None
    slots = self.free_slots[:need_size]
    self.free_slots = self.free_slots[need_size:]
    for conv in self.mamba_cache.conv:
        conv[:, slots] = 0
    for pool in self.mamba_cache.temporal.pages:
        pool.clear(slots)
    return slots


def pool_copy_from(original, self, src_index, dst_index):
    for conv in self.mamba_cache.conv:
        conv[:, dst_index] = conv[:, src_index]
    for pool in self.mamba_cache.temporal.pages:
        pool.copy(src_index, dst_index)


def pool_get_cpu_copy(original, self, indices):
    """Host copies for CPU offload (runtime.py:157-160): the convolution
    states and the raw page bytes of ``indices`` (compressed, as stored)."""
    torch.cuda.synchronize()
    return ([conv[:, indices].cpu() for conv in self.mamba_cache.conv],
            [pool.data[indices].cpu() for pool in self.mamba_cache.temporal.pages])


def pool_load_cpu_copy(original, self, mamba_cache_cpu, indices):
    convs, pages = mamba_cache_cpu
    for dst, src in zip(self.mamba_cache.conv, convs):
        dst[:, indices] = src.to(dst.device)
    for pool, src in zip(self.mamba_cache.temporal.pages, pages):
        pool.wait()
        pool.data[indices] = src.to(pool.data.device)


def pool_get_contiguous_buf_infos(original, self):
    raise NotImplementedError("STEPQuant v1 does not support disaggregated serving")


def kernel_decode(original, self, q, k, v, a, b, *, A_log, dt_bias, ssm_states, cache_indices, query_start_loc,
                  **kwargs):
    """Linear-attention decode (runtime.py:172-179): raw gates a, b and
    A_log/dt_bias go to the pool's fused step with L2-normalised q, k."""
    if not isinstance(ssm_states, PackedStatePool):
        return original(self, q, k, v, a, b, A_log=A_log, dt_bias=dt_bias, ssm_states=ssm_states,
                        cache_indices=cache_indices, query_start_loc=query_start_loc, **kwargs)
    out = ssm_states.step(q, k, v, a, b, cache_indices, normalize=True, scale=ssm_states.keys ** -.5,
                          a_log=A_log, dt_bias=dt_bias)
    return out.unsqueeze(0)


def kernel_packed_decode(original, self, mixed_qkv, a, b, *, A_log, dt_bias, scale, ssm_states, cache_indices,
                         num_v_heads, head_v_dim, **kwargs):
    """GDN decode on the fused qkv projection (runtime.py:182-190): q, k, v
    are column splits of ``mixed_qkv`` (strided rows, read in place)."""
    if not isinstance(ssm_states, PackedStatePool):
        return original(self, mixed_qkv, a, b, A_log=A_log, dt_bias=dt_bias, scale=scale, ssm_states=ssm_states,
                        cache_indices=cache_indices, num_v_heads=num_v_heads, head_v_dim=head_v_dim, **kwargs)
    value_width = num_v_heads * head_v_dim
    key_width = (mixed_qkv.shape[-1] - value_width) // 2
    q, k, v = mixed_qkv.split([key_width, key_width, value_width], -1)
    return ssm_states.step(q, k, v, a, b, cache_indices, normalize=True, scale=scale, a_log=A_log,
                           dt_bias=dt_bias).unsqueeze(0)


def _fused_extend(pool):
    return (type(pool) is PackedStatePool and pool.plan.architecture == "gdn" and pool.keys == 128
            and pool.values == 128 and pool.storage == "packed")


def kernel_extend(original, self, q, k, v, g, beta, *, ssm_states, cache_indices, query_start_loc, **kwargs):
    """Linear-attention prefill (runtime.py:193-202).

    GDN STEPQuant pools with K = V = 128 run the chunked prefill straight
    from and into the pages (``PackedStatePool.extend``: log-decay g, beta
    after the sigmoid, L2-normalised q and k, scale K^-0.5, the upstream
    chunk kernel's conventions).  Other pools take the reference's round
    trip: decode the active slots to V-first fp32, run the wrapped kernel on
    them, encode them back.
    """
    if not isinstance(ssm_states, PackedStatePool):
        return original(self, q, k, v, g, beta, ssm_states=ssm_states, cache_indices=cache_indices,
                        query_start_loc=query_start_loc, **kwargs)
    if _fused_extend(ssm_states):
        out = ssm_states.extend(q, k, v, g, beta, cache_indices, query_start_loc, normalize=True,
                                scale=ssm_states.keys ** -.5)
        return out.unsqueeze(0)
    active = ssm_states.decode(cache_indices).transpose(-1, -2).contiguous()
    local = torch.arange(cache_indices.numel(), device=cache_indices.device, dtype=cache_indices.dtype)
    output = original(self, q, k, v, g, beta, ssm_states=active, cache_indices=local,
                      query_start_loc=query_start_loc, **kwargs)
    ssm_states.encode(active.transpose(-1, -2), cache_indices)
    return output


def attention_forward(original, self, *args, **kwargs):
    """Decoder-layer forward hook: an attention layer marks a release window
    for deferred writeback chunks (runtime.py:205-208)."""
    from ..kernels.writeback import attention_window
    attention_window()
    return original(self, *args, **kwargs)


def size_pool(original, self, total_rest_memory):
    """Slot count from the compressed page size (runtime.py:297-324).

    Upstream sizes the mamba cache with dense fp32 states; this hook fixes
    ``max_mamba_cache_size`` from the real per-request bytes (convolution
    state plus every layer's page), takes the minimum over tensor-parallel
    ranks (mixed plans give ranks different page sizes), and returns the
    upstream result corrected from dense to compressed bytes (GiB), slot 0
    included.
    """
    params = self.mambaish_config.mamba2_cache_params
    heads, values, keys = params.shape.temporal
    plans = local_plans(params.layers, heads, "cpu", keys)
    conv_bytes = sum(math.prod(shape) for shape in params.shape.conv) * params.dtype.conv.itemsize * len(params.layers)
    spec = state_format()
    storage = os.environ.get("STEPQUANT_STATE_STORAGE", "packed")
    page_total = sum((packed_layout(p, values, storage) if spec.kind == "stepquant" else
                      format_layout(p, values, spec))[-1] for p in plans)
    compact = conv_bytes + page_total
    dense = params.mamba_cache_per_req
    server = self.server_args
    if server.max_mamba_cache_size is None and not (server.disable_radix_cache and
                                                    server.max_running_requests is not None):
        budget = total_rest_memory * server.mamba_full_memory_ratio / (1 + server.mamba_full_memory_ratio)
        count = max(0, int(budget * (1 << 30) // compact) - 1)
        count = _min_over_tensor_parallel(count)
        if count < 1:
            raise ValueError("insufficient memory for a STEPQuant request slot")
        server.max_mamba_cache_size = count * (server.dp_size if server.enable_dp_attention else 1)
    result = original(self, total_rest_memory)
    return result + (server.max_mamba_cache_size * (dense - compact) - compact) / (1 << 30)


def _min_over_tensor_parallel(count):
    """Every rank must expose the same number of request slots."""
    try:
        from sglang.srt.distributed import get_tp_group
    except ImportError:
        group = None
        if not (torch.distributed.is_available() and torch.distributed.is_initialized()):
            return count
        world = torch.distributed.get_world_size()
    else:
        tp = get_tp_group()
        group, world = tp.cpu_group, tp.world_size
    if world > 1:
        shared = torch.tensor(count, dtype=torch.int64)
        torch.distributed.all_reduce(shared, op=torch.distributed.ReduceOp.MIN, group=group)
        count = int(shared.item())
    return count
