"""Per-layer page pool of packed recurrent states on one MI355X GPU.

Mirrors ``stepquant.kernels.pool`` of the reference (pool.py:19-365): the
same constructor, methods, attributes and page byte layout, so the serving
adapter can use it unchanged.  All arithmetic runs in the HIP kernels of
``libstepquant_hip.so``, reached through the C ABI in include/stepquant_hip.h:

* ``step`` without a writeback stream is one fused kernel per call: read the
  tile, gated delta update, readout, requantise, store (``sq_decode_step``).
* ``step`` with a writeback stream splits into a foreground readout
  (``sq_decode_readout``) and a writer launched on the writeback stream
  (``sq_writeback``), eagerly or as a branch of the graph being captured,
  ordered by events with the reference's ``_schedule_writeback``/``wait``
  protocol (pool.py:284-356): ``ready`` orders consumers in the same capture
  or eager stream order, ``graph_ready`` (a ``GraphEvent``) consumers in
  other graphs.
* ``encode`` requantises dense fp32 states bit-identically to the CPU
  ``fit_state``; ``decode`` expands pages to fp32.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from .. import _native as N
from .events import GraphEvent, capture_id, wait_for


def packed_layout(plan, value_dim, storage="packed"):
    """Byte layout of one page (reference kernels/pool.py:19-66).

    Returns ``(offsets, rows, columns, page_bytes)``: per key row the byte
    offset of its first packed value (then one tile stride per head; for byte
    storage the per-head code-plane base), the byte offset of its fp16 row
    scale(s) (-1 for pivots), per head the fp16 column-scale offset (-1 when
    the head has no integer rows), and the page size.  Values are grouped in
    tiles of 16 (GDN) or 4 (KDA) along the value axis; one tile of every row
    of a head is stored contiguously, so a head's codes are one contiguous
    region.  FP16 pivot rows start at even offsets.
    """
    if storage not in ("packed", "byte"):
        raise ValueError("state storage must be packed or byte")
    widths = plan.bits.cpu().tolist()
    kda = plan.architecture == "kda"
    tile = min(4 if kda else 16, value_dim)
    offsets, rows, columns, heads_base = [], [], [], []
    cursor = 0
    for head in widths:
        if storage == "byte":
            base = cursor
            has_codes = any(w != 16 for w in head)
            if has_codes:
                cursor += len(head) * value_dim
            pivot_base = cursor
            n_pivot = 0
            for i, w in enumerate(head):
                if w == 16:
                    offsets.append(pivot_base + 2 * n_pivot * value_dim)
                    n_pivot += 1
                else:
                    offsets.append(base + i)
            cursor += 2 * n_pivot * value_dim
            heads_base.append(base)
        else:
            local = 0
            for w in head:
                if w == 16:
                    local += local & 1
                offsets.append(cursor + local)
                local += tile * w // 8
            stride = local + (local & 1)
            heads_base.append(stride)
            cursor += stride * (value_dim // tile)
    offsets.extend(heads_base)
    cursor += cursor & 1
    for head in widths:
        for w in head:
            if w == 16:
                rows.append(-1)
            else:
                rows.append(cursor)
                cursor += 2 * (value_dim // plan.value_group_size if (w == 2 and not kda) else 1)
    for head in widths:
        if any(w != 16 for w in head):
            columns.append(cursor)
            cursor += 2 * value_dim
        else:
            columns.append(-1)
    if storage == "byte":
        cursor = (cursor + 15) // 16 * 16
    return offsets, rows, columns, cursor


def _head_meta(plan, value_dim, offsets, rows, storage="packed"):
    """Per head: code-region start/bytes and row-scale region start/bytes.

    Packed pages: the head's tile blocks.  Byte pages: the head's int8 plane
    (when it has integer rows) followed by its FP16 pivot rows.
    """
    H, K = plan.bits.shape
    kda = plan.architecture == "kda"
    tile = min(4 if kda else 16, value_dim)
    meta = []
    for h in range(H):
        if storage == "byte":
            widths = plan.bits[h].tolist()
            n_pivot = sum(1 for w in widths if w == 16)
            start = offsets[H * K + h]
            nbytes = (K * value_dim if n_pivot < K else 0) + 2 * n_pivot * value_dim
        else:
            start = offsets[h * K]
            nbytes = offsets[H * K + h] * (value_dim // tile)
        row_offs = [rows[h * K + i] for i in range(K) if rows[h * K + i] >= 0]
        if row_offs:
            rstart = min(row_offs)
            widths = plan.bits[h].tolist()
            per = 2 * (value_dim // plan.value_group_size) if (not kda and widths[0] == 2) else 2
            rbytes = per * len(row_offs)
        else:
            rstart, rbytes = -1, 0
        meta.extend([start, nbytes, rstart, rbytes])
    return meta


def _check_offsets(first, drops):
    """Sequence offsets start at row 0 and never decrease, so every sequence's
    rows lie inside the q/k/v/out rows (cu_seqlens[-1] of them)."""
    if first != 0 or drops:
        raise ValueError("cu_seqlens must start at 0 and never decrease")


def _indices(slots, device):
    if isinstance(slots, torch.Tensor):
        t = slots.to(device)
        if t.dtype not in (torch.int32, torch.int64):
            t = t.to(torch.int64)
        return t.reshape(-1).contiguous()
    return torch.as_tensor(slots, dtype=torch.int64, device=device).reshape(-1).contiguous()


class PackedStatePool:
    def __init__(self, plan, slots, value_dim=128, writeback_stream=None, writeback_workspace=None,
                 writeback_chunk=64, storage="packed"):
        if plan.bits.device.type != "cuda":
            raise ValueError("HIP state pool requires a GPU (cuda) device")
        if storage not in ("packed", "byte"):
            raise ValueError("state storage must be packed or byte")
        if storage == "byte" and writeback_stream is None:
            raise ValueError("byte storage requires a writeback stream")
        self.storage = storage
        self.early_writeback = True
        self.plan = plan
        self.heads, self.keys = plan.bits.shape
        self.values = value_dim
        if self.keys & (self.keys - 1) or value_dim & (value_dim - 1) or value_dim % 4:
            raise ValueError("key/value dimensions must be powers of two, value_dim >= 4")
        if plan.architecture == "gdn" and value_dim % plan.value_group_size:
            raise ValueError("value dimension must be divisible by value_group_size")
        offsets, rows, columns, cursor = packed_layout(plan, value_dim, storage)
        self.page_bytes = cursor
        self.device = plan.bits.device
        dev = self.device
        self.offsets = torch.tensor(offsets, device=dev, dtype=torch.int32)
        self.rows = torch.tensor(rows, device=dev, dtype=torch.int32)
        self.columns = torch.tensor(columns, device=dev, dtype=torch.int32)
        meta = _head_meta(plan, value_dim, offsets, rows, storage)
        self.head_meta = torch.tensor(meta, device=dev, dtype=torch.int32)
        # Kernels over-read up to 15 bytes past a head region with 16-byte loads.
        self._pages = torch.zeros(slots * cursor + 64, device=dev, dtype=torch.uint8)
        self.data = self._pages[:slots * cursor].view(slots, cursor)
        self.bits = plan.bits.to(torch.int32).contiguous()
        self.impact = plan.impact.float().contiguous().to(dev)
        self.coefficients = None
        self.keep_prefill_states = False
        self._desc = N.Pool(
            data=self._pages.data_ptr(), page_bytes=cursor, num_slots=slots, bits=self.bits.data_ptr(),
            offsets=self.offsets.data_ptr(), rows=self.rows.data_ptr(), columns=self.columns.data_ptr(),
            impact=self.impact.data_ptr(), head_meta=self.head_meta.data_ptr(), heads=self.heads,
            keys=self.keys, values=value_dim, group=plan.value_group_size,
            kda=int(plan.architecture == "kda"), storage=int(storage == "byte"),
            max_code_bytes=max(meta[1::4]) if meta else 0, max_row_bytes=max(meta[3::4]) if meta else 0,
            flags=N.pool_flags(self.bits.cpu().reshape(-1).tolist(), meta, columns, self.heads, self.keys,
                               value_dim, plan.value_group_size, int(plan.architecture == "kda"),
                               int(storage == "byte"), cursor),
            reserved=0)
        self._init_writeback(writeback_stream, writeback_chunk)
        self._init_workspace(slots, writeback_workspace)

    # ----------------------------------------------------------- writer state
    def _init_writeback(self, writeback_stream, writeback_chunk):
        if writeback_chunk < 0:
            raise ValueError("writeback chunk must be nonnegative")
        self.writeback_chunk = writeback_chunk
        self.writeback_stream = writeback_stream
        self.pending = False
        self.captured_consumers = False
        self.consumer_dependencies = set()
        self.ready_capture = None
        self.deferred = None
        asynchronous = writeback_stream is not None
        # ready: a torch event, joined by consumers in the writer's own
        # capture (or stream order eagerly); graph_ready: a GraphEvent that
        # consumers in other graphs wait on through a graph node.
        self.ready = torch.cuda.Event() if asynchronous else None
        self.graph_ready = GraphEvent() if asynchronous else None
        self.completion = self.ready
        if asynchronous:
            self.graph_ready.record(torch.cuda.current_stream(self.device))

    def _init_workspace(self, slots, writeback_workspace):
        self.scratch = None
        stream = self.writeback_stream
        if stream is None:
            return
        # Writer inputs stay outside any graph's private pool: a captured
        # graph may otherwise alias them with a later layer's temporaries.
        dev, H, K, V = self.device, self.heads, self.keys, self.values
        self.scratch = (torch.empty((slots, H, K), device=dev, dtype=torch.float32),
                        torch.empty((slots, H, K), device=dev, dtype=torch.float32),
                        torch.empty((slots, H, V), device=dev, dtype=torch.float32),
                        torch.empty((slots, 1), device=dev, dtype=torch.float32),
                        torch.empty(slots, device=dev, dtype=torch.int64))
        for tensor in self.scratch:
            tensor.record_stream(stream)
        # Layers sharing one writer stream share this workspace entry, as in
        # the reference; the fused writer needs no row-coefficient planes.
        workspace = {} if writeback_workspace is None else writeback_workspace
        key = (self.device.index, stream.cuda_stream, slots, H, K)
        if key not in workspace:
            workspace[key] = torch.empty(slots, device=dev, dtype=torch.float32)
        self.coefficients = workspace[key]
        self.coefficients.record_stream(stream)

    @property
    def nbytes(self):
        return self.data.numel()

    def configure_writeback(self, stream, chunk):
        """Bind a capture's writer stream without replacing pages or scratch."""
        if self.writeback_stream is None or chunk < 0:
            raise ValueError("configuring writeback requires an asynchronous pool and nonnegative chunk")
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("select writeback resources before graph capture")
        self.wait()
        if stream != self.writeback_stream:
            for tensor in (*self.scratch, self.coefficients):
                tensor.record_stream(stream)
            self.writeback_stream = stream
        self.writeback_chunk = chunk

    # ------------------------------------------------------------- codecs
    def encode(self, state, slots):
        self.wait()
        if state.shape != (slots.numel(), self.heads, self.keys, self.values):
            raise ValueError("state must be [active slots, heads, key, value]")
        if slots.numel():
            self._writeback(state, slots)

    def _writeback(self, state, slots):
        state = state.to(device=self.device, dtype=torch.float32).contiguous()
        idx = _indices(slots, self.device)
        N.check(N.lib().sq_encode(self._desc, N.ptr(state), N.ptr(idx), N.dtype_code(idx), idx.numel(),
                                  N.stream_handle()), "encode")

    def decode(self, slots):
        self.wait()
        state = torch.empty((slots.numel(), self.heads, self.keys, self.values), device=self.device,
                            dtype=torch.float32)
        if slots.numel():
            idx = _indices(slots, self.device)
            N.check(N.lib().sq_decode_dense(self._desc, N.ptr(idx), N.dtype_code(idx), idx.numel(),
                                            N.ptr(state), N.stream_handle()), "decode")
        return state

    # ---------------------------------------------------------------- step
    def _step_args(self, q, k, v, g, beta, slots, out, normalize, scale, a_log, dt_bias, batch, hq):
        K, H, V = self.keys, self.heads, self.values
        if q.dtype != k.dtype or q.dtype != v.dtype or q.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            q, k, v = q.float(), k.float(), v.float()
        # one request's heads must sit K (V) elements apart for the kernels
        if q.stride(1) != K:
            q = q.contiguous()
        if k.stride(1) != K:
            k = k.contiguous()
        if v.stride(1) != V:
            v = v.contiguous()
        kda = self.plan.architecture == "kda"
        gate = [g, beta] + ([a_log, dt_bias] if a_log is not None else [])
        gdt = g.dtype if all(t.dtype == g.dtype for t in gate) and g.dtype in (
            torch.float32, torch.bfloat16, torch.float16) else torch.float32
        gate = [t.to(device=self.device, dtype=gdt).contiguous() for t in gate]
        g, beta = gate[0], gate[1]
        if g.numel() != batch * H * (K if kda else 1) or beta.numel() != batch * H:
            raise ValueError("gate shapes must be [batch, heads] (GDN) or [batch, heads, key] (KDA)")
        if a_log is not None:
            a_log, dt_bias = gate[2], gate[3]
            if a_log.numel() != H or dt_bias.numel() != H * (K if kda else 1):
                raise ValueError("a_log must be [heads] and dt_bias [heads] (GDN) or [heads*key] (KDA)")
        idx = _indices(slots, self.device)
        args = N.StepArgs(q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), g=g.data_ptr(), beta=beta.data_ptr(),
                          a_log=None if a_log is None else a_log.data_ptr(),
                          dt_bias=None if dt_bias is None else dt_bias.data_ptr(), out=out.data_ptr(),
                          slots=idx.data_ptr(), batch=batch, q_stride=q.stride(0), k_stride=k.stride(0),
                          v_stride=v.stride(0), key_heads=hq, qkv_dtype=N.dtype_code(q),
                          gate_dtype=N.dtype_code(g), out_dtype=N.dtype_code(out),
                          slots_dtype=N.dtype_code(idx), normalize=int(bool(normalize)), scale=float(scale),
                          reserved=0)
        keep = (q, k, v, g, beta, a_log, dt_bias, idx)
        return args, keep

    def step(self, q, k, v, g, beta, slots, *, normalize=False, scale=1., a_log=None, dt_bias=None):
        self.wait()
        if self.deferred is not None and not self.deferred.attention_windows:
            self.deferred.release_window()
        batch = slots.numel()
        if not batch:
            return torch.empty((0, self.heads, self.values), device=q.device, dtype=q.dtype)
        q = q.reshape(batch, -1, self.keys)
        k = k.reshape(batch, -1, self.keys)
        v = v.reshape(batch, self.heads, self.values)
        if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
            raise ValueError("head coordinates must be contiguous")
        hq = q.shape[1]
        if self.heads % hq or k.shape[1] != hq:
            raise ValueError("value heads must be divisible by query heads")
        out = torch.empty((batch, self.heads, self.values), device=q.device, dtype=q.dtype)
        args, keep = self._step_args(q, k, v, g, beta, slots, out, normalize, scale, a_log, dt_bias, batch, hq)
        if self.writeback_stream is None:
            N.check(N.lib().sq_decode_step(self._desc, args, N.stream_handle()), "decode step")
            return out
        if batch > self.scratch[0].shape[0]:
            raise ValueError("active batch exceeds the state pool workspace capacity")
        update_key, decay, delta, partial, stable_slots = (t[:batch] for t in self.scratch)
        scratch = self._scratch_desc(update_key, decay, delta, stable_slots)
        N.check(N.lib().sq_decode_readout(self._desc, args, scratch, N.stream_handle()), "decode readout")
        self._schedule_writeback(update_key, decay, delta, partial, stable_slots)
        return out

    def extend(self, q, k, v, g, beta, slots, cu_seqlens, *, checkpoints=None, checkpoint_slots=None,
               init_slots=None, normalize=False, scale=1., a_log=None, dt_bias=None, beta_logits=None,
               events=None, keep_states=None):
        """Chunked prefill of whole sequences straight from and into the pool.

        The behaviour of the serving adapter's ``kernel_extend``
        (reference sglang/runtime.py:193-202: decode the slots' states, run
        the chunked recurrence, encode the final states back) in one call:
        q, k ``[T, HK*K]`` (or ``[..., T, HK, K]``), v ``[T, H*V]``, g
        ``[T, H]`` (KDA: ``[T, H, K]``, per key channel), beta ``[T, H]``
        (with ``a_log``/``dt_bias``, ``g`` is the raw gate and the log decay
        is ``-exp(a_log) * softplus(g + dt_bias)``; ``beta_logits`` says
        whether beta holds logits, default: when ``a_log`` is given, as the
        decode step's convention),
        ``cu_seqlens`` ``[B+1]`` token offsets, ``slots`` ``[B]``.  Initial
        states come from ``init_slots`` (default ``slots``; ``None`` entries
        or slot <= 0 start from zero).  By default the final state is written
        to ``slots``; ``checkpoints`` ``[B, NC]`` (token counts, ascending;
        checked when they are host tensors) with ``checkpoint_slots``
        ``[B, NC]`` write intermediate prefix states as well.  ``cu_seqlens``
        must start at 0 and never decrease (ValueError otherwise).  Returns the outputs ``[T, H, V]`` in q's dtype.
        ``events`` (benchmarks): two ``torch.cuda.Event`` with timing, recorded
        once already, that the call records on the current stream right before
        and after the recurrence kernel.  ``keep_states`` (tests; default: the
        pool's ``keep_prefill_states``, False) keeps the call's device inputs
        and fp32 state workspaces in ``last_prefill``; otherwise the pool
        holds no reference to them after the call.
        """
        self.wait()
        if self.keys != 128 or self.values != 128:
            raise ValueError("prefill handles pools with K = V = 128")
        kda = self.plan.architecture == "kda"
        dev = self.device
        cu_host = None
        if isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.device.type != "cpu":
            cu = cu_seqlens.to(dev, torch.int32).reshape(-1).contiguous()
            total = 0
            if cu.numel() > 1:
                # one wait for the stream: the row count and the offsets' validity
                first, total, drops = torch.stack([cu[0], cu[-1], (cu[1:] < cu[:-1]).sum().to(torch.int32)]).tolist()
                _check_offsets(first, drops)
        else:
            # offsets known on the host: checked here, copied without a wait
            cu_host = torch.as_tensor(cu_seqlens).to(torch.int32).reshape(-1)
            total = int(cu_host[-1]) if cu_host.numel() > 1 else 0
            if cu_host.numel() > 1:
                _check_offsets(int(cu_host[0]), int((cu_host[1:] < cu_host[:-1]).sum()))
            cu = None  # copied below, with the checkpoints when they are host tensors too
        batch = (cu if cu_host is None else cu_host).numel() - 1
        if batch < 0:
            raise ValueError("cu_seqlens needs at least one entry")
        slots_t = _indices(slots, dev)
        if slots_t.numel() != batch:
            raise ValueError("one slot per sequence")
        q2 = q.reshape(-1, q.shape[-1] * (q.shape[-2] if q.dim() >= 3 else 1)) if q.dim() >= 3 else q
        k2 = k.reshape(-1, k.shape[-1] * (k.shape[-2] if k.dim() >= 3 else 1)) if k.dim() >= 3 else k
        v2 = v.reshape(-1, v.shape[-1] * (v.shape[-2] if v.dim() >= 3 else 1)) if v.dim() >= 3 else v
        if q2.shape[0] != total or k2.shape[0] != total or v2.shape[0] != total:
            raise ValueError("q, k, v need cu_seqlens[-1] token rows")
        if v2.shape[1] != self.heads * self.values or q2.shape[1] % self.keys or q2.shape[1] != k2.shape[1]:
            raise ValueError("q/k rows must hold HK*K values and v rows H*V")
        hk = q2.shape[1] // self.keys
        if self.heads % hk:
            raise ValueError("value heads must be divisible by key heads")
        qkv = []
        for t in (q2, k2, v2):
            t = t.to(torch.bfloat16)
            # the kernels take 16-byte aligned rows less than 2^23 elements apart
            if t.stride(-1) != 1 or t.stride(0) % 8 or t.stride(0) >= 1 << 23 or t.data_ptr() % 16:
                t = t.contiguous()
            qkv.append(t)
        q2, k2, v2 = qkv
        gate_dtype = torch.float32 if g.dtype == torch.float64 else g.dtype
        g2 = g.reshape(total, self.heads * (self.keys if kda else 1)).to(gate_dtype).contiguous()
        b2 = beta.reshape(total, self.heads).to(gate_dtype).contiguous()
        al = None if a_log is None else a_log.to(gate_dtype).contiguous()
        db = None if dt_bias is None else dt_bias.to(gate_dtype).contiguous()
        if (al is None) != (db is None):
            raise ValueError("a_log and dt_bias go together")
        if al is not None and (al.numel() != self.heads or db.numel() != self.heads * (self.keys if kda else 1)):
            raise ValueError("a_log must be [heads] and dt_bias [heads] (GDN) or [heads*key] (KDA)")
        on_host = cu_host is not None and checkpoints is not None and all(
            not isinstance(t, torch.Tensor) or t.device.type == "cpu" for t in (checkpoints, checkpoint_slots))
        if on_host:
            # checkpoints and their slots known on the host: masked there, copied without a wait
            ck_h = torch.as_tensor(checkpoints).to(torch.int32).reshape(batch, -1)
            if checkpoint_slots is None:
                raise ValueError("checkpoints need checkpoint_slots")
            cs_h = torch.as_tensor(checkpoint_slots).to(torch.int64).reshape(batch, -1)
            if cs_h.shape != ck_h.shape:
                raise ValueError("one slot per checkpoint")
            lengths_h = (cu_host[1:] - cu_host[:-1]).reshape(batch, 1)
            used = (ck_h > 0) & (ck_h <= lengths_h)
            # used positions must not decrease along a row: each one is at
            # least the largest used position before it (numpy: host work
            # here is on the step's critical path)
            ck_n, used_n = ck_h.numpy(), used.numpy()
            seen = np.maximum.accumulate(np.where(used_n, ck_n, 0), axis=1)
            if (used_n[:, 1:] & (ck_n[:, 1:] < seen[:, :-1])).any():
                raise ValueError("checkpoints of a sequence must be ascending")
            cs_h = torch.where(used, cs_h, torch.zeros_like(cs_h))
            # offsets, checkpoints and their slots in one pinned buffer: one copy
            n_cs, n_ck, n_cu = cs_h.numel(), ck_h.numel(), cu_host.numel()
            packed = torch.empty(n_cs + (n_ck + n_cu + 1) // 2, dtype=torch.int64, pin_memory=True)
            packed[:n_cs] = cs_h.reshape(-1)
            p32 = packed[n_cs:].view(torch.int32)
            p32[:n_cu] = cu_host
            p32[n_cu:n_cu + n_ck] = ck_h.reshape(-1)
            packed = packed.to(dev, non_blocking=True)
            ck_slots = packed[:n_cs].view(cs_h.shape)
            d32 = packed[n_cs:].view(torch.int32)
            cu = d32[:n_cu]
            ck = d32[n_cu:n_cu + n_ck].view(ck_h.shape)
        else:
            if cu is None:
                cu = cu_host.pin_memory().to(dev, non_blocking=True)
            lengths = (cu[1:] - cu[:-1]).to(torch.int32)
            if checkpoints is None:
                ck = lengths.reshape(batch, 1)
                ck_slots = slots_t.reshape(batch, 1)
            else:
                ck = torch.as_tensor(checkpoints, device=dev).to(torch.int32).reshape(batch, -1)
                if checkpoint_slots is None:
                    raise ValueError("checkpoints need checkpoint_slots")
                ck_slots = _indices(checkpoint_slots, dev).reshape(batch, -1)
                if ck_slots.shape != ck.shape:
                    raise ValueError("one slot per checkpoint")
            valid = (ck > 0) & (ck <= lengths[:, None])
            ck_slots = torch.where(valid, ck_slots, torch.zeros_like(ck_slots)).contiguous()
            ck = ck.contiguous()
        nc = ck.shape[1]
        init = slots_t if init_slots is None else _indices(init_slots, dev)
        out = torch.empty((total, self.heads, self.values), device=dev, dtype=q.dtype)
        # packed pools that the K = V = 128 kernels take are decoded inside
        # the recurrence kernel: no dense initial-state workspace
        page_init = bool(self._desc.flags & (N.POOL_FAST_GDN128 | N.POOL_FAST_KDA128))
        init_state = None if page_init else \
            torch.empty((batch, self.heads, self.keys, self.values), device=dev, dtype=torch.float32)
        keep = self.keep_prefill_states if keep_states is None else keep_states
        ck_state = torch.empty((batch * nc, self.heads, self.keys, self.values), device=dev, dtype=torch.float32)
        init = init.to(ck_slots.dtype)
        args = N.PrefillArgs(
            q=N.ptr(q2), k=N.ptr(k2), v=N.ptr(v2), g=N.ptr(g2), beta=N.ptr(b2), a_log=N.ptr(al),
            dt_bias=N.ptr(db), out=N.ptr(out), cu_seqlens=N.ptr(cu), checkpoints=N.ptr(ck),
            init_slots=N.ptr(init), slots=N.ptr(ck_slots), init_state=N.ptr(init_state),
            checkpoint_state=N.ptr(ck_state), batch=batch, q_stride=q2.stride(0), k_stride=k2.stride(0),
            v_stride=v2.stride(0), key_heads=hk, n_checkpoints=nc, qkv_dtype=N.BF16,
            gate_dtype=N.dtype_code(g2), out_dtype=N.dtype_code(out), slots_dtype=N.dtype_code(ck_slots),
            normalize=int(bool(normalize)), scale=float(scale),
            beta_logits=int(a_log is not None if beta_logits is None else bool(beta_logits)), reserved=0)
        if events is not None:
            # benchmark hook: two recorded torch.cuda.Event (torch creates them
            # at their first record) around the recurrence kernel
            handles = [int(e.cuda_event) for e in events]
            if len(handles) != 2 or not all(handles):
                raise ValueError("events must be two torch.cuda.Event that have been recorded once")
            ev = (ctypes.c_void_p * 2)(*handles)
            args.events = ctypes.cast(ev, ctypes.c_void_p)
        if batch:
            N.check(N.lib().sq_prefill(self._desc, args, N.stream_handle()), "prefill")
        if keep:
            self.last_prefill = (q2, k2, v2, g2, b2, al, db, cu, ck, init, ck_slots, init_state, ck_state)
        return out

    @staticmethod
    def _scratch_desc(update_key, decay, delta, stable_slots):
        return N.Scratch(key=update_key.data_ptr(), decay=decay.data_ptr(), delta=delta.data_ptr(),
                         stable_slots=stable_slots.data_ptr(), capacity=stable_slots.shape[0])

    def _schedule_writeback(self, update_key, decay, delta, partial, stable_slots):
        if self.deferred is not None:
            self.deferred.append((self, update_key, decay, delta, partial, stable_slots))
            return
        here = torch.cuda.current_stream(self.device)
        side = self.writeback_stream
        side.wait_stream(here)
        with torch.cuda.stream(side):
            self._finish_update(update_key, decay, delta, partial, stable_slots)
            self.graph_ready.record(side)
            self.ready.record(side)
        for tensor in (update_key, decay, delta, partial, stable_slots):
            tensor.record_stream(side)
        # Under capture the writer is a branch of the graph: consumers in the
        # same capture join it through `ready`, consumers anywhere else wait
        # on the graph_ready node every replay records.
        self.ready_capture = capture_id(here) if torch.cuda.is_current_stream_capturing() else None
        self.completion = self.graph_ready if self.ready_capture is not None else self.ready
        self.pending = True

    def _finish_update(self, update_key, decay, delta, partial, slots):
        """Writer for one chunk of requests (runs on the current stream)."""
        scratch = self._scratch_desc(update_key, decay, delta, slots)
        N.check(N.lib().sq_writeback(self._desc, scratch, slots.numel(), N.stream_handle()), "writeback")

    def wait(self):
        """Order the current stream after this pool's latest writer.

        Inside ``defer_writeback`` a paired capture waits on the previous
        replay's writer of this layer (its ``graph_ready`` node); a joined
        capture needs nothing, its replays finish their writers.  Otherwise,
        with a writer pending: eagerly, wait on ``completion``; inside the
        writer's own capture, join its branch; inside another capture, add a
        wait node on ``graph_ready`` (and on a graph's completion event, kept
        alive in ``consumer_dependencies``).  A wait orders only the stream
        it is issued on.
        """
        tasks = getattr(self, "deferred", None)
        if tasks is not None:
            if not tasks.joined:
                self.graph_ready.wait(torch.cuda.current_stream(self.device))
            return
        if not self.pending:
            return
        stream = torch.cuda.current_stream(self.device)
        if not torch.cuda.is_current_stream_capturing():
            wait_for(stream, self.completion)
            return
        if self.ready_capture is not None and self.ready_capture == capture_id(stream):
            stream.wait_event(self.ready)
            return
        self.captured_consumers = True
        if self.completion is not self.ready and self.completion is not self.graph_ready:
            self.consumer_dependencies.add(self.completion)
            wait_for(stream, self.completion)
        self.graph_ready.wait(stream)

    # ------------------------------------------------------------ slot ops
    def clear(self, slots):
        self.wait()
        idx = _indices(slots, self.device)
        if idx.numel():
            N.check(N.lib().sq_clear_slots(self._desc, N.ptr(idx), N.dtype_code(idx), idx.numel(),
                                           N.stream_handle()), "clear")

    def copy(self, source, destination):
        self.wait()
        src = _indices(source, self.device).to(torch.int64)
        dst = _indices(destination, self.device).to(torch.int64)
        if src.numel() != dst.numel():
            raise ValueError("copy needs as many destination slots as source slots")
        if src.numel():
            temp = torch.empty((src.numel(), self.page_bytes), device=self.device, dtype=torch.uint8)
            N.check(N.lib().sq_copy_slots(self._desc, N.ptr(src), N.ptr(dst), N.I64, src.numel(), N.ptr(temp),
                                          N.stream_handle()), "copy")
