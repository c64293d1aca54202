"""Pages of the paper's baseline state formats on one MI355X GPU.

Mirrors ``stepquant.kernels.format_pool`` of the reference
(format_pool.py:9-128): ``format_layout`` and ``FormatStatePool``, a
``PackedStatePool`` whose pages hold fp32 states (``fp32``), symmetric
absmax codes per 128-value group (``sym_int{4,6,8}_g128``) or DSQ dual-axis
codes (``dsq_int{4,6}``).  Encoding, decoding and the fused decode step run
in the HIP kernels behind ``sq_format_encode`` / ``sq_format_decode`` /
``sq_format_step``; clear and copy are the packed pool's page operations.
"""
from __future__ import annotations

import torch

from .. import _native as N
from .pool import PackedStatePool, _indices

_KINDS = {"fp32": N.FMT_FP32, "symmetric": N.FMT_SYMMETRIC, "dsq": N.FMT_DSQ}


def format_layout(plan, value_dim, spec):
    """Byte layout of one page (reference format_pool.py:9-25).

    Per key row its codes (``value_dim * bits / 8`` bytes; FP16 rows start at
    even bytes), then, 4-byte aligned, per row its metadata (symmetric: an
    fp16 scale and an fp16 zero point per value group; DSQ: one fp16 row
    scale; none for fp32), then, 4-byte aligned, per head the DSQ column
    metadata (an fp16 scale and an fp16 zero per column).  Returns
    ``(offsets, rows, columns, page_bytes)``; rows without metadata are -1.
    """
    widths = plan.bits.cpu().reshape(-1).tolist()
    floating, dual = spec.kind == "fp32", spec.kind == "dsq"
    offsets, rows, columns = [], [], []
    cursor = 0
    for w in widths:
        if w == 16:
            cursor += cursor & 1
        offsets.append(cursor)
        cursor += value_dim * w // 8
    cursor = -(-cursor // 4) * 4
    row_meta = 2 if dual else 4 * (value_dim // spec.group_size)
    for w in widths:
        if floating or w == 16:
            rows.append(-1)
        else:
            rows.append(cursor)
            cursor += row_meta
    cursor = -(-cursor // 4) * 4
    for _ in range(plan.bits.shape[0]):
        columns.append(cursor)
        cursor += 4 * value_dim if dual else 0
    return offsets, rows, columns, cursor


class FormatStatePool(PackedStatePool):
    """``PackedStatePool`` surface over baseline-format pages (format_pool.py:29-128).

    Synchronous only (no writeback stream).  Every row of the plan has the
    format's width.  This build's kernels take key dimensions up to 128 (and
    DSQ value dimensions up to 128).
    """

    def __init__(self, plan, slots, value_dim, spec, writeback_stream=None, layout=None):
        if writeback_stream is not None:
            raise ValueError("these fused formats require synchronous writeback")
        if not torch.isin(plan.bits, torch.tensor((spec.bits,), device=plan.bits.device)).all():
            raise ValueError(f"precision map incompatible with {spec.name}")
        self.plan, self.spec = plan, spec
        self.heads, self.keys = plan.bits.shape
        self.values, self.device = value_dim, plan.bits.device
        if self.device.type != "cuda":
            raise ValueError("fused format pool requires CUDA")
        if self.keys & (self.keys - 1) or value_dim & (value_dim - 1) or value_dim % 4:
            raise ValueError("key/value dimensions must be powers of two, value >= 4")
        if spec.kind == "dsq" and self.keys > 128:
            raise ValueError("dual-axis g128 requires key_dim <=128")
        if spec.kind not in ("dsq", "fp32") and value_dim % spec.group_size:
            raise ValueError("group size must divide value dimension")
        if spec.kind not in _KINDS:
            raise ValueError(f"{spec.name} is not a baseline page format")
        if self.keys > 128 or (spec.kind == "dsq" and value_dim > 128):
            raise ValueError("the HIP format kernels take key_dim <= 128 (and DSQ value_dim <= 128)")
        offsets, rows, columns, self.page_bytes = (format_layout(plan, value_dim, spec) if layout is None
                                                   else layout)
        dev = self.device
        self.offsets = torch.tensor(offsets, device=dev, dtype=torch.int32)
        self.rows = torch.tensor(rows, device=dev, dtype=torch.int32)
        self.columns = torch.tensor(columns, device=dev, dtype=torch.int32)
        self.bits = plan.bits.to(torch.int32).contiguous()
        self.impact = plan.impact.float().contiguous()
        self.storage = "packed"
        self.early_writeback = True
        self._pages = torch.zeros(slots * self.page_bytes + 64, device=dev, dtype=torch.uint8)
        self.data = self._pages[:slots * self.page_bytes].view(slots, self.page_bytes)
        self.floating = spec.kind == "fp32"
        self.float_data = self.data.view(torch.float32) if self.floating else None
        self.dual = spec.kind == "dsq"
        self.tile = value_dim if self.dual else min(value_dim, max(32, spec.group_size))
        self.coefficients = None
        self.scratch = None
        self._init_writeback(None, 64)
        self._fdesc = N.FormatPool(
            data=self._pages.data_ptr(), page_bytes=self.page_bytes, num_slots=slots,
            offsets=self.offsets.data_ptr(), rows=self.rows.data_ptr(), columns=self.columns.data_ptr(),
            heads=self.heads, keys=self.keys, values=value_dim, kind=_KINDS[spec.kind], bits=spec.bits,
            group=spec.group_size, kda=int(plan.architecture == "kda"),
            flags=N.FMT_ROWS_CONTIGUOUS if all(o == offsets[0] + r * (value_dim * spec.bits // 8)
                                               for r, o in enumerate(offsets)) else 0)
        # page operations (clear, copy) read only data, page_bytes and num_slots
        self._desc = N.Pool(data=self._pages.data_ptr(), page_bytes=self.page_bytes, num_slots=slots)

    def encode(self, state, slots):
        self.wait()
        if state.shape != (slots.numel(), self.heads, self.keys, self.values):
            raise ValueError("state shape mismatch")
        if slots.numel():
            state = state.to(device=self.device, dtype=torch.float32).contiguous()
            idx = _indices(slots, self.device)
            N.check(N.lib().sq_format_encode(self._fdesc, N.ptr(state), N.ptr(idx), N.dtype_code(idx),
                                             idx.numel(), N.stream_handle()), "format encode")

    def decode(self, slots):
        self.wait()
        state = torch.empty((slots.numel(), self.heads, self.keys, self.values), device=self.device,
                            dtype=torch.float32)
        if slots.numel():
            idx = _indices(slots, self.device)
            N.check(N.lib().sq_format_decode(self._fdesc, N.ptr(idx), N.dtype_code(idx), idx.numel(),
                                             N.ptr(state), N.stream_handle()), "format decode")
        return state

    def step(self, q, k, v, g, beta, slots, *, normalize=False, scale=1., a_log=None, dt_bias=None):
        batch = slots.numel()
        out = torch.empty((batch, self.heads, self.values), device=self.device, dtype=q.dtype)
        if batch:
            q, k = q.reshape(batch, -1, self.keys), k.reshape(batch, -1, self.keys)
            v = v.reshape(batch, self.heads, self.values)
            if self.heads % q.shape[1] or k.shape[1] != q.shape[1] or any(t.stride(-1) != 1 for t in (q, k, v)):
                raise ValueError("invalid head layout")
            args, keep = self._step_args(q, k, v, g, beta, slots, out, normalize, scale, a_log, dt_bias, batch,
                                         q.shape[1])
            N.check(N.lib().sq_format_step(self._fdesc, args, N.stream_handle()), "format step")
        return out

    def extend(self, *args, **kwargs):
        raise ValueError("chunked prefill writes STEPQuant pages; baseline formats use decode/encode")
