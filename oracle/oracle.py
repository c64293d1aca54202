"""STEPQuant CPU oracle: Python front end of oracle/stepquant_oracle.c.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module; the product
package ``stepquant_amd`` never does.  It is the checker, not the thing
measured or shipped.

Each function restates the reference algorithm it names (paths relative to
the reference repository):

* ``layout``          stepquant/kernels/pool.py:19-66 (``packed_layout``)
* ``fit_state``       stepquant/quantization.py:54-98
* ``initial_column_scales``/``column_refit``  the column half of fit_state
                      (quantization.py:80-98) for given row scales
* ``encode_page``     fit_state + page stores (kernels/fused.py:62-127, 251-282;
                      kernels/bitpack.py:6-30)
* ``decode_page``     kernels/fused.py:18-59 (``_read``), kernels/byte_codec.py:6-28
* ``prepare``         kernels/fused.py:155-179 (``prepare_inputs_kernel``)
* ``delta_step``      stepquant/core.py:5-15
* ``prefill``         the token recurrence of core.py:5-15 (``delta_step``,
                      GDN or KDA) applied to every token of a sequence, in
                      float64, with
                      the input preparation of kernels/fused.py:155-179; it is
                      the checker for the chunked prefill that replaces
                      sglang/runtime.py:193-202 (``kernel_extend``)
* ``pack``/``unpack`` stepquant/packing.py:6-22
* ``codec_encode``/``codec_decode``  stepquant/quantization.py:101-152 (``StateCodec``)
* ``format_layout``   stepquant/kernels/format_pool.py:9-25
* ``group_fit``/``dual_fit``  stepquant/formats.py:53-86 (baseline formats)
* ``format_encode_page``/``format_decode_page``  kernels/format_pool.py:68-90
                      with the page stores and reads of kernels/formats.py

Parity status: layout, fit_state, encode_page, decode_page, pack/unpack and
codec_encode are pinned by golden vectors written from the reference
(tests/golden) and by the known-answer tests of the reference's own test
suite.  delta_step and prepare are pinned by closed-form invariants and a
brute-force sequential check (tests/test_oracle_math.py).  prefill is pinned
by delta_step on single tokens and by the closed-form chunked (WY) form of
the same recurrence (tests/test_oracle_prefill.py).  The reference's own
chunked kernel lives in sglang==0.5.12 (not vendored, not installed here), so
its exact output is parity unpinned; the sequential recurrence is the oracle.
The baseline formats are pinned without the reference's code: group_fit by
brute force (every code is the nearest level of its group's grid, ties to
even) and closed forms; dual_fit through the same PyTorch-order row mean
that the fit_state golden vectors pin, plus brute force on its column step;
format_layout by closed-form region sizes (tests/test_oracle_formats.py).
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libsqoracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile the C oracle with its Makefile; returns the library path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int
        L = ctypes.c_int64
        F = ctypes.c_float
        _lib.sqo_layout.argtypes = [P, I, I, I, I, I, I, P, P, P]
        _lib.sqo_layout.restype = L
        _lib.sqo_fit_state.argtypes = [P, I, I, I, I, P, P, I, I, P, P, P, P, P]
        _lib.sqo_fit_state.restype = I
        _lib.sqo_encode_page.argtypes = [P, I, I, I, I, P, P, I, I, I, P, P, P, P, P, L]
        _lib.sqo_encode_page.restype = I
        _lib.sqo_decode_page.argtypes = [P, L, P, I, I, I, I, P, I, I, I, P, P, P, P]
        _lib.sqo_decode_page.restype = I
        _lib.sqo_prepare.argtypes = [P, P, L, L, P, P, P, P, I, I, I, I, I, I, F, P, P, P, P]
        _lib.sqo_prepare.restype = None
        _lib.sqo_delta_step.argtypes = [P, P, P, P, P, P, I, I, I, I, I, P, P]
        _lib.sqo_delta_step.restype = None
        _lib.sqo_torch_inner_sum.argtypes = [P, L]
        _lib.sqo_torch_inner_sum.restype = F
        _lib.sqo_torch_outer_sum.argtypes = [P, L, L, L, L]
        _lib.sqo_torch_outer_sum.restype = F
        _lib.sqo_f32_to_f16.argtypes = [F]
        _lib.sqo_f32_to_f16.restype = ctypes.c_uint16
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


@dataclass
class Plan:
    """Mirror of QuantizationPlan (quantization.py:7-30), numpy side."""
    architecture: str
    bits: np.ndarray  # [H,K] int32, 16 = pivot
    impact: np.ndarray  # [H,K] float32
    value_group_size: int = 32

    def __post_init__(self):
        self.bits = _c(self.bits, np.int32)
        self.impact = _c(self.impact, np.float32)

    @property
    def kda(self) -> int:
        return int(self.architecture == "kda")


@dataclass
class Layout:
    offsets: np.ndarray
    rows: np.ndarray
    columns: np.ndarray
    page_bytes: int


def layout(plan: Plan, value_dim: int, storage: str = "packed") -> Layout:
    lib = _load()
    H, K = plan.bits.shape
    off = np.zeros(H * K + H, np.int32)
    rows = np.zeros(H * K, np.int32)
    cols = np.zeros(H, np.int32)
    total = lib.sqo_layout(_ptr(plan.bits), H, K, value_dim, plan.kda, int(storage == "byte"),
                           plan.value_group_size, _ptr(off), _ptr(rows), _ptr(cols))
    return Layout(off, rows, cols, int(total))


def _two_heads(plan):
    if plan.kda:
        return np.zeros(plan.bits.shape[0], bool)
    return plan.bits[:, 0] == 2


def fit_state(x, plan: Plan):
    """Returns (z int16, r f16, c f16, r2 f16 or None, reconstructed f32)."""
    lib = _load()
    x = _c(x, np.float32)
    B, H, K, V = x.shape
    two = _two_heads(plan)
    G = plan.value_group_size if two.any() else V
    z = np.zeros(x.shape, np.int16)
    r = np.zeros((B, H, K), np.uint16)
    c = np.zeros((B, H, V), np.uint16)
    r2 = np.zeros((B, H, K, V // G), np.uint16)
    recon = np.zeros(x.shape, np.float32)
    rc = lib.sqo_fit_state(_ptr(x), B, H, K, V, _ptr(plan.bits), _ptr(plan.impact), plan.kda,
                           plan.value_group_size, _ptr(z), _ptr(r), _ptr(c), _ptr(r2), _ptr(recon))
    if rc:
        raise ValueError(f"oracle fit_state failed ({rc})")
    r2o = r2[:, two].view(np.float16) if two.any() else None
    return z, r.view(np.float16), c.view(np.float16), r2o, recon


def _row_constants(plan: Plan):
    """Per key row: qmax and norm of fit_state (quantization.py:63-72)."""
    bc = np.minimum(plan.bits, 8)
    qmax = (2.0 ** (bc - 1) - 1).astype(np.float32)
    norm = (2.0 ** (8 - bc) if plan.kda else np.ones_like(bc)).astype(np.float32)
    qmax[_two_heads(plan)] = 3.0
    return qmax, norm


def _fp16_scale(x):
    """quantization.py:49-51: clamp(2^-24, 65504).half().float()."""
    return np.clip(np.asarray(x, np.float32), np.float32(2.0 ** -24), np.float32(65504)) \
        .astype(np.float16).astype(np.float32)


def initial_column_scales(x, r_full, plan: Plan):
    """fit_state's c0 (quantization.py:80-82) for given row scales:
    fp16(amax over integer key rows of |x / r| / (qmax * norm)).

    x, r_full: [B, H, K, V] float32, r_full holding each value's row scale
    (the value-group scale on 2-bit GDN heads).  Returns [B, H, V]."""
    x = np.asarray(x, np.float32)
    qmax, norm = _row_constants(plan)
    t = np.abs(x / np.asarray(r_full, np.float32)) / (qmax * norm)[None, :, :, None]
    t = np.where((plan.bits != 16)[None, :, :, None], t, np.float32(0))
    return _fp16_scale(t.max(axis=2))


def column_refit(x, r_full, c0, plan: Plan):
    """The column half of fit_state (quantization.py:83-98) from given row
    scales and initial column scales: z = encode(c0) (rounded and clamped
    to [-qmax, qmax], or the 2-bit GDN levels +-1/+-3), then
    c = fp16(sum_K w^2 v x / sum_K w^2 v^2) with v = r * norm * z, or c0
    where the denominator is zero.

    x, r_full: [B, H, K, V] float32; c0: [B, H, V] float32.  The key sums
    run in float64 and are rounded once to float32, so a result can sit one
    fp16 ulp from fit_state's, which sums in PyTorch's float32 order."""
    x = np.asarray(x, np.float32)
    r_full = np.asarray(r_full, np.float32)
    c0 = np.asarray(c0, np.float32)
    qmax, norm = _row_constants(plan)
    qm = qmax[None, :, :, None]
    nm = norm[None, :, :, None]
    y = ((x / r_full) / c0[:, :, None, :]) / nm
    two = _two_heads(plan)[None, :, None, None]
    z = np.where(two, np.where(y >= 0, np.float32(1), np.float32(-1)) *
                 np.where(np.abs(y) >= 2, np.float32(3), np.float32(1)),
                 np.clip(np.rint(y), -qm, qm)).astype(np.float32)
    wsq = (plan.impact * plan.impact * (plan.bits != 16))[None, :, :, None].astype(np.float32)
    v = (r_full * nm) * z
    num = ((wsq * v) * x).astype(np.float64).sum(axis=2).astype(np.float32)
    den = (wsq * (v * v)).astype(np.float64).sum(axis=2).astype(np.float32)
    c = np.where(den > 0, num / np.maximum(den, np.float32(1e-30)), c0)
    return _fp16_scale(c)


def encode_page(x, slots, plan: Plan, lay: Layout, data, storage: str = "packed"):
    """Writes fit_state(x) into data[slots] in place (slot <= 0 skipped)."""
    lib = _load()
    x = _c(x, np.float32)
    B, H, K, V = x.shape
    slots = _c(slots, np.int64)
    assert data.dtype == np.uint8 and data.flags.c_contiguous and data.shape[-1] == lay.page_bytes
    rc = lib.sqo_encode_page(_ptr(x), B, H, K, V, _ptr(plan.bits), _ptr(plan.impact), plan.kda,
                             plan.value_group_size, int(storage == "byte"), _ptr(lay.offsets),
                             _ptr(lay.rows), _ptr(lay.columns), _ptr(slots), _ptr(data),
                             lay.page_bytes)
    if rc:
        raise ValueError(f"oracle encode_page failed ({rc})")
    return data


def decode_page(data, slots, plan: Plan, lay: Layout, value_dim: int, storage: str = "packed"):
    lib = _load()
    slots = _c(slots, np.int64)
    H, K = plan.bits.shape
    B = slots.size
    out = np.zeros((B, H, K, value_dim), np.float32)
    lib.sqo_decode_page(_ptr(data), lay.page_bytes, _ptr(slots), B, H, K, value_dim,
                        _ptr(plan.bits), plan.kda, plan.value_group_size, int(storage == "byte"),
                        _ptr(lay.offsets), _ptr(lay.rows), _ptr(lay.columns), _ptr(out))
    return out


def prepare(q, k, g, beta, H, K, kda, normalize=False, scale=1.0, a_log=None, dt_bias=None):
    """q,k: [B, HK*K] (rows may be padded: pass the full 2-D arrays)."""
    lib = _load()
    q = _c(q, np.float32).reshape(q.shape[0], -1)
    k = _c(k, np.float32).reshape(k.shape[0], -1)
    B = q.shape[0]
    HK = q.shape[1] // K
    g = _c(g, np.float32)
    beta = _c(beta, np.float32)
    qp = np.zeros((B, H, K), np.float32)
    kp = np.zeros((B, H, K), np.float32)
    ld = np.zeros((B, H, K) if kda else (B, H), np.float32)
    bo = np.zeros((B, H), np.float32)
    al = None if a_log is None else _c(a_log, np.float32)
    db = None if dt_bias is None else _c(dt_bias, np.float32)
    lib.sqo_prepare(_ptr(q), _ptr(k), q.shape[1], k.shape[1], _ptr(g), _ptr(beta), _ptr(al), _ptr(db),
                    B, H, HK, K, int(kda), int(normalize), float(scale), _ptr(qp), _ptr(kp),
                    _ptr(ld), _ptr(bo))
    return qp, kp, ld, bo


def delta_step(state, q, k, v, log_decay, beta):
    """core.py:5-15 on prepared fp32 inputs; returns (output, updated)."""
    lib = _load()
    state = _c(state, np.float32)
    B, H, K, V = state.shape
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    ld = _c(log_decay, np.float32)
    kda = int(ld.ndim == 3)
    beta = _c(beta, np.float32)
    out = np.zeros((B, H, V), np.float32)
    upd = np.zeros_like(state)
    lib.sqo_delta_step(_ptr(state), _ptr(q), _ptr(k), _ptr(v), _ptr(ld), _ptr(beta), B, H, K, V,
                       kda, _ptr(out), _ptr(upd))
    return out, upd


def inner_sum(x):
    """torch CPU order for x.sum(-1) of one contiguous float32 row."""
    x = _c(x, np.float32)
    return np.float32(_load().sqo_torch_inner_sum(_ptr(x), x.size))


def outer_sum(x):
    """torch CPU order for x.sum(-2) of a contiguous [n, ncols] float32 matrix."""
    x = _c(x, np.float32)
    n, ncols = x.shape
    lib = _load()
    out = np.zeros(ncols, np.float32)
    base = x.ctypes.data
    for j in range(ncols):
        out[j] = lib.sqo_torch_outer_sum(ctypes.c_void_p(base + 4 * j), n, ncols, ncols, j)
    return out


def f32_to_f16_bits(x):
    lib = _load()
    x = _c(x, np.float32).ravel()
    return np.array([lib.sqo_f32_to_f16(float(v)) for v in x], np.uint16)


# ---------------------------------------------------------------- packing.py

def pack(codes, bits):
    """packing.py:6-14: little-endian, n = 8/gcd(bits,8) codes per word."""
    if bits not in (2, 4, 6, 8):
        raise ValueError("supported code widths: 2, 4, 6, 8")
    flat = np.asarray(codes).reshape(-1).astype(np.int64)
    n = 8 // math.gcd(bits, 8)
    width = n * bits // 8
    flat = np.pad(flat, (0, (-flat.size) % n)).reshape(-1, n)
    word = (flat << (np.arange(n) * bits)).sum(-1)
    return ((word[:, None] >> (np.arange(width) * 8)) & 255).astype(np.uint8).reshape(-1)


def unpack(data, bits, count):
    """packing.py:17-22."""
    n = 8 // math.gcd(bits, 8)
    width = n * bits // 8
    word = (np.asarray(data).astype(np.int64).reshape(-1, width) << (np.arange(width) * 8)).sum(-1)
    codes = (word[:, None] >> (np.arange(n) * bits)) & ((1 << bits) - 1)
    return codes.reshape(-1)[:count].astype(np.int16)


# ------------------------------------------------------ StateCodec streams

def codec_encode(x, plan: Plan):
    """quantization.py:109-126: per-width code streams + scales + pivots."""
    x = _c(x, np.float32)
    z, r, c, r2, _ = fit_state(x, plan)
    B, H, K, V = x.shape
    flat_bits = plan.bits.reshape(-1)
    z = z.reshape(B, H * K, V).astype(np.int64)
    streams = {}
    for b in (2, 4, 6, 8):
        idx = np.nonzero(flat_bits == b)[0]
        codes = z[:, idx]
        if b == 2 and not plan.kda:
            codes = np.floor_divide(codes + 3, 2)
        else:
            codes = codes + (2 ** (b - 1) - 1)
        streams[b] = pack(codes, b)
    integer_rows = np.nonzero(flat_bits != 16)[0]
    integer_heads = np.nonzero((plan.bits != 16).any(-1))[0]
    pivots = x.reshape(B, H * K, V)[:, flat_bits == 16].astype(np.float16)
    return dict(codes=streams, rows=r.reshape(B, -1)[:, integer_rows],
                columns=c[:, integer_heads], pivots=pivots, two_bit_rows=r2, shape=x.shape)


# ------------------------------------------------------ baseline formats

def format_spec(name):
    """formats.py:30-44 (get_format) for the baseline names: (kind, bits, group)."""
    import re
    if name == "fp32":
        return "fp32", 32, 32
    m = re.fullmatch(r"sym_int([468])_g128", name)
    if m:
        return "symmetric", int(m[1]), 128
    m = re.fullmatch(r"dsq_int([46])", name)
    if m:
        return "dsq", int(m[1]), 128
    raise ValueError(f"unknown state format: {name}")


def format_layout(bits, value_dim, kind, group=128) -> Layout:
    """kernels/format_pool.py:9-25: row code offsets (FP16 rows at even
    bytes), then per-row metadata (symmetric: fp16 scale + fp16 zero point per
    value group; dsq: one fp16 row scale), then per-head dsq column metadata
    (fp16 scale + fp16 zero per column), each region 4-byte aligned."""
    flat = [int(b) for b in np.asarray(bits).reshape(-1)]
    H = np.asarray(bits).shape[0]
    offsets, rows, columns = [], [], []
    cursor = 0
    for b in flat:
        if b == 16:
            cursor += cursor & 1
        offsets.append(cursor)
        cursor += value_dim * b // 8
    cursor = -(-cursor // 4) * 4
    for b in flat:
        meta = b != 16 and kind != "fp32"
        rows.append(cursor if meta else -1)
        if meta:
            cursor += 2 if kind == "dsq" else value_dim // group * 4
    cursor = -(-cursor // 4) * 4
    for _ in range(H):
        columns.append(cursor)
        cursor += value_dim * 4 if kind == "dsq" else 0
    return Layout(np.array(offsets, np.int32), np.array(rows, np.int32), np.array(columns, np.int32), cursor)


def _half_scale(x):
    """formats.py:47-48: clamp(2^-24, 65504) -> fp16 (round to nearest even) -> fp32."""
    return np.clip(np.asarray(x, np.float32), np.float32(2.0 ** -24), np.float32(65504)).astype(
        np.float16).astype(np.float32)


def group_fit(x, bits, group=128):
    """formats.py:53-70 (symmetric kind): codes, scale s, zero point z, reconstruction."""
    x = _c(x, np.float32)
    y = x.reshape(x.shape[:-1] + (x.shape[-1] // group, group))
    limit = np.float32(2 ** (bits - 1) - 1)
    s = _half_scale(np.abs(y).max(-1, keepdims=True) / limit)
    z = np.full_like(s, limit)
    q = np.clip(np.round(y / s), -limit, limit) + z
    return q.reshape(x.shape), s[..., 0], z[..., 0], ((q - z) * s).reshape(x.shape)


def dual_fit(x, bits):
    """formats.py:73-86 (dsq kind, uniform widths): codes, r, c, reconstruction.

    r = fp16(sqrt(max(mean_j |x|, 1e-20))) with the mean in PyTorch's CPU
    order (sum / V), y = x / r, c = fp16(max_i |y| / L), q = clamp(rint(y / c)),
    reconstruction (r c) q."""
    x = _c(x, np.float32)
    B, H, K, V = x.shape
    levels = np.float32(2 ** (min(bits, 8) - 1) - 1)
    ax = np.abs(x)
    mean = np.array([inner_sum(row) for row in ax.reshape(-1, V)], np.float32).reshape(B, H, K, 1) / np.float32(V)
    r = _half_scale(np.sqrt(np.maximum(mean, np.float32(1e-20))))
    y = x / r
    c = _half_scale((np.abs(y) / levels).max(-2, keepdims=True))
    q = np.minimum(np.maximum(np.round(y / c), -levels), levels)
    return q + levels, r[..., 0], c[..., 0, :], (r * c) * q


def _put_half(data, slot, pos, values):
    v = np.asarray(values, np.float32).astype(np.float16).view(np.uint8).reshape(-1)
    data[slot, pos:pos + v.size] = v


def format_encode_page(x, slots, name, lay: Layout, data):
    """FormatStatePool.encode (format_pool.py:68-80 with kernels/formats.py
    store and kernels/bitpack.py store_words): x [B,H,K,V] into data[slots]."""
    kind, bits, group = format_spec(name)
    x = _c(x, np.float32)
    B, H, K, V = x.shape
    if kind == "symmetric":
        codes, s, z, _ = group_fit(x, bits, group)
    elif kind == "dsq":
        codes, r, c, _ = dual_fit(x, bits)
    for b, slot in enumerate(np.asarray(slots).reshape(-1)):
        if slot <= 0:
            continue
        for h in range(H):
            if kind == "dsq":
                for j in range(V):
                    _put_half(data, slot, lay.columns[h] + 4 * j, [c[b, h, j], 0.0])
            for i in range(K):
                off = lay.offsets[h * K + i]
                if kind == "fp32":
                    data[slot, off:off + 4 * V] = x[b, h, i].view(np.uint8)
                    continue
                row = pack(codes[b, h, i].astype(np.int64), bits)
                data[slot, off:off + row.size] = row
                if kind == "dsq":
                    _put_half(data, slot, lay.rows[h * K + i], [r[b, h, i]])
                else:
                    for g in range(V // group):
                        _put_half(data, slot, lay.rows[h * K + i] + 4 * g, [s[b, h, i, g], z[b, h, i, g]])
    return data


def format_decode_page(data, slots, name, lay: Layout, H, K, V):
    """FormatStatePool.decode (kernels/formats.py read): (code - z) s for
    symmetric pages, (r c)(code - L) for dsq pages; zeros for slot <= 0."""
    kind, bits, group = format_spec(name)
    slots = np.asarray(slots).reshape(-1)
    out = np.zeros((slots.size, H, K, V), np.float32)
    L = np.float32(2 ** (min(bits, 8) - 1) - 1)
    half = lambda slot, pos: np.float32(data[slot, pos:pos + 2].view(np.float16)[0])
    for b, slot in enumerate(slots):
        if slot <= 0:
            continue
        for h in range(H):
            cj = None
            if kind == "dsq":
                cj = np.array([half(slot, lay.columns[h] + 4 * j) for j in range(V)], np.float32)
            for i in range(K):
                off = lay.offsets[h * K + i]
                if kind == "fp32":
                    out[b, h, i] = data[slot, off:off + 4 * V].view(np.float32)
                    continue
                code = unpack(data[slot, off:off + V * bits // 8], bits, V).astype(np.float32)
                if kind == "dsq":
                    out[b, h, i] = (half(slot, lay.rows[h * K + i]) * cj) * (code - L)
                else:
                    for g in range(V // group):
                        m = lay.rows[h * K + i] + 4 * g
                        sl = slice(g * group, (g + 1) * group)
                        out[b, h, i, sl] = (code[sl] - half(slot, m + 2)) * half(slot, m)
    return out


def _softplus20(u):
    return np.where(u > 20.0, u, np.log1p(np.exp(np.minimum(u, 20.0))))


def prefill(q, k, v, g, beta, state0, cu_seqlens, checkpoints=None, normalize=False, scale=1.0,
            a_log=None, dt_bias=None, beta_logits=None):
    """Token-sequential GDN or KDA prefill in float64.

    q, k: [T, HK, K]; v: [T, H, V]; g: [T, H] (GDN) or [T, H, K] (KDA,
    per key channel) log decay, or the raw gate a when a_log is given:
    g = -exp(a_log[h]) softplus(a + dt_bias) with dt_bias [H] (GDN) or
    [H * K] (KDA); beta: [T, H], logits (beta = sigmoid(b)) when
    beta_logits is true (default: when a_log is given); state0: [B, H, K, V];
    cu_seqlens: [B + 1] token offsets; checkpoints: [B, NC] token counts
    after which the state is recorded (<= 0 or > length: unused).
    Per token (core.py:5-15): S <- e^g S (KDA: row i scaled by e^{g_i});
    delta = beta (v - S^T k);
    S <- S + k delta^T; o = S^T q, with q, k L2-normalised (eps 1e-6) and q
    scaled as kernels/fused.py:155-179 prepares them.
    Returns (out [T, H, V], states [B, NC, H, K, V], final [B, H, K, V]).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    T, HK, K = q.shape
    H, V = v.shape[1], v.shape[2]
    B = len(cu_seqlens) - 1
    if checkpoints is None:
        checkpoints = np.zeros((B, 0), np.int64)
    checkpoints = np.asarray(checkpoints).reshape(B, -1)
    NC = checkpoints.shape[1]
    kda = g.ndim == 3
    if a_log is not None:
        bias = np.asarray(dt_bias, np.float64)
        bias = bias.reshape(H, K)[None] if kda else bias[None, :]
        rate = np.exp(np.asarray(a_log, np.float64))
        rate = rate[None, :, None] if kda else rate[None, :]
        g = -rate * _softplus20(g + bias)
    if a_log is not None if beta_logits is None else beta_logits:
        beta = 1.0 / (1.0 + np.exp(-beta))
    head_of = np.arange(H) // (H // HK)
    out = np.zeros((T, H, V))
    states = np.zeros((B, NC, H, K, V))
    final = np.zeros((B, H, K, V))
    for b in range(B):
        s0, s1 = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        S = np.array(state0[b], np.float64)
        for t in range(s0, s1):
            qt, kt = q[t][head_of], k[t][head_of]
            if normalize:
                qt = qt / np.sqrt((qt * qt).sum(-1, keepdims=True) + 1e-6)
                kt = kt / np.sqrt((kt * kt).sum(-1, keepdims=True) + 1e-6)
            qt = qt * scale
            S = S * (np.exp(g[t])[:, :, None] if kda else np.exp(g[t])[:, None, None])
            delta = beta[t][:, None] * (v[t] - np.einsum("hk,hkv->hv", kt, S))
            S = S + kt[:, :, None] * delta[:, None, :]
            out[t] = np.einsum("hk,hkv->hv", qt, S)
            for c in range(NC):
                if checkpoints[b, c] == t - s0 + 1:
                    states[b, c] = S
        final[b] = S
    return out, states, final
