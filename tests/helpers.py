"""Shared helpers for the parity tests (oracle side and device side)."""
import numpy as np
import torch

from oracle import oracle as O


def dev():
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test selected but no HIP device is visible")
    return torch.device("cuda:0")


def make_plan(arch, bits, impact=None, group=32, seed=0):
    bits = np.asarray(bits, np.int32)
    if impact is None:
        impact = np.random.default_rng(seed).random(bits.shape).astype(np.float32) + .5
    return O.Plan(arch, bits, np.asarray(impact, np.float32), group)


def device_plan(oplan):
    from stepquant_amd.quantization import QuantizationPlan
    d = dev()
    return QuantizationPlan(oplan.architecture, torch.from_numpy(oplan.bits.astype(np.int64)).to(d),
                            torch.from_numpy(oplan.impact).to(d), oplan.value_group_size)


def page_codes(pages, slots, oplan, lay, V):
    """Integer codes [B,H,K,V] (pivots: fp16 bits) read from page bytes."""
    H, K = oplan.bits.shape
    tile = min(4 if oplan.kda else 16, V)
    out = np.zeros((len(slots), H, K, V), np.int64)
    for bi, s in enumerate(slots):
        if s <= 0:
            continue
        page = pages[s]
        bitsarr = np.unpackbits(page, bitorder="little")
        for h in range(H):
            stride = lay.offsets[H * K + h]
            for i in range(K):
                w = int(oplan.bits[h, i])
                off = int(lay.offsets[h * K + i])
                j = np.arange(V)
                start = (off + (j // tile) * stride) * 8 + (j % tile) * w
                idx = start[:, None] + np.arange(w)[None, :]
                out[bi, h, i] = (bitsarr[idx] << np.arange(w)[None, :]).sum(-1)
    return out


def scales(pages, slots, oplan, lay, V):
    """(row scales per row (and group), column scales) as float32 from pages."""
    H, K = oplan.bits.shape
    rs, cs = [], []
    for s in slots:
        page = pages[s]
        r = [page[o:o + 2 * (V // oplan.value_group_size if (not oplan.kda and oplan.bits[i // K, 0] == 2) else 1)]
             .view(np.float16).astype(np.float32) if o >= 0 else np.zeros(0, np.float32)
             for i, o in enumerate(lay.rows)]
        c = [page[o:o + 2 * V].view(np.float16).astype(np.float32) if o >= 0 else np.zeros(V, np.float32)
             for o in lay.columns]
        rs.append(r)
        cs.append(np.stack(c))
    return rs, np.stack(cs)


def _ordered_f16(bits):
    """fp16 bit patterns as integers whose difference counts ulps across signs."""
    bits = bits.astype(np.int64)
    mag = bits & 0x7FFF
    return np.where(bits & 0x8000, -mag, mag)


def scale_bytes_index(oplan, lay, V):
    """Byte offsets (within a page) of every stored scale: row scales (a
    GDN 2-bit head stores V/group per row) then column scales, each an fp16."""
    H, K = oplan.bits.shape
    idx = []
    for h in range(H):
        two = (not oplan.kda) and oplan.bits[h, 0] == 2
        n = V // oplan.value_group_size if two else 1
        for i in range(K):
            o = int(lay.rows[h * K + i])
            if o >= 0:
                idx.append(o + 2 * np.arange(n))
    rows = np.concatenate(idx) if idx else np.zeros(0, np.int64)
    cols = [int(o) + 2 * np.arange(V) for o in lay.columns if o >= 0]
    cols = np.concatenate(cols) if cols else np.zeros(0, np.int64)
    return rows, cols


def scale_ulps(got_pages, ref_pages, slots, oplan, lay, V):
    """fp16 ulp distance of the row and column scales of the live slots."""
    live = np.asarray([s for s in slots if s > 0], np.int64)
    out = []
    for idx in scale_bytes_index(oplan, lay, V):
        def read(p):
            lo = p[live][:, idx].astype(np.uint16)
            hi = p[live][:, idx + 1].astype(np.uint16)
            return _ordered_f16(lo | (hi << 8))
        out.append(np.abs(read(got_pages) - read(ref_pages)))
    return out[0], out[1]


def row_scales_full(pages, slots, oplan, lay, V):
    """[B, H, K, V] float32: every value's row scale read from the pages
    (the value-group scale on 2-bit GDN heads; 1 for pivot rows)."""
    H, K = oplan.bits.shape
    out = np.ones((len(slots), H, K, V), np.float32)
    for b, s in enumerate(slots):
        if s <= 0:
            continue
        for h in range(H):
            two = (not oplan.kda) and oplan.bits[h, 0] == 2
            n = V // oplan.value_group_size if two else 1
            for i in range(K):
                o = int(lay.rows[h * K + i])
                if o >= 0:
                    r = pages[s, o:o + 2 * n].view(np.float16).astype(np.float32)
                    out[b, h, i] = np.repeat(r, V // n)
    return out


def _shift_f16(x, k):
    return (x.astype(np.float16).view(np.int16) + k).view(np.float16).astype(np.float32)


def explained_by_initial_scale(got_pages, slots, oplan, lay, V, updated, b, h, j):
    """True when column j of head h (request index b) holds the least-squares
    refit that fit_state gives for the oracle's state with the page's row
    scales and an initial scale c0 one fp16 ulp either side (or at) the
    oracle's c0, within one fp16 ulp."""
    live = np.asarray(slots)[b:b + 1]
    full = row_scales_full(got_pages, live, oplan, lay, V)[:, h:h + 1]
    x = np.asarray(updated, np.float32)[b:b + 1, h:h + 1]
    sub = type(oplan)(oplan.architecture, oplan.bits[h:h + 1], oplan.impact[h:h + 1], oplan.value_group_size)
    c0 = O.initial_column_scales(x, full, sub)
    o = int(lay.columns[h]) + 2 * j
    got = got_pages[live[0], o:o + 2].view(np.int16).astype(np.int64)[0]
    for k in (-1, 0, 1):
        c = O.column_refit(x, full, _shift_f16(c0, k), sub)[0, 0, j]
        if abs(int(np.float16(c).view(np.int16)) - got) <= 1:
            return True
    return False


def check_scales(got_pages, ref_pages, slots, oplan, lay, V, budget, updated=None, c0_budget=0.01,
                 refit_budget=None):
    """Row and column scales equal the oracle's up to one fp16 ulp, and at
    most a ``budget`` fraction of them differ at all.

    With ``updated`` (the oracle's dense state that was requantised), a
    column scale further off is accepted on at most a ``c0_budget`` fraction
    of columns (rounded up), and only where it is the refit of an initial scale c0 one
    fp16 ulp from the oracle's: c0 = fp16(max|x/r|/L) rounds the other way
    when the step's state differs from the oracle's at the float32 ulp
    level, and the least-squares refit of a low-width column follows the
    codes of that c0 by several ulps.  With ``refit_budget`` (states that
    differ from the oracle's by more than float32 rounding, e.g. a chunked
    recurrence against the float64 one), at most that fraction of column
    scales may be further off: one flipped first-pass code moves the refit
    sum Σ z² by up to 2L - 1, which is many fp16 ulps of c when the column
    holds few large codes.  Returns the fractions off by one ulp."""
    rows, cols = scale_ulps(got_pages, ref_pages, slots, oplan, lay, V)
    fr = float((rows > 0).mean()) if rows.size else 0.0
    fc = float((cols > 0).mean()) if cols.size else 0.0
    far = np.argwhere(cols > 1)
    print(f"scales: rows {rows.size} max {rows.max(initial=0)} ulp, {fr:.2e} differ; "
          f"columns {cols.size} max {cols.max(initial=0)} ulp, {fc:.2e} differ, {len(far)} beyond one ulp",
          flush=True)
    assert rows.max(initial=0) <= 1, f"a row scale differs by {rows.max()} fp16 ulps"
    assert fr <= budget, f"{fr:.2e} of row scales differ"
    assert fc <= budget, f"{fc:.2e} of column scales differ"
    if len(far) and refit_budget is not None:
        assert len(far) <= np.ceil(refit_budget * cols.size), \
            f"{len(far)} column scales differ by more than one fp16 ulp (max {cols.max()})"
    elif len(far):
        assert updated is not None, f"a column scale differs by {cols.max()} fp16 ulps"
        live = [bi for bi, s in enumerate(slots) if s > 0]
        heads = [h for h in range(oplan.bits.shape[0]) if lay.columns[h] >= 0]
        for bl, idx in far:
            b, h, j = live[bl], heads[idx // V], idx % V
            assert explained_by_initial_scale(got_pages, slots, oplan, lay, V, updated, b, h, j), \
                f"request {b} head {h} column {j}: scale {cols[bl, idx]} fp16 ulps off, not a c0 rounding"
        assert len(far) <= np.ceil(c0_budget * cols.size), f"{len(far)} column scales differ by more than one fp16 ulp"
    return fr, fc


# row/column scales allowed one fp16 ulp off on at most this fraction
SCALE_BUDGET = 0.02
# prefill pages against the oracle's encoding of the float64 recurrence's
# states: column scales further than one fp16 ulp off on at most this
# fraction (the refit's response to first-pass code flips; measured at P6:
# 0.16%, max 15 ulps)
PREFILL_REFIT_BUDGET = 0.005


def check_requant(got_pages, slots, oplan, lay, V, updated, flip_budget=1e-3, storage="packed", refit_budget=None):
    """Pages requantised on the device against the oracle's encoding of the
    oracle's own state ``updated``: integer codes at most
    one level apart on at most ``flip_budget`` of them, pivots within
    rtol 1e-3, row and column scales per ``check_scales``, and dequantised
    values within rtol 1e-3 / atol 1e-4 except on at most ``flip_budget``.
    ``refit_budget`` is passed to ``check_scales``.
    Byte pages are held to the dequantised-value bar.  Returns the flipped
    fraction of integer codes (of dequantised values for byte pages)."""
    ref = np.zeros_like(got_pages)
    O.encode_page(np.asarray(updated, np.float32), slots, oplan, lay, ref, storage)
    live = np.broadcast_to((np.asarray(slots) > 0)[:, None, None, None], (len(slots),) + oplan.bits.shape + (V,))
    frac = None
    if storage == "packed":
        a = page_codes(got_pages, slots, oplan, lay, V)
        b = page_codes(ref, slots, oplan, lay, V)
        integer = np.broadcast_to(oplan.bits[None, :, :, None] != 16, a.shape)
        m = integer & live
        diff = np.abs(a[m] - b[m])
        assert diff.max(initial=0) <= 1, f"code differs by {diff.max()}"
        frac = float((diff > 0).mean()) if diff.size else 0.0
        print(f"codes: {frac:.2e} of {diff.size} flipped by one level", flush=True)
        assert frac <= flip_budget, f"{frac:.2e} of codes flipped"
        pv = (~integer) & live
        if pv.any():
            pa = a[pv].astype(np.uint16).view(np.float16).astype(np.float32)
            pb = b[pv].astype(np.uint16).view(np.float16).astype(np.float32)
            np.testing.assert_allclose(pa, pb, rtol=1e-3, atol=1e-5)
        check_scales(got_pages, ref, slots, oplan, lay, V, SCALE_BUDGET, updated, refit_budget=refit_budget)
    ga = O.decode_page(got_pages, slots, oplan, lay, V, storage)
    gb = O.decode_page(ref, slots, oplan, lay, V, storage)
    off = ~np.isclose(ga, gb, rtol=1e-3, atol=1e-4)
    print(f"dequantised: {off[live].mean():.2e} beyond rtol 1e-3 / atol 1e-4", flush=True)
    assert off[live].mean() <= flip_budget, f"{off[live].mean():.2e} of dequantised values differ"
    return frac if frac is not None else float(off[live].mean())


def sub_pages(pages, oplan, lay, heads, V):
    """The packed pages restricted to ``heads``: (plan, layout, pages) of a
    pool holding only those heads, each head's code region, row scales and
    column scales copied to their places in the smaller layout."""
    H, K = oplan.bits.shape
    tile = min(4 if oplan.kda else 16, V)
    sub = type(oplan)(oplan.architecture, oplan.bits[heads], oplan.impact[heads], oplan.value_group_size)
    sl = O.layout(sub, V)
    out = np.zeros((pages.shape[0], sl.page_bytes), np.uint8)
    for n, h in enumerate(heads):
        start, stride = int(lay.offsets[h * K]), int(lay.offsets[H * K + h])
        dst, size = int(sl.offsets[n * K]), (V // tile) * stride
        assert int(sl.offsets[len(heads) * K + n]) == stride
        out[:, dst:dst + size] = pages[:, start:start + size]
        two = (not oplan.kda) and oplan.bits[h, 0] == 2
        nr = 2 * (V // oplan.value_group_size if two else 1)
        for i in range(K):
            src, to = int(lay.rows[h * K + i]), int(sl.rows[n * K + i])
            if src >= 0:
                out[:, to:to + nr] = pages[:, src:src + nr]
        if lay.columns[h] >= 0:
            src, to = int(lay.columns[h]), int(sl.columns[n])
            out[:, to:to + 2 * V] = pages[:, src:src + 2 * V]
    return sub, sl, out


def check_prefill(out, ref_out, what="outputs"):
    """Prefill outputs against the float64 recurrence: rtol 1e-3 / atol 1e-4
    for fp32 outputs, rtol 2^-8 / atol 1e-4 for 16-bit ones (one rounding of
    the stored value on top of the kernel's own error)."""
    got = out.float().cpu().numpy() if isinstance(out, torch.Tensor) else np.asarray(out)
    rtol = 1e-3 if (not isinstance(out, torch.Tensor) or out.dtype == torch.float32) else 2 ** -8
    np.testing.assert_allclose(got, ref_out, rtol=rtol, atol=1e-4, err_msg=what)


def check_states(got, ref, what="states"):
    """Prefill states against the float64 recurrence, elementwise:
    rtol 1e-3 / atol 1e-4."""
    np.testing.assert_allclose(np.asarray(got), ref, rtol=1e-3, atol=1e-4, err_msg=what)
