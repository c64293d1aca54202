"""The CPU oracle against golden vectors written from the reference.

tests/golden/fit_state_vectors.npz holds inputs and outputs of the
reference's fit_state (stepquant/quantization.py:54-98) and StateCodec.encode
(quantization.py:109-126), produced by tests/golden/make_golden.py.
"""
import hashlib

import numpy as np
import pytest

from oracle import oracle as O


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _plan(data, meta, name):
    m = meta["cases"][name]
    return O.Plan(m["arch"], data[f"{name}/bits"], data[f"{name}/impact"], m["group"])


def test_golden_metadata(golden):
    data, meta = golden
    assert len(meta["cases"]) >= 14
    assert meta["cpu_capability"]  # recorded with the vectors


@pytest.mark.parametrize("name", [
    "c_config_gdn", "c_config_gdn_uniform6", "gdn_two_bit_g32", "gdn_mixed_v16_g4", "kda_mixed_v16",
    "kda_mixed_128", "kda_edges_v4", "kda_edges_v32", "gdn_v8_k4", "gdn_v32_k32", "zero_state",
    "scale_extremes", "kda_pivot_a", "kda_pivot_b"])
def test_fit_state_bit_exact(golden, name):
    data, meta = golden
    plan = _plan(data, meta, name)
    x = data[f"{name}/x"]
    z, r, c, r2, recon = O.fit_state(x, plan)
    np.testing.assert_array_equal(z.astype(np.int8), data[f"{name}/z"])
    np.testing.assert_array_equal(r.view(np.uint16), data[f"{name}/r"])
    np.testing.assert_array_equal(c.view(np.uint16), data[f"{name}/c"])
    if f"{name}/r2" in data:
        np.testing.assert_array_equal(r2.view(np.uint16), data[f"{name}/r2"])
    else:
        assert r2 is None
    assert _sha(recon) == meta["cases"][name]["recon_sha256"]
    if f"{name}/recon" in data:
        np.testing.assert_array_equal(recon, data[f"{name}/recon"])


@pytest.mark.parametrize("name", ["c_config_gdn", "gdn_two_bit_g32", "gdn_mixed_v16_g4", "kda_mixed_v16",
                                  "kda_mixed_128", "kda_edges_v4", "scale_extremes"])
def test_codec_streams_bit_exact(golden, name):
    data, meta = golden
    m = meta["cases"][name]
    enc = O.codec_encode(data[f"{name}/x"], _plan(data, meta, name))
    for b in (2, 4, 6, 8):
        assert _sha(enc["codes"][b]) == m["codec_sha256"][str(b)], b
        if f"{name}/codec{b}" in data:
            np.testing.assert_array_equal(enc["codes"][b], data[f"{name}/codec{b}"])
    assert _sha(enc["pivots"].view(np.uint16)) == m["codec_pivots_sha256"]
    assert _sha(enc["rows"].view(np.uint16)) == m["codec_rows_sha256"]
    assert _sha(enc["columns"].view(np.uint16)) == m["codec_columns_sha256"]


def test_kda_pivots_do_not_move_shared_columns(golden):
    """Reference invariant (tests/test_core.py:97-106), seen in the vectors."""
    data, _ = golden
    for key in ("c", "z"):
        a, b = data[f"kda_pivot_a/{key}"], data[f"kda_pivot_b/{key}"]
        if key == "z":
            a, b = a[:, :, :4], b[:, :, :4]
        np.testing.assert_array_equal(a, b)


def test_zero_state_decodes_to_zero(golden):
    data, meta = golden
    _, _, _, _, recon = O.fit_state(data["zero_state/x"], _plan(data, meta, "zero_state"))
    assert np.isfinite(recon).all() and np.abs(recon).max() < 1e-10


@pytest.mark.parametrize("name", ["c_config_gdn", "gdn_two_bit_g32", "gdn_mixed_v16_g4", "kda_mixed_v16",
                                  "kda_mixed_128", "kda_edges_v4", "kda_edges_v32", "gdn_v8_k4",
                                  "scale_extremes"])
@pytest.mark.parametrize("storage", ["packed", "byte"])
def test_page_round_trip_equals_reconstruction(golden, name, storage):
    """decode(encode(x)) through the pool page equals fit_state's reconstruction."""
    data, meta = golden
    plan = _plan(data, meta, name)
    x = data[f"{name}/x"]
    B, H, K, V = x.shape
    lay = O.layout(plan, V, storage)
    pages = np.zeros((B + 2, lay.page_bytes), np.uint8)
    slots = np.arange(B, 0, -1)
    O.encode_page(x, slots, plan, lay, pages, storage)
    assert not pages[0].any() and not pages[B + 1].any()
    out = O.decode_page(pages, slots, plan, lay, V, storage)
    # The page stores integer codes, so a -0.0 reconstruction decodes as +0.0.
    _, _, _, _, recon = O.fit_state(x, plan)
    assert _sha(recon) == meta["cases"][name]["recon_sha256"]
    np.testing.assert_array_equal(out, recon)
    assert _sha(out + np.float32(0)) == _sha(recon + np.float32(0))
    masked = O.decode_page(pages, np.zeros(2, np.int64), plan, lay, V, storage)
    assert not masked.any()


def _row_scales_full(plan, r, r2, V):
    """[B, H, K, V] float32 row scale of every value (group scales on 2-bit GDN heads)."""
    r = r.view(np.float16).astype(np.float32)
    full = np.repeat(r[..., None], V, axis=-1)
    two = (plan.bits[:, 0] == 2) & (not plan.kda)
    if two.any():
        g = plan.value_group_size
        full[:, two] = np.repeat(r2.view(np.float16).astype(np.float32), g, axis=-1)
    return full


@pytest.mark.parametrize("name", [
    "c_config_gdn", "c_config_gdn_uniform6", "gdn_two_bit_g32", "gdn_mixed_v16_g4", "kda_mixed_v16",
    "kda_mixed_128", "kda_edges_v4", "kda_edges_v32", "gdn_v8_k4", "gdn_v32_k32", "zero_state",
    "scale_extremes", "kda_pivot_a", "kda_pivot_b"])
def test_column_refit_against_golden(golden, name):
    """initial_column_scales + column_refit from the reference's own row
    scales give the reference's column scales (fit_state's c) within one
    fp16 ulp; all but a few exactly (the key sums run in another order)."""
    data, meta = golden
    plan = _plan(data, meta, name)
    x = data[f"{name}/x"]
    V = x.shape[-1]
    r2 = data[f"{name}/r2"] if f"{name}/r2" in data else None
    full = _row_scales_full(plan, data[f"{name}/r"], r2, V)
    c0 = O.initial_column_scales(x, full, plan)
    c = O.column_refit(x, full, c0, plan)
    ref = data[f"{name}/c"].view(np.float16).astype(np.float32)
    integer_heads = (plan.bits != 16).any(1)
    got_bits = c.astype(np.float16).view(np.int16).astype(np.int64)[:, integer_heads]
    ref_bits = ref.astype(np.float16).view(np.int16).astype(np.int64)[:, integer_heads]
    ulps = np.abs(got_bits - ref_bits)
    assert ulps.max(initial=0) <= 1
    assert (ulps > 0).mean() <= 0.01 if ulps.size else True


def test_column_refit_moves_with_initial_scale(golden):
    """A one-ulp change of c0 moves the least-squares refit of low-width
    columns by several fp16 ulps: the encode(c0) codes change by one level
    on values near a rounding boundary and the refit follows them.  A GPU
    step whose c0 rounds the other way (its state differs from the oracle's
    at the float32 ulp level) therefore yields such a column scale."""
    data, meta = golden
    name = "c_config_gdn"
    plan = _plan(data, meta, name)
    x = data[f"{name}/x"]
    full = _row_scales_full(plan, data[f"{name}/r"], None, x.shape[-1])
    c0 = O.initial_column_scales(x, full, plan)
    up = (c0.astype(np.float16).view(np.int16) + 1).view(np.float16).astype(np.float32)
    a = O.column_refit(x, full, c0, plan).astype(np.float16).view(np.int16).astype(np.int64)
    b = O.column_refit(x, full, up, plan).astype(np.float16).view(np.int16).astype(np.int64)
    assert np.abs(a - b).max() >= 3
