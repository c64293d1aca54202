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
