"""The baseline-format oracle (fp32, sym_int*_g128, dsq_int*) on the CPU.

Pins, without the reference's code:
* format_layout by the closed-form sizes of its regions (format_pool.py:9-25)
  and equality with the product's own layout function;
* group_fit by brute force: each scale recomputed in float64 (division is
  exact after one rounding to float32), each code the half-even rounding of
  the float64 quotient, clamped; reconstruction error at most s/2;
* dual_fit's row mean through ``inner_sum`` (PyTorch's CPU summation order,
  pinned by the fit_state golden vectors), its column scales and codes by
  the same brute force;
* page encode/decode round trips and the little-endian code stream of
  packing.py (test_core.py:36-43 pins ``pack``/``unpack``).
"""
import numpy as np
import pytest

from oracle import oracle as O

NAMES = ["fp32", "sym_int4_g128", "sym_int6_g128", "sym_int8_g128", "dsq_int4", "dsq_int6"]


def _bits(name, H, K):
    return np.full((H, K), O.format_spec(name)[1], np.int32)


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("H,K,V", [(2, 32, 128), (4, 128, 128), (1, 8, 256)])
def test_layout_closed_form(name, H, K, V):
    kind, b, group = O.format_spec(name)
    if kind == "dsq" and V > 128:
        V = 128
    lay = O.format_layout(_bits(name, H, K), V, kind, group)
    rows = H * K
    code = rows * V * b // 8
    assert np.array_equal(lay.offsets, np.arange(rows) * (V * b // 8))
    meta = {"fp32": 0, "symmetric": 4 * (V // group), "dsq": 2}[kind] * rows
    cols = 4 * V * H if kind == "dsq" else 0
    assert lay.page_bytes == -(-(-(-code // 4) * 4 + meta) // 4) * 4 + cols
    if kind == "fp32":
        assert (lay.rows == -1).all() and lay.page_bytes == rows * V * 4
    else:
        assert np.array_equal(lay.rows, -(-code // 4) * 4 + np.arange(rows) * (meta // rows))
    assert lay.page_bytes % 4 == 0


@pytest.mark.parametrize("name", NAMES)
def test_product_layout_matches_oracle(name):
    import torch
    from stepquant_amd.formats import FormatPlan, get_format
    from stepquant_amd.kernels.format_pool import format_layout
    spec = get_format(name)
    bits = _bits(name, 3, 32)
    plan = FormatPlan("gdn", torch.from_numpy(bits.astype(np.int64)), torch.ones(3, 32))
    off, rows, cols, total = format_layout(plan, 128, spec)
    lay = O.format_layout(bits, 128, spec.kind, spec.group_size)
    assert total == lay.page_bytes
    assert off == lay.offsets.tolist() and rows == lay.rows.tolist() and cols == lay.columns.tolist()


def _round_half_even(v):
    return np.vectorize(lambda t: float(round(t)))(v)


@pytest.mark.parametrize("bits", [4, 6, 8])
def test_group_fit_brute_force(bits):
    rng = np.random.default_rng(bits)
    x = (rng.standard_normal((2, 3, 8, 256)) * np.exp(rng.normal(0, 2, (2, 3, 8, 1)))).astype(np.float32)
    L = 2 ** (bits - 1) - 1
    s_grid = rng.integers(1, 40, (2, 3, 8, 2, 1)).astype(np.float32) * np.float32(2.0 ** -6)
    # plant exact ties (k + 1/2) s into some groups
    x[0, 0, 0, :128] = ((rng.integers(-L, L, 128) + .5) * s_grid[0, 0, 0, 0, 0]).astype(np.float32)
    x[0, 0, 0, 0] = L * s_grid[0, 0, 0, 0, 0]  # fixes that group's scale to s_grid
    codes, s, z, recon = O.group_fit(x, bits)
    g = x.reshape(2, 3, 8, 2, 128).astype(np.float64)
    amax = np.abs(g).max(-1)
    s_ref = np.clip((amax / L).astype(np.float32), 2.0 ** -24, 65504).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(z, np.full_like(s_ref, L))
    quot = (g / s_ref[..., None].astype(np.float64)).astype(np.float32)
    q = np.clip(_round_half_even(quot), -L, L)
    np.testing.assert_array_equal(codes.reshape(q.shape), q + L)
    # ties go to even levels
    assert s[0, 0, 0, 0] == s_grid[0, 0, 0, 0, 0]
    tie_codes = codes[0, 0, 0, 1:128] - L
    assert (np.abs(tie_codes) % 2 == 0).all()
    np.testing.assert_array_equal(recon.reshape(q.shape), (q * s_ref[..., None]).astype(np.float32))
    err = np.abs(recon.reshape(g.shape) - g)
    assert (err <= s_ref[..., None] / 2 * (1 + 1e-6)).all()


@pytest.mark.parametrize("bits", [4, 6])
def test_dual_fit_brute_force(bits):
    rng = np.random.default_rng(10 + bits)
    B, H, K, V = 2, 2, 32, 128
    x = (np.exp(rng.normal(0, .5, (B, H, K, 1))) * rng.standard_normal((B, H, K, V)) *
         np.exp(rng.normal(0, .5, (B, H, 1, V)))).astype(np.float32)
    x[1, 1, 3] = 0.0  # an all-zero row: r clamps to 2^-24, its codes sit at L
    L = 2 ** (bits - 1) - 1
    codes, r, c, recon = O.dual_fit(x, bits)
    mean = np.array([O.inner_sum(np.abs(row)) for row in x.reshape(-1, V)], np.float32).reshape(B, H, K) / np.float32(V)
    # the mean is a float32 sum in PyTorch's order: within a few ulps of the exact mean
    exact = np.abs(x.astype(np.float64)).mean(-1)
    assert (np.abs(mean - exact) <= 4e-7 * exact + 1e-30).all()
    r_ref = np.clip(np.sqrt(np.maximum(mean.astype(np.float64), 1e-20)).astype(np.float32), 2.0 ** -24,
                    65504).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(r, r_ref)
    y = (x.astype(np.float64) / r_ref[..., None]).astype(np.float32)
    c_ref = np.clip((np.abs(y).astype(np.float64).max(-2) / L).astype(np.float32), 2.0 ** -24,
                    65504).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(c, c_ref)
    q = np.clip(_round_half_even((y.astype(np.float64) / c_ref[:, :, None, :]).astype(np.float32)), -L, L)
    np.testing.assert_array_equal(codes, q + L)
    assert (codes[1, 1, 3] == L).all()
    np.testing.assert_array_equal(recon, ((r_ref[..., None] * c_ref[:, :, None, :]) * q).astype(np.float32))
    # every column reaches the top level (|q| = L) in its largest row
    assert (np.abs(q).max(-2) == L).all()


@pytest.mark.parametrize("name", NAMES)
def test_page_round_trip_and_code_stream(name):
    kind, b, group = O.format_spec(name)
    rng = np.random.default_rng(3)
    H, K, V = 2, 16, 128
    x = (rng.standard_normal((3, H, K, V)) * .3).astype(np.float32)
    lay = O.format_layout(_bits(name, H, K), V, kind, group)
    data = np.zeros((5, lay.page_bytes), np.uint8)
    slots = np.array([4, 0, 2])
    O.format_encode_page(x, slots, name, lay, data)
    assert not data[[0, 1, 3]].any(), "masked and unused slots stay empty"
    dec = O.format_decode_page(data, slots, name, lay, H, K, V)
    assert not dec[1].any()
    if kind == "fp32":
        np.testing.assert_array_equal(dec[[0, 2]], x[[0, 2]])
        return
    fit = O.group_fit(x, b, group) if kind == "symmetric" else O.dual_fit(x, b)
    np.testing.assert_array_equal(dec[[0, 2]], fit[-1][[0, 2]])
    # the first codes of head 1, row 5 of slot 4 as a little-endian bit stream
    codes = fit[0][0, 1, 5].astype(np.int64)
    off = int(lay.offsets[1 * K + 5])
    word = int.from_bytes(bytes(data[4, off:off + b // 2]), "little")
    assert [(word >> (j * b)) & ((1 << b) - 1) for j in range(4)] == codes[:4].tolist()
