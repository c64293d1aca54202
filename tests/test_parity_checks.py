"""The GPU parity checks themselves, exercised on the CPU: a mistake planted
in oracle-encoded pages must be caught by the scale check the decode-step
tests apply to the HIP pages."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import check_scales, make_plan, scale_bytes_index


def _pages(arch, bits, V=128, B=3):
    oplan = make_plan(arch, bits, seed=4)
    H, K = oplan.bits.shape
    lay = O.layout(oplan, V)
    x = (np.random.default_rng(0).standard_normal((B, H, K, V)) * .1).astype(np.float32)
    pages = np.zeros((B + 1, lay.page_bytes), np.uint8)
    slots = np.arange(1, B + 1)
    O.encode_page(x, slots, oplan, lay, pages)
    return oplan, lay, pages, slots


def _bump(pages, slot, byte, ulps):
    h = int(pages[slot, byte]) | (int(pages[slot, byte + 1]) << 8)
    h += ulps
    pages[slot, byte] = h & 0xFF
    pages[slot, byte + 1] = h >> 8


GDN = np.repeat(np.array([6, 2, 16, 4])[:, None], 128, 1)


def test_identical_pages_pass():
    oplan, lay, pages, slots = _pages("gdn", GDN)
    assert check_scales(pages, pages.copy(), slots, oplan, lay, 128, 0.0) == (0.0, 0.0)


def test_scale_index_covers_every_stored_scale():
    oplan, lay, _, _ = _pages("gdn", GDN)
    rows, cols = scale_bytes_index(oplan, lay, 128)
    # 6-, 4-bit heads: one scale per row; the 2-bit head: V/32 per row; pivot head none
    assert rows.size == 2 * 128 + 128 * 4
    assert cols.size == 3 * 128
    assert len(np.unique(np.concatenate([rows, cols]))) == rows.size + cols.size


@pytest.mark.parametrize("region", ["row", "group", "column"])
def test_two_ulp_scale_is_caught(region):
    oplan, lay, pages, slots = _pages("gdn", GDN)
    bad = pages.copy()
    K = 128
    if region == "row":
        byte = lay.rows[0 * K + 17]              # 6-bit head, row 17
    elif region == "group":
        byte = lay.rows[1 * K + 5] + 2 * 3       # 2-bit head, row 5, value group 3
    else:
        byte = lay.columns[3] + 2 * 100          # 4-bit head, column 100
    _bump(bad, 2, byte, 2)
    with pytest.raises(AssertionError, match="fp16 ulps"):
        check_scales(bad, pages, slots, oplan, lay, 128, 1.0)


def test_one_ulp_beyond_budget_is_caught():
    oplan, lay, pages, slots = _pages("kda", np.random.default_rng(1).choice([4, 6, 8], (2, 128)))
    bad = pages.copy()
    for j in range(0, 128, 4):                    # 32 of 768 column scales one ulp off
        _bump(bad, 1, lay.columns[0] + 2 * j, 1)
    check_scales(bad, pages, slots, oplan, lay, 128, 0.05)
    with pytest.raises(AssertionError, match="column scales differ"):
        check_scales(bad, pages, slots, oplan, lay, 128, 0.01)


def _state_pages(bits, seed=0):
    oplan = make_plan("gdn", bits, seed=4)
    H, K = oplan.bits.shape
    V, B = 128, 2
    lay = O.layout(oplan, V)
    x = (np.random.default_rng(seed).standard_normal((B, H, K, V)) * .1).astype(np.float32)
    pages = np.zeros((B + 1, lay.page_bytes), np.uint8)
    slots = np.arange(1, B + 1)
    O.encode_page(x, slots, oplan, lay, pages)
    return oplan, lay, pages, slots, x


def _far_column(oplan, lay, pages, slots, x, h):
    """(column, refit bits) of a column whose refit moves >1 ulp when c0 is one ulp up."""
    from tests.helpers import row_scales_full
    full = row_scales_full(pages, slots[:1], oplan, lay, 128)
    c0 = O.initial_column_scales(x[:1], full, oplan)
    up = (c0.astype(np.float16).view(np.int16) + 1).view(np.float16).astype(np.float32)
    a = O.column_refit(x[:1], full, c0, oplan).astype(np.float16).view(np.int16)
    b = O.column_refit(x[:1], full, up, oplan).astype(np.float16).view(np.int16)
    far = np.argwhere(np.abs(a[0, h].astype(int) - b[0, h].astype(int)) > 1)
    assert far.size, "some column's refit follows a one-ulp c0 by several ulps"
    j = int(far[0, 0])
    return j, int(b[0, h, j])


def test_far_column_scale_from_a_c0_rounding_is_accepted():
    oplan, lay, pages, slots, x = _state_pages(np.full((2, 128), 4))
    j, refit = _far_column(oplan, lay, pages, slots, x, 1)
    got = pages.copy()
    o = lay.columns[1] + 2 * j
    got[1, o:o + 2] = np.array([refit], np.int16).view(np.uint8)
    check_scales(got, pages, slots, oplan, lay, 128, 1.0, updated=x)
    with pytest.raises(AssertionError, match="fp16 ulps"):
        check_scales(got, pages, slots, oplan, lay, 128, 1.0)   # without the state: not explained


def test_far_column_scale_without_explanation_is_caught():
    oplan, lay, pages, slots, x = _state_pages(np.full((2, 128), 4))
    j, refit = _far_column(oplan, lay, pages, slots, x, 1)
    got = pages.copy()
    o = lay.columns[1] + 2 * j
    cur = int(pages[1, o:o + 2].view(np.int16)[0])
    wrong = cur - (refit - cur)                    # as far off, on the other side
    got[1, o:o + 2] = np.array([wrong], np.int16).view(np.uint8)
    with pytest.raises(AssertionError, match="not a c0 rounding"):
        check_scales(got, pages, slots, oplan, lay, 128, 1.0, updated=x)


@pytest.mark.parametrize("arch,bits", [("gdn", GDN), ("kda", None)])
def test_sub_pages_equal_the_encoding_of_those_heads(arch, bits):
    """sub_pages (the P6 parity check's head selection) gives exactly the
    pages a pool of only those heads holds for the same states."""
    from tests.helpers import sub_pages
    if bits is None:
        bits = np.where(np.random.default_rng(2).random((4, 128)) < .03, 16,
                        np.random.default_rng(3).choice([2, 4, 6, 8], (4, 128)))
    oplan = make_plan(arch, bits, seed=4)
    H, K, V, B = 4, 128, 128, 3
    lay = O.layout(oplan, V)
    x = (np.random.default_rng(0).standard_normal((B, H, K, V)) * .1).astype(np.float32)
    pages = np.zeros((B + 1, lay.page_bytes), np.uint8)
    slots = np.arange(1, B + 1)
    O.encode_page(x, slots, oplan, lay, pages)
    heads = [3, 1]
    sub, sl, got = sub_pages(pages, oplan, lay, heads, V)
    want = np.zeros_like(got)
    O.encode_page(x[:, heads], slots, sub, sl, want)
    assert np.array_equal(got, want)


def test_requant_check_catches_a_planted_code_flip_rate():
    """check_requant passes the oracle's own pages and fails when more than
    the budget of codes sit one level off (planted in the oracle's state)."""
    from tests.helpers import check_requant
    oplan, lay, pages, slots = _pages("gdn", np.full((4, 128), 8))
    x = (np.random.default_rng(0).standard_normal((3, 4, 128, 128)) * .1).astype(np.float32)  # as _pages
    assert check_requant(pages, slots, oplan, lay, 128, x) == 0.0
    # move 1% of the values by about one level: their codes flip
    rng = np.random.default_rng(1)
    step = np.abs(x).max(axis=2, keepdims=True) / 127
    moved = x + (rng.random(x.shape) < .01) * step * 1.01
    with pytest.raises(AssertionError, match="code|dequantised"):
        check_requant(pages, slots, oplan, lay, 128, moved)


def test_refit_budget_bounds_far_column_scales():
    """The prefill bar: column scales further than one ulp off are allowed on
    at most refit_budget of the columns, and no more."""
    oplan, lay, pages, slots = _pages("gdn", np.full((4, 128), 4))
    bad = pages.copy()
    for j in (3, 50, 99):                        # 3 of 1,536 column scales 5 ulps off
        _bump(bad, 2, lay.columns[1] + 2 * j, 5)
    check_scales(bad, pages, slots, oplan, lay, 128, 0.01, refit_budget=0.002)
    with pytest.raises(AssertionError, match="more than one fp16 ulp"):
        check_scales(bad, pages, slots, oplan, lay, 128, 0.01, refit_budget=0.001)
