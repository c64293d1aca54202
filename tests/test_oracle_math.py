"""Pins the oracle functions that the golden vectors do not cover.

* torch summation trees (restated from aten SumKernel.cpp) against torch;
* packed_layout against the reference's known-answer tests;
* delta_step against its closed form and the reference's error-propagation
  invariant (tests/test_core.py:11-27 of the reference);
* input preparation against a float64 formula;
* pack/unpack against hand-computed little-endian bytes and round trips.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O


@pytest.mark.parametrize("n", [4, 8, 16, 32, 64, 128, 256, 512])
def test_inner_sum_tree_matches_torch(n):
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(400, n, generator=g) * torch.rand(400, 1, generator=g) * 5).abs()
    expected = x.sum(-1).numpy()
    got = np.array([O.inner_sum(row) for row in x.numpy()])
    np.testing.assert_array_equal(got, expected)


@pytest.mark.parametrize("k,v", [(4, 4), (8, 8), (16, 16), (32, 8), (128, 16), (128, 32),
                                 (128, 128), (256, 64), (64, 256)])
def test_outer_sum_tree_matches_torch(k, v):
    g = torch.Generator().manual_seed(k * 1000 + v)
    x = torch.randn(3, k, v, generator=g) * torch.rand(3, k, 1, generator=g) * 3
    expected = x.sum(-2).numpy()
    got = np.stack([O.outer_sum(m) for m in x.numpy()])
    np.testing.assert_array_equal(got, expected)


def test_tree_differs_from_naive_order():
    # A plausible mistake (sequential order) must fail the tree test above.
    g = torch.Generator().manual_seed(5)
    x = torch.randn(200, 128, generator=g).abs()
    seq = np.array([np.float32(sum(np.float32(t) for t in row)) for row in x.numpy()])
    assert (seq != x.sum(-1).numpy()).any()


def test_half_rounding_matches_torch():
    g = torch.Generator().manual_seed(3)
    x = torch.cat([torch.randn(3000, generator=g) * 10 ** torch.randint(-9, 5, (3000,), generator=g),
                   torch.tensor([65504., 65519.99, 65520., 2. ** -24, 2. ** -25, 3 * 2. ** -26, 1e-30, 0.,
                                 -0., 1 + 2. ** -11, 1 + 3 * 2. ** -11])])
    got = O.f32_to_f16_bits(x.numpy())
    np.testing.assert_array_equal(got, x.half().numpy().view(np.uint16))


# ------------------------------------------------------------- layout KATs

def test_byte_layout_known_answer():
    """Reference tests/test_byte_layout.py:9-20."""
    bits = np.array([[2, 4, 6, 16], [16, 16, 16, 16]])
    plan = O.Plan("kda", bits, np.ones((2, 4)))
    lay = O.layout(plan, 32, "byte")
    payload = 4 * 32 + 5 * 32 * 2
    assert list(lay.offsets[8:]) == [0, 192]
    assert lay.offsets[3] == 128
    assert list(lay.columns) == [payload + 3 * 2, -1]
    assert list(lay.rows) == [payload, payload + 2, payload + 4, -1, -1, -1, -1, -1]
    assert lay.page_bytes == (payload + 3 * 2 + 32 * 2 + 15) // 16 * 16
    assert lay.page_bytes > O.layout(plan, 32, "packed").page_bytes


@pytest.mark.parametrize("arch", ["gdn", "kda"])
def test_six_bit_payload_has_no_padding(arch):
    """Reference tests/test_stepquant6.py:42-53."""
    H, K, V = 2, 128, 128
    plan = O.Plan(arch, np.full((H, K), 6), np.ones((H, K)))
    meta = 2 * H * (K + V)
    assert O.layout(plan, V).page_bytes - meta == H * K * V * 6 // 8
    assert O.layout(plan, V, "byte").page_bytes - meta == H * K * V


def test_headline_page_size():
    plan = O.Plan("gdn", np.full((32, 128), 6), np.ones((32, 128)))
    assert O.layout(plan, 128).page_bytes == 409600


@pytest.mark.parametrize("v", [4, 32])
def test_kda_half_aligned_pages(v):
    """Reference tests/test_kernel_edges.py:16."""
    plan = O.Plan("kda", np.array([[2, 4, 8, 16]]), np.ones((1, 4)))
    assert O.layout(plan, v).page_bytes % 4 == 2


@pytest.mark.parametrize("v", [8, 16, 32])
def test_gdn_word_aligned_pages(v):
    """Reference tests/test_kernel_edges.py:42."""
    plan = O.Plan("gdn", np.repeat(np.array([2, 4, 6, 8, 16])[:, None], 4, 1), np.ones((5, 4)), min(v, 32))
    assert O.layout(plan, v).page_bytes % 4 == 0


def test_packed_layout_address_formula():
    """Row offsets follow cursor + local with even pivot alignment; tile-major blocks."""
    bits = np.array([[4, 6, 16, 2, 8, 16, 6, 6]])
    plan = O.Plan("kda", bits, np.ones((1, 8)))
    lay = O.layout(plan, 8)
    local, expect = 0, []
    for b in bits[0]:
        if b == 16:
            local = (local + 1) // 2 * 2
        expect.append(local)
        local += 4 * b // 8
    stride = (local + 1) // 2 * 2
    assert list(lay.offsets[:8]) == expect and lay.offsets[8] == stride
    assert lay.rows[0] == stride * 2 and lay.rows[2] == -1


# --------------------------------------------------------- delta_step math

def _prepared(B, H, K, V, kda, seed):
    g = np.random.default_rng(seed)
    S = g.standard_normal((B, H, K, V)).astype(np.float32) * 0.1
    q = g.standard_normal((B, H, K)).astype(np.float32)
    k = g.standard_normal((B, H, K)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = g.standard_normal((B, H, V)).astype(np.float32)
    ld = -g.random((B, H, K) if kda else (B, H)).astype(np.float32)
    beta = g.random((B, H)).astype(np.float32)
    return S, q, k, v, ld, beta


@pytest.mark.parametrize("kda", [False, True])
def test_delta_step_closed_form(kda):
    S, q, k, v, ld, beta = _prepared(2, 3, 16, 8, kda, 1)
    out, upd = O.delta_step(S, q, k, v, ld, beta)
    d = np.exp(ld.astype(np.float64))
    d = d[..., None] if kda else d[..., None, None]
    ret = S.astype(np.float64) * (d if kda else d)
    if kda:
        ret = S.astype(np.float64) * np.exp(ld.astype(np.float64))[..., None]
    resid = v - np.einsum("bhk,bhkv->bhv", k.astype(np.float64), ret)
    ref_upd = ret + k[..., None] * (beta[..., None] * resid)[..., None, :]
    ref_out = np.einsum("bhk,bhkv->bhv", q.astype(np.float64), ref_upd)
    np.testing.assert_allclose(upd, ref_upd, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out, ref_out, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("kda", [False, True])
def test_delta_step_error_propagation(kda):
    """Reference tests/test_core.py:11-27: S'(S+e) - S'(S) = A e, A = (I - beta k k^T) D."""
    S, q, k, v, ld, beta = _prepared(2, 3, 7, 5, kda, 2)
    e = (np.random.default_rng(9).standard_normal(S.shape) * .01).astype(np.float32)
    y, s = O.delta_step(S, q, k, v, ld, beta)
    yh, sh = O.delta_step(S + e, q, k, v, ld, beta)
    d = np.exp(ld)[..., None] if kda else np.exp(ld)[..., None, None] * np.ones((1, 1, 7, 1))
    A = (np.eye(7) - beta[..., None, None] * k[..., :, None] * k[..., None, :]) * np.swapaxes(d, -1, -2)
    np.testing.assert_allclose(sh - s, A @ e, atol=1e-6, rtol=1e-4)
    transported = (np.swapaxes(A, -1, -2) @ q[..., None])[..., 0]
    np.testing.assert_allclose(yh - y, (np.swapaxes(e, -1, -2) @ transported[..., None])[..., 0],
                               atol=1e-6, rtol=1e-4)


def test_delta_step_sequential_brute_force():
    """Tiny case written as explicit scalar loops in float64."""
    S, q, k, v, ld, beta = _prepared(1, 1, 3, 2, False, 4)
    out, upd = O.delta_step(S, q, k, v, ld, beta)
    d = np.exp(np.float64(ld[0, 0]))
    R = [[float(S[0, 0, i, j]) * d for j in range(2)] for i in range(3)]
    for j in range(2):
        res = float(v[0, 0, j]) - sum(float(k[0, 0, i]) * R[i][j] for i in range(3))
        for i in range(3):
            R[i][j] += float(k[0, 0, i]) * float(beta[0, 0]) * res
        o = sum(float(q[0, 0, i]) * R[i][j] for i in range(3))
        assert abs(o - out[0, 0, j]) < 1e-5
    np.testing.assert_allclose(upd[0, 0], np.array(R), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kda", [False, True])
def test_prepare_raw_gates_and_gqa(kda):
    g = np.random.default_rng(3)
    B, H, HK, K = 3, 4, 2, 8
    q = g.standard_normal((B, HK * K)).astype(np.float32)
    k = g.standard_normal((B, HK * K)).astype(np.float32)
    a = g.standard_normal((B, H, K) if kda else (B, H)).astype(np.float32) * 10
    bias = g.standard_normal(H * K if kda else H).astype(np.float32)
    a_log = g.standard_normal(H).astype(np.float32)
    b = g.standard_normal((B, H)).astype(np.float32)
    qp, kp, ld, bo = O.prepare(q, k, a, b, H, K, kda, normalize=True, scale=K ** -.5, a_log=a_log,
                               dt_bias=bias)
    q64 = q.reshape(B, HK, K).astype(np.float64)
    k64 = k.reshape(B, HK, K).astype(np.float64)
    qn = q64 / np.sqrt((q64 ** 2).sum(-1, keepdims=True) + 1e-6) * K ** -.5
    kn = k64 / np.sqrt((k64 ** 2).sum(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(qp, np.repeat(qn, H // HK, 1), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(kp, np.repeat(kn, H // HK, 1), rtol=1e-5, atol=1e-6)
    u = a.astype(np.float64) + (bias.reshape(H, K) if kda else bias)
    sp = np.where(u > 20, u, np.log1p(np.exp(np.minimum(u, 20))))
    expect = -np.exp(a_log.astype(np.float64))[:, None] * sp if kda else -np.exp(a_log) * sp
    np.testing.assert_allclose(ld, expect, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(bo, 1 / (1 + np.exp(-b.astype(np.float64))), rtol=1e-6)


# --------------------------------------------------------------- packing

def test_pack_known_answers():
    assert list(O.pack(np.array([1, 2, 3, 0]), 2)) == [1 | 2 << 2 | 3 << 4]
    assert list(O.pack(np.array([0xA, 0x5]), 4)) == [0x5A]
    # 6-bit: four codes in three little-endian bytes
    c = np.array([0x3F, 0x01, 0x2A, 0x15])
    word = 0x3F | 0x01 << 6 | 0x2A << 12 | 0x15 << 18
    assert list(O.pack(c, 6)) == [word & 255, word >> 8 & 255, word >> 16 & 255]


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
@pytest.mark.parametrize("n", [0, 1, 7, 128, 513])
def test_pack_round_trip(bits, n):
    """Reference tests/test_core.py:36-43."""
    x = np.random.default_rng(n).integers(0, 2 ** bits, n)
    p = O.pack(x, bits)
    assert p.dtype == np.uint8
    np.testing.assert_array_equal(O.unpack(p, bits, n), x)
    assert p.size <= (n * bits + 7) // 8 + 2
