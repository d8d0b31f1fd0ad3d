"""The logits producer's checker (oracle/head_oracle.c) pinned on the CPU:
against the reference's own rmsnorm_f32 / matvec_f32_f32 / matvec_bf16_f32
compiled from its sources (oracle/_ref/libref_kernels.so, bit for bit), the
reference's known-answer cases (tests/unit/test_rmsnorm.cpp:22-36,
test_matvec.cpp:22-33), and float64 arithmetic (a transposed operand, a lost
term or a wrong scale fails these)."""
import numpy as np
import pytest

import oracle as O

needs_ref = pytest.mark.skipif(not O.ref_kernels_available(), reason="reference kernels not built")


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def test_rmsnorm_known_case():
    # reference tests/unit/test_rmsnorm.cpp:22-36: x = [1, 2, 3, 4], scale 1, eps 0
    y = O.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 0.0)
    rms = np.sqrt(np.float32(7.5))
    np.testing.assert_allclose(y, np.array([1, 2, 3, 4], np.float32) / rms, rtol=1e-5)


def test_matvec_identity_returns_input():
    # reference tests/unit/test_matvec.cpp:22-33
    x = np.arange(1, 9, dtype=np.float32)
    np.testing.assert_array_equal(O.matvec(np.eye(8, dtype=np.float32), x), x)
    np.testing.assert_array_equal(O.matvec(bf16_bits(np.eye(8, dtype=np.float32)), x), x)


@pytest.mark.parametrize("n", [1, 7, 8, 9, 131, 896, 4096, 5120])
def test_rmsnorm_close_to_float64(n):
    rng = np.random.default_rng(n)
    x = rng.uniform(-1.5, 1.5, n).astype(np.float32)
    s = rng.uniform(-1.5, 1.5, n).astype(np.float32)
    eps = 1e-6
    y = O.rmsnorm(x, s, eps)
    xd = x.astype(np.float64)
    want = xd * s / np.sqrt(np.mean(xd * xd) + eps)
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("M,K", [(37, 131), (16, 64), (5, 7), (64, 896), (40, 4096)])
def test_matvec_close_to_float64(M, K):
    rng = np.random.default_rng(M * K)
    w = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    x = rng.uniform(-1, 1, K).astype(np.float32)
    want = w.astype(np.float64) @ x.astype(np.float64)
    bound = 4 * K * np.finfo(np.float32).eps * (np.abs(w).astype(np.float64) @ np.abs(x).astype(np.float64))
    assert np.all(np.abs(O.matvec(w, x) - want) <= bound)
    wb = bf16_bits(w)
    want_b = bf16_to_f32(wb).astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(O.matvec(wb, x) - want_b) <= bound)


@needs_ref
@pytest.mark.parametrize("n", [1, 2, 4, 5, 6, 7, 8, 9, 10, 13, 14, 131, 134, 896, 2048, 4096, 4102])
def test_rmsnorm_matches_reference_bits(n):
    rng = np.random.default_rng(100 + n)
    for eps in (0.0, 1e-6, 1e-5):
        x = rng.normal(0, 3, n).astype(np.float32)
        s = rng.normal(1, 0.3, n).astype(np.float32)
        np.testing.assert_array_equal(O.rmsnorm(x, s, eps), O.rmsnorm(x, s, eps, use_ref=True))


@needs_ref
@pytest.mark.parametrize("M,K", [(37, 131), (16, 64), (5, 7), (3, 1), (4, 2), (4, 5), (4, 6), (7, 130), (7, 133),
                                 (7, 134), (64, 896), (48, 4096), (9, 4103)])
def test_matvec_matches_reference_bits(M, K):
    rng = np.random.default_rng(M + 7 * K)
    w = rng.normal(0, 0.05, (M, K)).astype(np.float32)
    x = rng.normal(0, 1, K).astype(np.float32)
    np.testing.assert_array_equal(O.matvec(w, x), O.matvec(w, x, use_ref=True))
    wb = bf16_bits(w)
    np.testing.assert_array_equal(O.matvec(wb, x), O.matvec(wb, x, use_ref=True))


@needs_ref
def test_evaluation_order_is_the_references():
    """Rows whose float32 sum depends on the order: the plain sequential sum
    differs from the compiled reference, the restatement does not."""
    K = 64
    x = np.ones(K, np.float32)
    w = np.zeros((2, K), np.float32)
    w[0, 0], w[0, 1:9] = 1e8, 3.0            # small terms absorbed one by one, not in partials
    w[1, ::8], w[1, 1::8], w[1, 2::8] = 1e7, -1e7, 0.75
    ref = O.matvec(w, x, use_ref=True)
    np.testing.assert_array_equal(O.matvec(w, x), ref)
    seq = []
    for row in w:
        acc = np.float32(0)
        for v in row:
            acc = np.float32(acc + v)
        seq.append(acc)
    assert np.all(np.asarray(seq, np.float32) != ref)


@needs_ref
@pytest.mark.parametrize("H,V,dtype,scale", [(896, 1000, "bf16", 1.0), (131, 77, "f32", 1.0),
                                             (4096, 300, "bf16", 8.0), (64, 50, "f32", 0.0)])
def test_lm_head_is_reference_rmsnorm_then_matvec(H, V, dtype, scale):
    rng = np.random.default_rng(H + V)
    rows = 3
    h = rng.normal(0, 2, (rows, H)).astype(np.float32)
    g = rng.normal(1, 0.2, H).astype(np.float32)
    w = rng.normal(0, 0.03, (V, H)).astype(np.float32)
    if dtype == "bf16":
        w = bf16_bits(w)
    logits, normed = O.lm_head(h, g, 1e-6, w, scale)
    for r in range(rows):
        xn = O.rmsnorm(h[r], g, 1e-6, use_ref=True)
        np.testing.assert_array_equal(normed[r], xn)
        y = O.matvec(w, xn, use_ref=True)
        if scale not in (0.0, 1.0):
            y = y * np.float32(1.0 / np.float32(scale))
        np.testing.assert_array_equal(logits[r], y)
