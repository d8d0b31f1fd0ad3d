"""The logits producer's checker (oracle/head_oracle.c) pinned on the CPU:
against the reference's own rmsnorm_f32 / matvec_f32_f32 / matvec_bf16_f32
compiled from its sources (oracle/_ref/libref_kernels.so, bit for bit), the
reference's known-answer cases (tests/unit/test_rmsnorm.cpp:22-36,
test_matvec.cpp:22-33), and float64 arithmetic (a transposed operand, a lost
term or a wrong scale fails these)."""
import numpy as np
import pytest

import oracle as O
import __graft_entry__

WL = __graft_entry__.load_package().workloads

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


# ---- quantised heads and the Hadamard fold --------------------------------------

QTYPES = {"q4k": O.HEAD_Q4_K, "q5k": O.HEAD_Q5_K, "q6k": O.HEAD_Q6_K, "q8_0": O.HEAD_Q8_0,
          "q4_1": O.HEAD_Q4_1, "q5_0": O.HEAD_Q5_0, "pq2_0": O.HEAD_PQ2_0}


def _f16(b, off):
    return (b[..., off].astype(np.uint16) | (b[..., off + 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float64)


def dequant64(w, dtype, H):
    """float64 weights [M, H] of a quantised head, from the GGUF block layouts
    (each value and scale exact in float64)."""
    M = w.shape[0]
    be, bb, _ = WL.QUANT_BLOCKS[dtype]
    b = w.reshape(M, H // be, bb)
    if dtype == O.HEAD_Q8_0:
        q = b[..., 2:34].view(np.int8).astype(np.float64)
        return (q * _f16(b, 0)[..., None]).reshape(M, H)
    if dtype == O.HEAD_Q4_1:
        qs = b[..., 4:20]
        q = np.concatenate([qs & 15, qs >> 4], axis=-1).astype(np.float64)
        return (q * _f16(b, 0)[..., None] + _f16(b, 2)[..., None]).reshape(M, H)
    if dtype == O.HEAD_Q5_0:
        qs = b[..., 6:22]
        qh = b[..., 2:6].copy().view(np.uint32)[..., 0]
        nib = np.concatenate([qs & 15, qs >> 4], axis=-1).astype(np.int64)
        bit = (qh[..., None] >> np.arange(32, dtype=np.uint32)) & 1
        return (((nib | (bit.astype(np.int64) << 4)) - 16) * _f16(b, 0)[..., None]).reshape(M, H)
    if dtype == O.HEAD_PQ2_0:
        codes = b[..., 2:34]
        c = np.stack([(codes >> (2 * j)) & 3 for j in range(4)], axis=-1).reshape(M, H // be, 128)
        return ((c.astype(np.float64) - 1) * _f16(b, 0)[..., None]).reshape(M, H)
    if dtype in (O.HEAD_Q4_K, O.HEAD_Q5_K):
        d, dmin = _f16(b, 0), _f16(b, 2)
        sm = b[..., 4:16].astype(np.int64)
        sc = np.zeros(sm.shape[:-1] + (8,), np.int64)
        mn = np.zeros_like(sc)
        for j in range(8):
            if j < 4:
                sc[..., j], mn[..., j] = sm[..., j] & 63, sm[..., j + 4] & 63
            else:
                sc[..., j] = (sm[..., j + 4] & 15) | ((sm[..., j - 4] >> 6) << 4)
                mn[..., j] = (sm[..., j + 4] >> 4) | ((sm[..., j] >> 6) << 4)
        ql = b[..., 16:144] if dtype == O.HEAD_Q4_K else b[..., 48:176]
        out = np.zeros(b.shape[:-1] + (256,), np.float64)
        for j in range(4):
            lo = (ql[..., 32 * j:32 * j + 32] & 15).astype(np.int64)
            hi = (ql[..., 32 * j:32 * j + 32] >> 4).astype(np.int64)
            if dtype == O.HEAD_Q5_K:
                qh = b[..., 16:48].astype(np.int64)
                lo |= ((qh >> (2 * j)) & 1) << 4
                hi |= ((qh >> (2 * j + 1)) & 1) << 4
            out[..., 64 * j:64 * j + 32] = lo * (d * sc[..., 2 * j])[..., None] - (dmin * mn[..., 2 * j])[..., None]
            out[..., 64 * j + 32:64 * j + 64] = (hi * (d * sc[..., 2 * j + 1])[..., None] -
                                                 (dmin * mn[..., 2 * j + 1])[..., None])
        return out.reshape(M, H)
    if dtype == O.HEAD_Q6_K:
        ql, qh = b[..., 0:128].astype(np.int64), b[..., 128:192].astype(np.int64)
        sc = b[..., 192:208].view(np.int8).astype(np.float64)
        d = _f16(b, 208)
        out = np.zeros(b.shape[:-1] + (256,), np.float64)
        for half in range(2):
            L, Hh = ql[..., 64 * half:64 * half + 64], qh[..., 32 * half:32 * half + 32]
            runs = [(L[..., :32] & 15) | ((Hh & 3) << 4), (L[..., 32:] & 15) | (((Hh >> 2) & 3) << 4),
                    (L[..., :32] >> 4) | (((Hh >> 4) & 3) << 4), (L[..., 32:] >> 4) | (((Hh >> 6) & 3) << 4)]
            for r, q in enumerate(runs):
                s = np.repeat(sc[..., 8 * half + 2 * r:8 * half + 2 * r + 2], 16, axis=-1)
                out[..., 128 * half + 32 * r:128 * half + 32 * r + 32] = (q - 32) * s * d[..., None]
        return out.reshape(M, H)
    raise ValueError(dtype)


@needs_ref
@pytest.mark.parametrize("name", sorted(QTYPES))
@pytest.mark.parametrize("M,H", [(8, 256), (37, 512), (64, 4096), (11, 1280), (9, 8192)])
def test_quant_matvec_is_the_references_bits(name, M, H):
    dt = QTYPES[name]
    if H % WL.QUANT_BLOCKS[dt][0]:
        pytest.skip("H is not a whole number of blocks")
    w = WL.quant_head(dt, M, H, seed=M * H + dt)
    x = np.random.default_rng(H + dt).normal(0, 1, H).astype(np.float32)
    got, ref = O.matvec(w, x, dtype=dt), O.matvec(w, x, dtype=dt, use_ref=True)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", sorted(QTYPES))
def test_quant_matvec_close_to_float64(name):
    """The dot product of the dequantised weights (float64), within a
    rounding bound: a wrong nibble, bit or scale order fails this."""
    dt = QTYPES[name]
    M, H = 24, 1024
    w = WL.quant_head(dt, M, H, seed=7 + dt, scale=0.5)
    x = np.random.default_rng(dt).normal(0, 1, H).astype(np.float32)
    W = dequant64(w, dt, H)
    want = W @ x.astype(np.float64)
    bound = 8 * H * np.finfo(np.float32).eps * (np.abs(W) @ np.abs(x.astype(np.float64))) + 1e-30
    got = O.matvec(w, x, dtype=dt).astype(np.float64)
    assert np.all(np.abs(got - want) <= bound), name


@needs_ref
@pytest.mark.parametrize("name", sorted(QTYPES))
def test_quant_evaluation_order_is_the_references(name):
    """Rows whose plain sequential float sum of the dequantised products
    differs from the reference's result: the restatement's partial-sum layout
    is what matches it."""
    dt = QTYPES[name]
    M, H = 16, 2048
    w = WL.quant_head(dt, M, H, seed=99 + dt, scale=1.0)
    x = np.random.default_rng(5).normal(0, 1, H).astype(np.float32) * np.float32(1e3)
    x[::7] *= np.float32(1e-4)
    ref = O.matvec(w, x, dtype=dt, use_ref=True)
    np.testing.assert_array_equal(O.matvec(w, x, dtype=dt).view(np.uint32), ref.view(np.uint32))
    W = dequant64(w, dt, H).astype(np.float32)
    seq = np.zeros(M, np.float32)
    for k in range(H):
        seq = (seq + W[:, k] * x[k]).astype(np.float32)
    assert np.sum(seq != ref) >= M // 2


def _block(dt, **f):
    be, bb, _ = WL.QUANT_BLOCKS[dt]
    return np.zeros(bb, np.uint8)


def _put16(b, off, v):
    h = np.float16(v).view(np.uint16)
    b[off], b[off + 1] = h & 0xFF, h >> 8


def test_quant_known_answers():
    """The reference's own known-answer cases (tests/unit/test_q6k.cpp:83-90,
    test_matvec_q4k.cpp:62-73, test_q8_0.cpp:83-93 and 128-146,
    test_q5_0.cpp:150-169, test_pq2_0.cpp:54-70)."""
    # Q6_K: every value q6 = 5, scales 3, d = 2 -> 30 each; dot with ones = 7680
    b = np.zeros(210, np.uint8)
    q6 = 5 + 32
    b[0:128] = (q6 & 15) | ((q6 & 15) << 4)
    hi2 = (q6 >> 4) & 3
    b[128:192] = hi2 | (hi2 << 2) | (hi2 << 4) | (hi2 << 6)
    b[192:208] = 3
    _put16(b, 208, 2.0)
    assert O.matvec(b[None], np.ones(256, np.float32), dtype=O.HEAD_Q6_K)[0] == 7680.0
    # Q4_K: d 1, dmin 0, every scale 1, nibbles l & 15 in each pair -> 1920
    b = np.zeros(144, np.uint8)
    _put16(b, 0, 1.0)
    b[4:8] = 1
    b[12:16] = 1
    nib = np.arange(32) & 15
    for j in range(4):
        b[16 + 32 * j:48 + 32 * j] = nib | (nib << 4)
    assert O.matvec(b[None], np.ones(256, np.float32), dtype=O.HEAD_Q4_K)[0] == 1920.0
    # Q8_0: d 1, every int8 1 -> 32; two rows of two blocks (1 and 2) -> 64, 128
    b = np.zeros(34, np.uint8)
    _put16(b, 0, 1.0)
    b[2:] = 1
    assert O.matvec(b[None], np.ones(32, np.float32), dtype=O.HEAD_Q8_0)[0] == 32.0
    r2 = np.zeros(34, np.uint8)
    _put16(r2, 0, 2.0)
    r2[2:] = 1
    w = np.stack([np.concatenate([b, b]), np.concatenate([r2, r2])])
    np.testing.assert_array_equal(O.matvec(w, np.ones(64, np.float32), dtype=O.HEAD_Q8_0), [64.0, 128.0])
    # Q5_0: nibbles 0 and fifth bits 0 -> -16 each, d 2 -> -1024 against ones
    b = np.zeros(22, np.uint8)
    _put16(b, 0, 2.0)
    assert O.matvec(b[None], np.ones(32, np.float32), dtype=O.HEAD_Q5_0)[0] == -1024.0
    # K not a whole number of blocks: zeros
    assert np.all(O.matvec(np.zeros((2, 40), np.uint8), np.ones(40, np.float32), dtype=O.HEAD_Q5_0) == 0)
    # PQ2_0: code c -> c - 1 (d 1); codes 0..3 spread over x = e_i picks each
    b = np.zeros(34, np.uint8)
    _put16(b, 0, 1.0)
    b[2:] = 0b11100100          # codes 0, 1, 2, 3 at positions 4i .. 4i + 3
    for j, want in enumerate([-1.0, 0.0, 1.0, 2.0]):
        x = np.zeros(128, np.float32)
        x[4 * 5 + j] = 1.0
        w8 = np.repeat(b[None], 8, axis=0)    # (eight rows: the vectorised path)
        assert O.matvec(w8, x, dtype=O.HEAD_PQ2_0)[0] == want


def _hadamard(n):
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("block", [2, 16, 1024])
def test_hadamard_fold_is_the_rotation(block):
    """The fold is, block by block, the orthonormal Sylvester-Hadamard rotation
    of x * signs (reference tests/unit/test_hadamard.cpp:31-53, 97-146); its
    own inverse; a constant block concentrates in its first coefficient."""
    H = 4 * block
    rng = np.random.default_rng(block)
    x = rng.normal(0, 1, H).astype(np.float32)
    s = np.where(rng.random(H) < 0.5, -1.0, 1.0).astype(np.float32)
    y = O.hadamard_fold(x, block, s)
    R = _hadamard(block) / np.sqrt(block)
    want = (R @ (x.astype(np.float64) * s).reshape(4, block).T).T.reshape(H)
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-5 * np.sqrt(block))
    back = O.hadamard_fold(y, block, None)
    np.testing.assert_allclose(back, x * s, atol=1e-5)
    c = O.hadamard_fold(np.full(block, 3.0, np.float32), block, None)
    assert c[0] == pytest.approx(3.0 * np.sqrt(block), rel=1e-6) and np.all(np.abs(c[1:]) < 1e-4)
    # a block that does not divide the width: the row as it is, signs not applied
    np.testing.assert_array_equal(O.hadamard_fold(x[: H - 1], block, s[: H - 1]), x[: H - 1])


@needs_ref
@pytest.mark.parametrize("H,block", [(4096, 1024), (2048, 2048), (1024, 64), (896, 128), (4096, 0), (1000, 64)])
def test_hadamard_fold_is_the_references_bits(H, block):
    rng = np.random.default_rng(H + block)
    x = rng.normal(0, 2, H).astype(np.float32)
    s = np.where(rng.random(H) < 0.5, -1.0, 1.0).astype(np.float32)
    for sg in (s, None):
        np.testing.assert_array_equal(O.hadamard_fold(x, block, sg).view(np.uint32),
                                      O.hadamard_fold(x, block, sg, use_ref=True).view(np.uint32))


@needs_ref
@pytest.mark.parametrize("name", ["q6k", "q8_0", "q4k", "bf16"])
def test_folded_lm_head_is_reference_norm_fold_matvec(name):
    """orc_lm_head with a fold: the reference's rmsnorm, hadamard_fold_f32 and
    matvec in sequence (qwen_model.cpp:182-207)."""
    dt = O.HEAD_NAMES[name]
    H, V, rows, block = 2048, 96, 2, 1024
    rng = np.random.default_rng(dt)
    h = rng.normal(0, 2, (rows, H)).astype(np.float32)
    g = rng.normal(1, 0.2, H).astype(np.float32)
    s = np.where(rng.random(H) < 0.5, -1.0, 1.0).astype(np.float32)
    if dt == O.HEAD_BF16:
        w = bf16_bits(rng.normal(0, 0.03, (V, H)))
    else:
        w = WL.quant_head(dt, V, H, seed=3)
    logits, normed = O.lm_head(h, g, 1e-6, w, 2.0, dtype=dt, fold_block=block, fold_signs=s)
    for r in range(rows):
        xn = O.hadamard_fold(O.rmsnorm(h[r], g, 1e-6, use_ref=True), block, s, use_ref=True)
        np.testing.assert_array_equal(normed[r], xn)
        y = O.matvec(w, xn, use_ref=True, dtype=dt) * np.float32(0.5)
        np.testing.assert_array_equal(logits[r], y)
