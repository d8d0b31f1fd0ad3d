"""Pins for the CPU oracle that do not depend on the oracle's own code.

Each stage is checked against something the mathematics or a library fixes:
closed-form IEEE single-op sequences computed here with numpy float32 scalars,
brute force over full sorts (numpy lexsort) for top-k / top-p, the libstdc++
discrete_distribution semantics (double partial sums + lower_bound, i.e.
numpy searchsorted) for the draw, and the C++ standard's mt19937_64 known
answer. Cases are chosen so that plausible mistakes (a fused multiply-add, the
wrong window, a dropped dedupe, an off-by-one cutoff, ties to the wrong index)
fail at least one assertion.
"""
import math

import numpy as np
import pytest

import oracle as O

f32 = np.float32
NEG_INF = f32(-np.inf)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---- RNG and the uniform -------------------------------------------------------

def test_mt19937_64_known_answer():
    # C++ standard [rand.predef]: 10000th output of a default-constructed mt19937_64.
    assert O.mt19937_64_nth(5489, 10000) == 9981545732273789042


@pytest.mark.parametrize("seed", [0, 1, 42, 5489, 2**63 + 12345])
def test_uniform_is_generate_canonical(seed):
    # generate_canonical<double,53> with one 64-bit draw: double(x) / 2^64.
    x = O.mt19937_64_nth(seed, 1)
    assert O.u_from_seed(seed) == float(x) / 2.0**64


# ---- penalties -----------------------------------------------------------------

def test_rep_penalty_closed_form_dedupe_and_range():
    l = np.array([2.0, -2.0, 0.0, -0.0, 3.0, 1.0], np.float32)
    p = O.identity_params(temperature=0.0, rep_penalty=1.5, repeat_last_n=64)
    hist = [0, 1, 2, 3, 0, 0, -1, 6, 100]      # duplicates of 0; -1/6/100 out of range
    tr = O.sample_row(l, p, hist=hist)
    exp = l.copy()
    r = f32(1.5)
    exp[0] = l[0] / r                          # once, despite three occurrences
    exp[1] = l[1] * r
    exp[2] = l[2] * r
    exp[3] = l[3] * r                          # -0 * 1.5 = -0 (bit pattern kept)
    np.testing.assert_array_equal(bits(tr.logits_after), bits(exp))


def test_rep_window_is_suffix():
    l = np.array([1.0, 1.0, 1.0, 0.5], np.float32)
    p = O.identity_params(temperature=0.0, rep_penalty=4.0, repeat_last_n=1)
    tr = O.sample_row(l, p, hist=[0, 1, 2])    # only id 2 is in the window
    assert tr.token == 0
    assert tr.logits_after[2] == f32(1.0) / f32(4.0)
    assert tr.logits_after[0] == f32(1.0) and tr.logits_after[1] == f32(1.0)


def _two_roundings(l, n, f, pp):
    return (f32(l) - f32(n) * f32(f)) - f32(pp)


def test_freq_presence_two_roundings_not_fused():
    # Find a case where fl(l - fl(n*f)) differs from a fused l - n*f, so a
    # contracted implementation would fail.
    rng = np.random.default_rng(3)
    for _ in range(10000):
        l = f32(rng.normal() * 4)
        f = f32(rng.uniform(0.01, 2))
        n = int(rng.integers(2, 50))
        fused = f32(np.float64(l) - np.float64(n) * np.float64(f))
        if fused != f32(l) - f32(n) * f32(f):
            break
    else:
        pytest.fail("no distinguishing case found")
    V = 4
    x = np.zeros(V, np.float32)
    x[1] = l
    p = O.identity_params(temperature=0.0, repeat_last_n=n, frequency_penalty=float(f),
                          presence_penalty=0.25)
    tr = O.sample_row(x, p, hist=[1] * n)
    assert bits(tr.logits_after[1]) == bits(_two_roundings(l, n, f, 0.25))


def test_freq_presence_window_is_max_of_rep_and_dry():
    # sampler.cpp:255: window = max(repeat_last_n, dry_last_n); DRY itself off.
    x = np.zeros(4, np.float32)
    p = O.identity_params(temperature=0.0, repeat_last_n=1, dry_last_n=3,
                          frequency_penalty=1.0, presence_penalty=0.5)
    tr = O.sample_row(x, p, hist=[1, 1, 2])
    assert tr.logits_after[1] == _two_roundings(0.0, 2, 1.0, 0.5)
    assert tr.logits_after[2] == _two_roundings(0.0, 1, 1.0, 0.5)
    assert tr.logits_after[0] == 0.0 and tr.logits_after[3] == 0.0


def test_identity_windows_silence_freq_presence():
    x = np.zeros(4, np.float32)
    p = O.identity_params(temperature=0.0, frequency_penalty=1.0, presence_penalty=1.0)
    tr = O.sample_row(x, p, hist=[1, 1, 2])
    np.testing.assert_array_equal(tr.logits_after, x)


def test_dry_closed_form():
    x = np.array([1.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    p = O.identity_params(temperature=0.0, dry_multiplier=0.8, dry_base=1.75,
                          dry_allowed_len=2, dry_last_n=8)
    hist = [1, 1, 1, 1, 2, 2, 2, 3]           # counts: 1->4, 2->3, 3->1
    tr = O.sample_row(x, p, hist=hist)
    pen1 = f32(0.8) * f32(O.powf(1.75, 2.0))
    pen2 = f32(0.8) * f32(O.powf(1.75, 1.0))
    assert tr.logits_after[1] == f32(1.0) - pen1
    assert tr.logits_after[2] == f32(1.0) - pen2
    assert tr.logits_after[3] == f32(1.0)     # n <= allowed_len
    # a window shorter than two ids disables DRY (sampler.cpp:69)
    tr2 = O.sample_row(x, dict(p, dry_last_n=1), hist=hist)
    np.testing.assert_array_equal(tr2.logits_after, x)


def test_stage_order_bias_then_rep_then_fp():
    x = np.array([0.0, -1.0, 0.0], np.float32)
    p = O.identity_params(temperature=0.0, rep_penalty=2.0, repeat_last_n=4,
                          frequency_penalty=0.5, presence_penalty=0.25)
    tr = O.sample_row(x, p, hist=[1, 1], bias={1: 3.0})
    v = f32(-1.0) + f32(3.0)                  # bias first: 2.0 > 0 -> divided
    v = v / f32(2.0)
    v = _two_roundings(v, 2, 0.5, 0.25)
    assert tr.logits_after[1] == v


def test_mask_equals_neg_inf_bias():
    rng = np.random.default_rng(11)
    V = 300
    for trial in range(20):
        x = rng.normal(size=V).astype(np.float32) * 2
        allowed = rng.random(V) < 0.1
        allowed[rng.integers(V)] = True
        mask = np.zeros((V + 31) // 32, np.uint32)
        for t in np.nonzero(allowed)[0]:
            mask[t >> 5] |= np.uint32(1 << (t & 31))
        p = O.identity_params(temperature=0.9, top_k=7, top_p=0.9)
        u = float(rng.random())
        a = O.sample_row(x, p, mask=mask, u=u)
        b = O.sample_row(x, p, bias={int(t): -np.inf for t in np.nonzero(~allowed)[0]}, u=u)
        assert a.token == b.token
        np.testing.assert_array_equal(bits(a.logits_after), bits(b.logits_after))
        assert allowed[a.token]


# ---- temperature, top-k, softmax, top-p, draw ----------------------------------

def test_temperature_multiplies_by_rounded_reciprocal():
    rng = np.random.default_rng(5)
    x = rng.normal(size=257).astype(np.float32) * 3
    for T in (0.7, 0.3, 1.7, 1.0):
        tr = O.sample_row(x, O.identity_params(temperature=T), u=0.3)
        exp = x if T == 1.0 else x * (f32(1.0) / f32(T))
        np.testing.assert_array_equal(bits(tr.logits_after), bits(exp))


def brute_topk(v, k):
    order = np.lexsort((np.arange(v.size), -v.astype(np.float64)))  # value desc, index asc
    return np.sort(order[:k])


@pytest.mark.parametrize("k", [1, 2, 5, 20, 63])
def test_topk_matches_full_sort_with_ties(k):
    rng = np.random.default_rng(k)
    for _ in range(10):
        x = np.round(rng.normal(size=200) * 2, 1).astype(np.float32)   # many ties
        x[rng.integers(200, size=5)] = -0.0
        x[rng.integers(200, size=5)] = 0.0
        tr = O.sample_row(x, O.identity_params(temperature=0.8, top_k=k), u=0.5)
        v = x * (f32(1.0) / f32(0.8))
        np.testing.assert_array_equal(tr.topk_idx, brute_topk(v, k))
        np.testing.assert_array_equal(tr.kept_idx, brute_topk(v, k))


def softmax64(v):
    fin = np.isfinite(v)
    e = np.zeros(v.size)
    e[fin] = np.exp(v[fin].astype(np.float64) - v[fin].max())
    return e / e.sum()


def test_softmax_probabilities_match_float64():
    rng = np.random.default_rng(9)
    x = rng.normal(size=1000).astype(np.float32) * 3
    tr = O.sample_row(x, O.identity_params(temperature=0.5, top_k=100), u=0.5)
    v = x * (f32(1.0) / f32(0.5))
    ref = softmax64(np.where(np.isin(np.arange(1000), tr.kept_idx), v, -np.inf))[tr.kept_idx]
    np.testing.assert_allclose(tr.kept_prob, ref, rtol=1e-6)
    assert abs(float(np.sum(tr.kept_prob, dtype=np.float64)) - 1.0) < 1e-6


def float_softmax(v):
    """Spec of sampler.cpp:124-142 with numpy float32 scalars and libm expf."""
    fin = v != NEG_INF
    m = v[fin].max()
    e = np.zeros(v.size, np.float32)
    e[fin] = O.expf_many((v[fin] - m).astype(np.float32))
    s = np.add.accumulate(e)[-1]              # sequential float32 sum, index order
    return e * (f32(1.0) / s)


@pytest.mark.parametrize("top_p", [0.1, 0.5, 0.8, 0.9, 0.95, 0.999])
def test_top_p_matches_sorted_float_cumsum(top_p):
    rng = np.random.default_rng(int(top_p * 1000))
    for _ in range(5):
        x = (rng.normal(size=500) * 1.5).astype(np.float32)
        tr = O.sample_row(x, O.identity_params(top_p=top_p), u=0.5)
        p = float_softmax(x)
        order = np.lexsort((np.arange(p.size), -p.astype(np.float64)))
        cum = np.add.accumulate(p[order])
        hit = np.nonzero(cum >= f32(top_p))[0]
        cutoff = hit[0] + 1 if hit.size else p.size
        np.testing.assert_array_equal(tr.kept_idx, np.sort(order[:cutoff]))


def cdf_draw(prob_full, u):
    q = prob_full.astype(np.float64)
    q = q / np.add.accumulate(q)[-1]
    cp = np.add.accumulate(q)
    cp[-1] = 1.0
    return int(np.searchsorted(cp, u, side="left"))


@pytest.mark.parametrize("seed", range(8))
def test_draw_is_lower_bound_on_double_cdf(seed):
    rng = np.random.default_rng(100 + seed)
    V = 64
    x = rng.normal(size=V).astype(np.float32)
    for u in list(rng.random(20)) + [0.0, 1.0 - 2.0**-53]:
        tr = O.sample_row(x, O.identity_params(top_k=10, temperature=1.3), u=u)
        full = np.zeros(V, np.float32)
        full[tr.kept_idx] = tr.kept_prob
        assert tr.token == cdf_draw(full, u)
        assert tr.u_consumed


def test_draw_edge_quirks():
    x = np.array([0.0, 0.0, 0.0, 5.0, 0.0], np.float32)
    p = O.identity_params(top_k=1)
    assert O.sample_row(x, p, u=0.0).token == 0          # u == 0 -> index 0 even with p0 = 0
    assert O.sample_row(x, p, u=0.5).token == 3
    # all logits -inf -> uniform over V (sampler.cpp:127-130)
    mask = np.zeros(1, np.uint32)
    uni = np.full(5, f32(1.0) / f32(5.0), np.float32)
    for u in (0.99, 0.2, 0.5, 0.0, 0.7999999999):
        tr = O.sample_row(x, O.identity_params(), mask=mask, u=u)
        assert tr.token == cdf_draw(uni, u) and tr.kept_idx.size == 0


def test_u_consumption_rules():
    assert O.sample_row([1.0], O.identity_params(), u=0.9).token == 0
    assert not O.sample_row([1.0], O.identity_params(), u=0.9).u_consumed
    tr = O.sample_row([1.0, 2.0], O.identity_params(temperature=0.0), u=0.9)
    assert tr.token == 1 and not tr.u_consumed
    assert O.sample_row(np.zeros(0, np.float32), O.identity_params()).token == -1


def test_argmax_first_max_and_signed_zero():
    assert O.argmax([0.0, -0.0, 0.0]) == 0
    assert O.argmax([-0.0, 0.0]) == 0
    assert O.argmax([-np.inf, -np.inf]) == 0
    assert O.argmax([1.0, 3.0, 3.0]) == 1


def test_expf_is_glibc():
    # The oracle calls libm through std::exp(float); spot values are exact.
    assert O.expf(0.0) == 1.0
    assert O.expf(-np.inf) == 0.0
    assert O.expf(-200.0) == 0.0
    assert abs(O.expf(-1.0) - math.exp(-1.0)) < 1e-7


def test_stage_clock_leaves_results_unchanged(orc, wl):
    """The CPU baseline's per-stage breakdown runs the same ladder: tokens equal
    the plain batch call's, and every stage of a config-2 row is timed."""
    w = wl.config(2, seed=4, rows=3, V=20000)
    x1, x2 = w.logits_f32().copy(), w.logits_f32().copy()
    t1 = orc.sample_batch(x1, w.params, w.hist, w.hist_len, None, w.u)
    t2, st = orc.sample_batch_stages(x2, w.params, w.hist, w.hist_len, None, w.u)
    np.testing.assert_array_equal(t1, t2)
    np.testing.assert_array_equal(x1.view(np.uint32), x2.view(np.uint32))
    assert set(st) == set(orc.STAGES)
    assert all(v >= 0.0 for v in st.values())
    assert st["penalties"] > 0 and st["top_k"] > 0 and st["draw"] > 0
