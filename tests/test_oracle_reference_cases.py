"""The reference's own sampler tests, restated against the CPU oracle.

/root/reference/tests/unit/test_sampler.cpp:21-117 holds the only known-answer
cases for this path (tiny V, fixed seeds). Each case runs the restatement with
the uniform the reference would draw from SamplerContext(seed), checks the
reference test's assertion, and -- where the reference was compiled into
oracle/_ref -- checks that the reference itself returns the same token and
leaves the same logits.

One expectation is tightened: test_sampler.cpp:90-100 accepts {0, 1} for
top_p = 0.5 over {10, 9, 0, 0, 0}, but p0 = 0.731 >= 0.5 already, so only token
0 survives and the exact answer is 0.
"""
import numpy as np
import pytest

import oracle as O


def run(logits, params, seed, recent=None, bias=None):
    u = O.u_from_seed(seed)
    tr = O.sample_row(np.array(logits, np.float32), params, hist=recent, bias=bias, u=u)
    if O.ref_available():
        tok, after = O.ref_sample_row(np.array(logits, np.float32), params, hist=recent,
                                      bias=bias, seed=seed)
        assert tok == tr.token
        np.testing.assert_array_equal(after.view(np.uint32), tr.logits_after.view(np.uint32))
    return tr


def test_argmax_returns_max_index():
    # test_sampler.cpp:21-24
    l = [0.1, 0.3, 0.2, 0.9, 0.5]
    assert O.argmax(l) == 3
    if O.ref_available():
        assert O.ref_argmax(l) == 3


def test_temperature_zero_is_argmax_after_penalties():
    # test_sampler.cpp:26-32
    tr = run([1.0, 5.0, 2.0, 3.0], O.identity_params(temperature=0.0), 42)
    assert tr.token == 1 and tr.greedy and not tr.u_consumed


def test_identity_draw_in_range_and_exact():
    # test_sampler.cpp:34-42; the exact token follows from softmax + the CDF draw.
    l = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    tr = run(l, O.identity_params(temperature=1.0), 7)
    assert 0 <= tr.token < 4
    e = np.exp(l.astype(np.float64) - 4.0)
    cp = np.cumsum(e / e.sum())
    assert tr.token == int(np.searchsorted(cp, O.u_from_seed(7), side="left"))


def test_same_seed_same_token():
    # test_sampler.cpp:44-55
    l = [0.5, 0.7, 0.3, 0.9, 0.6, 0.4, 0.8, 0.2]
    p = O.identity_params(temperature=1.0)
    assert run(l, p, 123456).token == run(l, p, 123456).token


def test_top_k_one_is_argmax():
    # test_sampler.cpp:57-64
    assert run([0.1, 0.4, 0.3, 0.9, 0.2], O.identity_params(top_k=1), 1).token == 3


def test_repetition_penalty_demotes_recent():
    # test_sampler.cpp:66-78
    p = O.identity_params(temperature=0.0, rep_penalty=2.0, repeat_last_n=8)
    assert run([0.1, 2.0, 2.5], p, 1, recent=[2]).token == 1


def test_min_p_filters_tail():
    # test_sampler.cpp:80-88
    tr = run([10.0, -5.0, -6.0, -7.0, -8.0], O.identity_params(min_p=0.5), 42)
    assert tr.token == 0
    assert list(tr.kept_idx) == [0]


def test_top_p_half_keeps_only_token0():
    # test_sampler.cpp:90-100 (expectation tightened to {0}, see module docstring)
    tr = run([10.0, 9.0, 0.0, 0.0, 0.0], O.identity_params(top_p=0.5), 5)
    assert tr.token == 0
    assert list(tr.kept_idx) == [0]


def test_logit_bias_pushes_token():
    # test_sampler.cpp:102-109
    tr = run([0.1, 0.2, 0.3], O.identity_params(temperature=0.0), 1, bias={0: 100.0})
    assert tr.token == 0


@pytest.mark.parametrize("seed", [99, 1, 2, 3])
def test_default_params_valid_token(seed):
    # test_sampler.cpp:111-117 (seed 99), plus a few more seeds
    l = [0.1, 0.5, 0.9, 0.3, 0.7, 0.2, 0.4, 0.6, 0.8, 0.15]
    tr = run(l, O.default_params(), seed)
    assert 0 <= tr.token < 10
