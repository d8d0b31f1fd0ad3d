"""The restatement against the reference's own sampler.

oracle/_ref/libref_sampler.so is /root/reference/src/sampler/sampler.cpp
compiled from its sources (oracle/Makefile). On seeded tie-free cases
(tests/case_gen.py) that switch every stage on and off, the restatement given
the uniform of SamplerContext(seed) must return the reference's token and leave
bit-identical logits. The committed fixture tests/golden/ref_cases.npz holds
reference outputs for such cases so the restatement stays pinned where the
reference sources are absent (the GPU box).
"""
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from case_gen import make_case

GOLD = Path(__file__).resolve().parent / "golden" / "ref_cases.npz"


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference sources)")
@pytest.mark.parametrize("seed", range(400))
def test_restatement_equals_reference(seed):
    x, hist, bias, p = make_case(seed)
    tok, after = O.ref_sample_row(x, p, hist=hist, bias=bias, seed=seed)
    tr = O.sample_row(x, p, hist=hist, bias=bias, u=O.u_from_seed(seed))
    assert tr.token == tok
    np.testing.assert_array_equal(tr.logits_after.view(np.uint32), after.view(np.uint32))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (no reference sources)")
@pytest.mark.parametrize("seed", range(6))
def test_restatement_equals_reference_full_vocab(seed):
    # Realistic V with the server defaults (DRY on) and the CLI's identity + T.
    rng = np.random.default_rng(seed)
    V = 151936
    x = (rng.normal(size=V) * 2).astype(np.float32)
    hist = rng.integers(0, V, size=600).astype(np.int32)
    hist[-50:] = hist[-100:-50]                     # a repeated span for DRY
    for p in (O.default_params(), O.identity_params(temperature=0.8),
              O.identity_params(temperature=0.7, top_k=50, rep_penalty=1.1, repeat_last_n=2048,
                                frequency_penalty=0.5, presence_penalty=0.3)):
        tok, after = O.ref_sample_row(x, p, hist=hist, seed=seed)
        tr = O.sample_row(x, p, hist=hist, u=O.u_from_seed(seed))
        assert tr.token == tok
        np.testing.assert_array_equal(tr.logits_after.view(np.uint32), after.view(np.uint32))


def test_restatement_reproduces_golden_reference_outputs():
    g = np.load(GOLD, allow_pickle=False)
    n = int(g["n"])
    assert n >= 100
    for i in range(n):
        x = g["logits"][i]
        hist = g["hist"][i][: int(g["hist_len"][i])]
        nb = int(g["bias_n"][i])
        bias = {int(a): float(b) for a, b in zip(g["bias_ids"][i][:nb], g["bias_vals"][i][:nb])}
        p = {k: g["p_" + k][i].item() for k in O.PARAM_FIELDS}
        seed = int(g["seed"][i])
        tr = O.sample_row(x, p, hist=hist, bias=bias, u=O.u_from_seed(seed))
        assert tr.token == int(g["token"][i]), i
        np.testing.assert_array_equal(tr.logits_after.view(np.uint32),
                                      g["after"][i].view(np.uint32))
