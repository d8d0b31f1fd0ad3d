"""GPU parity: the HIP sampler through its C ABI against the CPU oracle.

Bar: token ids and top-k index sets bit-exact, ties to
the lower index; probabilities within 1e-6 relative (this build reproduces
glibc expf, so they are asserted bit-exact as well); the logits left behind
with in-place writeback bit-exact. Inputs are the seeded BASELINE
configurations (ultima.cpp_amd/workloads.py) at full V = 151936 and the edge
cases the reference's own tests and semantics call for.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
from gpu_helpers import compare_rows, run_gpu, to_device

pytestmark = pytest.mark.gpu


# ---- the BASELINE configurations ----------------------------------------------

@pytest.mark.parametrize("cfg,rows", [(1, 1), (2, 8), (4, 8), (5, 24)])
def test_config_rows_match_oracle(sampler, wl, cfg, rows, kernel_mode):
    w = wl.config(cfg, seed=11, rows=rows)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == rows


def test_config2_full_batch(sampler, hs, wl, kernel_mode):
    w = wl.config(2, seed=1)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == 64
    # penalties on random histories never push the top-k below the stream's
    # bounds (general kernels); exact lists never read a row again
    assert not np.any(g["row_flags"] & hs.ROW_REREAD)


def test_config4_full_batch(sampler, wl, kernel_mode):
    w = wl.config(4, seed=1)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == 128


def test_config5_full_batch(sampler, wl, kernel_mode):
    """Every one of the 1024 rows with the library's own kernels; every third
    row in the forced kernel modes."""
    w = wl.config(5, seed=1)
    g = run_gpu(sampler, w)
    rows = range(1024) if kernel_mode == "default" else range(0, 1024, 3)
    assert compare_rows(w, g, rows=rows) == len(rows)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_exact_lists_large_k(sampler, wl, dtype, kernel_mode):
    """Top-k above 64 in batches the exact lists take (every row samples,
    penalties that only lower): the stream's block-level bound over its chunk
    maxima, lists merged by the large-k merge. k at 65, in between and at the
    1024 limit next to small k; histories of each row's top tokens (hundreds
    of penalised candidates, some pushed below the bound); a constant row
    (every chunk at the bound) and a rounded row (ties across slices)."""
    rng = np.random.default_rng(77 if dtype == "f32" else 78)
    B, V, H = 10, 151936, 512
    x = rng.normal(0.0, 2.5, size=(B, V)).astype(np.float32)
    x[3] = np.float32(1.0)
    x[7] = np.round(x[7] * 2) / 2
    hist = np.empty((B, H), np.int32)
    for r in range(B):
        top = np.argsort(-x[r], kind="stable")[:1200]
        hist[r] = rng.permutation(np.concatenate([rng.choice(top, 400), rng.integers(0, V, H - 400)]))
    ks = (65, 100, 257, 500, 1000, 1024, 1, 64, 700, 333)
    plist = [wl.identity_params(top_k=k, temperature=float(rng.uniform(0.3, 1.5)),
                                top_p=float(rng.choice([1.0, 0.9, 0.6])), rep_penalty=1.3, repeat_last_n=512,
                                frequency_penalty=0.2, presence_penalty=0.4) for k in ks]
    xs = x if dtype == "f32" else wl.to_bf16_bits(x)
    w = _wl_from(wl, xs, plist, rng.random(B), dtype=dtype)
    w.hist, w.hist_len = hist, np.full(B, H, np.int64)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == B


@pytest.mark.parametrize("cfg", [2, 4])
def test_writeback_leaves_reference_state(sampler, wl, cfg):
    w = wl.config(cfg, seed=5, rows=4)
    if w.dtype != "f32":
        pytest.skip("writeback is defined for float32 logits")
    g = run_gpu(sampler, w, writeback=True)
    compare_rows(w, g, writeback=True)


@pytest.mark.parametrize("kind", ["server", "cli_topk", "greedy", "mixed"])
def test_writeback_on_the_exact_lists(hs, sampler, wl, kind, kernel_mode):
    """The drop-in's calls write their logits back (sample() works in place):
    batches the exact lists take keep taking them with write-back (the
    library's choice: ULTIMA_HSAMP_KERNELS_EXACT), and the logits left behind
    are the reference's bits -- kept ids at their post-penalty,
    post-temperature value and the rest -inf, greedy rows' whole post-penalty
    row -- in every kernel mode."""
    import torch
    rng = np.random.default_rng({"server": 1, "cli_topk": 2, "greedy": 3, "mixed": 4}[kind])
    B, V, H = 6, 151936, 600
    x = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[:, -30:] = np.argsort(-x, axis=1)[:, :30]          # the likely ids in the windows
    if kind == "server":
        plist = [wl.default_params(temperature=0.8) for _ in range(B)]
    elif kind == "cli_topk":
        plist = [wl.identity_params(temperature=0.7, top_k=40) for _ in range(B)]
    elif kind == "greedy":
        plist = [wl.default_params(temperature=0.0) for _ in range(B)]
    else:
        plist = [wl.default_params(temperature=t) for t in (0.0, 0.5, 0.9, 0.0, 1.2, 0.3)]
    w = _wl_from(wl, x, plist, rng.random(B), hist=hist)
    if kernel_mode == "default":
        xd, ud, hd, _ = to_device(w)
        k = sampler.query_kernels(xd, plist, ud, hist=hd, hist_len=w.hist_len, writeback=True)
        assert k & hs.KERNELS_EXACT and k & hs.KERNELS_WRITEBACK and not k & hs.KERNELS_GENERAL, k
    g = run_gpu(sampler, w, writeback=True)
    compare_rows(w, g, writeback=True)


def test_repeated_launches_are_stable(sampler, wl):
    w = wl.config(2, seed=2, rows=16)
    first = run_gpu(sampler, w)["token"]
    for _ in range(5):
        np.testing.assert_array_equal(run_gpu(sampler, w)["token"], first)


# ---- edge cases ----------------------------------------------------------------

def _wl_from(wl, x, plist, u, hist=None, mask=None, dtype="f32"):
    B = x.shape[0]
    hl = None if hist is None else np.full(B, hist.shape[1], np.int64)
    return wl.Workload("edge", dtype, x, plist, np.asarray(u, np.float64), hist, hl, mask)


def test_ties_break_to_lower_index(sampler, wl, kernel_mode):
    rng = np.random.default_rng(0)
    V = 151936
    rows = []
    x = np.round(rng.normal(size=(6, V)) * 2, 1).astype(np.float32)   # massive ties
    x[1] = 0.5                                                          # constant row
    x[2, ::2] = -0.0
    x[2, 1::2] = 0.0
    x[3] = np.float32(1.0)
    x[3, 1000:1100] = 2.0
    plist = [wl.identity_params(top_k=k, temperature=t) for k, t in
             ((50, 0.7), (40, 1.0), (10, 1.0), (64, 1.3), (1000, 0.9), (7, 0.3))]
    w = _wl_from(wl, x, plist, rng.random(6))
    g = run_gpu(sampler, w)
    compare_rows(w, g)


def test_bf16_ties_and_top_p(sampler, wl, kernel_mode):
    rng = np.random.default_rng(1)
    x = wl.to_bf16_bits(rng.normal(size=(8, 151936)).astype(np.float32) * 2.5)
    plist = [wl.identity_params(top_k=int(k), top_p=float(p), temperature=1.0)
             for k, p in zip((1, 5, 20, 100, 500, 1000, 999, 257), (0.5, 0.8, 0.9, 0.95, 0.6, 0.99, 1.0, 0.3))]
    w = _wl_from(wl, x, plist, rng.random(8), dtype="bf16")
    g = run_gpu(sampler, w)
    compare_rows(w, g)


def test_mask_sparser_than_k_and_all_masked(sampler, wl, kernel_mode):
    rng = np.random.default_rng(2)
    B, V = 4, 151936
    x = rng.normal(size=(B, V)).astype(np.float32)
    allowed = np.zeros((B, V), bool)
    allowed[0, rng.choice(V, 5, replace=False)] = True     # fewer allowed than k
    allowed[1, :] = False                                   # nothing allowed: uniform over V
    allowed[2, [0, V - 1]] = True
    allowed[3, rng.random(V) < 0.001] = True
    mask = wl.mask_from_allowed(allowed)
    plist = [wl.identity_params(top_k=20, top_p=0.8)] * B
    w = _wl_from(wl, x, plist, [0.3, 0.77, 0.99, 0.5], mask=mask)
    g = run_gpu(sampler, w)
    compare_rows(w, g)
    assert int(g["row_flags"][1]) & 16   # uniform draw flagged


def test_greedy_and_sampling_rows_mixed(sampler, wl):
    rng = np.random.default_rng(3)
    B, V = 6, 151936
    x = rng.normal(size=(B, V)).astype(np.float32) * 2
    x[4, :] = -np.inf
    x[4, 77] = 1.0
    hist = rng.integers(0, V, size=(B, 300)).astype(np.int32)
    plist = [wl.identity_params(temperature=0.0, rep_penalty=1.3, repeat_last_n=300),
             wl.identity_params(top_k=40, temperature=0.8),
             wl.identity_params(temperature=-1.0),
             wl.default_params(),
             wl.identity_params(temperature=0.0),
             wl.identity_params(top_k=3, min_p=0.5, temperature=2.0)]
    w = _wl_from(wl, x, plist, rng.random(B), hist=hist)
    g = run_gpu(sampler, w)
    compare_rows(w, g)


def test_penalties_dry_bias_and_out_of_range_history(sampler, wl):
    rng = np.random.default_rng(4)
    B, V = 5, 151936
    x = rng.normal(size=(B, V)).astype(np.float32) * 2
    hist = rng.integers(-5, V + 5, size=(B, 700)).astype(np.int32)
    hist[:, 600:] = hist[:, 500:600]                      # repeats for DRY
    hist[2, :] = 12345                                    # one id, many times
    bias = [{1: 5.0, 2: -3.0, V - 1: 10.0}, None, {12345: 7.5, -3: 1.0, V + 2: 1.0}, None,
            {int(t): float(v) for t, v in zip(rng.choice(V, 200, replace=False), rng.normal(size=200))}]
    plist = [wl.default_params(temperature=0.9),
             wl.default_params(top_k=100, dry_allowed_len=0, dry_last_n=700, frequency_penalty=0.2),
             wl.default_params(rep_penalty=0.8, presence_penalty=-0.5, frequency_penalty=0.01),
             wl.identity_params(top_k=50, rep_penalty=1.5, repeat_last_n=10, dry_multiplier=1.2,
                                dry_last_n=650, dry_base=2.0),
             wl.default_params(min_p=0.0, top_p=0.5)]
    w = _wl_from(wl, x, plist, rng.random(B), hist=hist)
    g = run_gpu(sampler, w, bias=bias)
    compare_rows(w, g, bias=bias)


def test_uniform_edges(sampler, wl, kernel_mode):
    rng = np.random.default_rng(5)
    B, V = 4, 151936
    x = np.repeat(rng.normal(size=(1, V)).astype(np.float32), B, axis=0)
    plist = [wl.identity_params(top_k=30)] * B
    w = _wl_from(wl, x, plist, [0.0, 1.0 - 2.0**-53, 0.5, 2.0**-60])
    g = run_gpu(sampler, w)
    compare_rows(w, g)


@pytest.mark.parametrize("k", [20, 300])
def test_u_on_and_beside_cdf_boundaries(sampler, wl, k, kernel_mode):
    """u placed exactly on, and 1e-12 either side of, interior partial sums
    of the reference's CDF (double sum S of the kept p in index order,
    q = p / S, sequential partial sums): the finalize must leave its tree
    fast path for the reference's sequential sums there, so every token must
    match exactly (no CDF_NEAR tolerance). k = 20 takes the one-wave
    finalize, k = 300 the block finalize of the general merge."""
    rng = np.random.default_rng(123)
    V = 151936
    base = rng.normal(0, 1.5, size=(1, V)).astype(np.float32)
    params = wl.identity_params(top_k=k, temperature=0.9)
    probe = _wl_from(wl, base, [params], [0.5])
    tr = O.sample_row(probe.logits_f32()[0], params, hist=None, mask=None, bias=None, u=0.5)
    p = tr.kept_prob.astype(np.float64)
    S = 0.0
    for v in p:
        S += v
    cp, acc = [], 0.0
    for v in p:
        acc += v / S
        cp.append(acc)
    us = []
    for j in (0, 3, 9, 15) + ((100, 250, len(cp) - 2) if k > 64 else ()):
        for d in (0.0, 1e-12, -1e-12):
            us.append(min(max(cp[j] + d, 0.0), 1.0 - 2.0**-53))
    B = len(us)
    w = _wl_from(wl, np.repeat(base, B, axis=0), [params] * B, us)
    g = run_gpu(sampler, w)
    # the fallback replays the reference's sums: every token matches exactly
    assert compare_rows(w, g, strict_token=True) == B


@pytest.mark.parametrize("k,top_p,min_p,sigma", [(1000, 0.5, 0.0, 0.01), (900, 0.97, 0.0, 0.3),
                                                 (700, 1.0, 0.9, 0.02), (1024, 0.8, 0.5, 0.05)])
def test_general_finalize_long_sums(sampler, wl, k, top_p, min_p, sigma):
    """Rows with hundreds of near-equal probabilities through the block
    finalize (k > 64): the index-order softmax sum and the top-p running sum
    over up to 1024 values are the reference's sequential float sums, exact
    to the bit, and the cut falls where the reference's does."""
    rng = np.random.default_rng(k)
    V = 151936
    B = 8
    x = rng.normal(0, sigma, size=(B, V)).astype(np.float32)
    params = [wl.identity_params(top_k=k, top_p=top_p, min_p=min_p, temperature=1.0) for _ in range(B)]
    us = list(rng.random(B))
    w = _wl_from(wl, x, params, us)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g, strict_token=True) == B


@pytest.mark.parametrize("V", [2, 5, 31, 33, 1000, 50257])
def test_small_and_unaligned_vocab(sampler, wl, V, kernel_mode):
    rng = np.random.default_rng(V)
    B = 3
    x = rng.normal(size=(B, V)).astype(np.float32) * 3
    k = min(V - 1, 40)
    plist = [wl.identity_params(top_k=k, temperature=0.7), wl.identity_params(temperature=0.0),
             wl.default_params(top_k=max(1, V // 2))]
    w = _wl_from(wl, x, plist, rng.random(B))
    g = run_gpu(sampler, w, set_cap=V)     # row 2 keeps up to V/2 ids
    compare_rows(w, g)


@pytest.mark.parametrize("V,dtype", [(5, "f32"), (33, "f32"), (1001, "f32"), (50257, "f32"), (151939, "f32"),
                                     (50257, "bf16"), (151941, "bf16")])
def test_sampling_penalties_ragged_end(sampler, wl, V, dtype, kernel_mode):
    """Sampling rows with penalties over vocabularies that are not a multiple
    of the 16-byte load width: the row's last ids, which the stream's vector
    loads leave out, hold high logits and sit in the history many times, so
    their true values decide the top-k."""
    rng = np.random.default_rng(V + 17)
    B, H = 4, 256
    xf = (rng.normal(size=(B, V)) * 2).astype(np.float32)
    xf[:, -7:] += 6.0
    hist = rng.integers(0, V, size=(B, H)).astype(np.int32)
    hist[:, :8] = V - 1
    hist[:, 8:12] = V - 2
    hist[:, 12] = V - 3
    k = min(V - 1, 50)
    pen = dict(rep_penalty=1.2, repeat_last_n=H, frequency_penalty=0.3, presence_penalty=0.2)
    plist = [wl.identity_params(top_k=k, temperature=0.8, **pen),
             wl.identity_params(top_k=max(1, k // 2), top_p=0.9, temperature=1.3, **pen),
             wl.identity_params(top_k=k, temperature=1.0),
             wl.identity_params(top_k=1, temperature=0.5, **pen)]
    x = xf if dtype == "f32" else wl.to_bf16_bits(xf)
    w = _wl_from(wl, x, plist, rng.random(B), hist=hist, dtype=dtype)
    for align in (None, 8):   # contiguous rows, and rows with a padded 16-byte aligned stride
        g = run_gpu(sampler, w, row_align=align)
        assert compare_rows(w, g) == B


def test_top64_ties_and_zero_signs(sampler, wl, kernel_mode):
    """Tie-heavy rows with every top-k at most 64 (the batch qualifies for
    exact lists): rounded logits, a constant row (every list runs past the
    merge's window), -0 and +0 alternating, a plateau above a constant."""
    rng = np.random.default_rng(10)
    V = 151936
    x = np.round(rng.normal(size=(6, V)) * 2, 1).astype(np.float32)
    x[1] = 0.5
    x[2, ::2] = -0.0
    x[2, 1::2] = 0.0
    x[3] = np.float32(1.0)
    x[3, 1000:1100] = 2.0
    x[5] = np.round(x[5] * 4) / 4
    plist = [wl.identity_params(top_k=k, temperature=t, top_p=p) for k, t, p in
             ((50, 0.7, 1.0), (40, 1.0, 0.9), (10, 1.0, 1.0), (64, 1.3, 0.95), (1, 0.9, 1.0), (7, 0.3, 0.5))]
    w = _wl_from(wl, x, plist, rng.random(6))
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == 6


def test_nan_logits_flagged_and_left_out(sampler, wl, kernel_mode):
    """NaN logits are outside the contract: the row is flagged (bit 8) and its
    NaN ids count as -inf, so the rest of the row samples exactly as the
    oracle does with those ids at -inf. NaNs sit next to the row's largest
    logits (same 16-byte chunk), in a row's ragged end, and fill one row
    except for a few ids."""
    rng = np.random.default_rng(31)
    V = 151936
    x = rng.normal(0, 2, size=(5, V)).astype(np.float32)
    top = np.argsort(-x[0])[:40]
    x[0, top[::3] ^ 1] = np.nan              # neighbours of some top ids
    x[1, V - 3:] = np.nan                     # the ragged end
    x[1, 12345] = np.nan
    x[2, :] = np.nan
    x[2, [7, 70000, 151935]] = [1.0, 2.0, 0.5]
    x[3, ::1000] = np.nan
    plist = [wl.identity_params(top_k=k, temperature=t, top_p=p) for k, t, p in
             ((50, 0.7, 1.0), (40, 1.0, 0.9), (10, 1.0, 1.0), (64, 1.3, 0.95), (20, 0.8, 1.0))]
    w = _wl_from(wl, x, plist, rng.random(5))
    g = run_gpu(sampler, w)
    for r in range(4):
        assert int(g["row_flags"][r]) & 8, f"row {r}: NaN not flagged"
    assert not (int(g["row_flags"][4]) & 8)
    ref = _wl_from(wl, np.where(np.isnan(x), np.float32(-np.inf), x), plist, w.u)
    assert compare_rows(ref, g) == 5


def test_single_token_vocab(sampler, wl):
    x = np.array([[3.0], [-np.inf]], np.float32)
    plist = [wl.identity_params(top_k=5), wl.identity_params(temperature=2.0)]
    w = _wl_from(wl, x, plist, [0.9, 0.1])
    g = run_gpu(sampler, w)
    compare_rows(w, g)


# ---- the C ABI's host-row entry and its errors ----------------------------------

REF_CASES = [
    ([1.0, 5.0, 2.0, 3.0], dict(temperature=0.0), 42, None, None),
    ([1.0, 2.0, 3.0, 4.0], dict(), 7, None, None),
    ([0.5, 0.7, 0.3, 0.9, 0.6, 0.4, 0.8, 0.2], dict(), 123456, None, None),
    ([0.1, 0.4, 0.3, 0.9, 0.2], dict(top_k=1), 1, None, None),
    ([0.1, 2.0, 2.5], dict(temperature=0.0, rep_penalty=2.0, repeat_last_n=8), 1, [2], None),
    ([10.0, -5.0, -6.0, -7.0, -8.0], dict(min_p=0.5), 42, None, None),
    ([10.0, 9.0, 0.0, 0.0, 0.0], dict(top_p=0.5), 5, None, None),
    ([0.1, 0.2, 0.3], dict(temperature=0.0), 1, None, {0: 100.0}),
]


@pytest.mark.parametrize("case", range(len(REF_CASES)))
def test_reference_cases_through_sample_host(sampler, case):
    l, over, seed, recent, bias = REF_CASES[case]
    p = O.identity_params(**over)
    u = O.u_from_seed(seed)
    tok, after = sampler.sample_host(np.array(l, np.float32), p, hist=recent, bias=bias, u=u,
                                     writeback=True)
    tr = O.sample_row(np.array(l, np.float32), p, hist=recent, bias=bias, u=u)
    assert tok == tr.token
    np.testing.assert_array_equal(after.view(np.uint32), tr.logits_after.view(np.uint32))


def test_default_params_sample_host(sampler):
    l = np.array([0.1, 0.5, 0.9, 0.3, 0.7, 0.2, 0.4, 0.6, 0.8, 0.15], np.float32)
    for seed in range(20):
        u = O.u_from_seed(seed)
        tok, after = sampler.sample_host(l, O.default_params(), u=u, writeback=True)
        tr = O.sample_row(l, O.default_params(), u=u)
        assert tok == tr.token
        np.testing.assert_array_equal(after.view(np.uint32), tr.logits_after.view(np.uint32))


def test_run_rejects_invalid_requests(sampler, hs, wl):
    import torch
    w = wl.config(2, seed=1, rows=2)
    x, u, h, m = to_device(w)
    bad = [dict(w.params[0], temperature=float("nan")), w.params[1]]
    with pytest.raises(hs.HsampError) as e:
        sampler.run(x, bad, u, hist=h, hist_len=w.hist_len)
    assert e.value.status == hs.ERR_INVALID
    with pytest.raises(hs.HsampError) as e:
        sampler.run(x, w.params, u, hist=h, hist_len=[5000, 5000])   # longer than the stride
    assert e.value.status == hs.ERR_INVALID
    with pytest.raises(hs.HsampError) as e:
        sampler.run(x, w.params, u, hist=None, hist_len=w.hist_len)
    assert e.value.status == hs.ERR_INVALID
    xb = x.to(torch.bfloat16)
    with pytest.raises(hs.HsampError) as e:
        sampler.run(xb, w.params, u, hist=h, hist_len=w.hist_len, writeback=True)
    assert e.value.status == hs.ERR_UNSUPPORTED
    dup = [{1: 1.0, 2: 2.0}, None]
    b = hs.Batch()
    parr, bids, bvals = hs.make_params(w.params, w.hist_len, dup)
    bids[1] = 1                                                          # duplicate id
    tok = torch.empty(2, dtype=torch.int32, device=x.device)
    b.rows, b.vocab, b.dtype = 2, w.vocab, hs.F32
    b.logits, b.logits_stride = x.data_ptr(), x.stride(0)
    b.hist, b.hist_stride = h.data_ptr(), h.stride(0)
    b.u, b.token = u.data_ptr(), tok.data_ptr()
    b.params = ctypes.cast(parr, ctypes.POINTER(hs.Params))
    b.bias_ids, b.bias_vals = bids.ctypes.data, bvals.ctypes.data
    assert hs.lib().ultima_hsamp_run(sampler.h, ctypes.byref(b), None) == hs.ERR_INVALID
    big = wl.config(2, seed=1, rows=2)
    with pytest.raises(hs.HsampError) as e:
        sampler.run(x, [dict(p, repeat_last_n=40000) for p in big.params], u, hist=torch.zeros(
            (2, 40000), dtype=torch.int32, device=x.device), hist_len=[40000, 40000])
    assert e.value.status == hs.ERR_CAPACITY
    torch.cuda.synchronize()


def test_penalties_below_the_stream_bounds(sampler, hs, wl, kernel_mode):
    """Sampling rows whose histories hold their 1500 highest logits under heavy
    penalties: the true top-k lies far below every slice's survival bound on
    pre-penalty keys. The general merge's bound check fails and it reads each
    row again in full; exact lists resolve the penalised ids in the stream
    (about 1500 per row, all at or above the unpenalised bound) and never read
    a row again."""
    rng = np.random.default_rng(99)
    B, V, H = 4, 40000, 2048
    x = rng.normal(size=(B, V)).astype(np.float32)
    hist = np.empty((B, H), np.int32)
    for r in range(B):
        top = np.argsort(-x[r])[:1500]
        hist[r] = rng.permutation(np.concatenate([top, rng.choice(top, H - 1500)]))
    plist = [wl.identity_params(temperature=0.9, top_k=40, top_p=0.9, rep_penalty=50.0, repeat_last_n=2048,
                                frequency_penalty=2.0, presence_penalty=1.0) for _ in range(B)]
    w = _wl_from(wl, x, plist, rng.random(B))
    w.hist, w.hist_len = hist, np.full(B, H, np.int64)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == B
    if kernel_mode == "general":
        assert np.all(g["row_flags"] & hs.ROW_REREAD)
    else:
        assert not np.any(g["row_flags"] & hs.ROW_REREAD)


def test_penalty_windows_of_different_lengths(sampler, wl, kernel_mode):
    """Exact lists keep a plain count per id when the repetition and the
    frequency/presence windows coincide (or one stage is off) and a count
    plus a repetition bit otherwise. Rows: repetition window shorter than the
    frequency/presence window (DRY off but dry_last_n widening it), equal
    windows, repetition off, frequency/presence off, and a DRY window shorter
    than the repetition window. Histories repeat the rows' top ids so that
    every kind of count reaches the kept set."""
    rng = np.random.default_rng(77)
    B, V, H = 5, 60000, 1024
    x = rng.normal(0, 2, size=(B, V)).astype(np.float32)
    hist = np.empty((B, H), np.int32)
    for r in range(B):
        top = np.argsort(-x[r])[:60]
        hist[r] = rng.permutation(np.concatenate([rng.choice(top, 400), rng.integers(0, V, H - 400)]))
    base = dict(temperature=0.8, top_k=50, top_p=0.95)
    plist = [wl.identity_params(**base, rep_penalty=1.3, repeat_last_n=64, dry_last_n=700,
                                frequency_penalty=0.4, presence_penalty=0.2),
             wl.identity_params(**base, rep_penalty=1.3, repeat_last_n=700, frequency_penalty=0.4,
                                presence_penalty=0.2),
             wl.identity_params(**base, repeat_last_n=300, dry_last_n=300, frequency_penalty=0.7),
             wl.identity_params(**base, rep_penalty=1.5, repeat_last_n=900),
             wl.identity_params(**base, rep_penalty=1.2, repeat_last_n=500, dry_last_n=100,
                                presence_penalty=0.6)]
    w = _wl_from(wl, x, plist, rng.random(B))
    w.hist, w.hist_len = hist, np.full(B, H, np.int64)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == B


def test_greedy_flagged_past_the_window(sampler, wl):
    """Greedy rows whose 2048 penalised ids hold the largest logits of the
    first slice: that slice hands over more flagged ids than the merge's
    window, and the ones past it still take part in the argmax."""
    rng = np.random.default_rng(7)
    B, V, H = 4, 40000, 2048
    x = rng.normal(size=(B, V)).astype(np.float32)
    x[:, :H] += 8.0
    hist = np.stack([rng.permutation(H) for _ in range(B)]).astype(np.int32)
    plist = [wl.identity_params(temperature=0.0, rep_penalty=1.5, repeat_last_n=2048,
                                frequency_penalty=0.3 * (r + 1), presence_penalty=0.5) for r in range(B)]
    w = _wl_from(wl, x, plist, rng.random(B))
    w.hist, w.hist_len = hist, np.full(B, H, np.int64)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == B


@pytest.mark.parametrize("greedy_rows", [0, 6, 12])
def test_long_history_of_top_tokens(sampler, wl, greedy_rows, kernel_mode):
    """2048-id histories drawn mostly from each row's 300 highest logits, ids
    repeated many times over the frequency, presence and repetition windows:
    hundreds of penalised candidates per row reach the merge (flag mode), and
    a batch mixing greedy and sampling rows takes both stream kernels."""
    rng = np.random.default_rng(4242 + greedy_rows)
    B, V, H = 12, 151936, 2048
    x = rng.normal(size=(B, V)).astype(np.float32)
    hist = np.empty((B, H), np.int32)
    for r in range(B):
        top = np.argsort(-x[r])[:300]
        pool = np.concatenate([rng.choice(top, 1600), rng.integers(0, V, 448)])
        hist[r] = rng.permutation(pool)
    plist = []
    for r in range(B):
        if r < greedy_rows:
            plist.append(wl.identity_params(temperature=0.0, rep_penalty=1.1, repeat_last_n=2048,
                                            frequency_penalty=0.5, presence_penalty=0.3))
        else:
            plist.append(wl.identity_params(temperature=0.7, top_k=50, rep_penalty=1.1, repeat_last_n=1024,
                                            frequency_penalty=0.5, presence_penalty=0.3))
    w = _wl_from(wl, x, plist, rng.random(B))
    w.hist, w.hist_len = hist, np.full(B, H, np.int64)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == B


@pytest.mark.parametrize("greedy_rows", [0, 2])
def test_penalised_top_tokens_flag_mode(sampler, wl, greedy_rows):
    """Histories that hold the rows' highest logits, repeated: the penalised ids
    compete for the top-k (and the argmax) after their penalties. All knobs
    only lower logits, so the stream hands penalised ids over as flagged
    candidates and the merge finds their true values."""
    rng = np.random.default_rng(77 + greedy_rows)
    B, V, H = 8, 40000, 600
    x = (rng.normal(size=(B, V)) * 2.5).astype(np.float32)
    hist = np.empty((B, H), np.int32)
    for r in range(B):
        top = np.argsort(-x[r])[:40]
        pool = np.concatenate([top, top[:10], top[:5], rng.integers(0, V, H)])
        hist[r] = rng.permutation(pool)[:H]
    plist = []
    for r in range(B):
        if r < greedy_rows:
            plist.append(wl.identity_params(temperature=0.0, rep_penalty=1.3, repeat_last_n=200,
                                            frequency_penalty=0.4, presence_penalty=0.2))
        else:
            plist.append(wl.identity_params(temperature=0.8, top_k=50, top_p=0.95, rep_penalty=1.3,
                                            repeat_last_n=200, frequency_penalty=0.4, presence_penalty=0.2,
                                            dry_multiplier=0.8, dry_base=1.75, dry_allowed_len=2,
                                            dry_last_n=H))
    w = _wl_from(wl, x, plist, rng.random(B))
    w.hist, w.hist_len = hist, np.full(B, H, np.int64)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == B


# ---- handle scratch limits and graph capture ----------------------------------

def test_slice_override_beyond_the_handle_is_refused(hs, wl, monkeypatch):
    """ULTIMA_HSAMP_SLICES (diagnostics) may ask for more slices than the
    handle's per-slice counters hold (rows x slices > max(4104, max_rows)):
    the run is refused before any kernel is launched."""
    import torch
    # (the overrides are read when a handle is created)
    monkeypatch.setenv("ULTIMA_HSAMP_SLICES", "256")
    s = hs.Sampler(0, max_rows=64, max_vocab=151936)
    monkeypatch.delenv("ULTIMA_HSAMP_SLICES")
    s2 = hs.Sampler(0, max_rows=64, max_vocab=151936)
    try:
        w = wl.config(2, seed=1)
        x, u, h, m = to_device(w)
        with pytest.raises(hs.HsampError) as e:
            s.run(x, w.params, u, hist=h, hist_len=w.hist_len)
        assert e.value.status == hs.ERR_CAPACITY
        g = s2.run(x, w.params, u, hist=h, hist_len=w.hist_len)
        torch.cuda.synchronize()
        want = [O.sample_row(w.logits[r], w.params[r], hist=w.hist[r], u=float(w.u[r])).token for r in range(4)]
        assert list(g["token"][:4].cpu().numpy()) == want
    finally:
        s.close()
        s2.close()


def test_graph_replay_after_scratch_grows(hs, wl):
    """A graph captured from a handle keeps the scratch it was captured with:
    a later, larger batch grows the handle's scratch (the old areas are kept
    until destroy), and replaying the first graph still gives its tokens."""
    import torch
    s = hs.Sampler(0, max_rows=256, max_vocab=151936)
    try:
        small = wl.config(2, seed=21, rows=8)
        x, u, h, m = to_device(small)
        out = {"token": torch.empty(8, dtype=torch.int32, device=x.device),
               "row_flags": torch.empty(8, dtype=torch.int32, device=x.device)}
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            s.run(x, small.params, u, hist=h, hist_len=small.hist_len, outputs=out, stream=stream)
        stream.synchronize()
        want = out["token"].clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            s.run(x, small.params, u, hist=h, hist_len=small.hist_len, outputs=out, stream=stream)
        stream.synchronize()
        # a larger batch, uncaptured: more candidate and overflow scratch
        big = wl.config(5, seed=3, rows=256)
        xb, ub, hb, mb = to_device(big)
        gb = s.run(xb, big.params, ub, hist=hb, hist_len=big.hist_len)
        torch.cuda.synchronize()
        for r in (0, 100, 255):
            tr = O.sample_row(big.logits_f32()[r], big.params[r], hist=big.hist[r][: int(big.hist_len[r])],
                              u=float(big.u[r]))
            assert int(gb["token"][r]) == tr.token or tr.cdf_margin <= 1e-6
        for _ in range(3):
            out["token"].fill_(-7)
            with torch.cuda.stream(stream):
                graph.replay()
            stream.synchronize()
            assert torch.equal(out["token"], want)
        del graph
    finally:
        s.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("kmix", [40, 300])
def test_greedy_rows_with_sampling_rows(sampler, wl, kernel_mode, dtype, kmix):
    """Greedy rows (argmax, sampler.cpp:220-228) batched with sampling rows of
    top-k <= 64 (k_pick) or above (k_pick_l), exact lists or general kernels:
    NaN at id 0 (id 0 wins), NaN elsewhere (left out), a maximum of zero held
    as -0 at a lower id than +0 (the lower id wins), a row of -inf but one
    NaN past id 0 (id 0), penalised top ids, a mask that leaves out id 0's NaN."""
    rng = np.random.default_rng(61 + kmix)
    B, V = 8, 151936
    x = rng.normal(size=(B, V)).astype(np.float32) * 2
    x[0, 0] = np.nan
    x[1, 5000] = np.nan
    x[1, 77] = 40.0
    x[2, :] = -5.0
    x[2, 3] = -0.0
    x[2, 9000] = 0.0
    x[3, :] = -np.inf
    x[3, 1234] = np.nan
    mask_rows = np.ones((B, (V + 31) // 32), np.uint32) * np.uint32(0xFFFFFFFF)
    x[4, 0] = np.nan
    mask_rows[4, 0] &= np.uint32(0xFFFFFFFE)             # id 0 (NaN) not allowed
    hist = rng.integers(0, V, size=(B, 256)).astype(np.int32)
    top5 = np.argsort(-x[5])[:40]
    hist[5, -40:] = top5
    plist = [wl.identity_params(temperature=0.0),
             wl.identity_params(temperature=0.0, rep_penalty=1.2, repeat_last_n=64),
             wl.identity_params(temperature=0.0),
             wl.identity_params(temperature=-1.0),
             wl.identity_params(temperature=0.0),
             wl.identity_params(temperature=0.0, rep_penalty=3.0, repeat_last_n=64, frequency_penalty=0.5,
                                presence_penalty=0.5),
             wl.identity_params(top_k=kmix, temperature=0.8, top_p=0.9),
             wl.default_params(top_k=kmix)]
    xs = x if dtype == "f32" else wl.to_bf16_bits(x)
    w = wl.Workload("edge", dtype, xs, plist, rng.random(B), hist, np.full(B, 256, np.int64), mask_rows)
    g = run_gpu(sampler, w)
    assert compare_rows(w, g) == B
    tok = g["token"]
    assert tok[0] == 0 and tok[3] == 0 and tok[2] == 3 and tok[1] == 77 and tok[4] != 0


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("kmix", [40, 300])
@pytest.mark.parametrize("signs", ["lowering", "mixed"])
def test_bias_with_penalties(sampler, wl, kernel_mode, dtype, kmix, signs):
    """Logit bias (bans at -inf, negative values on the top tokens, zeros;
    with "mixed" also boosts that lift ids from far below the slices' bounds
    to the top, among them the ragged end and id 0; up to 256 entries a row)
    beside repetition, DRY and frequency/presence penalties: the exact lists
    evaluate the bias ids on their own with every stage (sampler.cpp:28-34)."""
    rng = np.random.default_rng(91 + kmix + (7 if signs == "mixed" else 0))
    B, V = 6, 151936
    x = rng.normal(size=(B, V)).astype(np.float32) * 2
    hist = rng.integers(0, V, size=(B, 512)).astype(np.int32)
    bias = []
    for r in range(B):
        top = np.argsort(-x[r])[:300]
        b = {int(t): float("-inf") for t in top[:20]}                       # bans
        b.update({int(t): float(-rng.uniform(0.1, 4.0)) for t in top[20:120]})
        b.update({int(t): 0.0 for t in rng.choice(V, 30, replace=False)})
        b.update({int(t): -1.5 for t in (0, V - 1, V - 2)})                # edges, the ragged end
        if signs == "mixed":
            low = np.argsort(x[r])[:5000]
            b.update({int(t): float(rng.uniform(8.0, 20.0)) for t in rng.choice(low, 40, replace=False)})
            b.update({int(t): float(rng.uniform(0.5, 3.0)) for t in top[150:200]})
            b.update({int(t): 25.0 for t in (0, V - 1)} if r % 2 else {})
        bias.append(dict(list(b.items())[-256:]))
        hist[r, -60:] = top[100:160]
    bias[3] = None
    plist = [wl.identity_params(top_k=kmix, temperature=0.7),
             wl.default_params(top_k=kmix),
             wl.identity_params(top_k=kmix, temperature=1.2, top_p=0.9, rep_penalty=1.3, repeat_last_n=256,
                                frequency_penalty=0.3, presence_penalty=0.2),
             wl.identity_params(top_k=kmix, temperature=0.9),
             wl.identity_params(temperature=0.0, rep_penalty=1.2, repeat_last_n=64),
             wl.default_params(top_k=kmix, dry_last_n=512, repeat_last_n=512, frequency_penalty=0.1)]
    xs = x if dtype == "f32" else wl.to_bf16_bits(x)
    w = wl.Workload("edge", dtype, xs, plist, rng.random(B), hist, np.full(B, 512, np.int64), None)
    g = run_gpu(sampler, w, bias=bias)
    assert compare_rows(w, g, bias=bias) == B


@pytest.mark.parametrize("cfg", [2, 5])
def test_one_history_shared_by_every_row(sampler, wl, cfg, kernel_mode):
    """hist_stride 0: every row reads the same history array, row r its first
    hist_len[r] ids (a drafted block's positions over the sequence's ids and
    drafts); each row equal to the oracle with that prefix as its history."""
    import torch
    w = wl.config(cfg, seed=7, rows=24)
    rng = np.random.default_rng(cfg)
    L = w.hist.shape[1]
    w.hist = np.tile(w.hist[0], (w.hist.shape[0], 1))
    w.hist_len = rng.integers(0, L + 1, w.hist.shape[0]).astype(np.int64)
    w.hist_len[:2] = (0, L)
    x, u, h, m = to_device(w)
    shared = h[0].contiguous().unsqueeze(0).expand(h.shape[0], L)
    assert shared.stride(0) == 0
    out = sampler.run(x, w.params, u, hist=shared, hist_len=w.hist_len, mask=m, want_sets=True, set_cap=2048)
    torch.cuda.synchronize()
    g = {k: v.cpu().numpy() for k, v in out.items()}
    assert compare_rows(w, g) == w.hist.shape[0]
