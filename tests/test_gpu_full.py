"""Rows over the whole vocabulary (top-k off or above 1024): the k_full path.

Every row is compared with the CPU oracle (tests/gpu_helpers.compare_rows):
token, top-k set, kept set and probabilities bit for bit, row flags. The
kept sets are large, so the set outputs are sized to V.
"""
import numpy as np
import pytest

from gpu_helpers import compare_rows, run_gpu

pytestmark = pytest.mark.gpu


def _wl(wl, V, rows, params, seed=3, sigma=2.0, dtype="f32", hist_len=0, mask=None):
    x = wl._rows_normal(seed, rows, V, sigma)
    hist = hl = None
    if hist_len:
        hist = (wl.splitmix64(seed * 7 + 1, rows * hist_len) % np.uint64(V)).astype(np.int32).reshape(rows, hist_len)
        hl = np.full(rows, hist_len, np.int64)
    logits = x if dtype == "f32" else wl.to_bf16_bits(x)
    return wl.Workload("full", dtype, logits, [dict(p) for p in params], wl.uniform53(seed + 9, rows),
                       hist, hl, mask)


def test_config3_spike_and_flat_rows(sampler, wl):
    """BASELINE config 3 at its size, B = 256: 128 rows N(0, 1) with 16 spike
    ids at +15 (exact ties, a nucleus of the 16), 128 near-flat rows N(0, 0.1)
    (a nucleus of about 1e5 ids), top-p 0.9 over the full vocabulary. Every
    row is compared with the oracle: token, kept set and probabilities."""
    w = wl.config(3, seed=5)
    assert w.rows == 256
    g = run_gpu(sampler, w, set_cap=w.vocab)
    assert compare_rows(w, g) == 256


@pytest.mark.parametrize("knobs", [
    dict(temperature=1.0),                                   # identity(): plain draw over V
    dict(temperature=0.8, top_p=0.95),
    dict(temperature=1.3, min_p=0.05),
    dict(temperature=0.7, top_p=0.9, min_p=0.02),
    dict(temperature=0.9, top_k=1500, top_p=0.97),            # k above the top-k path's limit
    dict(temperature=0.9, top_k=3000),
])
def test_full_vocab_knobs(sampler, wl, knobs):
    V, rows = 20011, 6
    p = wl.identity_params(**knobs)
    w = _wl(wl, V, rows, [p] * rows)
    g = run_gpu(sampler, w, set_cap=V)
    assert compare_rows(w, g) == rows


def test_full_vocab_with_penalties_and_bf16(sampler, wl):
    V, rows = 30000, 4
    p = wl.identity_params(temperature=0.8, top_p=0.9, rep_penalty=1.15, repeat_last_n=256,
                           frequency_penalty=0.4, presence_penalty=0.2)
    for dtype in ("f32", "bf16"):
        w = _wl(wl, V, rows, [p] * rows, dtype=dtype, hist_len=300)
        g = run_gpu(sampler, w, set_cap=V)
        assert compare_rows(w, g) == rows


def test_full_vocab_mixed_with_topk_and_greedy_rows(sampler, wl):
    V, rows = 12000, 6
    plist = [wl.identity_params(temperature=1.0, top_p=0.9),
             wl.identity_params(temperature=0.7, top_k=40),
             wl.identity_params(temperature=0.0),
             wl.identity_params(temperature=1.2),
             wl.identity_params(temperature=0.9, top_k=2048, min_p=0.01),
             wl.identity_params(temperature=0.6, top_k=8, top_p=0.8)]
    w = _wl(wl, V, rows, plist, seed=8)
    g = run_gpu(sampler, w, set_cap=V)
    assert compare_rows(w, g) == rows


@pytest.mark.parametrize("pen", [True, False])
def test_full_vocab_writeback(sampler, wl, pen):
    V, rows = 9000, 3
    if pen:
        p = wl.identity_params(temperature=0.75, top_p=0.8, rep_penalty=1.2, repeat_last_n=64)
    else:   # a plain transform: the many-block passes ahead of k_full
        p = wl.identity_params(temperature=0.75, top_p=0.8)
    w = _wl(wl, V, rows, [p] * rows, hist_len=64)
    g = run_gpu(sampler, w, writeback=True, set_cap=V)
    assert compare_rows(w, g, writeback=True) == rows


def test_full_vocab_all_masked_row_draws_uniformly(sampler, wl):
    V, rows = 4096, 2
    mask = np.zeros((rows, V // 32), np.uint32)
    mask[1, 5] = 1 << 3          # row 1: one allowed id
    p = wl.identity_params(temperature=1.0, top_p=0.9)
    w = _wl(wl, V, rows, [p] * rows, mask=mask)
    g = run_gpu(sampler, w, set_cap=V)
    assert compare_rows(w, g) == rows
    assert int(g["row_flags"][0]) & 16          # nothing finite: uniform over V


@pytest.mark.parametrize("rows,dtype", [(1, "f32"), (3, "f32"), (2, "bf16")])
def test_cli_identity_rows_at_full_vocab(hs, sampler, wl, rows, dtype):
    """The CLI's call (SamplerParams::identity() + temperature,
    apps/ultima-cli/main.cpp:661-674) at V = 151936: its whole-row passes run
    over many blocks (k_fs_*) ahead of k_full; in the bf16 case with a masked
    row."""
    import torch
    V = 151936
    p = wl.identity_params(temperature=0.8)
    mask = None
    if dtype == "bf16":
        mask = np.full((rows, V // 32), 0xFFFFFFFF, np.uint32)
        mask[1, ::3] = 0x0F0F0F0F
    w = _wl(wl, V, rows, [p] * rows, seed=31 + rows, dtype=dtype, mask=mask)
    from gpu_helpers import to_device
    x, u, h, m = to_device(w)
    k = sampler.query_kernels(x, w.params, u, mask=m)
    assert k & hs.KERNELS_FULL
    g = run_gpu(sampler, w, set_cap=V)
    assert compare_rows(w, g) == rows


def test_cli_row_with_nan_logits_is_flagged(hs, sampler, wl):
    """NaN logits in a whole-vocabulary row count as -inf and flag the row
    (the reference's softmax would turn every probability into NaN): the
    token is one of the finite ids, drawn as if the NaN ids were masked."""
    V = 151936
    p = wl.identity_params(temperature=0.8)
    w = _wl(wl, V, 1, [p], seed=41)
    w.logits[0, 5::1000] = np.nan
    g = run_gpu(sampler, w, set_cap=V)
    assert int(g["row_flags"][0]) & hs.ROW_NAN
    assert not np.isnan(w.logits[0, int(g["token"][0])])
    masked = w.logits.copy()
    masked[0, 5::1000] = -np.inf
    wm = _wl(wl, V, 1, [p], seed=41)
    wm.logits[:] = masked
    gm = run_gpu(sampler, wm, set_cap=V)
    assert int(g["token"][0]) == int(gm["token"][0])
    assert int(g["kept_count"][0]) == int(gm["kept_count"][0]) == V - 152


@pytest.mark.parametrize("V", [32000, 151936, 262144])
def test_plain_transform_rows_exact_sums(hs, sampler, wl, V):
    """Rows that take the whole-row passes over many blocks (plain transform:
    temperature and mask only) with sums that leave their binade in different
    places: flat rows (the sum doubles window after window), wide rows (a few
    ids carry it), a constant row (the sum lands on powers of two exactly at
    window ends), rows with long masked-out ranges (empty windows) and a row
    of one allowed id per 4096. The kept probabilities are e * fl(1/S) for
    every id, so they pin the exact index-order sum S bit for bit."""
    rows = 6
    sig = [0.3, 2.0, 8.0, 0.0, 1.0, 3.0]
    x = wl._rows_normal(77, rows, V, sig)
    x[3] = 0.5                                  # constant row
    temps = [1.0, 0.8, 1.7, 1.0, 0.6, 1.1]
    params = [wl.identity_params(temperature=t) for t in temps]
    mask = np.full((rows, (V + 31) // 32), 0xFFFFFFFF, np.uint32)
    lo, hi = V // 10 // 32, V // 2 // 32
    mask[4, lo:hi] = 0                          # a long masked-out range
    mask[5, :] = 0
    mask[5, ::128] = 1                          # one id per 4096
    w = wl.Workload("full", "f32", x, params, wl.uniform53(78, rows), None, None, mask)
    g = run_gpu(sampler, w, set_cap=V)
    assert compare_rows(w, g) == rows


def test_full_vocab_draw_without_sets(sampler, wl):
    """With no kept set asked for, rows whose top-p or min-p removed ids take
    the draw's window sums from the numerators alone and their kept count from
    the stages' own counts: token, row flags and kept count must equal those of
    the run that writes the sets (checked against the oracle). Rows: cfg3's
    spike rows (the cut splits ids of equal p at the top) and flat rows, top-p
    and min-p knobs, and min_p 2 (every id removed: the uniform draw)."""
    import torch
    V = 151936
    w3 = wl.config(3, seed=11, rows=4)
    knobs = [dict(temperature=0.8, top_p=0.5), dict(temperature=1.2, min_p=0.05),
             dict(temperature=0.7, top_p=0.95, min_p=0.02), dict(temperature=1.5, min_p=2.0)]
    wk = _wl(wl, V, len(knobs), [wl.identity_params(**k) for k in knobs], seed=19)
    for w in (w3, wk):
        g = run_gpu(sampler, w, set_cap=V)
        assert compare_rows(w, g) == w.rows
        from gpu_helpers import to_device
        x, u, h, m = to_device(w)
        out = {"kept_count": torch.empty(w.rows, dtype=torch.int32, device=x.device)}
        o = sampler.run(x, w.params, u, hist=h, hist_len=w.hist_len, mask=m, outputs=out)
        torch.cuda.synchronize()
        for k in ("token", "row_flags", "kept_count"):
            assert np.array_equal(o[k].cpu().numpy(), g[k]), (w.name, k)
