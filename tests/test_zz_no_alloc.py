"""ultima_hsamp_run_noalloc: the handle-free, allocation-free entry point
against ultima_hsamp_run on the same batches.

The no-alloc entry takes its scratch from the library's fixed device array
(ULTIMA_HSAMP_NOALLOC_SCRATCH_BYTES per GPU); its results must equal the
handle path's bit for bit (token, flags, top-k set, kept set and
probabilities). Two calls in a row, the second with a smaller batch, show
that what the first call left in the shared array does not leak into the
second; a batch whose scratch does not fit is refused before any launch.
"""
import numpy as np
import pytest

from gpu_helpers import to_device

pytestmark = pytest.mark.gpu

SET_CAP = 1024


def _both(hs, sampler, w):
    import torch
    x, u, h, m = to_device(w)
    ref = sampler.run(x, w.params, u, hist=h, hist_len=w.hist_len, mask=m, want_sets=True, set_cap=SET_CAP)
    torch.cuda.synchronize()
    ref = {k: v.cpu().numpy() for k, v in ref.items()}
    got = hs.run_noalloc(x, w.params, u, hist=h, hist_len=w.hist_len, mask=m, want_sets=True, set_cap=SET_CAP)
    torch.cuda.synchronize()
    got = {k: v.cpu().numpy() for k, v in got.items()}
    return ref, got


def _same(ref, got, B):
    np.testing.assert_array_equal(got["token"], ref["token"])
    np.testing.assert_array_equal(got["row_flags"], ref["row_flags"])
    np.testing.assert_array_equal(got["topk_count"], ref["topk_count"])
    np.testing.assert_array_equal(got["kept_count"], ref["kept_count"])
    for r in range(B):
        n = int(ref["topk_count"][r])
        if n > 0:
            np.testing.assert_array_equal(got["topk_idx"][r][:n], ref["topk_idx"][r][:n])
        n = min(int(ref["kept_count"][r]), SET_CAP)
        np.testing.assert_array_equal(got["kept_idx"][r][:n], ref["kept_idx"][r][:n])
        np.testing.assert_array_equal(got["kept_prob"][r][:n].view(np.uint32), ref["kept_prob"][r][:n].view(np.uint32))


def test_noalloc_matches_run_on_two_calls(hs, wl):
    s = hs.Sampler(0, max_rows=256, max_vocab=151936)
    try:
        # the headline batch, then a smaller one with other kernels (bf16,
        # allowed-token mask), then a small mixed batch (greedy rows, k up to
        # 1000: the general kernels), then the first batch again
        cases = [wl.config(2, seed=41), wl.config(4, seed=42, rows=16), wl.config(5, seed=43, rows=24),
                 wl.config(2, seed=41)]
        for w in cases:
            ref, got = _both(hs, s, w)
            _same(ref, got, w.rows)
    finally:
        s.close()


def test_noalloc_refuses_batches_beyond_its_array(hs, wl):
    import torch
    w = wl.config(4, seed=44)          # 128 bf16 rows: candidate lists alone exceed the array
    x, u, h, m = to_device(w)
    with pytest.raises(hs.HsampError) as e:
        hs.run_noalloc(x, w.params, u, hist=h, hist_len=w.hist_len, mask=m)
    assert e.value.status == hs.ERR_CAPACITY
    torch.cuda.synchronize()
