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


def test_noalloc_graph_keeps_its_knobs_after_other_calls(hs, wl):
    """A graph captured through the no-alloc entry replays with the knobs it was
    captured with, after eager no-alloc calls with other knobs on the same GPU
    (among them rows over the whole vocabulary, which the captured batch has
    none of); capturing knobs that no uncaptured call used first is refused."""
    import torch
    s = hs.Sampler(0, max_rows=256, max_vocab=151936)
    stream = torch.cuda.Stream()
    try:
        wa = wl.config(2, seed=51, rows=8)
        wb = wl.config(3, seed=52, rows=4)           # top-p over the whole vocabulary
        ref_a, _ = _both(hs, s, wa)
        ref_b, _ = _both(hs, s, wb)
        xa, ua, ha, ma = to_device(wa)
        xb, ub, hb, mb = to_device(wb)
        out_a = None
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            out_a = hs.run_noalloc(xa, wa.params, ua, hist=ha, hist_len=wa.hist_len, mask=ma, want_sets=True,
                                   set_cap=SET_CAP, stream=stream)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            hs.run_noalloc(xa, wa.params, ua, hist=ha, hist_len=wa.hist_len, mask=ma, want_sets=True,
                           set_cap=SET_CAP, stream=stream, outputs=out_a)
        stream.synchronize()
        for v in out_a.values():
            v.zero_()
        for rep in range(3):
            # another batch with other knobs, eagerly, then the graph again
            got_b = hs.run_noalloc(xb, wb.params, ub, hist=hb, hist_len=wb.hist_len, mask=mb, want_sets=True,
                                   set_cap=SET_CAP)
            torch.cuda.synchronize()
            _same(ref_b, {k: v.cpu().numpy() for k, v in got_b.items()}, wb.rows)
            g.replay()
            torch.cuda.synchronize()
            _same(ref_a, {k: v.cpu().numpy() for k, v in out_a.items()}, wa.rows)
            for v in out_a.values():
                v.zero_()
        # knobs no uncaptured call used: refused under capture, nothing recorded
        wc = wl.config(2, seed=53, rows=8)
        wc.params[0]["temperature"] = 0.55
        xc, uc, hc, mc = to_device(wc)
        g2 = torch.cuda.CUDAGraph()
        status = None
        with torch.cuda.graph(g2, stream=stream):
            try:
                hs.run_noalloc(xc, wc.params, uc, hist=hc, hist_len=wc.hist_len, mask=mc, stream=stream)
            except hs.HsampError as e:
                status = e.status
        stream.synchronize()
        assert status == hs.ERR_UNSUPPORTED
        del g2
    finally:
        s.close()
