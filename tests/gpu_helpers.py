"""Helpers for the GPU parity tests: run a workload through the C ABI and
through the CPU oracle, and compare what each leaves behind."""
from __future__ import annotations

import numpy as np

import oracle as O


def to_device(wl):
    import torch
    dev = torch.device("cuda:0")
    if wl.dtype == "f32":
        x = torch.from_numpy(np.ascontiguousarray(wl.logits)).to(dev)
    else:
        x = torch.from_numpy(np.ascontiguousarray(wl.logits).view(np.int16)).to(dev).view(torch.bfloat16)
    u = torch.from_numpy(np.ascontiguousarray(wl.u, dtype=np.float64)).to(dev)
    h = None if wl.hist is None else torch.from_numpy(np.ascontiguousarray(wl.hist)).to(dev)
    m = None if wl.mask is None else torch.from_numpy(np.ascontiguousarray(wl.mask).view(np.int32)).to(dev)
    return x, u, h, m


def run_gpu(sampler, wl, bias=None, writeback=False, set_cap=2048, row_align=None):
    """row_align: place the rows in a buffer whose row stride is V rounded up
    to this many elements (a padded, 16-byte aligned stride when V is not a
    multiple of the load width)."""
    import torch
    x, u, h, m = to_device(wl)
    if row_align:
        V = x.shape[1]
        xp = torch.zeros((x.shape[0], (V + row_align - 1) // row_align * row_align), dtype=x.dtype, device=x.device)
        xp[:, :V] = x
        x = xp[:, :V]
    out = sampler.run(x, wl.params, u, hist=h, hist_len=wl.hist_len, mask=m, bias=bias,
                      writeback=writeback, want_sets=True, set_cap=set_cap)
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy() for k, v in out.items()}
    if writeback:
        res["logits_after"] = x.cpu().numpy()
    return res


def run_oracle(wl, r, bias=None, cap=None):
    x = wl.logits_f32()[r]
    return O.sample_row(x, wl.params[r], hist=None if wl.hist is None else wl.hist[r][: int(wl.hist_len[r])],
                        mask=None if wl.mask is None else wl.mask[r],
                        bias=None if bias is None else bias[r], u=float(wl.u[r]), cap=cap)


def compare_rows(wl, g, rows=None, bias=None, writeback=False, exact_probs=True, strict_token=False):
    """Assert GPU == oracle on each row; returns the number of rows checked.

    The top-k set, the kept set and its probabilities are fixed before the
    draw, so they are compared on every row. The token may differ only where
    u lies within 1e-6 of a CDF boundary (flagged CDF_NEAR by the GPU); with
    strict_token even that is an error (the finalize then has to replay the
    reference's sequential sums exactly)."""
    rows = range(wl.rows) if rows is None else rows
    n = 0
    for r in rows:
        tr = run_oracle(wl, r, bias=bias)
        ctx = f"row {r} of {wl.name}"
        flags = int(g["row_flags"][r])
        if tr.topk_idx is not None:
            cnt = int(g["topk_count"][r])
            assert cnt == tr.topk_idx.size, f"{ctx}: top-k count {cnt} != {tr.topk_idx.size}"
            np.testing.assert_array_equal(g["topk_idx"][r][:cnt], tr.topk_idx, err_msg=ctx)
        kc = int(g["kept_count"][r])
        assert kc == tr.kept_idx.size, f"{ctx}: kept {kc} != {tr.kept_idx.size}"
        np.testing.assert_array_equal(g["kept_idx"][r][:kc], tr.kept_idx, err_msg=ctx)
        gp, op = g["kept_prob"][r][:kc], tr.kept_prob
        # contract: 1e-6 relative; this build reproduces glibc expf, so bits match
        np.testing.assert_allclose(gp, op, rtol=1e-6, atol=0, err_msg=ctx)
        if exact_probs:
            np.testing.assert_array_equal(gp.view(np.uint32), op.view(np.uint32), err_msg=ctx)
        assert bool(flags & 1) == tr.greedy, ctx
        assert bool(flags & 2) == tr.u_consumed, ctx
        if int(g["token"][r]) != tr.token:
            # the one tolerated mismatch: u within 1e-6 of a CDF boundary, flagged by the GPU
            assert not strict_token, f"{ctx}: token {g['token'][r]} != oracle {tr.token} (strict)"
            assert (flags & 4) and tr.cdf_margin <= 1e-6, \
                f"{ctx}: token {g['token'][r]} != oracle {tr.token} (cdf margin {tr.cdf_margin})"
        if writeback:
            np.testing.assert_array_equal(g["logits_after"][r][: wl.vocab].view(np.uint32),
                                          tr.logits_after.view(np.uint32), err_msg=ctx)
        n += 1
    return n
