"""Device-side history (ultima_hsamp_history_push, batch.hist_len_dev): the
recent-token window kept on the GPU and appended with each step's sampled
token, against the reference's SamplerContext, whose recent_ grows without
bound and whose penalties slice its last repeat_last_n / dry_last_n ids
(reference src/sampler/sampler.cpp:213-217, 16-99). Bar: every step's token
equal to the oracle's on the full host-side history (a u within 1e-6 of a
CDF boundary aside, flagged by the GPU), including steps after the rows
were compacted, and when the step (sample + push) is replayed from a
captured graph."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

ROW_CDF_NEAR = 1


def test_push_appends_and_compacts(hs):
    import torch
    dev = torch.device("cuda:0")
    stride, keep = 8, 4
    model = [[], [100, 101, 102, 103, 104], list(range(200, 208))]
    hist = torch.full((3, stride), -7, dtype=torch.int32, device=dev)
    for r, row in enumerate(model):
        if row:
            hist[r, :len(row)] = torch.tensor(row, dtype=torch.int32)
    lens = torch.tensor([len(m) for m in model], dtype=torch.int32, device=dev)
    for step in range(13):
        tok = [1000 * step + r for r in range(3)]
        hs.history_push(hist, lens, torch.tensor(tok, dtype=torch.int32, device=dev), keep)
        for r in range(3):
            if len(model[r]) >= stride:
                model[r] = model[r][-keep:]
            model[r].append(tok[r])
        torch.cuda.synchronize()
        got_len = lens.cpu().numpy()
        got = hist.cpu().numpy()
        for r in range(3):
            assert got_len[r] == len(model[r]), (step, r)
            np.testing.assert_array_equal(got[r, :len(model[r])], model[r])


def _knobs(kind):
    if kind == "penalties":   # the exact-list kernels take these rows
        return O.identity_params(temperature=0.9, top_k=40, rep_penalty=1.3, repeat_last_n=48,
                                 frequency_penalty=0.4, presence_penalty=0.5)
    return O.default_params(temperature=1.1, top_k=80, top_p=0.95, rep_penalty=1.2, repeat_last_n=48,
                            dry_multiplier=0.8, dry_base=1.75, dry_allowed_len=2, dry_last_n=32,
                            frequency_penalty=0.2, presence_penalty=0.1)


def _step_inputs(rng, base):
    """Logits near a fixed per-row profile (the same ids stay on top, so the
    penalties decide among them) and a fresh u per row."""
    x = (base + rng.normal(0.0, 0.35, base.shape)).astype(np.float32)
    u = rng.random(base.shape[0])
    return x, u


def _check_token(g_tok, g_flags, x, p, host_hist, u, where):
    t = O.sample_row(x, p, hist=np.asarray(host_hist, np.int32), u=float(u))
    if g_tok != t.token:
        assert (g_flags & ROW_CDF_NEAR) and t.cdf_margin <= 1e-6, f"{where}: gpu {g_tok} oracle {t.token}"


@pytest.mark.parametrize("kind", ["penalties", "dry"])
def test_decode_loop_with_device_history(hs, sampler, kernel_mode, kind):
    import torch
    dev = torch.device("cuda:0")
    B, V, W = 4, 4096, 48
    stride, keep = 2 * W, W
    rng = np.random.default_rng(11 if kind == "penalties" else 12)
    base = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    p = _knobs(kind)
    params = [dict(p) for _ in range(B)]
    hist = torch.zeros((B, stride), dtype=torch.int32, device=dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    host = [[] for _ in range(B)]
    x_d = torch.empty((B, V), dtype=torch.float32, device=dev)
    u_d = torch.empty(B, dtype=torch.float64, device=dev)
    out = None
    for step in range(2 * stride + 10):          # two compactions
        x, u = _step_inputs(rng, base)
        x_d.copy_(torch.from_numpy(x))
        u_d.copy_(torch.from_numpy(u))
        # the plan's length: the exact one while filling, then the window
        hl = [min(len(h), W) for h in host]
        out = sampler.run(x_d, params, u_d, hist=hist, hist_len=hl, hist_len_dev=lens, outputs=out)
        hs.history_push(hist, lens, out["token"], keep)
        torch.cuda.synchronize()
        tok = out["token"].cpu().numpy()
        fl = out["row_flags"].cpu().numpy()
        for r in range(B):
            _check_token(int(tok[r]), int(fl[r]), x[r], p, host[r], u[r], f"step {step} row {r}")
            host[r].append(int(tok[r]))
    got_len = lens.cpu().numpy()
    got = hist.cpu().numpy()
    for r in range(B):
        n = int(got_len[r])
        assert keep < n <= stride
        np.testing.assert_array_equal(got[r, :n], host[r][-n:])


def test_captured_step_with_device_history(hs, sampler):
    """Sample + push captured once in the steady state (the plan no longer
    changes), replayed with new logits and uniforms written into the captured
    buffers between replays; every replay checked against the oracle."""
    import torch
    dev = torch.device("cuda:0")
    B, V, W = 8, 8192, 48
    stride, keep = 2 * W, W
    rng = np.random.default_rng(13)
    base = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    p = _knobs("penalties")
    params = [dict(p) for _ in range(B)]
    hist = torch.zeros((B, stride), dtype=torch.int32, device=dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    host = [[] for _ in range(B)]
    x_d = torch.empty((B, V), dtype=torch.float32, device=dev)
    u_d = torch.empty(B, dtype=torch.float64, device=dev)
    out = None
    stream = torch.cuda.Stream(dev)

    def eager_step(hl):
        nonlocal out
        x, u = _step_inputs(rng, base)
        x_d.copy_(torch.from_numpy(x))
        u_d.copy_(torch.from_numpy(u))
        with torch.cuda.stream(stream):
            out = sampler.run(x_d, params, u_d, hist=hist, hist_len=hl, hist_len_dev=lens, outputs=out,
                              stream=stream)
            hs.history_push(hist, lens, out["token"], keep, stream=stream)
        stream.synchronize()
        tok, fl = out["token"].cpu().numpy(), out["row_flags"].cpu().numpy()
        for r in range(B):
            _check_token(int(tok[r]), int(fl[r]), x[r], p, host[r], u[r], f"eager row {r}")
            host[r].append(int(tok[r]))

    while min(len(h) for h in host) < W + 2:    # fill, then one steady step uncaptured
        eager_step([min(len(h), W) for h in host])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        sampler.run(x_d, params, u_d, hist=hist, hist_len=[W] * B, hist_len_dev=lens, outputs=out,
                    stream=stream)
        hs.history_push(hist, lens, out["token"], keep, stream=stream)
    stream.synchronize()
    # the capture ran nothing: lengths and histories are as the eager steps left them
    np.testing.assert_array_equal(lens.cpu().numpy(), [min(len(h), stride) for h in host])
    for step in range(stride + 5):               # through a compaction
        x, u = _step_inputs(rng, base)
        x_d.copy_(torch.from_numpy(x))
        u_d.copy_(torch.from_numpy(u))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        tok, fl = out["token"].cpu().numpy(), out["row_flags"].cpu().numpy()
        for r in range(B):
            _check_token(int(tok[r]), int(fl[r]), x[r], p, host[r], u[r], f"replay {step} row {r}")
            host[r].append(int(tok[r]))
    got_len = lens.cpu().numpy()
    got = hist.cpu().numpy()
    for r in range(B):
        n = int(got_len[r])
        np.testing.assert_array_equal(got[r, :n], host[r][-n:])


def test_graph_from_the_first_token(hs, sampler, kernel_mode):
    """One decode step (sample + push) captured right after the first step of a
    10-id prompt, with the server's defaults (SamplerParams{}: DRY over 512
    ids, repetition over 64, min_p .05), then replayed 600 times: the windows
    are taken on the device from each row's current length, so every step
    equals the oracle on the full host history while the windows grow from
    10 ids to their caps (compactions: the other loops here)."""
    import torch
    dev = torch.device("cuda:0")
    B, V, P0 = 4, 4096, 10
    stride, keep = 1024, 512
    rng = np.random.default_rng(600)
    params = [O.default_params(temperature=t) for t in (0.2, 0.7, 1.0, 1.3)]
    base = rng.normal(0.0, 2.5, (B, V)).astype(np.float32)
    host = [list(rng.integers(0, V, P0)) for _ in range(B)]
    hist = torch.zeros((B, stride), dtype=torch.int32, device=dev)
    hist[:, :P0] = torch.from_numpy(np.asarray(host, np.int32)).to(dev)
    lens = torch.full((B,), P0, dtype=torch.int32, device=dev)
    x_d = torch.empty((B, V), dtype=torch.float32, device=dev)
    u_d = torch.empty(B, dtype=torch.float64, device=dev)
    stream = torch.cuda.Stream(dev)
    out = None

    def step():
        nonlocal out
        # (hist_len is ignored with device lengths: any value)
        out = sampler.run(x_d, params, u_d, hist=hist, hist_len=[0] * B, hist_len_dev=lens, outputs=out,
                          stream=stream)
        hs.history_push(hist, lens, out["token"], keep, stream=stream)

    graph = None
    for s in range(601):
        x, u = _step_inputs(rng, base)
        x_d.copy_(torch.from_numpy(x))
        u_d.copy_(torch.from_numpy(u))
        torch.cuda.synchronize()
        if s == 0:
            with torch.cuda.stream(stream):
                step()
        else:
            if graph is None:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=stream):
                    step()
                stream.synchronize()
            graph.replay()
        torch.cuda.synchronize()
        tok, fl = out["token"].cpu().numpy(), out["row_flags"].cpu().numpy()
        for r in range(B):
            _check_token(int(tok[r]), int(fl[r]), x[r], params[r], host[r], u[r], f"step {s} row {r}")
            host[r].append(int(tok[r]))
    got_len = lens.cpu().numpy()
    got = hist.cpu().numpy()
    for r in range(B):
        n = int(got_len[r])
        assert n == P0 + 601
        np.testing.assert_array_equal(got[r, :n], host[r][-n:])
