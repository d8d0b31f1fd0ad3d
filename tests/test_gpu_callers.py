"""Batched callers of the sampler on the GPU, against the reference's
one-token-at-a-time loop restated on the CPU oracle:
 - ultima_hsamp_verify_block: a drafted block's target logits -> the tokens the
   loop (sample(), push_recent; src/server/http_server.cpp:174-201) emits with
   the same uniforms;
 - ultima_hsamp_decode_commit: the loop's stop rules (-1, eos / im_end, and
   max_tokens) applied to many slots per step, histories kept on the device.
Bar: every emitted token equal to the oracle's (a u within 1e-6 of a CDF
boundary aside, flagged by the GPU), histories and lengths equal."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

ROW_CDF_NEAR = 1


def _knobs(wl, kind):
    if kind == "penalties":
        return wl.identity_params(temperature=0.8, top_k=40, top_p=0.9, rep_penalty=1.3, repeat_last_n=64,
                                  frequency_penalty=0.3, presence_penalty=0.4)
    if kind == "server":
        return wl.default_params(temperature=0.7, top_p=0.95, rep_penalty=1.1, repeat_last_n=64)
    return wl.identity_params(temperature=1.0, top_k=200)


def _loop(xs, p, hist, u, draft):
    """The reference loop over the block: sample position i with the history so
    far, stop after the first sample that differs from its draft."""
    h = list(hist)
    out, margins = [], []
    for i in range(xs.shape[0]):
        t = O.sample_row(xs[i], p, hist=np.asarray(h, np.int32), u=float(u[i]))
        out.append(t.token)
        margins.append(t.cdf_margin)
        if i == xs.shape[0] - 1 or t.token != draft[i]:
            break
        h.append(t.token)
    return out, margins


def _verify_case(hs, sampler, wl, xs, p, hist, u, draft, dtype, one_buffer=False):
    """one_buffer: the drafts follow the history in one device array (the
    rows read it in place), else two separate arrays (prefix rows built)."""
    import torch
    dev = torch.device("cuda:0")
    if dtype == "bf16":
        bits = wl.to_bf16_bits(xs)
        xs = wl.bf16_to_f32(bits)
        xd = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xd = torch.from_numpy(xs).to(dev)
    if one_buffer:
        seq = torch.from_numpy(np.concatenate([np.asarray(hist, np.int32), np.asarray(draft, np.int32)])).to(dev)
        hd = seq[:len(hist)] if len(hist) else None
        dd = seq[len(hist):] if len(draft) else None
    else:
        dd = torch.from_numpy(np.asarray(draft, np.int32)).to(dev) if len(draft) else None
        hd = torch.from_numpy(np.asarray(hist, np.int32)).to(dev) if len(hist) else None
    toks, count, flags = sampler.verify_block(xd, p, torch.from_numpy(u).to(dev), draft=dd, hist=hd)
    torch.cuda.synchronize()
    want, margins = _loop(xs, p, hist, u, draft)
    got = toks.cpu().numpy()[: int(count.cpu()[0])].tolist()
    fl = flags.cpu().numpy()
    if got != want:
        # only a draw within 1e-6 of a CDF boundary may differ, and then the
        # first difference is at that position
        i = next(j for j in range(min(len(got), len(want))) if got[j] != want[j])
        assert (fl[i] & ROW_CDF_NEAR) and margins[i] <= 1e-6, (got, want)
        return None
    assert np.all(toks.cpu().numpy()[len(got):] == -1)
    return got


@pytest.mark.parametrize("layout", ["separate", "one_buffer", "no_history"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("kind", ["penalties", "server", "plain"])
def test_verify_block_equals_the_sequential_loop(hs, sampler, wl, dtype, kind, layout):
    rng = np.random.default_rng({"penalties": 1, "server": 2, "plain": 3}[kind] + (10 if dtype == "bf16" else 0)
                                + {"separate": 0, "one_buffer": 20, "no_history": 40}[layout])
    V, n, L = 32000, 8, (0 if layout == "no_history" else 120)
    p = _knobs(wl, kind)
    base = rng.normal(0.0, 2.0, V).astype(np.float32)
    seen = set()
    for accept in (0, 3, n - 1):
        xs = (base + rng.normal(0.0, 0.6, (n, V))).astype(np.float32)
        hist = rng.integers(0, V, L).astype(np.int32)
        if L:
            hist[-20:] = np.argsort(-base)[:20]      # recent ids among the likely ones: penalties matter
        u = rng.random(n)
        # drafts that the loop accepts up to position `accept`, then one it rejects
        xs_eff = xs if dtype == "f32" else wl.bf16_to_f32(wl.to_bf16_bits(xs))
        h = list(hist)
        draft = []
        for i in range(n - 1):
            t = O.sample_row(xs_eff[i], p, hist=np.asarray(h, np.int32), u=float(u[i])).token
            if i < accept:
                draft.append(t)
                h.append(t)
            else:
                draft.append((t + 1 + i) % V)
        got = _verify_case(hs, sampler, wl, xs, p, hist, u, draft, dtype, one_buffer=layout == "one_buffer")
        if got is not None:
            assert len(got) == accept + 1
            seen.add(accept)
    assert seen   # at least one block decided away from a CDF boundary


def test_verify_block_single_position_and_empty_history(hs, sampler, wl):
    rng = np.random.default_rng(4)
    V = 5000
    xs = rng.normal(0.0, 1.5, (1, V)).astype(np.float32)
    u = rng.random(1)
    got = _verify_case(hs, sampler, wl, xs, _knobs(wl, "plain"), [], u, [], "f32")
    assert got is None or len(got) == 1


def test_verify_block_long_block_over_many_lists(hs, sampler, wl):
    """65 positions (more than one wave of the accept kernel), every draft the
    loop's own sample: all accepted, the last position's sample emitted."""
    rng = np.random.default_rng(5)
    V, n, L = 151936, 65, 300
    p = _knobs(wl, "penalties")
    xs = rng.normal(0.0, 2.0, (n, V)).astype(np.float32)
    hist = rng.integers(0, V, L).astype(np.int32)
    u = rng.random(n)
    h = list(hist)
    draft = []
    for i in range(n - 1):
        t = O.sample_row(xs[i], p, hist=np.asarray(h, np.int32), u=float(u[i])).token
        draft.append(t)
        h.append(t)
    for one_buffer in (False, True):
        got = _verify_case(hs, sampler, wl, xs, p, hist, u, draft, "f32", one_buffer=one_buffer)
        assert got is None or len(got) == n


def _commit_oracle(x, params, u, host, active, budget, stop):
    """One step of the server loop on every slot: (tokens, margins)."""
    toks, margins = [], []
    for r in range(len(params)):
        if not active[r] or (budget is not None and budget[r] <= 0):
            # an ended slot, or one started with no budget (max_tokens 0), emits nothing
            active[r] = False
            toks.append(-1)
            margins.append(1.0)
            continue
        t = O.sample_row(x[r], params[r], hist=np.asarray(host[r], np.int32), u=float(u[r]))
        toks.append(t.token)
        margins.append(t.cdf_margin)
        if t.token < 0 or t.token in stop:
            active[r] = False
            continue
        host[r].append(t.token)
        if budget is not None:
            budget[r] -= 1
            if budget[r] <= 0:
                active[r] = False
    return toks, margins


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("captured", [False, True])
def test_decode_commit_runs_the_server_loop_on_many_slots(hs, sampler, wl, captured, fused):
    """fused: ultima_hsamp_run_commit (the rules applied where each token is
    decided); else ultima_hsamp_run then ultima_hsamp_decode_commit."""
    import torch
    dev = torch.device("cuda:0")
    B, V, W = 7, 4096, 64
    stride, keep = 2 * W, W
    eos, im_end = 7, 11
    stop = (eos, im_end)
    out = None
    rng = np.random.default_rng(21 + int(captured) + 2 * int(fused))

    def step_fn(hl):
        nonlocal out
        if fused:
            out = sampler.run_commit(x_d, params, u_d, hist, hl, lens, active, keep, stop, budget, outputs=out,
                                     stream=stream)
        else:
            out = sampler.run(x_d, params, u_d, hist=hist, hist_len=hl, hist_len_dev=lens, outputs=out,
                              stream=stream)
            hs.decode_commit(hist, lens, out["token"], active, keep, stop, budget, stream=stream)

    # (the server's knobs with DRY looking back 48 ids: every window within W,
    # as the device-history plan requires)
    params = [_knobs(wl, k) for k in ("penalties", "server", "plain", "penalties", "server", "plain", "plain")]
    for r in (1, 4):
        params[r]["dry_last_n"] = 48
    base = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    base[:, [eos, im_end]] = -10.0
    # slots 1 and 4 drift towards a stop token, slot 2 has a small budget
    ramp = np.zeros((B, V), np.float32)
    hist = torch.zeros((B, stride), dtype=torch.int32, device=dev)
    lens = torch.zeros(B, dtype=torch.int32, device=dev)
    active = torch.ones(B, dtype=torch.int32, device=dev)
    budget_h = [200, 200, 9, 200, 200, 200, 0]          # slot 6: max_tokens 0
    budget = torch.tensor(budget_h, dtype=torch.int32, device=dev)
    host = [[] for _ in range(B)]
    act_h = [True] * B
    x_d = torch.empty((B, V), dtype=torch.float32, device=dev)
    u_d = torch.empty(B, dtype=torch.float64, device=dev)
    stream = torch.cuda.Stream(dev)
    graph = None
    steps = 2 * stride + 10                   # through a compaction
    for step in range(steps):
        ramp[1, eos] = 0.15 * step
        ramp[4, im_end] = 0.1 * step
        x = (base + ramp + rng.normal(0.0, 0.5, (B, V))).astype(np.float32)
        u = rng.random(B)
        x_d.copy_(torch.from_numpy(x))
        u_d.copy_(torch.from_numpy(u))
        hl = [min(len(h), W) for h in host]
        # (an ended slot's row is still sampled and its token dropped: its
        # history may be shorter than the plan's windows)
        steady = all(hl[r] == W or not act_h[r] for r in range(B))
        if captured and graph is None and steady:
            # this step runs eagerly with the steady-state plan, then the same
            # step is captured once (its plan no longer changes) and replayed
            # from the next step on
            with torch.cuda.stream(stream):
                step_fn([W] * B)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            snap = [t.clone() for t in (hist, lens, active, budget)]
            with torch.cuda.graph(graph, stream=stream):
                step_fn([W] * B)
            stream.synchronize()
            for t, c in zip((hist, lens, active, budget), snap):   # (capture does not run the kernels)
                assert torch.equal(t, c)
        elif graph is not None:
            torch.cuda.synchronize()
            graph.replay()
        else:
            with torch.cuda.stream(stream):
                step_fn(hl)
        torch.cuda.synchronize()
        want, margins = _commit_oracle(x, params, u, host, act_h, budget_h, stop)
        got = out["token"].cpu().numpy()
        fl = out["row_flags"].cpu().numpy()
        for r in range(B):
            if got[r] != want[r]:
                assert (fl[r] & ROW_CDF_NEAR) and margins[r] <= 1e-6, f"step {step} slot {r}: {got[r]} {want[r]}"
                pytest.skip("a draw within 1e-6 of a CDF boundary; the slots' paths part")
        np.testing.assert_array_equal(active.cpu().numpy().astype(bool), act_h, err_msg=f"step {step}")
    assert not act_h[2] and len(host[2]) == 9            # budget spent
    assert not act_h[6] and len(host[6]) == 0            # no budget: nothing emitted
    assert not act_h[1] and not act_h[4]                 # stopped on eos / im_end
    got_len = lens.cpu().numpy()
    got_hist = hist.cpu().numpy()
    for r in range(B):
        n = int(got_len[r])
        np.testing.assert_array_equal(got_hist[r, :n], host[r][-n:])
        if len(host[r]) >= stride:
            assert keep < n <= stride
    np.testing.assert_array_equal(budget.cpu().numpy(), budget_h)


def test_decode_commit_64_slots_server_defaults_full_vocab(hs, sampler, wl):
    """The benchmarked decode step at its real shape: 64 slots, V = 151936,
    SamplerParams{} (DRY over 512 ids, repetition over 64, min_p .05; a
    quarter of the slots at temperature 0.9), histories already past the
    longest window; steps eager, then captured once and replayed, each step's
    tokens and every slot's history against the server loop on the oracle."""
    import torch
    dev = torch.device("cuda:0")
    B, V, H0 = 64, 151936, 600
    stride, keep = 1024, 512
    rng = np.random.default_rng(64)
    params = [wl.default_params() if r % 4 else wl.default_params(temperature=0.9) for r in range(B)]
    base = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    host = [list(rng.integers(0, V, H0)) for _ in range(B)]
    hist = torch.zeros((B, stride), dtype=torch.int32, device=dev)
    hist[:, :H0] = torch.from_numpy(np.asarray(host, np.int32)).to(dev)
    lens = torch.full((B,), H0, dtype=torch.int32, device=dev)
    active = torch.ones(B, dtype=torch.int32, device=dev)
    act_h = [True] * B
    stop = (151643, 151645)
    x_d = torch.empty((B, V), dtype=torch.float32, device=dev)
    u_d = torch.empty(B, dtype=torch.float64, device=dev)
    stream = torch.cuda.Stream(dev)
    out = None
    win = [512] * B          # every window full: the plan is the same at every step

    def step_fn():
        nonlocal out
        out = sampler.run_commit(x_d, params, u_d, hist, win, lens, active, keep, stop, None, outputs=out,
                                 stream=stream)

    graph = None
    for step in range(7):
        x = (base + rng.normal(0.0, 0.5, (B, V))).astype(np.float32)
        u = rng.random(B)
        x_d.copy_(torch.from_numpy(x))
        u_d.copy_(torch.from_numpy(u))
        torch.cuda.synchronize()
        if step == 3:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                step_fn()
            stream.synchronize()
        if graph is not None:
            graph.replay()
        else:
            with torch.cuda.stream(stream):
                step_fn()
        torch.cuda.synchronize()
        print(f"64-slot decode step {step}", flush=True)
        want, margins = _commit_oracle(x, params, u, host, act_h, None, stop)
        got = out["token"].cpu().numpy()
        fl = out["row_flags"].cpu().numpy()
        for r in range(B):
            if got[r] != want[r]:
                assert (fl[r] & ROW_CDF_NEAR) and margins[r] <= 1e-6, f"step {step} slot {r}: {got[r]} {want[r]}"
                pytest.skip("a draw within 1e-6 of a CDF boundary; the slots' paths part")
    got_len = lens.cpu().numpy()
    got_hist = hist.cpu().numpy()
    for r in range(B):
        n = int(got_len[r])
        np.testing.assert_array_equal(got_hist[r, :n], host[r][-n:])
