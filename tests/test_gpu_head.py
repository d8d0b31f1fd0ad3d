"""GPU parity of the logits producer (ultima_hsamp_lm_head: final rmsnorm +
lm-head matvec, reference src/model/qwen_model.cpp:182-207) against its CPU
checker oracle/head_oracle.c, which the CPU tests pin bit for bit to the
reference's own AVX2 kernels. Bar: normed rows and logits bit-exact; the
tokens sampled from the device logits equal the oracle's on its logits."""
import numpy as np
import pytest

import oracle as O
from test_oracle_head import bf16_bits

pytestmark = pytest.mark.gpu


def _head(hs, h, g, w, scale=1.0, eps=1e-6):
    import torch
    dev = torch.device("cuda:0")
    ht = torch.from_numpy(h).to(dev)
    gt = torch.from_numpy(g).to(dev)
    if w.dtype == np.uint16:
        wt = torch.from_numpy(w.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        wt = torch.from_numpy(w).to(dev)
    logits, normed = hs.lm_head(ht, gt, eps, wt, scale)
    torch.cuda.synchronize()
    return logits.cpu().numpy(), normed.cpu().numpy()


@pytest.mark.parametrize("rows,H,V,dtype,scale", [
    (1, 896, 151936, "bf16", 1.0),     # Qwen2.5-0.5B head
    (3, 4096, 5003, "bf16", 1.0),      # a Qwen3-8B hidden size, ragged vocab tile
    (6, 2048, 3000, "f32", 1.0),       # two batch groups
    (2, 131, 777, "f32", 8.0),         # hidden % 8 == 3 (fused tail), unaligned rows, logit scale
    (2, 132, 500, "f32", 1.0),         # hidden % 8 == 4 (vectorised tail)
    (1, 7, 33, "bf16", 0.0),           # hidden < 8: tail only
    (5, 4100, 257, "bf16", 2.5),       # hidden % 8 == 4 with bf16 (fused tail)
    (1, 137, 100, "f32", 1.0),         # hidden % 8 == 1
    (1, 10, 40, "f32", 1.0),           # hidden % 8 == 2
    (1, 133, 70, "bf16", 1.0),         # hidden % 8 == 5
    (2, 262, 90, "bf16", 1.0),         # hidden % 8 == 6
    (2, 200, 64, "bf16", 1.0),         # norm chains: one 16-step group and 9 single steps
    (1, 8192, 1000, "bf16", 1.0),      # a Qwen2.5-72B hidden size: one full norm pass
    (2, 8212, 300, "f32", 1.0),        # two norm passes (the second 2 steps), vectorised tail
])
def test_lm_head_matches_oracle_bits(hs, rows, H, V, dtype, scale):
    rng = np.random.default_rng(rows * 1000 + H + V)
    h = rng.normal(0, 2.0, (rows, H)).astype(np.float32)
    g = rng.normal(1.0, 0.2, H).astype(np.float32)
    w = rng.normal(0, 0.04, (V, H)).astype(np.float32)
    if dtype == "bf16":
        w = bf16_bits(w)
    got, normed = _head(hs, h, g, w, scale)
    want, want_n = O.lm_head(h, g, 1e-6, w, scale)
    np.testing.assert_array_equal(normed, want_n)
    np.testing.assert_array_equal(got, want)


def test_lm_head_feeds_the_sampler(hs, sampler, wl):
    """Device hidden states -> device logits -> sampled tokens, no host round
    trip in between: equal to the oracle's tokens on the oracle's logits."""
    import torch
    rng = np.random.default_rng(77)
    rows, H, V = 4, 896, 151936
    h = rng.normal(0, 2.0, (rows, H)).astype(np.float32)
    g = rng.normal(1.0, 0.1, H).astype(np.float32)
    w = bf16_bits(rng.normal(0, 0.08, (V, H)).astype(np.float32))
    dev = torch.device("cuda:0")
    wt = torch.from_numpy(w.view(np.int16)).to(dev).view(torch.bfloat16)
    logits, _ = hs.lm_head(torch.from_numpy(h).to(dev), torch.from_numpy(g).to(dev), 1e-6, wt)
    params = [wl.identity_params(temperature=0.8, top_k=40, top_p=0.95) for _ in range(rows)]
    u = rng.random(rows)
    out = sampler.run(logits, params, torch.from_numpy(u).to(dev))
    torch.cuda.synchronize()
    want_logits, _ = O.lm_head(h, g, 1e-6, w)
    for r in range(rows):
        tr = O.sample_row(want_logits[r], params[r], u=float(u[r]))
        assert int(out["token"][r]) == tr.token


def test_lm_head_rejects_invalid(hs):
    import ctypes
    h = hs.Head()
    assert hs.lib().ultima_hsamp_lm_head(ctypes.byref(h), None) == hs.ERR_INVALID
    assert hs.lib().ultima_hsamp_lm_head(None, None) == hs.ERR_INVALID
