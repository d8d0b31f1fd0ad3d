"""GPU parity of the logits producer (ultima_hsamp_lm_head: final rmsnorm +
lm-head matvec, reference src/model/qwen_model.cpp:182-207) against its CPU
checker oracle/head_oracle.c, which the CPU tests pin bit for bit to the
reference's own AVX2 kernels. Bar: normed rows and logits bit-exact; the
tokens sampled from the device logits equal the oracle's on its logits."""
import numpy as np
import pytest

import oracle as O
from test_oracle_head import WL, bf16_bits

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


# ---- quantised heads and the Hadamard fold ----------------------------------------

QNAMES = ["q4k", "q5k", "q6k", "q8_0", "q4_1", "q5_0", "pq2_0"]


def _qhead(hs, h, g, w, dtype, scale=1.0, fold_block=0, signs=None, offset=0, eps=1e-6):
    """Device run of a quantised (or dense, fold) head; `offset` places the
    weights `offset` bytes into their buffer (rows not dword-aligned)."""
    import torch
    dev = torch.device("cuda:0")
    ht = torch.from_numpy(h).to(dev)
    gt = torch.from_numpy(g).to(dev)
    if dtype >= O.HEAD_Q4_K:
        flat = np.zeros(w.size + 64, np.uint8)
        flat[offset:offset + w.size] = w.reshape(-1)
        buf = torch.from_numpy(flat).to(dev)
        wt = buf[offset:offset + w.size].view(w.shape)
    elif dtype == O.HEAD_BF16:
        wt = torch.from_numpy(w.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        wt = torch.from_numpy(w).to(dev)
    st = None if signs is None else torch.from_numpy(signs).to(dev)
    logits, normed = hs.lm_head(ht, gt, eps, wt, scale, weight_dtype=dtype, fold_block=fold_block, fold_signs=st)
    torch.cuda.synchronize()
    return logits.cpu().numpy(), normed.cpu().numpy()


@pytest.mark.parametrize("name", QNAMES)
@pytest.mark.parametrize("rows,H,V,scale,offset", [
    (1, 4096, 151936, 1.0, 0),     # a Qwen3-8B head, one row (the decode step)
    (2, 2048, 5003, 8.0, 0),       # two batch rows share the tile, ragged vocabulary tile, logit scale
    (3, 1024, 700, 1.0, 0),        # three rows in a four-wave block
    (5, 512, 130, 0.0, 0),         # two batch groups
    (1, 1280, 300, 1.0, 2),        # rows two bytes off dword alignment
    (2, 768, 257, 2.5, 1),         # rows at odd byte addresses
])
def test_quant_head_matches_oracle_bits(hs, name, rows, H, V, scale, offset):
    dt = O.HEAD_NAMES[name]
    be = WL.QUANT_BLOCKS[dt][0]
    if H % be:
        H = H // be * be if H >= be else be
    print(f"quant head {name} rows={rows} H={H} V={V} offset={offset}", flush=True)
    rng = np.random.default_rng(rows * 7 + H + V + dt)
    h = rng.normal(0, 2.0, (rows, H)).astype(np.float32)
    g = rng.normal(1.0, 0.2, H).astype(np.float32)
    w = WL.quant_head(dt, V, H, seed=H + V + dt)
    got, normed = _qhead(hs, h, g, w, dt, scale, offset=offset)
    want, want_n = O.lm_head(h, g, 1e-6, w, scale, dtype=dt)
    np.testing.assert_array_equal(normed, want_n)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", ["q8_0", "q4_1", "q5_0", "pq2_0"])
@pytest.mark.parametrize("H", [96, 1056, 384])
def test_quant_head_partial_chunks(hs, name, H):
    """Hidden sizes whose last chunk holds fewer blocks than the others."""
    dt = O.HEAD_NAMES[name]
    if H % WL.QUANT_BLOCKS[dt][0]:
        pytest.skip("not a whole number of blocks")
    rng = np.random.default_rng(H + dt)
    h = rng.normal(0, 2.0, (2, H)).astype(np.float32)
    g = rng.normal(1.0, 0.2, H).astype(np.float32)
    w = WL.quant_head(dt, 200, H, seed=H * 3 + dt)
    got, _ = _qhead(hs, h, g, w, dt)
    want, _ = O.lm_head(h, g, 1e-6, w, dtype=dt)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quant_head_not_whole_blocks_gives_zeros(hs):
    """As the reference's matvecs: a hidden size that is not a whole number of
    the type's blocks gives logits of 0 (normed rows still written)."""
    H, V = 100, 64
    rng = np.random.default_rng(3)
    h = rng.normal(0, 1, (1, H)).astype(np.float32)
    g = np.ones(H, np.float32)
    w = np.full((V, 4 * 22), 0x55, np.uint8)
    got, normed = _qhead(hs, h, g, w, O.HEAD_Q5_0)
    assert np.all(got == 0.0)
    np.testing.assert_array_equal(normed, O.rmsnorm(h[0], g, 1e-6)[None])


def test_quant_head_special_scales(hs):
    """Blocks with fp16 scales that are subnormal, zero, negative, infinite and
    NaN: converted exactly (NaN logits compared as NaN)."""
    H, V = 512, 128
    rng = np.random.default_rng(11)
    h = rng.normal(0, 1, (1, H)).astype(np.float32)
    g = np.ones(H, np.float32)
    for name in QNAMES:
        dt = O.HEAD_NAMES[name]
        w = WL.quant_head(dt, V, H, seed=5 + dt)
        be, bb, fields = WL.QUANT_BLOCKS[dt]
        blocks = w.reshape(-1, bb)
        specials = np.array([0x0001, 0x03FF, 0x0000, 0x8000, 0xBC00, 0x7C00, 0xFC00, 0x7E00, 0x7C01], np.uint16)
        for k in range(0, blocks.shape[0], 3):
            v = specials[(k // 3) % specials.size]
            blocks[k, fields[0]] = v & 0xFF
            blocks[k, fields[0] + 1] = v >> 8
        got, _ = _qhead(hs, h, g, w, dt)
        want, _ = O.lm_head(h, g, 1e-6, w, dtype=dt)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), name
        np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32), err_msg=name)


@pytest.mark.parametrize("name", ["f32", "bf16", "q6k", "q8_0", "q4k"])
@pytest.mark.parametrize("H,block,signed", [(4096, 1024, True), (2048, 2048, False), (1024, 64, True),
                                            (1000, 64, True)])
def test_folded_head_matches_oracle_bits(hs, name, H, block, signed):
    """The Hadamard-folded head (qwen_model.cpp:189-196): norm, signs, the
    blockwise rotation, matvec; a block that does not divide H leaves the rows
    unfolded, as the reference does."""
    dt = O.HEAD_NAMES[name]
    if dt >= O.HEAD_Q4_K and H % WL.QUANT_BLOCKS[dt][0]:
        pytest.skip("not a whole number of blocks")
    print(f"folded head {name} H={H} block={block} signed={signed}", flush=True)
    rows, V = 2, 3001
    rng = np.random.default_rng(H + block + dt)
    h = rng.normal(0, 2.0, (rows, H)).astype(np.float32)
    g = rng.normal(1.0, 0.2, H).astype(np.float32)
    s = np.where(rng.random(H) < 0.5, -1.0, 1.0).astype(np.float32) if signed else None
    if dt == O.HEAD_F32:
        w = rng.normal(0, 0.04, (V, H)).astype(np.float32)
    elif dt == O.HEAD_BF16:
        w = bf16_bits(rng.normal(0, 0.04, (V, H)).astype(np.float32))
    else:
        w = WL.quant_head(dt, V, H, seed=H + dt)
    got, normed = _qhead(hs, h, g, w, dt, 2.0, fold_block=block, signs=s)
    want, want_n = O.lm_head(h, g, 1e-6, w, 2.0, dtype=dt, fold_block=block, fold_signs=s)
    np.testing.assert_array_equal(normed, want_n)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quant_head_feeds_the_sampler(hs, sampler, wl):
    """A Q6_K head's device logits sampled on the device: the oracle's tokens."""
    import torch
    rng = np.random.default_rng(78)
    rows, H, V = 3, 1024, 151936
    h = rng.normal(0, 2.0, (rows, H)).astype(np.float32)
    g = rng.normal(1.0, 0.1, H).astype(np.float32)
    w = WL.quant_head(O.HEAD_Q6_K, V, H, seed=9, scale=0.05)
    dev = torch.device("cuda:0")
    logits, _ = hs.lm_head(torch.from_numpy(h).to(dev), torch.from_numpy(g).to(dev), 1e-6,
                           torch.from_numpy(w).to(dev), weight_dtype=O.HEAD_Q6_K)
    params = [wl.identity_params(temperature=0.8, top_k=40, top_p=0.95) for _ in range(rows)]
    u = rng.random(rows)
    out = sampler.run(logits, params, torch.from_numpy(u).to(dev))
    torch.cuda.synchronize()
    want_logits, _ = O.lm_head(h, g, 1e-6, w, dtype=O.HEAD_Q6_K)
    for r in range(rows):
        tr = O.sample_row(want_logits[r], params[r], u=float(u[r]))
        assert int(out["token"][r]) == tr.token


def test_lm_head_rejects_bad_types_and_folds(hs):
    import ctypes
    import torch
    dev = torch.device("cuda:0")
    H, V = 64, 32
    x = torch.zeros((1, H), device=dev)
    g = torch.ones(H, device=dev)
    w = torch.zeros((V, H), device=dev)
    lo = torch.zeros((1, V), device=dev)
    n = torch.zeros((1, H), device=dev)
    h = hs.Head()
    h.hidden, h.hidden_stride, h.rows, h.hidden_dim, h.vocab = x.data_ptr(), H, 1, H, V
    h.norm_scale, h.eps, h.logit_scale, h.weight = g.data_ptr(), 1e-6, 1.0, w.data_ptr()
    h.normed, h.logits, h.logits_stride = n.data_ptr(), lo.data_ptr(), V
    for dt, fb, want in [(9, 0, hs.ERR_INVALID), (-1, 0, hs.ERR_INVALID), (0, 3, hs.ERR_INVALID),
                         (0, -2, hs.ERR_INVALID), (0, 16384, hs.ERR_UNSUPPORTED), (0, 64, hs.OK)]:
        h.weight_dtype, h.fold_block = dt, fb
        assert hs.lib().ultima_hsamp_lm_head(ctypes.byref(h), None) == want, (dt, fb)
    torch.cuda.synchronize()
