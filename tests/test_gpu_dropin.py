"""The ultima::sampler C++ drop-in (libultima_sampler.so) on the GPU.

`dropin_driver refcases` compiles the reference's own test cases
(/root/reference/tests/unit/test_sampler.cpp:21-117) against the drop-in
header; `dropin_driver replay` runs seeded random cases (tests/case_gen.py)
through sample(), which works in place like the reference's, and the tokens
and logits must equal the CPU oracle given the uniform SamplerContext(seed)
draws. `dropin_driver cli` runs the reference CLI's generation loop
(apps/ultima-cli/main.cpp:661-679: identity() + temperature at V = 151936);
`dropin_driver batch` calls sample_batch() on device buffers.
"""
import struct
import subprocess

import numpy as np
import pytest

import oracle as O
from case_gen import make_case

pytestmark = pytest.mark.gpu


def driver(pkg):
    return str(pkg.hsamp.PKG / "dropin_driver")


def test_reference_test_cases_pass(pkg, hs):
    r = subprocess.run([driver(pkg), "refcases"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


def _write_cases(path, cases):
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(cases)))
        for x, hist, bias, p, seed in cases:
            f.write(struct.pack("<i", x.size))
            f.write(np.asarray(x, np.float32).tobytes())
            f.write(struct.pack("<i", hist.size))
            f.write(np.asarray(hist, np.int32).tobytes())
            f.write(struct.pack("<i", len(bias)))
            for t, v in bias.items():
                f.write(struct.pack("<if", t, v))
            f.write(struct.pack("<fQffQQfffQffQ", p["rep_penalty"], p["repeat_last_n"],
                                p["dry_multiplier"], p["dry_base"], p["dry_allowed_len"],
                                p["dry_last_n"], p["frequency_penalty"], p["presence_penalty"],
                                p["temperature"], p["top_k"], p["top_p"], p["min_p"], seed))


def test_replay_matches_oracle(pkg, hs, tmp_path):
    cases = []
    for seed in range(300):
        x, hist, bias, p = make_case(seed)
        cases.append((x, hist, bias, p, seed))
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    _write_cases(fin, cases)
    r = subprocess.run([driver(pkg), "replay", str(fin), str(fout)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    data = open(fout, "rb").read()
    off = 0
    for i, (x, hist, bias, p, seed) in enumerate(cases):
        tok = struct.unpack_from("<i", data, off)[0]
        off += 4
        after = np.frombuffer(data, np.float32, x.size, off)
        off += 4 * x.size
        tr = O.sample_row(x, p, hist=hist, bias=bias, u=O.u_from_seed(seed))
        assert tok == tr.token, f"case {i}"
        np.testing.assert_array_equal(after.view(np.uint32), tr.logits_after.view(np.uint32),
                                      err_msg=f"case {i}")


def _u_of(x: int) -> float:
    """generate_canonical<double, 53> of one mt19937_64 output (clamped below 1)."""
    u = float(x) / 2.0**64
    return u if u < 1.0 else float(np.nextafter(1.0, 0.0))


@pytest.mark.parametrize("temperature", [0.8, 1.0, 0.0])
def test_cli_generation_loop_full_vocab(pkg, hs, wl, tmp_path, temperature):
    """The CLI's exact call for every generated token: identity() with only
    the temperature set, over the full V = 151936 row, one context whose
    history grows by each sampled id; argmax when T <= 0."""
    V, steps, seed = 151936, 6, 20240917
    prompt = np.arange(1, 9, dtype=np.int32) * 1000
    rows = np.stack([wl._rows_normal(100 + i, 1, V, 3.0)[0] for i in range(steps)])
    fin, fout = tmp_path / "cli.bin", tmp_path / "cli_out.bin"
    with open(fin, "wb") as f:
        f.write(struct.pack("<iifQi", V, steps, temperature, seed, prompt.size))
        f.write(prompt.tobytes())
        f.write(rows.astype(np.float32).tobytes())
    r = subprocess.run([driver(pkg), "cli", str(fin), str(fout)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    data = open(fout, "rb").read()
    p = O.identity_params(temperature=temperature)
    hist = list(prompt)
    off = 0
    for i in range(steps):
        tok = struct.unpack_from("<i", data, off)[0]
        off += 4
        after = np.frombuffer(data, np.float32, V, off)
        off += 4 * V
        if temperature <= 0.0:
            assert tok == O.argmax(rows[i]), f"step {i}"
        else:
            # one mt19937_64 call per sample(): step i draws output i + 1
            u = _u_of(O.mt19937_64_nth(seed, i + 1))
            tr = O.sample_row(rows[i], p, hist=np.array(hist, np.int32), u=u)
            assert tok == tr.token, f"step {i}: {tok} != {tr.token}"
            np.testing.assert_array_equal(after.view(np.uint32), tr.logits_after.view(np.uint32),
                                          err_msg=f"step {i}")
        hist.append(tok)


def test_sample_batch_device_rows(pkg, hs, wl, tmp_path):
    """sample_batch() (the drop-in's native batched entry) on device copies of
    config-2-like rows with mixed knobs, checked row by row against the oracle."""
    B, V, H = 12, 151936, 512
    rng = np.random.default_rng(77)
    x = wl._rows_normal(7, B, V, 2.0)
    hist = rng.integers(0, V, size=(B, H)).astype(np.int32)
    hist_len = np.array([H, 0, 100, H, 1, 300, H, 64, 2, H, 10, H], np.int64)
    u = rng.random(B)
    plist = []
    for r in range(B):
        plist.append(O.identity_params(
            temperature=[0.7, 0.0, 1.2, 0.9][r % 4], top_k=[50, 0, 40, 1000, 5, 0][r % 6],
            top_p=[1.0, 0.9, 0.95][r % 3], min_p=[0.0, 0.05][r % 2],
            rep_penalty=[1.1, 1.0, 1.3][r % 3], repeat_last_n=int(hist_len[r]),
            frequency_penalty=[0.5, 0.0][r % 2], presence_penalty=[0.3, 0.0, 0.1][r % 3],
            dry_multiplier=[0.0, 0.8][r % 2], dry_last_n=[0, 256][r % 2]))
    fin, fout = tmp_path / "batch.bin", tmp_path / "batch_out.bin"
    with open(fin, "wb") as f:
        f.write(struct.pack("<iii", B, V, H))
        f.write(x.astype(np.float32).tobytes())
        f.write(hist.tobytes())
        f.write(hist_len.tobytes())
        f.write(u.astype(np.float64).tobytes())
        for p in plist:
            f.write(struct.pack("<fQffQQfffQffQ", p["rep_penalty"], p["repeat_last_n"],
                                p["dry_multiplier"], p["dry_base"], p["dry_allowed_len"],
                                p["dry_last_n"], p["frequency_penalty"], p["presence_penalty"],
                                p["temperature"], p["top_k"], p["top_p"], p["min_p"], 0))
    r = subprocess.run([driver(pkg), "batch", str(fin), str(fout)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    tok = np.frombuffer(open(fout, "rb").read(), np.int32)
    for i in range(B):
        tr = O.sample_row(x[i], plist[i], hist=hist[i, : hist_len[i]], u=float(u[i]))
        assert tok[i] == tr.token or tr.cdf_margin <= 1e-6, f"row {i}: {tok[i]} != {tr.token}"
