"""Write tests/golden/ref_cases.npz: inputs and the reference's outputs.

Runs the reference's own sampler (oracle/_ref/libref_sampler.so, compiled
from /root/reference/src/sampler/sampler.cpp by oracle/Makefile) on the seeded
cases of tests/case_gen.py and stores each case's inputs, token and the logits
sample() leaves behind. Run in the container that has the reference sources:
    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "oracle"), str(ROOT / "tests")]
import oracle as O  # noqa: E402
from case_gen import make_case  # noqa: E402

N, V, HMAX, BMAX = 160, 257, 300, 8
SEED0 = 10_000


def main():
    out = {k: [] for k in ("logits", "hist", "hist_len", "bias_ids", "bias_vals", "bias_n",
                           "seed", "token", "after")}
    params = {k: [] for k in O.PARAM_FIELDS}
    for i in range(N):
        seed = SEED0 + i
        x, hist, bias, p = make_case(seed, V)
        tok, after = O.ref_sample_row(x, p, hist=hist, bias=bias, seed=seed)
        h = np.zeros(HMAX, np.int32)
        h[: hist.size] = hist
        bi = np.zeros(BMAX, np.int32)
        bv = np.zeros(BMAX, np.float32)
        for j, (a, b) in enumerate(bias.items()):
            bi[j], bv[j] = a, b
        for k, v in (("logits", x), ("hist", h), ("hist_len", hist.size), ("bias_ids", bi),
                     ("bias_vals", bv), ("bias_n", len(bias)), ("seed", seed), ("token", tok),
                     ("after", after)):
            out[k].append(v)
        for k in O.PARAM_FIELDS:
            params[k].append(p[k])
    arrs = {k: np.array(v) for k, v in out.items()}
    arrs["seed"] = arrs["seed"].astype(np.uint64)
    for k, v in params.items():
        arrs["p_" + k] = np.array(v, dtype=np.float32 if isinstance(v[0], float) else np.uint64)
    arrs["n"] = np.array(N)
    np.savez_compressed(Path(__file__).with_name("ref_cases.npz"), **arrs)
    print(f"wrote {N} reference cases")


if __name__ == "__main__":
    main()
