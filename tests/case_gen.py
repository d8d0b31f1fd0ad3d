"""Seeded random cases for oracle-vs-reference comparisons (test helper).

Each case is a small row with continuous logits (ties in top-k / top-p are
practically absent, so the reference's unspecified tie order cannot matter),
a history with repeats, optional logit bias and a knob set drawn from a grid
that switches every stage on and off.
"""
import numpy as np


def make_case(seed: int, V: int = 257):
    rng = np.random.default_rng(seed)
    x = (rng.normal(size=V) * rng.choice([0.5, 2.0, 4.0])).astype(np.float32)
    H = int(rng.choice([0, 1, 5, 40, 300]))
    hist = rng.integers(-2, min(V + 3, 40 if rng.random() < 0.5 else V + 3), size=H).astype(np.int32)
    bias = {}
    if rng.random() < 0.3:
        for t in rng.choice(V, size=int(rng.integers(1, 6)), replace=False):
            bias[int(t)] = float(np.float32(rng.normal() * 3))
    p = dict(
        rep_penalty=float(rng.choice([1.0, 1.1, 0.9, 1.5])),
        repeat_last_n=int(rng.choice([0, 8, 64, 1000])),
        dry_multiplier=float(rng.choice([0.0, 0.8])),
        dry_base=float(rng.choice([1.75, 2.0])),
        dry_allowed_len=int(rng.choice([0, 2, 3])),
        dry_last_n=int(rng.choice([0, 16, 512])),
        frequency_penalty=float(rng.choice([0.0, 0.5, -0.25])),
        presence_penalty=float(rng.choice([0.0, 0.3])),
        temperature=float(rng.choice([0.0, 0.2, 0.7, 1.0, 1.5])),
        top_k=int(rng.choice([0, 1, 5, 40, V, V + 1])),
        top_p=float(rng.choice([1.0, 0.9, 0.5, 0.0, 0.999])),
        min_p=float(rng.choice([0.0, 0.05, 0.3])),
    )
    return x, hist, bias, p
