"""Seeded synthetic sampler workloads (the five BASELINE configurations).

Inputs are generated once on the host with a build-specified generator so the
CPU checker and the GPU see identical bits: SplitMix64 (counter mode) ->
53-bit uniforms -> Box-Muller normals in float64, scaled and rounded to float32
(and to bfloat16, round-to-nearest-even, for the bf16 configurations).
History ids are uniform in [0, V); mask bits use integer thresholds; the draw
uniforms are 53-bit SplitMix64 uniforms.

Per-row knobs start from SamplerParams::identity() (reference
src/sampler/sampler.cpp:192-205) and set only the listed knobs.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

V_QWEN = 151936
_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n outputs of SplitMix64 started at `seed`, from position `offset`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & (2**64 - 1)) + i * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform53(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Uniforms in [0, 1) with 53 random bits."""
    return (splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, n: int, sigma: float) -> np.ndarray:
    """float32 N(0, sigma^2) by Box-Muller in float64."""
    m = (n + 1) // 2
    u1 = 1.0 - uniform53(seed, m, 0)          # (0, 1]
    u2 = uniform53(seed ^ 0x5DEECE66D, m, 0)  # [0, 1)
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return (z * sigma).astype(np.float32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bfloat16 bit patterns to float32."""
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def identity_params(**over) -> dict:
    """SamplerParams::identity() (reference src/sampler/sampler.cpp:192-205)."""
    p = dict(rep_penalty=1.0, repeat_last_n=0, dry_multiplier=0.0, dry_base=1.75,
             dry_allowed_len=2, dry_last_n=0, frequency_penalty=0.0, presence_penalty=0.0,
             temperature=1.0, top_k=0, top_p=1.0, min_p=0.0)
    p.update(over)
    return p


def default_params(**over) -> dict:
    """SamplerParams{} (reference include/ultima/sampler/sampler.hpp:16-52)."""
    p = dict(rep_penalty=1.1, repeat_last_n=64, dry_multiplier=0.8, dry_base=1.75,
             dry_allowed_len=2, dry_last_n=512, frequency_penalty=0.0, presence_penalty=0.0,
             temperature=0.2, top_k=40, top_p=0.95, min_p=0.05)
    p.update(over)
    return p


@dataclass
class Workload:
    name: str
    dtype: str                       # "f32" or "bf16"
    logits: np.ndarray               # [B, V] float32, or uint16 bf16 bits
    params: list                     # B dicts
    u: np.ndarray                    # [B] float64
    hist: np.ndarray | None = None   # [B, H] int32
    hist_len: np.ndarray | None = None  # [B] int64
    mask: np.ndarray | None = None   # [B, ceil(V/32)] uint32
    meta: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return self.logits.shape[0]

    @property
    def vocab(self) -> int:
        return self.logits.shape[1]

    def logits_f32(self) -> np.ndarray:
        return self.logits if self.dtype == "f32" else bf16_to_f32(self.logits)

    def algorithmic_bytes(self) -> int:
        """One read of every input byte plus the outputs (tokens)."""
        n = self.logits.nbytes + self.u.nbytes + 4 * self.rows
        if self.hist is not None:
            n += int(sum(int(h) for h in self.hist_len)) * 4
        if self.mask is not None:
            n += self.mask.nbytes
        return n


def _rows_normal(seed: int, B: int, V: int, sigma) -> np.ndarray:
    out = np.empty((B, V), np.float32)
    for r in range(B):
        s = sigma[r] if np.ndim(sigma) else sigma
        out[r] = normal(seed * 1_000_003 + r, V, s)
    return out


def _hist(seed: int, B: int, H: int, V: int) -> np.ndarray:
    return (splitmix64(seed ^ 0x41C64E6D, B * H) % np.uint64(V)).astype(np.int32).reshape(B, H)


def config(cfg: int, seed: int = 1, V: int = V_QWEN, rows: int | None = None) -> Workload:
    """BASELINE configuration `cfg` (1..5). `rows` / `V` shrink it for tests."""
    if cfg == 1:
        B = rows or 1
        x = _rows_normal(seed, B, V, 3.0)
        H = 64
        hist = _hist(seed, B, H, V)
        p = identity_params(temperature=0.8, top_k=40, top_p=0.95, rep_penalty=1.1,
                            repeat_last_n=64)
        return Workload("cfg1", "f32", x, [dict(p) for _ in range(B)], uniform53(seed + 7, B),
                        hist, np.full(B, H, np.int64))
    if cfg == 2:
        B = rows or 64
        x = _rows_normal(seed, B, V, 2.0)
        H = 2048
        hist = _hist(seed, B, H, V)
        p = identity_params(temperature=0.7, top_k=50, top_p=1.0, rep_penalty=1.1,
                            repeat_last_n=2048, frequency_penalty=0.5, presence_penalty=0.3)
        return Workload("cfg2", "f32", x, [dict(p) for _ in range(B)], uniform53(seed + 7, B),
                        hist, np.full(B, H, np.int64))
    if cfg == 3:
        B = rows or 256
        half = B // 2
        x = np.empty((B, V), np.float32)
        x[:half] = _rows_normal(seed, half, V, 1.0)
        x[half:] = _rows_normal(seed + 1, B - half, V, 0.1)
        for r in range(half):
            ids = np.unique(splitmix64(seed * 31 + r, 64) % np.uint64(V))[:16]
            x[r, ids.astype(np.int64)] = 15.0
        p = identity_params(temperature=1.0, top_k=0, top_p=0.9)
        return Workload("cfg3", "f32", x, [dict(p) for _ in range(B)], uniform53(seed + 7, B))
    if cfg == 4:
        B = rows or 128
        x = to_bf16_bits(_rows_normal(seed, B, V, 2.0))
        bits = splitmix64(seed ^ 0x1234567, B * V).reshape(B, V)
        allowed = bits < np.uint64(int(0.01 * 2**64))          # Bernoulli(0.01)
        for r in range(B):
            if not allowed[r].any():
                allowed[r, int(splitmix64(seed + r, 1)[0] % np.uint64(V))] = True
        mask = mask_from_allowed(allowed[:, :V])
        p = identity_params(temperature=1.0, top_k=20, top_p=0.8)
        return Workload("cfg4", "bf16", x, [dict(p) for _ in range(B)], uniform53(seed + 7, B),
                        mask=np.ascontiguousarray(mask, dtype=np.uint32))
    if cfg == 5:
        B = rows or 1024
        x = to_bf16_bits(_rows_normal(seed, B, V, 2.5))
        H = 512
        hist = _hist(seed, B, H, V)
        uu = uniform53(seed ^ 0xC0FFEE, 4 * B).reshape(4, B)
        kk = splitmix64(seed ^ 0xBEEF, B) % np.uint64(1000) + np.uint64(1)
        plist = []
        for r in range(B):
            plist.append(identity_params(
                temperature=float(np.float32(0.2 + 1.3 * uu[0, r])),
                top_k=int(kk[r]),
                top_p=float(np.float32(0.5 + 0.5 * uu[1, r])),
                rep_penalty=float(np.float32(1.0 + 0.3 * uu[2, r])),
                repeat_last_n=512))
        return Workload("cfg5", "bf16", x, plist, uniform53(seed + 7, B), hist,
                        np.full(B, H, np.int64))
    raise ValueError(f"unknown config {cfg}")


def mask_from_allowed(allowed: np.ndarray) -> np.ndarray:
    """[B, V] bool -> [B, ceil(V/32)] uint32 words, bit t of word t>>5."""
    B, V = allowed.shape
    W = (V + 31) // 32
    pad = np.zeros((B, W * 32), bool)
    pad[:, :V] = allowed
    w = np.zeros((B, W), np.uint64)
    bits = pad.reshape(B, W, 32).astype(np.uint64)
    for b in range(32):
        w |= bits[:, :, b] << np.uint64(b)
    return w.astype(np.uint32)


# ---- quantised lm-head weights (GGUF block layouts) -------------------------------

# weight type -> (values per block, bytes per block, byte offsets of the block's
# fp16 scale fields); the type numbers are include/ultima_hsamp.h's
# ULTIMA_HSAMP_HEAD_* values
QUANT_BLOCKS = {
    2: (256, 144, (0, 2)),    # Q4_K: d, dmin, 12 B scales/mins, 128 B nibbles
    3: (256, 176, (0, 2)),    # Q5_K: d, dmin, 12 B scales/mins, 32 B fifth bits, 128 B nibbles
    4: (256, 210, (208,)),    # Q6_K: 128 B low nibbles, 64 B high bits, 16 int8 scales, d
    5: (32, 34, (0,)),        # Q8_0: d, 32 int8
    6: (32, 20, (0, 2)),      # Q4_1: d, m, 16 B nibbles
    7: (32, 22, (0,)),        # Q5_0: d, 32 fifth bits, 16 B nibbles
    8: (128, 34, (0,)),       # PQ2_0: d, 32 B of 2-bit codes
}


def quant_row_bytes(dtype: int, H: int) -> int:
    be, bb, _ = QUANT_BLOCKS[dtype]
    if H % be:
        raise ValueError(f"H={H} is not a multiple of the type's {be}-value blocks")
    return H // be * bb


def quant_head(dtype: int, V: int, H: int, seed: int, scale: float = 0.02) -> np.ndarray:
    """Random [V, row_bytes] uint8 head of a quantised type: uniform random
    quant bytes, the fp16 scale fields finite values ~ U(0, scale) (the second
    field, a min, ~ U(0, scale / 4))."""
    be, bb, fields = QUANT_BLOCKS[dtype]
    rb = quant_row_bytes(dtype, H)
    nb = V * (H // be)
    u = splitmix64(seed, (nb * bb + 7) // 8)
    w = u.view(np.uint8)[: nb * bb].reshape(nb, bb).copy()
    for i, off in enumerate(fields):
        v = uniform53(seed + 101 + i, nb) * (scale if i == 0 else scale / 4)
        h = v.astype(np.float16).view(np.uint16)
        w[:, off] = (h & 0xFF).astype(np.uint8)
        w[:, off + 1] = (h >> 8).astype(np.uint8)
    return w.reshape(V, rb)
