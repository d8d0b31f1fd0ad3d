"""The exact-sum engine of k_full on the GPU (tests/cpp/xsum_kit.hip).

softmax_probs (reference src/sampler/sampler.cpp:124-142) and apply_top_p
(:146-164) take float32 running sums over up to V values; k_full reproduces
them in parallel from integer increments per binade. Here the engine runs on
sequences built to stress it -- sums that cross many binades, values exactly
half-way between two multiples of the running sum's ulp (round half to even),
subnormals, zeros, equal values, single huge values, a sequence longer than
one window table (512-id windows of two steps) -- and must give numpy's
sequential float32 sums (np.add.accumulate is a plain left-to-right loop)
bit for bit, and the top-p driver the exact cutoff of the descending order.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _kit(pkg):
    import torch  # noqa: F401  (first: the kit binds to torch's HIP runtime, one per process)
    lib = ctypes.CDLL(str(pkg.hsamp.PKG.parent / "tests" / "cpp" / "libxsum_kit.so"))
    lib.xsum_run.restype = ctypes.c_int
    lib.xsum_run.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                             ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    lib.xinc_run.restype = ctypes.c_int
    lib.xinc_run.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    return lib


def _run(kit, x, thr, known_range=False):
    import torch
    n = x.size
    w512 = (n + 511) // 512
    G = max(1, (w512 + 2047) // 2048)
    ws = 512 * G
    Vp = (n + ws - 1) // ws * ws
    xp = np.zeros(Vp, np.float32)
    xp[:n] = x
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(xp).to(dev)
    out = torch.zeros(4, dtype=torch.float32, device=dev)
    outi = torch.zeros(4, dtype=torch.int32, device=dev)
    rlo = rhi = 0
    if known_range and np.any(x > 0):
        pos = x[x > 0]
        rlo, rhi = int(pos.min().view(np.uint32)), int(pos.max().view(np.uint32))
    rc = kit.xsum_run(xd.data_ptr(), n, Vp, G, float(thr), rlo, rhi, out.data_ptr(), outi.data_ptr())
    assert rc == 0, f"xsum_run: HIP status {rc}"
    return out.cpu().numpy(), outi.cpu().numpy()


def _seq(x):
    return np.add.accumulate(x.astype(np.float32), dtype=np.float32)


def _cases():
    rng = np.random.default_rng(2024)
    c = {}
    c["flat"] = np.exp(rng.normal(0, 0.1, 151936)).astype(np.float32)
    c["spiky"] = np.exp(rng.normal(0, 1, 151936) - 15).astype(np.float32)
    c["spiky"][rng.choice(151936, 16, replace=False)] = 1.0
    # multiples of 2^-20: increments land exactly half-way once the sum passes 2^4
    c["halfway"] = (rng.integers(1, 64, 120000) * 2.0**-20).astype(np.float32)
    c["halfway"][::7] = 2.0**-20
    c["subnormal"] = (rng.random(50000) * 1e-39).astype(np.float32)
    z = np.exp(rng.normal(0, 3, 80000)).astype(np.float32)
    z[rng.random(80000) < 0.3] = 0.0
    c["zeros_wide"] = z
    c["equal"] = np.full(151936, np.float32(6.5e-6))
    w = np.exp(rng.normal(0, 0.1, 151936)).astype(np.float32)
    w[1234] = np.float32(3e4)
    c["one_huge"] = w
    t = np.exp(rng.normal(-30, 0.1, 151936)).astype(np.float32)
    t[5] = np.float32(1e-44)
    c["outlier_range"] = t
    # nearly equal values: the sum crosses many binades inside buckets of one increment
    c["narrow"] = np.exp(rng.normal(0, 0.01, 151936)).astype(np.float32)
    # mantissas ending in 12 or more zero bits: the crossing add and half-way values at every binade
    c["coarse"] = (rng.integers(2**11, 2**12, 151936) * 2.0**-12).astype(np.float32)
    c["long"] = np.exp(rng.normal(0, 0.5, 1_200_000)).astype(np.float32)     # 2-step windows
    c["tiny"] = np.array([3.0, 0.0, 1e-8], np.float32)
    return c


CASES = _cases()


@pytest.mark.parametrize("name", list(CASES))
def test_exact_index_sum(pkg, name):
    kit = _kit(pkg)
    x = CASES[name]
    out, _ = _run(kit, x, 0.0)
    want = _seq(x)[-1]
    assert out[0].view(np.uint32) == want.view(np.uint32), f"{name}: {out[0]!r} != {want!r}"


@pytest.mark.parametrize("known_range", [False, True])
@pytest.mark.parametrize("name", [n for n in CASES if n not in ("long", "tiny")])
@pytest.mark.parametrize("frac", [0.9, 0.5, 0.999])
def test_top_p_cutoff(pkg, name, frac, known_range):
    kit = _kit(pkg)
    x = CASES[name]
    xs = np.sort(x)[::-1]
    cum = _seq(xs)
    thr = np.float32(frac * float(cum[-1]))
    out, outi = _run(kit, x, float(thr), known_range)
    hit = np.nonzero(cum >= thr)[0]
    assert outi[0] == (1 if hit.size else 0), name
    if hit.size:
        j = int(hit[0])
        assert outi[1] == j + 1, f"{name}: cut after {outi[1]} values, want {j + 1}"
        assert out[1].view(np.uint32) == xs[j].view(np.uint32), name
        assert out[2].view(np.uint32) == cum[j].view(np.uint32), name
        # the values above the cut's and equal to it (the removal's tie rule)
        assert outi[2] == int(np.count_nonzero(x > xs[j])), name
        assert outi[3] == int(np.count_nonzero(x == xs[j])), name


@pytest.mark.parametrize("E", [-126, -40, -17, -1, 0, 9, 16, 30])
def test_float_increments_match_integer_ones(pkg, E):
    """The increments k_fs_exp takes by float arithmetic (ldexp, floor; and
    the plain increment away from one half, by rounding to nearest) are the
    integer ones (xinc2) for every kind of value at binade E: far below the
    sum's ulp, exactly half-way between two multiples of it at every scale,
    just beside half-way, within the binade, at and past its top, zeros and
    subnormals."""
    import torch
    kit = _kit(pkg)
    rng = np.random.default_rng(1000 + E)
    vals = [np.float32(0.0), np.float32(1e-45), np.float32(1e-39)]
    for d in range(-3, 27):           # x = m * 2^(E - d) for mantissas m in [1, 2)
        sc = np.float32(2.0) ** np.float32(np.clip(E - d, -149, 127))
        m = rng.uniform(1.0, 2.0, 64).astype(np.float32)
        vals += list((m * sc).astype(np.float32))
    for top in (4, 12, 20):           # (k + 1/2) ulps of binade E, k < 2^top, and their neighbours
        k = rng.integers(0, 1 << top, 32)
        h = ((k * 2 + 1).astype(np.float64) * 2.0 ** (E - 24)).astype(np.float32)
        vals += list(h) + list(np.nextafter(h, np.float32(np.inf))) + list(np.nextafter(h, np.float32(0)))
    x = np.array([v for v in vals if np.isfinite(v)], np.float32)
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(x).to(dev)
    out = torch.zeros(4 * x.size, dtype=torch.int32, device=dev)
    rc = kit.xinc_run(xd.data_ptr(), x.size, E, out.data_ptr())
    assert rc == 0
    o = out.cpu().numpy().view(np.uint32).reshape(-1, 4)
    bad = np.nonzero((o[:, 0] != o[:, 2]) | (o[:, 1] != o[:, 3]))[0]
    assert bad.size == 0, f"E={E}: x={x[bad[:4]]!r} int={o[bad[:4], :2]} float={o[bad[:4], 2:]}"
