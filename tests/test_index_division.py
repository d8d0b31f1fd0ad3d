"""The kernels divide block and row indices by the slice count S with a
32-bit reciprocal: umulhi(g, m) with m = floor(2^32 / S) + 1 (S > 1; S = 1
divides by 1 directly), and window positions by W the same way. The host
accepts a batch only when every index the kernels divide stays below
2^32 / S. These checks pin that arithmetic (numpy, exhaustive at the edges
of each quotient and dense random samples) against integer division."""
import numpy as np


def umulhi(g, m):
    return (g.astype(np.uint64) * np.uint64(m)) >> np.uint64(32)


def magic(d):
    return (1 << 32) // d + 1


def test_reciprocal_division_is_exact_below_the_bound():
    rng = np.random.default_rng(0)
    for d in list(range(2, 300)) + [1000, 4096, 65535]:
        m = magic(d)
        assert m < (1 << 32)
        limit = (1 << 32) // d          # the host keeps every index below this
        g = rng.integers(0, limit, size=20000, dtype=np.uint64)
        q = np.arange(0, limit // d + 1, max(1, limit // d // 2000), dtype=np.uint64)
        edges = np.concatenate([q * d, q * d + d - 1, g])
        edges = edges[edges < limit]
        np.testing.assert_array_equal(umulhi(edges, m), edges // np.uint64(d), err_msg=f"d={d}")


def test_host_bound_covers_the_largest_indices():
    # (B + 2) * S * (S + 8) < 2^32 on the host: the largest block index
    # (rows * S rounded up to 8 XCDs) plus S, times S, stays below 2^32
    for B in (1, 64, 1024, 4096):
        for S in (1, 2, 12, 19, 64, 256):
            if (B + 2) * S * (S + 8) >= (1 << 32):
                continue
            g_max = ((B * S + 7) // 8) * 8 + S
            assert g_max * S < (1 << 32)
