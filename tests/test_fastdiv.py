"""The multiply-high division the kernels use for point -> batch / camera /
pixel indices (``FastDiv`` in ``csrc/bevpool.hip``; Granlund & Montgomery,
"Division by invariant integers using multiplication", 1994):

    s = ceil(log2 d),  m = floor(2^32 (2^s - d) / d) + 1,
    n / d = (mulhi32(n, m) + n) >> s          for 0 <= n < 2^31, 1 <= d <= 2^31.

Checked against exact integer division over every divisor up to 4096, all
powers of two and their neighbours, the divisors the benchmark shapes use,
and random divisors, at numerators chosen where an off-by-one would show:
0, multiples of d and their neighbours, and the top of the range."""
from __future__ import annotations

import numpy as np


def magic(d: int):
    s = 0
    while (1 << s) < d:
        s += 1
    m = ((1 << 32) * ((1 << s) - d)) // d + 1
    assert 0 <= m < (1 << 32)
    return m, s


def fast_div(n: np.ndarray, d: int) -> np.ndarray:
    m, s = magic(d)
    hi = (n.astype(np.uint64) * np.uint64(m)) >> np.uint64(32)
    total = hi + n.astype(np.uint64)
    assert int(total.max()) < (1 << 32)  # the 32-bit sum does not overflow
    return (total >> np.uint64(s)).astype(np.int64)


def numerators(d: int, rng) -> np.ndarray:
    top = (1 << 31) - 1
    k = np.unique(np.concatenate([np.arange(0, 64), rng.integers(0, top // d + 1, 512),
                                  [top // d - 1, top // d]]))
    k = k[(k >= 0) & (k <= top // d)]
    base = k * d
    n = np.concatenate([base, base - 1, base + 1, base + d - 1,
                        [0, 1, top, top - 1, top - d], rng.integers(0, top, 256)])
    return np.unique(n[(n >= 0) & (n <= top)]).astype(np.int64)


def divisors(rng):
    ds = set(range(1, 4097))
    for e in range(1, 32):
        ds.update({(1 << e) - 1, 1 << e, (1 << e) + 1})
    # det / hires frustum: D*fH*fW, cameras per batch, points per batch
    ds.update({118 * 32 * 88, 118 * 64 * 176, 6, 6 * 118 * 32 * 88, 6 * 118 * 64 * 176,
               32 * 88, 64 * 176, 118})
    ds.update(int(v) for v in rng.integers(1, 1 << 31, 2000))
    return sorted(d for d in ds if 1 <= d <= (1 << 31))


def test_fast_div_matches_integer_division():
    rng = np.random.default_rng(7)
    for d in divisors(rng):
        n = numerators(d, rng)
        np.testing.assert_array_equal(fast_div(n, d), n // d, err_msg=f'd={d}')


def test_fast_div_catches_a_wrong_magic():
    """A magic number one too small breaks the identity for some divisor:
    the check above can fail."""
    rng = np.random.default_rng(8)
    broken = 0
    for d in (3, 7, 11, 118 * 32 * 88, 100003):
        m, s = magic(d)
        n = numerators(d, rng)
        hi = (n.astype(np.uint64) * np.uint64(m - 1)) >> np.uint64(32)
        q = ((hi + n.astype(np.uint64)) >> np.uint64(s)).astype(np.int64)
        broken += int(np.any(q != n // d))
    assert broken > 0
