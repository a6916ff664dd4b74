"""The requantization lookup tables of the HIP library against the oracle's
literal searchsorted + nearest rule (no GPU: the tables are built by host
code in librfadam8.so and evaluated there with the same lookup the kernels
use).

The window test covers dense ranges of f32 bit patterns around every
codebook entry and every decision point, plus random windows; the exhaustive
test walks every f32 pattern in [-1, 1] for both codebooks (about 3.2e9
patterns, half a minute on 8 cores).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from rollfast_amd import _lib


def _windows(cb: np.ndarray, half: int, rng, n_random: int, sign_bit: int):
    cb = cb[cb > 0] if sign_bit == 0 else -cb[cb < 0]
    mids = ((cb[:-1].astype(np.float64) + cb[1:]) / 2).astype(np.float32)
    centres = np.concatenate([cb.astype(np.float32), mids]).view(np.uint32).astype(np.int64)
    centres = np.concatenate([centres, rng.integers(0, 0x3F800000, n_random)])
    out = []
    for c in centres:
        lo = max(0, int(c) - half)
        hi = min(0x3F800000, int(c) + half)
        out.append((sign_bit | lo, hi - lo + 1))
    return out


@pytest.mark.parametrize("q,signed", [(orc.Q_SIGNED, True), (orc.Q_UNSIGNED, False)])
def test_table_codes_match_oracle_windows(q, signed):
    cb = orc.codebook(signed)
    rng = np.random.default_rng(11)
    spans = _windows(cb, 2048, rng, 64, 0)
    if signed:
        spans += _windows(cb, 2048, rng, 64, 0x80000000)
    checked = 0
    for first, count in spans:
        got = _lib.host_table_codes(q, first, count)
        want = orc.nearest_codes_bits(q, first, count)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"q={q} first=0x{first + int(bad[0]):08x} got {got[bad[0]]} want {want[bad[0]]}"
        checked += count
    assert checked > 1_000_000


@pytest.mark.parametrize("q", [orc.Q_SIGNED, orc.Q_UNSIGNED])
def test_table_codes_special_values(q):
    """+-0, denormals, values at and beyond +-1 (clipped to the end codes),
    +-Inf and NaN (code 254, the literal rule's result)."""
    pats = np.array([0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x3F800000, 0xBF800000,
                     0x3F800001, 0x40000000, 0xC0000000, 0x7F800000, 0xFF800000, 0x7FC00000,
                     0xFFC00000, 0x7F800001], np.uint32)
    got = np.array([_lib.host_table_codes(q, int(b), 1)[0] for b in pats])
    want = orc.nearest_codes_list(q, pats)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("q,lo,hi", [(orc.Q_UNSIGNED, 0x00000000, 0x3F800000),
                                     (orc.Q_SIGNED, 0x00000000, 0x3F800000),
                                     (orc.Q_SIGNED, 0x80000000, 0xBF800000)])
def test_table_codes_exhaustive(q, lo, hi):
    chunk = 1 << 26
    start = lo
    while start <= hi:
        count = min(chunk, hi - start + 1)
        got = _lib.host_table_codes(q, start, count)
        want = orc.nearest_codes_bits(q, start, count)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"first mismatch at 0x{start + int(bad[0]):08x}"
        start += count



def _search_want(cb: np.ndarray, first: int, count: int) -> np.ndarray:
    """numpy's searchsorted (side left) of n clipped to [cb[0], cb[255]] for
    the f32 patterns first .. first+count-1: the reference's ui
    (adam8.py:549-550) for finite n."""
    n = np.arange(first, first + count, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.searchsorted(cb, np.clip(n, cb[0], cb[255]), side="left").astype(np.uint16)


@pytest.mark.parametrize("q,signed", [(orc.Q_SIGNED, True), (orc.Q_UNSIGNED, False)])
def test_search_index_windows(q, signed):
    """The moment-SR lookup's searchsorted index, and the oracle's, around
    every codebook entry (where the count steps) and in random windows,
    against numpy's searchsorted on the oracle's codebook."""
    cb = orc.codebook(signed)
    rng = np.random.default_rng(12)
    spans = _windows(cb, 4096, rng, 64, 0)
    if signed:
        spans += _windows(cb, 4096, rng, 64, 0x80000000)
    for first, count in spans:
        want = _search_want(cb, first, count)
        for got in (_lib.host_search_index(q, first, count), orc.search_index_bits(q, first, count)):
            bad = np.nonzero(got != want)[0]
            assert bad.size == 0, f"q={q} first=0x{first + int(bad[0]):08x} got {got[bad[0]]} want {want[bad[0]]}"


def test_search_index_special_values():
    """+-0, denormals, +-1 and beyond (clipped), +-Inf; NaN sorts last and
    clips to 255."""
    pats = np.array([0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x3F800000, 0xBF800000,
                     0x3F800001, 0x40000000, 0xC0000000, 0x7F800000, 0xFF800000, 0x7FC00000], np.uint32)
    for q in (orc.Q_SIGNED, orc.Q_UNSIGNED):
        got = np.array([_lib.host_search_index(q, int(b), 1)[0] for b in pats])
        want = np.array([orc.search_index_bits(q, int(b), 1)[0] for b in pats])
        np.testing.assert_array_equal(got, want)
    cb = orc.codebook(True)
    assert orc.search_index_bits(orc.Q_SIGNED, 0x00000000, 1)[0] == 127   # cb[127] = 0 >= +0
    assert orc.search_index_bits(orc.Q_SIGNED, 0x80000000, 1)[0] == 127   # -0 == +0
    assert orc.search_index_bits(orc.Q_SIGNED, 0x00000001, 1)[0] == 128   # 0 < denormal <= cb[128]
    assert orc.search_index_bits(orc.Q_SIGNED, 0xBF800000, 1)[0] == 0     # -1 clips to cb[0]
    assert orc.search_index_bits(orc.Q_SIGNED, 0x7FC00000, 1)[0] == 255   # NaN
    assert cb[127] == 0.0


@pytest.mark.parametrize("q,lo,hi", [(orc.Q_UNSIGNED, 0x00000000, 0x3F800000),
                                     (orc.Q_SIGNED, 0x00000000, 0x3F800000),
                                     (orc.Q_SIGNED, 0x80000000, 0xBF800000)])
def test_search_index_exhaustive(q, lo, hi):
    """Every f32 pattern of [-1, 1] (the moment-SR kernels' range of n)
    against the oracle's searchsorted."""
    chunk = 1 << 26
    start = lo
    while start <= hi:
        count = min(chunk, hi - start + 1)
        got = _lib.host_search_index(q, start, count)
        want = orc.search_index_bits(q, start, count)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"first mismatch at 0x{start + int(bad[0]):08x}: got {got[bad[0]]} want {want[bad[0]]}"
        start += count


@pytest.mark.parametrize("q,signed", [(orc.Q_SIGNED, True), (orc.Q_UNSIGNED, False)])
def test_sr_records_and_reciprocal_quotient(q, signed):
    """The moment-SR neighbour records: per ui >= 1, cb[li], the f32 gap
    cb[ui] - cb[li] times 2^-16 and the f32 nearest to 1/gap times 2^16
    (exact rationals), so that the kernels' quotient fma(fma(-d', a*y',
    a), y', a*y') comes out as x = 65536 p.  Against IEEE a / d (numpy
    float32) over dense samples of a in [0, d] for every gap, x / 65536
    must decide the Bernoulli draw (uniform < p, uniform a multiple of
    2^-23, adam8.py:558-564) alike for every uniform value.  ui = 0
    (n <= cb[0]) holds {-2, 0, 65536}: x >= 131072 for every such n, so
    the kernel's "upper" pick is ui = 0 = li."""
    from fractions import Fraction

    cb = orc.codebook(signed)
    rec = _lib.host_sr_records(q)
    assert rec[0].tolist() == [-2.0, 0.0, 65536.0, 0.0]
    below = np.array([cb[0], np.nextafter(cb[0], np.float32(-2)), -1.0 if signed else -0.0], np.float32)
    below = below[below >= -1]
    x0 = orc.recip_quotient(below - np.float32(rec[0, 0]), float(rec[0, 1]), float(rec[0, 2]))
    assert (x0 >= 131072.0).all(), x0
    rng = np.random.default_rng(21)
    exact_equal = total = 0
    for ui in range(1, 256):
        li = ui - 1
        d = np.float32(cb[ui]) - np.float32(cb[li])
        assert d > 0.0, ui
        assert rec[ui, 0] == cb[li] and rec[ui, 1] == d * np.float32(2.0 ** -16) and rec[ui, 3] == 0.0, ui
        y = np.float32(rec[ui, 2] / np.float32(65536.0))
        assert np.float32(y * np.float32(65536.0)) == rec[ui, 2], ui
        inv = 1 / Fraction(float(d))
        err = abs(Fraction(float(y)) - inv)
        for c in (np.nextafter(y, np.float32(0)), np.nextafter(y, np.float32(np.inf))):
            assert abs(Fraction(float(c)) - inv) >= err, ui
        # a: rounded multiples k * 2^-23 * d (where p crosses the draw's grid)
        # and their neighbours, random patterns in [0, d], and the ends
        k = rng.integers(0, 1 << 23, 4000).astype(np.float64)
        base = (k * 2.0 ** -23 * float(d)).astype(np.float32)
        near = [base]
        for step in (1, 2, 3):
            up, down = base.copy(), base.copy()
            for _ in range(step):
                up = np.nextafter(up, np.float32(np.inf))
                down = np.nextafter(down, np.float32(0))
            near += [up, down]
        rand = rng.integers(0, int(np.float32(d).view(np.uint32)) + 1, 8000).astype(np.uint32).view(np.float32)
        ends = np.array([0.0, 1e-45, 2e-45, 1.2e-38, d, np.nextafter(d, np.float32(0))], np.float32)
        a = np.concatenate(near + [rand, ends])
        a = a[(a >= 0) & (a <= d)]
        got = orc.recip_quotient(a, float(rec[ui, 1]), float(rec[ui, 2])).astype(np.float64)
        want = (a / d).astype(np.float32).astype(np.float64)
        bad = np.nonzero(np.ceil(got * 2.0 ** 7) != np.ceil(want * 2.0 ** 23))[0]
        assert bad.size == 0, f"ui={ui} a={a[bad[0]]!r} x={got[bad[0]]!r} ieee={want[bad[0]]!r}"
        assert (got >= 0).all() and (got <= 65536).all()
        assert ((got > 0) == (want > 0)).all(), ui
        # x is 65536 times the IEEE quotient itself wherever p >= 2^-90;
        # below, a subnormal a makes the correction term inexact (p < 2^-96
        # there), which only the sign of p could show to the draw
        big = want >= 2.0 ** -90
        diff = np.nonzero(big & (got != want * 65536.0))[0]
        assert diff.size == 0, f"ui={ui} a={a[diff[0]]!r} x={got[diff[0]]!r} ieee={want[diff[0]]!r}"
        exact_equal += int(np.sum(got == want * 65536.0))
        total += a.size
    assert exact_equal > 0.99 * total, (exact_equal, total)
