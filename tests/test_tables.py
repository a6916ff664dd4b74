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
