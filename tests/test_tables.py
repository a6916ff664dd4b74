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
