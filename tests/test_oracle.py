"""Pinning of the CPU oracle (no GPU).

Each test fixes one oracle function by something other than the oracle's own
formula: published known-answer vectors (Random123), exact rational
arithmetic (codebooks), brute force over all 256 codebook entries (nearest
code), the exact expectation over every noise value (bf16 stochastic
rounding), float64 textbook AdamW (fallback moments), and the reference's
own tolerance and property tests (rollfast tests/test_adam8.py,
tests/test_utils.py).
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as orc


# ------------------------------------------------------------ threefry ----
# Random123 kat_vectors, threefry2x32 with 20 rounds (the cipher under
# jax.random's default PRNG; the same three vectors appear in JAX's own
# random tests).
THREEFRY_KATS = [
    ((0x00000000, 0x00000000), (0x00000000, 0x00000000), (0x6B200159, 0x99BA4EFE)),
    ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
    ((0x13198A2E, 0x03707344), (0x243F6A88, 0x85A308D3), (0xC4923A9C, 0x483DF7A0)),
]


@pytest.mark.parametrize("key,ctr,want", THREEFRY_KATS)
def test_threefry2x32_known_answers(key, ctr, want):
    assert orc.threefry2x32(key, ctr) == want


def test_random_bits_and_split_layout():
    """bits[i] = y0 ^ y1 of threefry(key, (hi32(i), lo32(i))); split(key)[i] =
    threefry(key, (0, i)).  Checked element by element against the KAT-pinned
    block function, including an offset that crosses 2^32."""
    key = (0x13198A2E, 0x03707344)
    bits = orc.random_bits(key, 8, offset=(1 << 32) - 4)
    for i, b in enumerate(bits):
        idx = (1 << 32) - 4 + i
        y0, y1 = orc.threefry2x32(key, (idx >> 32, idx & 0xFFFFFFFF))
        assert int(b) == y0 ^ y1
    sub = orc.split(key, 5)
    for i in range(5):
        assert tuple(int(v) for v in sub[i]) == orc.threefry2x32(key, (0, i))


# jax.random.split(jax.random.PRNGKey(0)) as JAX prints it (uint32[2, 2]):
# under the default jax_threefry_partitionable layout (JAX >= 0.5, the
# reference's jax>=0.6.2), and under the legacy layout JAX used before.
SPLIT_KEY0_PARTITIONABLE = [[1797259609, 2579123966], [928981903, 3453687069]]
SPLIT_KEY0_LEGACY = [[4146024105, 967050713], [2718843009, 1272950319]]


def test_split_of_prngkey0_is_jax_partitionable_value():
    """The oracle's split (adam8.py:274, :306, :645; utils.py:682) gives JAX's
    published split(PRNGKey(0)).  Counters (i, 0) instead of (0, i), or the
    legacy iota layout, give other words and fail here."""
    assert orc.split((0, 0), 2).tolist() == SPLIT_KEY0_PARTITIONABLE
    swapped = [list(orc.threefry2x32((0, 0), (i, 0))) for i in range(2)]
    assert swapped != SPLIT_KEY0_PARTITIONABLE
    assert SPLIT_KEY0_LEGACY != SPLIT_KEY0_PARTITIONABLE


def test_legacy_split_layout_cross_checks_the_block_function():
    """The legacy layout of split(key, n): counters iota(2n) cut in halves
    (x0 = 0..n-1, x1 = n..2n-1), the cipher's y0 words then its y1 words,
    reshaped to [n, 2].  Built from the oracle's block function it gives
    JAX's published legacy split(PRNGKey(0)): a second published vector
    through the same cipher, with other counters than the Random123 ones."""
    n = 2
    ys = [orc.threefry2x32((0, 0), (i, n + i)) for i in range(n)]
    flat = [y[0] for y in ys] + [y[1] for y in ys]
    assert [flat[0:2], flat[2:4]] == SPLIT_KEY0_LEGACY


def test_uniform_of_prngkey0_legacy_value():
    """jax.random.uniform(PRNGKey(0)) of the legacy layout is 0.41845703
    (JAX's printed value): the scalar's bits are y0 of threefry(key, (0, 0)),
    the Random123 zero vector's 0x6B200159, and uniform's mantissa fill
    (bits >> 9 | 0x3F800000) - 1 (the Bernoulli draw of adam8.py:458, :564)
    maps it to 3510272 / 2^23 exactly."""
    y0, _ = orc.threefry2x32((0, 0), (0, 0))
    assert y0 == 0x6B200159
    u = orc.uniform01(np.array([y0], np.uint32))[0]
    assert u == np.float32(3510272 / 2 ** 23)
    assert abs(float(u) - 0.41845703) < 5e-9


# ------------------------------------------------------------ codebooks ---
def _exact_codebook(signed: bool) -> np.ndarray:
    """The dynamic codebook of rollfast optim/adam8.py:465-503 in exact
    rational arithmetic: 7 decades 10^(index-6) times the midpoints of
    linspace(0.1, 1, k) (k = 2^index + 1 signed, 2^(index+1) + 1 unsigned),
    mirrored when signed, plus 0 and 1; then rounded once to f32."""
    vals = []
    for index in range(7):
        scale = Fraction(10) ** (index - 6)
        points = 2 ** index + 1 if signed else 2 ** (index + 1) + 1
        step = (Fraction(1) - Fraction(1, 10)) / (points - 1)
        for k in range(points - 1):
            mid = Fraction(1, 10) + step * k + step / 2
            vals.append(scale * mid)
            if signed:
                vals.append(-scale * mid)
    vals += [Fraction(0), Fraction(1)]
    assert len(vals) == 256
    vals.sort()
    return np.array([float(v) for v in vals], dtype=np.float64).astype(np.float32)


@pytest.mark.parametrize("signed", [True, False])
def test_codebook_matches_exact_rational_construction(signed):
    got = orc.codebook(signed)
    want = _exact_codebook(signed)
    assert got.dtype == np.float32 and got.shape == (256,)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_codebook_reference_facts():
    s = orc.codebook(True)
    u = orc.codebook(False)
    assert np.all(np.diff(s) > 0) and np.all(np.diff(u) > 0)
    assert s[0] == np.float32(-0.99296874) and s[127] == 0.0 and s[255] == 1.0
    assert s[128] == np.float32(5.5e-7) and s[126] == np.float32(-5.5e-7)
    assert u[0] == 0.0 and u[1] == np.float32(3.25e-7) and u[255] == 1.0
    assert u[254] == np.float32(0.9964844)
    # zero codes: argmin |cb| (adam8.py:532-539; tests/test_adam8.py:62,82)
    assert int(np.argmin(np.abs(s))) == 127 and int(np.argmin(np.abs(u))) == 0


# ---------------------------------------------------------- nearest code --
def _brute_nearest(cb: np.ndarray, n: np.ndarray) -> np.ndarray:
    """argmin_i fl(|cb_i - clip(n)|) over all 256 entries, ties to the lower
    index (np.argmin returns the first minimum)."""
    n = np.clip(n.astype(np.float32), cb[0], cb[255]).astype(np.float32)
    d = np.abs(cb[None, :] - n[:, None]).astype(np.float32)
    return np.argmin(d, axis=1).astype(np.uint8)


def _probe_values(cb: np.ndarray, rng) -> np.ndarray:
    """Every codebook entry and every f32 midpoint of neighbours, each with
    its 3 f32 neighbours either side, plus uniform and log-uniform samples."""
    pts = [cb]
    mids = ((cb[:-1].astype(np.float64) + cb[1:].astype(np.float64)) / 2).astype(np.float32)
    pts.append(mids)
    base = np.concatenate(pts).astype(np.float32)
    near = [base]
    for k in range(1, 4):
        up = base.copy()
        dn = base.copy()
        for _ in range(k):
            up = np.nextafter(up, np.float32(np.inf))
            dn = np.nextafter(dn, np.float32(-np.inf))
        near += [up, dn]
    lo = float(cb[0])
    near.append(rng.uniform(lo, 1.0, 20000).astype(np.float32))
    mag = np.exp(rng.uniform(np.log(1e-9), 0.0, 20000)).astype(np.float32)
    near.append(mag if lo >= 0 else mag * rng.choice([-1, 1], mag.size).astype(np.float32))
    near.append(np.array([-2.0, -1.0, 1.5, 3.0, 0.0, -0.0], np.float32))  # clipped to the ends
    return np.concatenate(near).astype(np.float32)


@pytest.mark.parametrize("q,signed", [(orc.Q_SIGNED, True), (orc.Q_UNSIGNED, False)])
def test_nearest_code_brute_force(q, signed):
    cb = orc.codebook(signed)
    vals = _probe_values(cb, np.random.default_rng(1))
    got = orc.nearest_codes_list(q, vals.view(np.uint32))
    np.testing.assert_array_equal(got, _brute_nearest(cb, vals))


def test_nearest_code_ties_go_to_the_lower_code():
    """An input exactly halfway (in f32 distances) between two entries takes
    the lower code (adam8.py:566-569 uses a strict <)."""
    cb = orc.codebook(True)
    found = 0
    for i in range(255):
        lo, hi = cb[i], cb[i + 1]
        m = np.float32((np.float64(lo) + np.float64(hi)) / 2)
        if np.float32(abs(hi - m)) == np.float32(abs(m - lo)):
            assert orc.nearest_code(orc.Q_SIGNED, m) == i
            found += 1
    assert found > 100


def test_nearest_code_nan_is_code_254():
    """searchsorted puts NaN past the end (index 256 -> clipped 255); the
    strict compare against NaN is false, so the lower neighbour 254 wins.
    Documented choice: jnp.searchsorted on NaN is parity unpinned."""
    assert orc.nearest_code(orc.Q_SIGNED, float("nan")) == 254
    assert orc.nearest_code(orc.Q_UNSIGNED, float("nan")) == 254


# ------------------------------------------------ quantize / dequantize ---
def test_symmetric_int8_error_bounded_by_half_scale():
    """tests/test_adam8.py:18-42: linspace(-3, 2, 513), block 128."""
    x = np.linspace(-3.0, 2.0, 513, dtype=np.float32)
    codes, scales = orc.quantize(x, 128, orc.Q_SYMMETRIC)
    assert codes.dtype == np.int8 and scales.dtype == np.float32
    assert codes.min() >= -127 and codes.max() <= 127
    back = orc.dequantize(codes, scales, x.size, 128, orc.Q_SYMMETRIC)
    assert np.max(np.abs(back - x)) <= np.max(scales) / 2 + 1e-6


def test_dynamic_signed_error_bound():
    """tests/test_adam8.py:45-65."""
    x = np.linspace(-3.0, 2.0, 513, dtype=np.float32)
    codes, scales = orc.quantize(x, 128, orc.Q_SIGNED)
    assert codes.dtype == np.uint8 and codes.shape == (5, 128)
    back = orc.dequantize(codes, scales, x.size, 128, orc.Q_SIGNED)
    assert np.max(np.abs(back - x)) <= np.max(scales) * 0.01


def test_dynamic_unsigned_nonnegative_and_error_bound():
    """tests/test_adam8.py:68-84."""
    x = np.linspace(0.0, 3.0, 513, dtype=np.float32)
    codes, scales = orc.quantize(x, 128, orc.Q_UNSIGNED)
    back = orc.dequantize(codes, scales, x.size, 128, orc.Q_UNSIGNED)
    assert back.min() >= 0.0
    assert np.max(np.abs(back - x)) <= np.max(scales) * 0.01


def test_quantize_literal_definition():
    """scale = absmax (1 for an all-zero block), code = nearest(clip(x /
    scale)) with IEEE f32 division, padding codes = the zero code
    (adam8.py:113-187)."""
    rng = np.random.default_rng(3)
    bs = 64
    x = (rng.standard_normal(5 * bs - 17) * 0.3).astype(np.float32)
    x[bs:2 * bs] = 0.0  # a zero block
    cb = orc.codebook(True)
    codes, scales = orc.quantize(x, bs, orc.Q_SIGNED)
    xp = np.zeros(5 * bs, np.float32)
    xp[:x.size] = x
    blocks = xp.reshape(5, bs)
    amax = np.max(np.abs(blocks), axis=1)
    want_scales = np.where(amax > 0, amax, np.float32(1.0)).astype(np.float32)
    np.testing.assert_array_equal(scales, want_scales)
    norm = (blocks / want_scales[:, None]).astype(np.float32)
    want_codes = _brute_nearest(cb, norm.reshape(-1)).reshape(5, bs)
    np.testing.assert_array_equal(codes, want_codes)
    assert np.all(codes.reshape(-1)[x.size:] == 127)
    assert np.all(codes[1] == 127) and scales[1] == 1.0


def test_dequantize_closed_form():
    rng = np.random.default_rng(4)
    bs = 32
    codes = rng.integers(0, 256, size=(3, bs), dtype=np.uint8)
    scales = rng.uniform(0.1, 2.0, 3).astype(np.float32)
    for q, signed in ((orc.Q_SIGNED, True), (orc.Q_UNSIGNED, False)):
        cb = orc.codebook(signed)
        got = orc.dequantize(codes, scales, 3 * bs - 5, bs, q)
        want = (cb[codes] * scales[:, None]).astype(np.float32).reshape(-1)[:3 * bs - 5]
        np.testing.assert_array_equal(got, want)
    sym = codes.view(np.int8)
    got = orc.dequantize(sym, scales, 3 * bs, bs, orc.Q_SYMMETRIC)
    np.testing.assert_array_equal(got, (sym.astype(np.float32) * scales[:, None]).reshape(-1))


def test_moment_sr_upper_probability():
    """Codebook SR picks the upper neighbour with probability
    (n - cb_l) / (cb_u - cb_l) (adam8.py:557-564): a fixed value repeated
    over 2^17 random draws lands within 5 sigma of that rate."""
    cb = orc.codebook(True)
    i = 200
    n = np.float32(cb[i] + np.float32(0.3) * (cb[i + 1] - cb[i]))
    p = float((np.float64(n) - cb[i]) / (np.float64(cb[i + 1]) - cb[i]))
    bs = 1024
    count = 128 * bs
    x = np.full(count, n, np.float32)
    x[::bs] = 1.0  # absmax of every block is exactly 1: normalised value stays n
    bits = orc.random_bits((7, 11), count)
    codes, _ = orc.quantize(x, bs, orc.Q_SIGNED, bits=bits)
    sel = np.ones(count, bool)
    sel[::bs] = False
    c = codes.reshape(-1)[sel]
    assert set(np.unique(c).tolist()) <= {i, i + 1}
    rate = np.mean(c == i + 1)
    sigma = np.sqrt(p * (1 - p) / c.size)
    assert abs(rate - p) < 5 * sigma


# ------------------------------------------------------------ bf16 SR -----
def test_sr_bf16_exhaustive_noise_is_exactly_unbiased():
    """Over all 2^16 noise values, (x + noise) & 0xFFFF0000 averages to x
    exactly for every finite x (utils.py:365-371)."""
    rng = np.random.default_rng(5)
    xs = np.concatenate([
        rng.standard_normal(24).astype(np.float32),
        (rng.standard_normal(8) * 1e-30).astype(np.float32),
        np.array([1.0 + 2.0 ** -9, -3.0e38, 1e-40, -1e-42, 0.0], np.float32),
    ]).astype(np.float32)
    noise = np.arange(1 << 16, dtype=np.uint32)
    for x in xs:
        out = orc.sr_bf16(np.full(noise.size, x, np.float32), noise)
        vals = orc.bf16_bits_to_f32(out).astype(np.float64)
        assert vals.sum() == np.float64(x) * (1 << 16), x


def test_sr_bf16_specials():
    noise = np.array([0, 1, 0x7FFF, 0x8000, 0xFFFF, 0x12345678], np.uint32)
    for x, want in ((np.inf, 0x7F80), (-np.inf, 0xFF80)):
        out = orc.sr_bf16(np.full(noise.size, x, np.float32), noise)
        assert np.all(out == want)
    # NaN: the noise is zeroed and the low 16 bits truncated, so a quiet NaN
    # stays a NaN and a payload only in the low half collapses to Inf.
    q = np.array([0x7FC00000], np.uint32).view(np.float32)
    assert np.all(orc.sr_bf16(np.repeat(q, 6), noise) == 0x7FC0)
    low = np.array([0x7F800001], np.uint32).view(np.float32)
    assert np.all(orc.sr_bf16(np.repeat(low, 6), noise) == 0x7F80)
    # the largest finite value can round up to +Inf (no saturation)
    big = np.array([0x7F7FFFFF], np.uint32).view(np.float32)
    assert orc.sr_bf16(big, np.array([1], np.uint32))[0] == 0x7F80


def test_sr_bf16_sub_ulp_signal_kat():
    """tests/test_utils.py:89-103: ones(4096) bf16 + 2^-9 stays 1.0 under
    nearest-even and moves up under stochastic rounding."""
    n = 4096
    p = orc.f32_to_bf16_bits(np.ones(n, np.float32))
    det = p.copy()
    orc.apply_updates(det, orc.BF16, np.full(n, 2.0 ** -9, np.float32))
    assert np.all(det == 0x3F80)
    sr = p.copy()
    orc.apply_updates(sr, orc.BF16, np.full(n, 2.0 ** -9, np.float32), bits=orc.random_bits((0, 0), n))
    v = orc.bf16_bits_to_f32(sr)
    assert np.any(v > 1.0) and v.mean() > 1.0
    # E[SR] = 1 + 2^-9: 1/4 of the draws move to 1 + 2^-7
    assert abs(np.mean(v > 1.0) - 0.25) < 5 * np.sqrt(0.25 * 0.75 / n)


def test_f32_to_bf16_round_to_nearest_even():
    x = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20, -2.5, np.inf], np.float32)
    want = np.array([0x3F80, 0x3F82, 0x3F81, 0xC020, 0x7F80], np.uint16)
    np.testing.assert_array_equal(orc.f32_to_bf16_bits(x), want)


# ---------------------------------------------------------- the step ------
def _textbook_adamw(p, grads, *, b1, b2, eps, eps_root, wd, lr):
    """float64 AdamW as optax.adamw defines it (tests/test_adam.py:32-47)."""
    p = p.astype(np.float64).copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for t, g in enumerate(grads, start=1):
        g = g.astype(np.float64)
        m = b1 * m + (1 - b1) * g
        v = b2 * v + (1 - b2) * g * g
        mh = m / (1 - b1 ** t)
        vh = v / (1 - b2 ** t)
        u = mh / (np.sqrt(vh + eps_root) + eps) + wd * p
        p = p - lr * u
    return p


def test_fallback_leaf_matches_textbook_adamw():
    """f32 params with f32 (unquantized) moments: three oracle steps agree
    with float64 AdamW to f32 rounding (reference anchor: exact fallback
    check, tests/finetune/test_adamw8_from_plan.py:196-201, atol 1e-7)."""
    rng = np.random.default_rng(6)
    n = 3000
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    grads = [(rng.standard_normal(n) * 1e-2).astype(np.float32) for _ in range(3)]
    p = p0.copy()
    mu = np.zeros(n, np.float32)
    nu = np.zeros(n, np.float32)
    for t, g in enumerate(grads, start=1):
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=t, decay=True, apply=True)
        orc.adam8_leaf(hp, p, orc.F32, g, orc.F32, orc.MOM_F32, mu, None, nu, None)
    want = _textbook_adamw(p0, grads, b1=0.9, b2=0.999, eps=1e-8, eps_root=0.0, wd=0.01, lr=1e-3)
    np.testing.assert_allclose(p, want, rtol=0, atol=1e-7)


def test_adamw8_second_step_is_close_to_fp32_adamw():
    """tests/test_adam8.py:121-149: 64x64 linspace params, grads 0.125,
    eps 1e-6, block 256, min_size 1; the second step's updates of the
    quantized optimizer match fp32 AdamW within rtol 0.03, atol 3e-4."""
    n = 4096
    p0 = np.linspace(-1.0, 1.0, n, dtype=np.float32)
    g = np.full(n, 0.125, np.float32)
    kw = dict(b1=0.9, b2=0.999, eps=1e-6, weight_decay=0.01, lr=1e-3, decay=True)
    # quantized
    mu = np.full(n, 127, np.uint8)
    nu = np.zeros(n, np.uint8)
    ms = np.ones(16, np.float32)
    vs = np.ones(16, np.float32)
    p = p0.copy()
    upd = np.empty(n, np.float32)
    orc.adam8_leaf(orc.make_hparams(count=1, **kw), p, orc.F32, g, orc.F32, orc.MOM_QUANT, mu, ms, nu, vs, 256,
                   updates_out=upd)
    p1 = (p0 + upd).astype(np.float32)
    upd_q = np.empty(n, np.float32)
    orc.adam8_leaf(orc.make_hparams(count=2, **kw), p1.copy(), orc.F32, g, orc.F32, orc.MOM_QUANT, mu, ms, nu, vs,
                   256, updates_out=upd_q)
    # fp32 reference, float64 arithmetic
    b1, b2, eps, wd, lr = 0.9, 0.999, 1e-6, 0.01, 1e-3
    m = (1 - b1) * 0.125
    v = (1 - b2) * 0.125 ** 2
    u1 = -lr * ((m / (1 - b1)) / (np.sqrt(v / (1 - b2)) + eps) + wd * p0.astype(np.float64))
    pf = p0 + u1
    m = b1 * m + (1 - b1) * 0.125
    v = b2 * v + (1 - b2) * 0.125 ** 2
    u2 = -lr * ((m / (1 - b1 ** 2)) / (np.sqrt(v / (1 - b2 ** 2)) + eps) + wd * pf)
    np.testing.assert_allclose(upd_q, u2, rtol=0.03, atol=3e-4)


def test_quantized_moments_track_fp32_moments():
    """After 5 quantized steps the dequantized moments stay within the
    accumulated codebook resolution of the float64 moments: each
    requantization adds at most 0.01 * scale (the reference's quantizer
    bound, tests/test_adam8.py:65,84) and the EMA scales earlier errors by
    b < 1, so 5 steps stay within 5 * 0.01 * max scale."""
    rng = np.random.default_rng(8)
    n, bs = 8192, 2048
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    mu = np.full(n, 127, np.uint8)
    nu = np.zeros(n, np.uint8)
    ms = np.ones(n // bs, np.float32)
    vs = np.ones(n // bs, np.float32)
    m = np.zeros(n)
    v = np.zeros(n)
    for t in range(1, 6):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        m = 0.9 * m + 0.1 * g
        v = 0.999 * v + 0.001 * g.astype(np.float64) ** 2
        orc.adam8_leaf(orc.make_hparams(count=t, lr=1e-3, apply=True), p, orc.F32, g, orc.F32, orc.MOM_QUANT,
                       mu, ms, nu, vs, bs)
    md = orc.dequantize(mu, ms, n, bs, orc.Q_SIGNED)
    vd = orc.dequantize(nu, vs, n, bs, orc.Q_UNSIGNED)
    for got, want, sc in ((md, m, ms), (vd, v, vs)):
        err = np.abs(got - want).reshape(-1, bs).max(axis=1)
        assert np.all(err <= 5 * 0.01 * sc), (err, sc)
        assert np.all(err > 0)  # the moments really are quantized


# ------------------------------------------- full-precision AdamW (adam.py) --
def _bc(b, t) -> float:
    """1 - b**t as JAX evaluates it for a Python-float b and an int32 count:
    in f32 from f32(b) (optax and rollfast alike; its bits against XLA's pow
    are parity unpinned)."""
    return float(np.float32(1.0) - np.power(np.float32(b), np.float32(t)))


def _textbook_adam_updates(p, grads, *, b1, b2, eps, wd=0.0, lr=None, mask=True, nesterov=False):
    """optax.scale_by_adam / optax.adamw direction in float64 (bias-correction
    factors as JAX computes them), params advanced by the updates when lr is
    given."""
    p = p.astype(np.float64).copy()
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    outs = []
    for t, g in enumerate(grads, start=1):
        g = g.astype(np.float64)
        m = b1 * m + (1 - b1) * g
        v = b2 * v + (1 - b2) * g * g
        if nesterov:
            mh = b1 * m / _bc(b1, t + 1) + (1 - b1) * g / _bc(b1, t)
        else:
            mh = m / _bc(b1, t)
        u = mh / (np.sqrt(v / _bc(b2, t)) + eps)
        if lr is not None:
            u = -lr * (u + (wd * p if mask else 0.0))
            p = p + u
        outs.append(u)
    return outs


def _oracle_adam_steps(p, grads, *, lr=None, wd=0.0, decay=False, nesterov=False, eps=1e-8):
    p = p.astype(np.float32).copy()
    mu = np.zeros(p.size, np.float32)
    nu = np.zeros(p.size, np.float32)
    outs = []
    for t, g in enumerate(grads, start=1):
        upd = np.empty(p.size, np.float32)
        hp = orc.make_hparams(eps=eps, weight_decay=wd, lr=lr, count=t, decay=decay, nesterov=nesterov,
                              ema_weight_f32=True)
        orc.adam8_leaf(hp, p.copy(), orc.F32, g.astype(np.float32), orc.F32, orc.MOM_F32, mu, None, nu, None,
                       updates_out=upd)
        outs.append(upd)
        p = (p + upd).astype(np.float32)
    return outs


@pytest.mark.parametrize("nesterov", [False, True])
def test_scale_by_adam_matches_textbook_direction(nesterov):
    """tests/test_adam.py:32-47: three steps of scale_by_adam against
    optax.scale_by_adam's direction (float64 textbook here), atol 1e-6."""
    p = np.array([1.0, -2.0], np.float32)
    grads = [np.array([0.1, -0.2], np.float32)] * 3
    got = _oracle_adam_steps(p, grads, nesterov=nesterov)
    want = _textbook_adam_updates(p, grads, b1=0.9, b2=0.999, eps=1e-8, nesterov=nesterov)
    for a, b in zip(got, want):
        np.testing.assert_allclose(a, b, atol=1e-6)


def test_adamw_masked_decoupled_weight_decay_matches_textbook():
    """tests/test_adam.py:87-116: adamw(lr 0.01, wd 0.1, mask w only) over
    three steps against optax.adamw (float64 textbook here), atol 1e-6."""
    pw = np.array([1.0, -2.0], np.float32)
    pb = np.array([0.5], np.float32)
    gw = [np.array([0.1, -0.2], np.float32)] * 3
    gb = [np.array([0.0], np.float32)] * 3
    got_w = _oracle_adam_steps(pw, gw, lr=0.01, wd=0.1, decay=True)
    got_b = _oracle_adam_steps(pb, gb, lr=0.01, wd=0.1, decay=False)
    want_w = _textbook_adam_updates(pw, gw, b1=0.9, b2=0.999, eps=1e-8, wd=0.1, lr=0.01, mask=True)
    want_b = _textbook_adam_updates(pb, gb, b1=0.9, b2=0.999, eps=1e-8, wd=0.1, lr=0.01, mask=False)
    for a, b in zip(got_w + got_b, want_w + want_b):
        np.testing.assert_allclose(a, b, atol=1e-6)


def test_adam_ema_weight_conventions_differ_where_expected():
    """optim/adam.py weights the gradient by 1 - f32(b1) computed in f32
    (utils.py:327-335); adam8.py by the double 1.0 - b1.  For b1 = 0.9 the
    two f32 weights differ (0x3dccccd0 vs 0x3dcccccd), so the stored first
    moment differs in the last bits for generic gradients: the double weight
    stays within 2^-23 (relative) of 0.1 * g, the f32 weight, itself 2.4e-7
    off, within 2^-21."""
    a = orc.make_hparams(ema_weight_f32=True)
    b = orc.make_hparams()
    assert np.float32(a.one_minus_b1).view(np.uint32) == 0x3DCCCCD0
    assert np.float32(b.one_minus_b1).view(np.uint32) == 0x3DCCCCCD
    assert a.nest_one_minus_b1 == b.nest_one_minus_b1 == np.float32(0.1)
    rng = np.random.default_rng(9)
    g = rng.standard_normal(4096).astype(np.float32)
    ms = []
    for hp in (a, b):
        mu = np.zeros(g.size, np.float32)
        nu = np.zeros(g.size, np.float32)
        orc.adam8_leaf(hp, np.zeros(g.size, np.float32), orc.F32, g, orc.F32, orc.MOM_F32, mu, None, nu, None,
                       updates_out=np.empty(g.size, np.float32))
        ms.append(mu)
    assert np.count_nonzero(ms[0] != ms[1]) > 1000
    exact = 0.1 * g.astype(np.float64)
    rel = [np.abs(m - exact) / np.abs(exact) for m in ms]
    assert rel[1].max() <= 2.0 ** -23 and rel[0].max() <= 2.0 ** -21
    assert rel[0].max() > 2.0 ** -23  # the f32 weight really is the other convention


def test_bf16_moment_store_sr_is_the_sr_of_the_f32_moments():
    """mu_dtype=bfloat16 (adam.py:219-222): the stored bf16 moments are
    _stochastic_round_bf16 of the f32 moments with the fed bits."""
    rng = np.random.default_rng(10)
    n = 5000
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    mb = orc.random_bits((1, 2), n)
    vb = orc.random_bits((3, 4), n)
    hp32 = orc.make_hparams(ema_weight_f32=True)
    mu32 = np.zeros(n, np.float32)
    nu32 = np.zeros(n, np.float32)
    orc.adam8_leaf(hp32, np.zeros(n, np.float32), orc.F32, g, orc.F32, orc.MOM_F32, mu32, None, nu32, None,
                   updates_out=np.empty(n, np.float32))
    hp16 = orc.make_hparams(ema_weight_f32=True, store_sr=True)
    mu16 = np.zeros(n, np.uint16)
    nu16 = np.zeros(n, np.uint16)
    orc.adam8_leaf(hp16, np.zeros(n, np.float32), orc.F32, g, orc.F32, orc.MOM_BF16, mu16, None, nu16, None,
                   mu_bits=mb, nu_bits=vb, updates_out=np.empty(n, np.float32))
    np.testing.assert_array_equal(mu16, orc.sr_bf16(mu32, mb))
    np.testing.assert_array_equal(nu16, orc.sr_bf16(nu32, vb))
    # without store_sr the bf16 moments are rounded to nearest even (adam8.py:688)
    hp_rne = orc.make_hparams(ema_weight_f32=True)
    mu16[:] = 0
    nu16[:] = 0
    orc.adam8_leaf(hp_rne, np.zeros(n, np.float32), orc.F32, g, orc.F32, orc.MOM_BF16, mu16, None, nu16, None,
                   updates_out=np.empty(n, np.float32))
    np.testing.assert_array_equal(mu16, orc.f32_to_bf16_bits(mu32))


# ----------------------------------------------- global-norm clipping -----
def test_global_norm_clip_scale_closed_forms():
    """finetune/transforms.py:57-82: a 3-4-12 tree has norm 13; scale =
    max_norm / (13 + 1e-6) below 1, exactly 1 above; NaN and Inf propagate
    as jnp.minimum and sqrt do."""
    grads = [np.array([3.0], np.float32), np.array([4.0, 0.0], np.float32), np.array([12.0], np.float32)]
    scale, norm = orc.global_norm_clip_scale(grads, 1.0)
    assert norm == np.float32(13.0)
    assert scale == np.float32(np.float32(1.0) / np.float32(np.float32(13.0) + np.float32(1e-6)))
    assert orc.global_norm_clip_scale(grads, 100.0)[0] == np.float32(1.0)
    nan_scale, nan_norm = orc.global_norm_clip_scale([np.array([np.nan], np.float32)], 1.0)
    assert np.isnan(nan_scale) and np.isnan(nan_norm)
    inf_scale, inf_norm = orc.global_norm_clip_scale([np.array([np.inf], np.float32)], 1.0)
    assert inf_scale == 0.0 and np.isinf(inf_norm)


def test_global_norm_matches_float64_and_leaf_order_f32_sum():
    rng = np.random.default_rng(12)
    grads = [rng.standard_normal(n).astype(np.float32) * np.float32(s)
             for n, s in ((100000, 1e-3), (7, 5.0), (4096, 1e-2), (33333, 0.3))]
    scale, norm = orc.global_norm_clip_scale(grads, 1.0)
    exact = np.sqrt(sum(np.sum(g.astype(np.float64) ** 2) for g in grads))
    assert abs(float(norm) - exact) <= 4 * 2.0 ** -24 * exact
    # the leaf sums are added in f32 in leaf order
    tot = np.float32(0.0)
    for g in grads:
        tot = np.float32(tot + np.float32(np.sum(g.astype(np.float64) ** 2)))
    assert norm == np.sqrt(tot, dtype=np.float32)
    assert scale < 1.0


def test_clip_leaf_bf16_rounds_once_with_bf16_scale():
    """bf16 leaves: leaf * scale.astype(bf16) -- the scale is first rounded to
    bf16, the product of two bf16 values is exact in f32 and rounded once."""
    rng = np.random.default_rng(13)
    g = orc.f32_to_bf16_bits(rng.standard_normal(10000).astype(np.float32))
    scale = np.float32(0.0123456)
    s16 = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(np.array([scale], np.float32)))[0]
    assert s16 != scale
    got = orc.clip_leaf(g, orc.BF16, scale)
    exact = orc.bf16_bits_to_f32(g).astype(np.float64) * np.float64(s16)
    assert np.all(exact.astype(np.float32).astype(np.float64) == exact)  # the product is exact in f32
    np.testing.assert_array_equal(got, orc.f32_to_bf16_bits(exact.astype(np.float32)))
    f = rng.standard_normal(100).astype(np.float32)
    np.testing.assert_array_equal(orc.clip_leaf(f, orc.F32, scale), f * scale)


def test_apply_if_finite_decision_known_sequence():
    """optax.apply_if_finite, documented behaviour: non-finite steps are
    skipped until more than max_consecutive_errors of them come in a row,
    then the update is let through; a finite step resets the consecutive
    count but not the total."""
    seq = [True, False, False, False, True, False, True]
    want = {  # max_consecutive_errors -> (applied, notfinite_count, total_notfinite) per step
        1: ([1, 0, 1, 1, 1, 0, 1], [0, 1, 2, 3, 0, 1, 0], [0, 1, 2, 3, 3, 4, 4]),
        2: ([1, 0, 0, 1, 1, 0, 1], [0, 1, 2, 3, 0, 1, 0], [0, 1, 2, 3, 3, 4, 4]),
    }
    for mce, (w_apply, w_count, w_total) in want.items():
        count = total = 0
        got_apply, got_count, got_total = [], [], []
        for fin in seq:
            a, count, total = orc.apply_if_finite_decision(count, total, fin, mce)
            got_apply.append(int(a))
            got_count.append(count)
            got_total.append(total)
        assert (got_apply, got_count, got_total) == (w_apply, w_count, w_total), mce
    # the counters saturate at the int32 maximum (optax.numerics.safe_increment)
    assert orc.apply_if_finite_decision(2**31 - 1, 2**31 - 1, False, 1) == (True, 2**31 - 1, 2**31 - 1)


def test_all_finite_and_reject_params():
    f = np.array([0.5, -1.0, 3.0e38], np.float32)
    b = orc.f32_to_bf16_bits(np.array([0.5, 2.0], np.float32))
    assert orc.all_finite([f, b], [orc.F32, orc.BF16])
    for bad in (np.nan, np.inf, -np.inf):
        g = f.copy()
        g[1] = bad
        assert not orc.all_finite([g, b], [orc.F32, orc.BF16])
        gb = orc.f32_to_bf16_bits(np.array([0.5, bad], np.float32))
        assert not orc.all_finite([f, gb], [orc.F32, orc.BF16])
    assert orc.all_finite([], [])
    # IEEE 754 round-to-nearest: x + (+0) is x for every x except -0, which gives +0
    p = np.array([-0.0, 0.0, 1.5, -2.0, np.inf, -np.inf, 1e-45, -1e-45], np.float32)
    want = p.copy()
    want[0] = 0.0
    orc.reject_params(p, orc.F32)
    np.testing.assert_array_equal(p.view(np.uint32), want.view(np.uint32))
    h = np.array([0x8000, 0x0000, 0x3FC0, 0xC000, 0x7F80, 0xFF80, 0x0001, 0x8001], np.uint16)
    want_h = h.copy()
    want_h[0] = 0
    orc.reject_params(h, orc.BF16)
    np.testing.assert_array_equal(h, want_h)


# ----------------------------------------------------------------- Magma --
def test_uniform01_known_bits():
    """jax.random.uniform's mantissa fill: bits 0 -> 0, all ones -> 1 - 2^-23,
    the top 23 bits set the mantissa, the low 9 bits are dropped."""
    u = orc.uniform01(np.array([0, 0xFFFFFFFF, 1 << 31, 0x1FF], np.uint32))
    assert u[0] == np.float32(0.0)
    assert u[1] == np.float32(1.0 - 2.0 ** -23)
    assert u[2] == np.float32(0.5)
    assert u[3] == np.float32(0.0)


def test_magma_leaf_closed_forms():
    """magma.py:98-118: a moment parallel to the gradient has cosine 1, an
    antiparallel one -1, an orthogonal one and an all-zero leaf 0 (the
    1e-12 floor), a NaN gradient 0 (nan_to_num); the score is
    0.9 * s_prev + 0.1 * sigmoid(cos / tau), here against float64."""
    key = orc.split(np.array([0, 7], np.uint32), 1)[0]
    g = np.array([1.0, -2.0, 3.0], np.float32)

    def want(cos, tau, s_prev):
        return 0.9 * s_prev + 0.1 / (1.0 + np.exp(-cos / tau))

    for mu, cos in ((3 * g, 1.0), (-0.5 * g, -1.0), (np.array([2.0, 1.0, 0.0], np.float32), 0.0),
                    (np.zeros(3, np.float32), 0.0)):
        for tau, s_prev in ((2.0, 0.5), (0.25, 0.9)):
            s, _keep = orc.magma_leaf(g, mu, s_prev, key, 0.5, tau)
            assert s.dtype == np.float32 and abs(float(s) - want(cos, tau, s_prev)) < 2e-7, (mu, tau, s)
    s, _ = orc.magma_leaf(np.array([np.nan, 1.0], np.float32), np.ones(2, np.float32), 0.5, key, 0.5, 2.0)
    assert abs(float(s) - want(0.0, 2.0, 0.5)) < 2e-7


def test_magma_bernoulli_mask():
    """bernoulli(key, p) = uniform(key) < p: never at p = 0, always at p = 1,
    and at p = 0.3 the keep frequency over 4,000 keys lies within 4 sigma."""
    keys = orc.split(np.array([0, 42], np.uint32), 4000)
    g = np.ones(4, np.float32)
    for p, rate in ((0.0, 0.0), (1.0, 1.0)):
        kept = [orc.magma_leaf(g, g, 0.5, k, p, 2.0)[1] for k in keys[:200]]
        assert np.mean(kept) == rate
    kept = np.array([orc.magma_leaf(g, g, 0.5, k, 0.3, 2.0)[1] for k in keys])
    sigma = np.sqrt(0.3 * 0.7 / keys.shape[0])
    assert abs(kept.mean() - 0.3) < 4 * sigma


def test_magma_apply_masks_and_scales():
    """magma.py:120-122 and scale_by_learning_rate: a dropped leaf's update
    is exactly zero; a kept one is s * delta, then times -lr."""
    delta = np.array([1.0, -2.0, 0.5], np.float32)
    assert (orc.magma_apply(delta, np.float32(0.7), False) == 0.0).all()
    np.testing.assert_array_equal(orc.magma_apply(delta, np.float32(0.5), True), delta * np.float32(0.5))
    np.testing.assert_array_equal(orc.magma_apply(delta, np.float32(0.5), True, np.float32(-0.1)),
                                  np.float32(-0.1) * (delta * np.float32(0.5)))


def _symmetric_tie_block():
    """A block whose absmax is 127, so scale = 127 / 127 = 1 exactly and
    x / scale = x: every k + 0.5 for k in -127..126 (exact ties of
    jnp.round), then 127 and -127 themselves (256 values)."""
    halves = np.arange(-127, 127, dtype=np.float32) + np.float32(0.5)
    x = np.concatenate([halves, np.float32([127.0, -127.0])])
    return x, x.size


def test_symmetric_round_half_even_exact_ties():
    """adam8.py:455 jnp.round rounds halves to the even neighbour: 0.5 -> 0,
    1.5 -> 2, 2.5 -> 2, -0.5 -> 0, -1.5 -> -2, 126.5 -> 126.  Round half
    away from zero (1, 2, 3, -1, ...) or half up fails here."""
    x, n = _symmetric_tie_block()
    codes, scales = orc.quantize(x, 256, orc.Q_SYMMETRIC)
    assert scales[0] == np.float32(1.0)
    got = codes.reshape(-1)[:n].astype(np.int64)
    k = np.arange(-127, 127)
    even = np.where(k % 2 == 0, k, k + 1)          # the even one of k and k + 1
    np.testing.assert_array_equal(got[:254], even)
    assert list(got[254:]) == [127, -127]
    assert got[127] == 0 and got[128] == 2 and got[129] == 2 and got[126] == 0 and got[125] == -2


def _bits_for_uniform(u: np.ndarray) -> np.ndarray:
    """Raw words whose jax.random.uniform value is exactly u (u a multiple
    of 2^-23 in [0, 1)): mantissa = u * 2^23 in bits 9..31."""
    m = np.round(np.asarray(u, np.float64) * (1 << 23)).astype(np.uint64)
    return (m << np.uint64(9)).astype(np.uint32)


def test_symmetric_sr_floor_plus_bernoulli_closed_form():
    """adam8.py:456-458: r = floor(s) + bernoulli(s - floor(s)), bernoulli =
    uniform < p.  With scale 1, s = x: for s = 2.25 the draw u < 0.25 gives
    3, u >= 0.25 gives 2; for s = -2.25, floor is -3 and p = 0.75, so
    u < 0.75 gives -2 and u >= 0.75 gives -3 (a truncating floor would give
    -2 there); integers never move.  u sits one step below, at and above p."""
    step = 2.0 ** -23
    cases = []   # (s, u, expected)
    for s, lo in ((2.25, 2), (-2.25, -3), (0.75, 0), (-0.75, -1), (126.5, 126), (-126.5, -127)):
        p = s - lo
        cases += [(s, p - step, lo + 1), (s, p, lo), (s, min(p + step, 1 - step), lo), (s, 0.0, lo + 1)]
    cases += [(3.0, 0.0, 3), (3.0, 1 - step, 3), (-5.0, 0.0, -5), (0.0, 0.0, 0)]
    s = np.float32([c[0] for c in cases])
    x = np.concatenate([s, np.float32([127.0])])       # absmax 127: scale 1
    bits = np.zeros(x.size, np.uint32)
    bits[:s.size] = _bits_for_uniform([c[1] for c in cases])
    assert np.all(orc.uniform01(bits[:s.size]) == np.float32([c[1] for c in cases]))
    codes, scales = orc.quantize(x, x.size, orc.Q_SYMMETRIC, bits=bits)
    assert scales[0] == np.float32(1.0)
    np.testing.assert_array_equal(codes.reshape(-1)[:s.size].astype(np.int64), [c[2] for c in cases])


def test_zero_weight_decay_term_closed_form():
    """optim/adam.py's weight-0 decay term (``u + 0 * f32(p)``, utils.py:79-90)
    in the oracle: for finite params the updates equal those without it
    except that a -0 update becomes +0 when the param is positive; a
    non-finite param makes the update NaN."""
    rng = np.random.default_rng(4)
    n = 4096
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    p[:4] = [np.inf, -np.inf, np.nan, 0.5]
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    g[3] = -0.0   # with a -0 first moment: m = b1*(-0) + (1-b1)*(-0) = -0, a -0 direction

    def run(zero):
        hp = orc.make_hparams(count=1, apply=False, ema_weight_f32=True, zero_decay=zero)
        m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
        m[3] = -0.0
        out = np.empty(n, np.float32)
        orc.adam8_leaf(hp, p.copy(), orc.F32, g, orc.F32, orc.MOM_F32, m, None, v, None, 2048, updates_out=out)
        return out

    base, zero = run(False), run(True)
    assert np.isnan(zero[:3]).all() and np.isfinite(base[:3]).all()
    np.testing.assert_array_equal(zero[4:], base[4:] + np.float32(0.0))
    assert np.signbit(base[3]) and not np.signbit(zero[3])


def test_f16_widening_all_patterns_against_numpy():
    """The oracle's binary16 -> f32 over all 65,536 patterns against numpy's
    float16 (NaN positions and every other value bit for bit)."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def _f16_narrowing_cases():
    """f32 patterns that decide binary16 rounding: a stride-61 sweep of every
    pattern, and +-3 patterns around every midpoint between adjacent f16
    values (including 65504 | 65536 and the subnormal steps)."""
    sweep = np.arange(0, 1 << 32, 61, dtype=np.uint64).astype(np.uint32)
    pos = np.arange(0, 0x7C01, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    pos = np.append(pos, 65536.0)   # the rounding target just above 65504 (Inf in f16)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32).view(np.uint32).astype(np.int64)
    near = (mids[:, None] + np.arange(-3, 4)[None, :]).reshape(-1)
    near = np.concatenate([near, near | (1 << 31)]).astype(np.uint32)
    return [sweep[i:i + (1 << 24)] for i in range(0, sweep.size, 1 << 24)] + [near]


def test_f16_narrowing_against_numpy():
    """The oracle's f32 -> binary16 (round to nearest even, overflow to Inf
    from 65520, subnormals) against numpy's astype(float16)."""
    for bits in _f16_narrowing_cases():
        x = bits.view(np.float32)
        got = orc.f32_to_f16_bits(x)
        with np.errstate(over="ignore"):
            want = x.astype(np.float16).view(np.uint16)
        nan = np.isnan(x)
        np.testing.assert_array_equal(got[~nan], want[~nan])
        assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


@pytest.mark.parametrize("quantizer", [orc.Q_SIGNED, orc.Q_UNSIGNED, orc.Q_SYMMETRIC])
def test_scale_dtype_changes_only_the_stored_scales(quantizer):
    """quantize_blocks codes with the f32 scale and stores
    scales.astype(scale_dtype) (adam8.py:167-186): the codes do not depend on
    scale_dtype, and the stored scales are the f32 ones rounded (numpy's
    bfloat16-free check: bf16 rounding through the bit patterns, f16 through
    numpy's float16)."""
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(5 * 256 + 9) * np.exp(rng.uniform(-30, 12, 5 * 256 + 9))).astype(np.float32)
    if quantizer == orc.Q_UNSIGNED:
        x = np.abs(x)
    c32, s32 = orc.quantize(x, 256, quantizer)
    cb, sb = orc.quantize(x, 256, quantizer, scale_dtype=orc.BF16)
    ch, sh = orc.quantize(x, 256, quantizer, scale_dtype=orc.F16)
    np.testing.assert_array_equal(cb, c32)
    np.testing.assert_array_equal(ch, c32)
    np.testing.assert_array_equal(sb, orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(s32)))
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(sh, s32.astype(np.float16).astype(np.float32))


def test_step_with_16_bit_scales_reads_the_stored_scale():
    """One adam8 step with bf16 block scales from a state whose scales are
    bf16 values: the new moments and codes equal the f32-scale step's (same
    old scales), and only the stored new scales are rounded."""
    rng = np.random.default_rng(12)
    n, bs = 4 * 2048, 2048
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    mc = rng.integers(0, 256, n).astype(np.uint8)
    vc = rng.integers(0, 256, n).astype(np.uint8)
    ms = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(rng.uniform(1e-4, 1e-2, 4).astype(np.float32)))
    vs = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(rng.uniform(1e-7, 1e-5, 4).astype(np.float32)))
    outs = []
    for sd in (orc.F32, orc.BF16):
        hp = orc.make_hparams(count=3, apply=False, scale_dtype=sd)
        a = [p.copy(), mc.copy(), ms.copy(), vc.copy(), vs.copy(), np.empty(n, np.float32)]
        orc.adam8_leaf(hp, a[0], orc.F32, g, orc.F32, orc.MOM_QUANT, a[1], a[2], a[3], a[4], bs, updates_out=a[5])
        outs.append(a)
    (f, b) = outs
    np.testing.assert_array_equal(b[1], f[1])
    np.testing.assert_array_equal(b[3], f[3])
    np.testing.assert_array_equal(b[5].view(np.uint32), f[5].view(np.uint32))
    np.testing.assert_array_equal(b[2], orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(f[2])))
    np.testing.assert_array_equal(b[4], orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(f[4])))


def test_f16_params_round_the_f32_step():
    """An f16 param leaf: without the weak-typed decay its new params are
    the f32 step's params (on the same values) rounded to f16 by numpy; with
    it, the decay term is f16(f16(wd) * p) (numpy float16 arithmetic, exact
    products)."""
    rng = np.random.default_rng(13)
    n = 3000
    p16 = (rng.standard_normal(n) * 0.5).astype(np.float16)
    g16 = (rng.standard_normal(n) * 1e-2).astype(np.float16)
    p32, g32 = p16.astype(np.float32), g16.astype(np.float32)
    for weak in (False, True):
        hp = orc.make_hparams(count=1, weight_decay=0.01, lr=1e-3, decay=True, decay_weak=weak, apply=True)
        a16 = p16.view(np.uint16).copy()
        orc.adam8_leaf(hp, a16, orc.F16, g16.view(np.uint16).copy(), orc.F16, orc.MOM_F32,
                       np.zeros(n, np.float32), None, np.zeros(n, np.float32), None)
        if not weak:
            a32 = p32.copy()
            orc.adam8_leaf(hp, a32, orc.F32, g32, orc.F32, orc.MOM_F32, np.zeros(n, np.float32), None,
                           np.zeros(n, np.float32), None)
            np.testing.assert_array_equal(a16, a32.astype(np.float16).view(np.uint16))
        else:
            hp0 = orc.make_hparams(count=1, apply=False)
            u = np.empty(n, np.float32)
            orc.adam8_leaf(hp0, p32.copy(), orc.F32, g32, orc.F32, orc.MOM_F32, np.zeros(n, np.float32), None,
                           np.zeros(n, np.float32), None, updates_out=u)
            wdp = (np.float16(0.01) * p16).astype(np.float32)          # f16 product, rounded once
            want = (p32 + np.float32(-1e-3) * (u + wdp)).astype(np.float16)
            np.testing.assert_array_equal(a16, want.view(np.uint16))


def _rn_bf16(q: Fraction) -> Fraction:
    """An exact rational rounded to the nearest bfloat16 (8 significant bits,
    ties to even; subnormal spacing 2^-133), as an exact rational."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1                      # now 2^e <= a < 2^(e+1)
    ulp = Fraction(2) ** max(e - 7, -133)
    k, rem = divmod(a, ulp)
    k = int(k)
    if rem * 2 > ulp or (rem * 2 == ulp and k % 2 == 1):
        k += 1
    return sign * k * ulp


def test_rn_bf16_helper_against_the_bit_rounding():
    """The rational rounding above against the oracle's f32 -> bf16
    (round-to-nearest-even on the bit pattern) for f32 inputs."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(5000) * np.exp(rng.uniform(-20, 20, 5000))).astype(np.float32)
    got = np.array([float(_rn_bf16(Fraction(float(v)))) for v in x], np.float32)
    np.testing.assert_array_equal(got, orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(x)))


def test_weak_typed_bf16_decay_term_closed_form():
    """optax add_decayed_weights ``u + wd * p`` with a Python-scalar wd and
    bf16 params (adam8.py:433-443; H5): JAX's weak typing keeps ``wd * p`` in
    bf16, so the decay term is RN_bf16(RN_bf16(wd) * p), the exact product
    rounded once, added to the f32 update in f32.  Computed here in exact
    rationals and checked bit for bit against the oracle's update-only output
    on inputs where the f32 product (a non-weak oracle) gives another sum for
    most elements."""
    rng = np.random.default_rng(17)
    n = 4096
    wd = 0.0123
    p32 = (rng.standard_normal(n) * 0.7).astype(np.float32)
    pbits = orc.f32_to_bf16_bits(p32)
    p = orc.bf16_bits_to_f32(pbits)
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)

    def update(**kw):
        hp = orc.make_hparams(count=1, apply=False, **kw)
        u = np.empty(n, np.float32)
        orc.adam8_leaf(hp, pbits.copy(), orc.BF16, g.copy(), orc.F32, orc.MOM_F32, np.zeros(n, np.float32), None,
                       np.zeros(n, np.float32), None, updates_out=u)
        return u

    u0 = update()                                                   # no decay link
    u_weak = update(weight_decay=wd, decay=True, decay_weak=True)
    u_strong = update(weight_decay=wd, decay=True, decay_weak=False)
    wd16 = _rn_bf16(Fraction(float(np.float32(wd))))               # the Python float is first an f32 weak scalar
    assert wd16 == _rn_bf16(Fraction(wd))                           # (the same bf16 either way for this wd)
    term = np.array([float(_rn_bf16(wd16 * Fraction(float(v)))) for v in p], np.float32)
    want = (u0 + term).astype(np.float32)
    np.testing.assert_array_equal(u_weak.view(np.uint32), want.view(np.uint32))
    f32_term = (np.float32(wd) * p).astype(np.float32)
    want_strong = (u0 + f32_term).astype(np.float32)
    np.testing.assert_array_equal(u_strong.view(np.uint32), want_strong.view(np.uint32))
    assert np.count_nonzero(want != want_strong) > n // 2


# ------------------------------------------------------ optax.MultiSteps --
def _acc_run(mode, grads, gdtype, adtype, acc0=None):
    """Feeds the grads one micro-step at a time; returns the accumulator's
    f32 values after each."""
    n = np.asarray(grads[0]).size
    acc = np.zeros(n, np.float32) if adtype == orc.F32 else np.zeros(n, np.uint16)
    if acc0 is not None:
        acc[:] = acc0
    out = []
    for i, g in enumerate(grads):
        orc.accumulate(mode, i, g, gdtype, acc, adtype)
        out.append(orc.to_f32(acc.copy(), adtype))
    return out


def test_accumulate_mean_dyadic_sequence_and_sum():
    """Welford's running mean of 1, 2, 3, 4 is 1, 1.5, 2, 2.5 exactly (every
    intermediate is dyadic); the sum mode gives 1, 3, 6, 10.  A divisor of
    n_acc instead of n_acc + 1, or a dropped term, fails both."""
    seq = [np.full(5, v, np.float32) for v in (1.0, 2.0, 3.0, 4.0)]
    for got, want in zip(_acc_run(orc.ACC_MEAN, seq, orc.F32, orc.F32), (1.0, 1.5, 2.0, 2.5)):
        np.testing.assert_array_equal(got, np.full(5, want, np.float32))
    for got, want in zip(_acc_run(orc.ACC_SUM, seq, orc.F32, orc.F32), (1.0, 3.0, 6.0, 10.0)):
        np.testing.assert_array_equal(got, np.full(5, want, np.float32))


def test_accumulate_mean_of_a_constant_is_the_constant():
    """(g - g) = 0 after the first micro-step, so the running mean of a
    constant stream is that constant, bit for bit, in every dtype."""
    rng = np.random.default_rng(3)
    v = rng.standard_normal(257).astype(np.float32)
    for dt in (orc.F32, orc.BF16, orc.F16):
        g = orc.from_f32(v, dt)
        for got in _acc_run(orc.ACC_MEAN, [g] * 6, dt, dt):
            np.testing.assert_array_equal(got, orc.to_f32(g, dt))


def test_accumulate_f32_matches_numpy_float32_per_op():
    """f32 accumulation against numpy's own float32 arithmetic, one
    correctly rounded operation at a time."""
    rng = np.random.default_rng(4)
    grads = [(rng.standard_normal(1000) * 10.0 ** rng.integers(-3, 3, 1000)).astype(np.float32) for _ in range(7)]
    a = np.zeros(1000, np.float32)
    s = np.zeros(1000, np.float32)
    for i, (got_m, got_s, g) in enumerate(zip(_acc_run(orc.ACC_MEAN, grads, orc.F32, orc.F32),
                                              _acc_run(orc.ACC_SUM, grads, orc.F32, orc.F32), grads)):
        a = a + (g - a) / np.float32(i + 1)
        s = g + s
        np.testing.assert_array_equal(got_m.view(np.uint32), a.view(np.uint32))
        np.testing.assert_array_equal(got_s.view(np.uint32), s.view(np.uint32))


def test_accumulate_f16_rounds_every_operation():
    """Same-dtype f16 accumulation against numpy float16 arithmetic, which
    rounds each operation to binary16; rounding once at the end (an f32
    computation) differs on part of the sample, so the check can fail."""
    rng = np.random.default_rng(5)
    grads16 = [rng.standard_normal(4000).astype(np.float16) for _ in range(5)]
    got = _acc_run(orc.ACC_MEAN, [g.view(np.uint16) for g in grads16], orc.F16, orc.F16)
    a = np.zeros(4000, np.float16)
    a32 = np.zeros(4000, np.float16)
    differs = 0
    for i, g in enumerate(grads16):
        once = (a32.astype(np.float32) + (g.astype(np.float32) - a32.astype(np.float32)) / np.float32(i + 1))
        a32 = a.copy()
        a = a + (g - a) / np.float16(i + 1)
        np.testing.assert_array_equal(got[i], a.astype(np.float32))
        differs += int(np.sum(once.astype(np.float16) != a))
    assert differs > 0
    s = np.zeros(4000, np.float16)
    for i, (g, gs) in enumerate(zip(grads16, _acc_run(orc.ACC_SUM, [g.view(np.uint16) for g in grads16],
                                                       orc.F16, orc.F16))):
        s = g + s
        np.testing.assert_array_equal(gs, s.astype(np.float32))


def test_accumulate_bf16_grads_into_f32_widen_exactly():
    """bf16 grads into an f32 accumulator (the builders' default
    accumulate_dtype) compute in f32 on the exactly widened grads."""
    rng = np.random.default_rng(6)
    v = [rng.standard_normal(333).astype(np.float32) for _ in range(4)]
    gb = [orc.f32_to_bf16_bits(x) for x in v]
    wide = [orc.bf16_bits_to_f32(h) for h in gb]
    for mode in (orc.ACC_MEAN, orc.ACC_SUM):
        for x, y in zip(_acc_run(mode, gb, orc.BF16, orc.F32), _acc_run(mode, wide, orc.F32, orc.F32)):
            np.testing.assert_array_equal(x.view(np.uint32), y.view(np.uint32))


def test_accumulate_reset_is_zero_times_acc():
    """(1 - emit) * acc on the emitting micro-step: finite values become a
    zero of their sign, Inf and NaN become NaN, which the next window's
    running mean keeps (NaN + (g - NaN) / 1)."""
    vals = np.array([1.5, -2.0, 0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45], np.float32)
    for dt in (orc.F32, orc.BF16, orc.F16):
        acc = orc.from_f32(vals, dt).copy()
        orc.accumulate(orc.ACC_ZERO, 0, None, dt, acc, dt)
        got = orc.to_f32(acc, dt)
        finite = np.isfinite(vals)
        src = orc.to_f32(orc.from_f32(vals, dt), dt)
        np.testing.assert_array_equal(got[finite], 0.0)
        np.testing.assert_array_equal(np.signbit(got[finite]), np.signbit(src[finite]))
        assert np.isnan(got[~finite]).all()
        orc.accumulate(orc.ACC_MEAN, 0, orc.from_f32(np.full(vals.size, 3.0, np.float32), dt), dt, acc, dt)
        got = orc.to_f32(acc, dt)
        np.testing.assert_array_equal(got[finite], 3.0)
        assert np.isnan(got[~finite]).all()


def test_multisteps_counters_known_sequence():
    """optax.MultiSteps: with k = 3 the third, sixth, ... micro-steps emit;
    mini_step cycles 0, 1, 2 and gradient_step counts the emits."""
    mini = grad = 0
    emits, minis, grads = [], [], []
    for _ in range(7):
        e, mini, grad = orc.multisteps_counters(mini, grad, 3)
        emits.append(int(e))
        minis.append(mini)
        grads.append(grad)
    assert emits == [0, 0, 1, 0, 0, 1, 0]
    assert minis == [1, 2, 0, 1, 2, 0, 1]
    assert grads == [0, 0, 1, 1, 1, 2, 2]
    assert orc.multisteps_counters(0, 5, 1) == (True, 0, 6)


# ------------------------------------------------------ packed bit source --
def test_packed_param_bits_definition():
    """The packed source's param bits (no reference counterpart), element by
    element from the KAT-pinned block function: element e takes half (e & 1)
    of word (e & 2 ? y1 : y0) of the block at counter e >> 2, including
    offsets whose block counter crosses 2^32 and unaligned offsets."""
    key = (0x13198A2E, 0x03707344)
    for offset in (0, 3, (1 << 34) - 6):
        got = orc.packed_param_bits(key, 13, offset)
        for i, b in enumerate(got):
            e = offset + i
            q = e >> 2
            y = orc.threefry2x32(key, (q >> 32, q & 0xFFFFFFFF))
            w = y[1] if e & 2 else y[0]
            assert int(b) == ((w >> 16) if e & 1 else (w & 0xFFFF))
    # four consecutive elements use the four halves of one block, once each
    y0, y1 = orc.threefry2x32(key, (0, 5))
    assert orc.packed_param_bits(key, 4, 20).tolist() == [y0 & 0xFFFF, y0 >> 16, y1 & 0xFFFF, y1 >> 16]


def test_packed_moment_bits_definition():
    """The packed source's moment words (no reference counterpart), element
    by element from the KAT-pinned block function: element e's word is
    (main << 16) | fill, with main and fill the half (e & 1) of y0 (first
    moment) or y1 (second) of the blocks at counters e >> 1 and
    2^63 + (e >> 1); the storage noise is the main half.  Offsets cross
    2^32 and 2^33 and start on odd elements."""
    key = (7, 11)
    for offset in (0, 5, (1 << 33) - 3):
        m, v = orc.packed_moment_bits(key, 7, offset)
        sm, sv = orc.packed_store_bits(key, 7, offset)
        for i in range(7):
            e = offset + i
            q = e >> 1
            y0, y1 = orc.threefry2x32(key, (q >> 32, q & 0xFFFFFFFF))
            z0, z1 = orc.threefry2x32(key, ((q >> 32) | 0x80000000, q & 0xFFFFFFFF))
            half = (lambda w: w >> 16) if e & 1 else (lambda w: w & 0xFFFF)
            assert int(m[i]) == (half(y0) << 16) | half(z0)
            assert int(v[i]) == (half(y1) << 16) | half(z1)
            assert (int(sm[i]), int(sv[i])) == (half(y0), half(y1))
    # a pair of elements uses the four halves of one main block, once each
    y0, y1 = orc.threefry2x32(key, (0, 9))
    m, v = orc.packed_moment_bits(key, 2, 18)
    assert [int(w) >> 16 for w in m] + [int(w) >> 16 for w in v] == [y0 & 0xFFFF, y0 >> 16, y1 & 0xFFFF, y1 >> 16]


def test_packed_main_half_settles_the_draw():
    """The kernel decides a packed moment draw from its 16-bit main half m
    alone when m + 127/128 < x = 65536 p ("upper") or m >= x ("lower"),
    with x - 127/128 computed in f32, and reads the fill only in between.
    For every main half and all 128 fill values, a settled decision equals
    the whole word's (uniform of the top 23 bits < p), over probabilities
    at and beside every 2^-23 step near sampled main-half boundaries, 0,
    the smallest subnormal, 1 and random values; and the fill is needed
    for one main half per probability, none when x's fraction is 0 or
    above 127/128."""
    rng = np.random.default_rng(3)
    ps = [0.0, 1.0, float(np.float32(2.0 ** -149)), float(np.float32(2.0 ** -23)), float(np.float32(0.5))]
    for m0 in rng.integers(0, 65536, 8).tolist() + [0, 1, 65535]:
        for f0 in (0, 1, 126, 127, 128):
            k = m0 * 128 + f0
            for d in (-1, 0, 1):
                ps.append(float(np.nextafter(np.float32(k * 2.0 ** -23), np.float32(2.0), dtype=np.float32)
                                if d > 0 else np.nextafter(np.float32(k * 2.0 ** -23), np.float32(-1.0),
                                                           dtype=np.float32) if d < 0 else np.float32(k * 2.0 ** -23)))
    ps += rng.random(32).astype(np.float32).tolist()
    hm = np.arange(65536, dtype=np.float32)
    fills = np.arange(128, dtype=np.float64)
    for p in ps:
        p32 = np.float32(min(max(p, 0.0), 1.0))
        x = np.float32(p32 * np.float32(65536.0))
        up = hm < np.float32(x - np.float32(0.9921875))
        open_ = ~up & (hm < x)
        # whole-word decision for every (m, f): (128 m + f) * 2^-23 < p, exact in float64
        whole = ((hm.astype(np.float64)[:, None] * 128.0 + fills[None, :]) * 2.0 ** -23) < np.float64(p32)
        settled = ~open_
        assert np.all(whole[settled & up]), p
        assert not np.any(whole[settled & ~up]), p
        frac = float(x) - np.floor(float(x))
        assert int(open_.sum()) == (1 if 0.0 < frac <= 127.0 / 128.0 else 0), p
