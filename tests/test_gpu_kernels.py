"""GPU parity of the standalone kernels against the CPU oracle:
quantize_blocks / dequantize_blocks (rollfast optim/adam8.py:113-204),
_stochastic_round_bf16 (utils.py:342-371) and apply_updates (:648-708).
Integer/byte outputs (codes, bf16 bit patterns) must be bit-exact; f32
outputs (scales, dequantized values) are compared bit for bit as well."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import bf16_bits, to_device, to_host

pytestmark = pytest.mark.gpu

QUANTIZERS = {"dynamic_signed": orc.Q_SIGNED, "dynamic_unsigned": orc.Q_UNSIGNED, "symmetric_int8": orc.Q_SYMMETRIC}


def _rf():
    import rollfast_amd as rf

    return rf


def _edge_values(rng, n):
    """Log-uniform magnitudes 1e-8..1e2 with random sign, plus zeros,
    denormals, exact ties and +-absmax."""
    mag = np.exp(rng.uniform(np.log(1e-8), np.log(1e2), size=n)).astype(np.float32)
    x = np.where(rng.random(n) < 0.5, -mag, mag).astype(np.float32)
    x[rng.random(n) < 0.02] = 0.0
    x[rng.random(n) < 0.01] = np.float32(-0.0)
    den = rng.random(n) < 0.01
    x[den] = (rng.integers(1, 1 << 23, size=den.sum()).astype(np.uint32)).view(np.float32)
    return x


def _check_quantize(x, block_size, quantizer, sr=False):
    import torch

    rf = _rf()
    key = rf.prng.PRNGKey(11)
    xd = to_device(x, "f32")
    qb = rf.quantize_blocks(xd, block_size=block_size, quantizer=quantizer, stochastic_rounding=sr,
                            key=key if sr else None)
    torch.cuda.synchronize()
    nb = max(1, -(-x.size // block_size))
    bits = orc.random_bits(key, nb * block_size) if sr else None
    codes, scales = orc.quantize(x, block_size, QUANTIZERS[quantizer], bits=bits)
    got = to_host(qb.values)
    np.testing.assert_array_equal(got.view(np.uint8), codes.reshape(-1).view(np.uint8))
    np.testing.assert_array_equal(to_host(qb.scales).view(np.uint32), scales.view(np.uint32))
    back = rf.dequantize_blocks(qb)
    torch.cuda.synchronize()
    ref = orc.dequantize(codes, scales, x.size, block_size, QUANTIZERS[quantizer])
    np.testing.assert_array_equal(to_host(back).view(np.uint32), ref.view(np.uint32))
    assert tuple(back.shape) == tuple(xd.shape)


@pytest.mark.parametrize("quantizer", list(QUANTIZERS))
@pytest.mark.parametrize("block_size,size", [(2048, 2048 * 37), (2048, 2048 * 5 + 777), (128, 513), (1000, 4321)])
def test_quantize_dequantize_parity(quantizer, block_size, size):
    rng = np.random.default_rng(size + block_size)
    _check_quantize(_edge_values(rng, size), block_size, quantizer)


@pytest.mark.parametrize("quantizer", list(QUANTIZERS))
def test_quantize_stochastic_rounding_parity(quantizer):
    rng = np.random.default_rng(9)
    _check_quantize(_edge_values(rng, 2048 * 9 + 5), 2048, quantizer, sr=True)


def test_quantize_special_blocks():
    """Zero blocks (scale 1), a block with -absmax (clipped to code 0), NaN and
    Inf blocks, a tiny-scale block below the fast range, exact ties."""
    bs = 2048
    blocks = []
    blocks.append(np.zeros(bs, np.float32))
    b = np.linspace(-1, 1, bs).astype(np.float32)
    b[0] = -2.0
    b[1] = 2.0
    blocks.append(b)
    b = np.linspace(-1, 1, bs).astype(np.float32)
    b[5] = np.nan
    blocks.append(b)
    b = np.linspace(-1, 1, bs).astype(np.float32)
    b[7] = np.inf
    blocks.append(b)
    b = np.linspace(-1, 1, bs).astype(np.float32)
    b[9] = -np.inf
    blocks.append(b)
    blocks.append((np.linspace(-1, 1, bs) * 1e-30).astype(np.float32))   # scale < 2^-70
    blocks.append((np.linspace(-1, 1, bs) * 1e-40).astype(np.float32))   # subnormal scale
    cb = orc.codebook(True)
    mids = ((cb[:-1].astype(np.float64) + cb[1:]) / 2).astype(np.float32)
    b = np.resize(np.concatenate([mids, cb, [1.0]]).astype(np.float32), bs)
    blocks.append(b)
    x = np.concatenate(blocks)
    for q in QUANTIZERS:
        _check_quantize(x, bs, q)


def _decision_patterns(q):
    """Bit patterns of normalised values that probe the kernel's lookup: a
    stride-61 sweep of [-1, 1] ([0, 1] unsigned) plus +-64 patterns around
    every midpoint of adjacent codebook entries (where the thresholds are)."""
    cb = orc.codebook(q == orc.Q_SIGNED)
    pats = [np.arange(0, 0x3F800001, 61, dtype=np.uint64)]
    if q == orc.Q_SIGNED:
        pats.append(np.arange(0x80000000, 0xBF800001, 61, dtype=np.uint64))
    mids = ((cb[:-1].astype(np.float64) + cb[1:]) / 2).astype(np.float32).view(np.uint32).astype(np.int64)
    near = (mids[:, None] + np.arange(-64, 65)[None, :]).reshape(-1)
    pats.append(near.astype(np.uint64))
    pats.append(cb.view(np.uint32).astype(np.uint64))
    bits = np.unique(np.concatenate(pats)).astype(np.uint32)
    vals = bits.view(np.float32)
    keep = np.abs(vals) <= 1.0
    if q == orc.Q_UNSIGNED:
        keep &= vals >= 0
    return bits[keep]


@pytest.mark.parametrize("quantizer", ["dynamic_signed", "dynamic_unsigned"])
def test_quantize_normalised_values_through_table_lookup(quantizer):
    """Normalised values pass through the kernel's table lookup with scale 1
    (each block holds 1.0) and must equal the oracle's searchsorted code."""
    import torch

    rf = _rf()
    q = QUANTIZERS[quantizer]
    bits = _decision_patterns(q)
    n = bits.size
    nb = -(-n // 2047)
    body = np.zeros(nb * 2047, np.uint32)
    body[:n] = bits
    x = np.zeros((nb, 2048), np.float32)
    x[:, :2047] = body.reshape(nb, 2047).view(np.float32)
    x[:, 2047] = 1.0
    qb = rf.quantize_blocks(to_device(x.reshape(-1), "f32"), quantizer=quantizer)
    torch.cuda.synchronize()
    got = to_host(qb.values).reshape(nb, 2048)[:, :2047].reshape(-1)[:n]
    want = orc.nearest_codes_list(q, bits)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{quantizer}: code mismatch at bits {hex(int(bits[bad[0]]))}"


def test_sr_bf16_parity_fed_and_threefry():
    import torch

    from rollfast_amd.utils import _stochastic_round_bf16

    rf = _rf()
    rng = np.random.default_rng(1)
    n = 1 << 20
    x = _edge_values(rng, n)
    x[:4] = [np.inf, -np.inf, np.nan, np.float32(3.0e38)]
    key = rf.prng.PRNGKey(5)
    bits = orc.random_bits(key, n)
    want = orc.sr_bf16(x, bits)
    got = _stochastic_round_bf16(to_device(x, "f32"), key)
    got_fed = _stochastic_round_bf16(to_device(x, "f32"), key, random_bits=to_device(bits, "u32"))
    torch.cuda.synchronize()
    w = want.copy()
    for arr in (to_host(got), to_host(got_fed)):
        nan = np.isnan(orc.bf16_bits_to_f32(w))
        np.testing.assert_array_equal(arr[~nan], w[~nan])
        assert np.isnan(orc.bf16_bits_to_f32(arr[nan])).all()


@pytest.mark.parametrize("stochastic", [False, True])
def test_apply_updates_parity(stochastic):
    import torch

    rf = _rf()
    rng = np.random.default_rng(2)
    sizes = [(4096,), (33, 7), (1,), (2048 * 3 + 5,)]
    dtypes = ["bf16", "f32", "bf16", "f32"]
    params, host = {}, []
    ups, uhost = {}, []
    for i, (s, dt) in enumerate(zip(sizes, dtypes)):
        n = int(np.prod(s))
        p = (rng.standard_normal(n) * 0.5).astype(np.float32)
        p = bf16_bits(p) if dt == "bf16" else p
        u = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        params[f"p{i}"] = to_device(p, dt).reshape(s)
        ups[f"p{i}"] = to_device(u, "f32").reshape(s)
        host.append(p.copy())
        uhost.append(u)
    key = rf.prng.PRNGKey(0)
    out = rf.apply_updates(params, ups, key=key if stochastic else None, stochastic=stochastic)
    torch.cuda.synchronize()
    keys = orc.split(key, len(sizes))
    for i, dt in enumerate(dtypes):
        pd = orc.BF16 if dt == "bf16" else orc.F32
        bits = orc.random_bits(keys[i], host[i].size) if stochastic else None
        orc.apply_updates(host[i], pd, uhost[i], bits=bits)
        np.testing.assert_array_equal(to_host(out[f"p{i}"]).view(np.uint8), host[i].view(np.uint8))


def test_apply_updates_sub_ulp_signal():
    """tests/test_utils.py:89-103: ones(4096) bf16 + 2^-9 stays 1 under RNE
    and rises in mean under stochastic rounding."""
    import torch

    rf = _rf()
    p1 = {"w": torch.ones((4096,), dtype=torch.bfloat16, device="cuda")}
    p2 = {"w": torch.ones((4096,), dtype=torch.bfloat16, device="cuda")}
    u = {"w": torch.full((4096,), 2.0**-9, dtype=torch.float32, device="cuda")}
    det = rf.apply_updates(p1, u, stochastic=False)
    sto = rf.apply_updates(p2, u, key=rf.prng.PRNGKey(0))
    assert torch.all(det["w"] == 1.0)
    assert torch.any(sto["w"] > det["w"])
    assert sto["w"].float().mean() > det["w"].float().mean()


def test_apply_updates_skips_none_and_masked():
    import torch

    rf = _rf()
    params = {"w": torch.ones((2,), device="cuda"), "none": torch.ones((2,), device="cuda"),
              "masked": torch.ones((2,), device="cuda")}
    updates = {"w": torch.ones((2,), device="cuda"), "none": None, "masked": rf.MaskedNode()}
    out = rf.apply_updates(params, updates, key=rf.prng.PRNGKey(0), stochastic=False)
    torch.cuda.synchronize()
    assert torch.allclose(out["w"], torch.full((2,), 2.0, device="cuda"))
    assert torch.allclose(out["none"], torch.ones((2,), device="cuda"))
    assert torch.allclose(out["masked"], torch.ones((2,), device="cuda"))


def test_apply_updates_prefix_skips_subtrees():
    import torch

    rf = _rf()
    params = {"train": {"w": torch.ones((2,), device="cuda"), "b": torch.full((2,), 3.0, device="cuda")},
              "static": {"name": "layer"}}
    updates = {"train": {"w": torch.ones((2,), device="cuda"), "b": None}, "static": None}
    out = rf.apply_updates_prefix(params, updates, stochastic=False)
    torch.cuda.synchronize()
    assert torch.allclose(out["train"]["w"], torch.full((2,), 2.0, device="cuda"))
    assert torch.allclose(out["train"]["b"], torch.full((2,), 3.0, device="cuda"))
    assert out["static"] == {"name": "layer"}


def test_tree_stochastic_cast_keys_and_passthrough():
    """utils.py:374-409: keys are split over every leaf of the flatten with
    is_leaf=None/MaskedNode, so aux leaves consume subkeys too; aux leaves and
    bf16 leaves come back unchanged, complex leaves become complex64, f32
    leaves are stochastically rounded with their own subkey."""
    import torch

    from rollfast_amd._base import MaskedNode
    from rollfast_amd.utils import _tree_stochastic_cast

    rf = _rf()
    rng = np.random.default_rng(7)
    a = _edge_values(rng, 5000)
    d = bf16_bits(rng.standard_normal(300).astype(np.float32))
    e = rng.standard_normal(777).astype(np.float32)
    mask = MaskedNode()
    tree = {"a": to_device(a, "f32"), "b": None, "c": mask, "d": to_device(d, "bf16"),
            "e": to_device(e, "f32"), "z": torch.ones(3, dtype=torch.complex128, device="cuda")}
    key = rf.prng.PRNGKey(11)
    out = _tree_stochastic_cast(tree, torch.bfloat16, key)
    torch.cuda.synchronize()
    # flatten order with aux leaves as leaves: a, b, c, d, e, z -> 6 subkeys
    keys = orc.split(tuple(int(k) for k in key), 6)
    for name, x, i in (("a", a, 0), ("e", e, 4)):
        want = orc.sr_bf16(x, orc.random_bits(tuple(keys[i]), x.size))
        got = to_host(out[name])
        nan = np.isnan(orc.bf16_bits_to_f32(want))
        np.testing.assert_array_equal(got[~nan], want[~nan], err_msg=name)
    assert out["b"] is None and out["c"] is mask
    assert out["d"] is tree["d"]
    assert out["z"].dtype == torch.complex64
    f32 = _tree_stochastic_cast({"a": tree["a"]}, torch.float32, key)["a"]
    assert f32.dtype == torch.float32


def test_apply_updates_nested_tree_native_and_python_walks():
    """apply_updates over a nested dict / list / tuple tree with None and
    MaskedNode leaves: the native walk (f32 updates) and the Python walk
    (bf16 updates, converted) give the oracle's result with the per-leaf key
    of each leaf's flatten position; the returned tree has new containers
    around the same tensors."""
    import torch

    rf = _rf()
    rng = np.random.default_rng(9)

    def tree(seed_shift):
        r = np.random.default_rng(100 + seed_shift)
        p = [bf16_bits((r.standard_normal(n) * 0.5).astype(np.float32)) for n in (300, 70, 5000)]
        pf = (r.standard_normal(64) * 0.5).astype(np.float32)
        return p, pf

    hp, hpf = tree(0)
    u = [(rng.standard_normal(n) * 1e-3).astype(np.float32) for n in (300, 70, 5000)]
    uf = (rng.standard_normal(64) * 1e-3).astype(np.float32)
    key = rf.prng.PRNGKey(5)
    results = []
    for native in (True, False):
        params = {"a": [to_device(hp[0], "bf16"), (to_device(hp[1], "bf16"), None)],
                  "b": {"x": to_device(hpf, "f32"), "y": to_device(hp[2], "bf16")}}
        udt = torch.float32 if native else torch.bfloat16
        ups = {"a": [torch.from_numpy(u[0]).cuda().to(udt), (torch.from_numpy(u[1]).cuda().to(udt), None)],
               "b": {"x": torch.from_numpy(uf).cuda().to(udt), "y": rf.MaskedNode()}}
        out = rf.apply_updates(params, ups, key=key)
        torch.cuda.synchronize()
        assert out is not params and out["a"] is not params["a"] and out["a"][0] is params["a"][0]
        assert out["a"][1][1] is None and out["b"]["y"] is params["b"]["y"]
        results.append(out)
    # flatten order: a/0, a/1/0, a/1/1 (None), b/x, b/y -> indices 0, 1, 2, 3, 4
    keys = orc.split(key, 5)
    for native, out in zip((True, False), results):
        uu = [u[0], u[1], uf] if native else [orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(x)) for x in (u[0], u[1], uf)]
        want0, want1, wantx = hp[0].copy(), hp[1].copy(), hpf.copy()
        orc.apply_updates(want0, orc.BF16, uu[0], bits=orc.random_bits(keys[0], 300))
        orc.apply_updates(want1, orc.BF16, uu[1], bits=orc.random_bits(keys[1], 70))
        orc.apply_updates(wantx, orc.F32, uu[2], bits=orc.random_bits(keys[3], 64))
        np.testing.assert_array_equal(to_host(out["a"][0]), want0)
        np.testing.assert_array_equal(to_host(out["a"][1][0]), want1)
        np.testing.assert_array_equal(to_host(out["b"]["x"]).view(np.uint32), wantx.view(np.uint32))
        np.testing.assert_array_equal(to_host(out["b"]["y"]), hp[2])


def test_symmetric_int8_exact_ties_and_sr_closed_form():
    """The kernel's symmetric quantizer on exact ties of jnp.round (half to
    even, adam8.py:455) and on the floor + Bernoulli rule with fed words
    placed one step below, at and above p (adam8.py:456-458); both against
    the closed forms the oracle is pinned to."""
    from tests.test_oracle import _bits_for_uniform, _symmetric_tie_block

    rf = _rf()
    x, n = _symmetric_tie_block()
    qb = rf.quantize_blocks(to_device(x, "f32"), block_size=256, quantizer="symmetric_int8")
    got = to_host(qb.values).view(np.int8).astype(np.int64)[:n]
    k = np.arange(-127, 127)
    np.testing.assert_array_equal(got[:254], np.where(k % 2 == 0, k, k + 1))
    assert list(got[254:]) == [127, -127]
    step = 2.0 ** -23
    s_vals, us, want = [], [], []
    for s, lo in ((2.25, 2), (-2.25, -3), (0.75, 0), (-0.75, -1), (126.5, 126), (-126.5, -127)):
        p = s - lo
        for u, w in ((p - step, lo + 1), (p, lo), (min(p + step, 1 - step), lo), (0.0, lo + 1)):
            s_vals.append(s)
            us.append(u)
            want.append(w)
    xs = np.concatenate([np.float32(s_vals), np.float32([127.0])])
    bits = np.zeros(xs.size, np.uint32)
    bits[:len(us)] = _bits_for_uniform(us)
    qb = rf.quantize_blocks(to_device(xs, "f32"), block_size=xs.size, quantizer="symmetric_int8",
                            stochastic_rounding=True, random_bits=to_device(bits, "u32"))
    got = to_host(qb.values).view(np.int8).astype(np.int64)[:len(want)]
    np.testing.assert_array_equal(got, want)
