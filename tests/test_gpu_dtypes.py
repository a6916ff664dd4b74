"""GPU parity for the dtypes beyond f32/bf16: block scales stored as
``scale_dtype`` bfloat16 or float16 (adam8.py:167-186, :202), float16 params
and grads (adam8.py:620 takes any inexact dtype; apply_updates rounds
non-bf16 params to nearest, utils.py:700), float16 fallback moments
(``fallback_dtype``, adam8.py:688) and float16 ``mu_dtype`` in the
full-precision AdamW (optim/adam.py).

Bars as everywhere: codes, scales and moments bit-exact; params bit-exact
with ``exact=True`` (IEEE direction), within one ulp of their dtype
otherwise.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import OracleTree, bf16_ulp_distance, to_device, to_host

pytestmark = pytest.mark.gpu

DT = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}


def _rf():
    import rollfast_amd as rf

    return rf


def _values(rng, n, dtype, std):
    x = (rng.standard_normal(n) * std).astype(np.float32)
    return orc.from_f32(x, DT[dtype])


@pytest.mark.parametrize("scale_dtype", ["bf16", "f16"])
@pytest.mark.parametrize("quantizer", ["dynamic_signed", "dynamic_unsigned", "symmetric_int8"])
@pytest.mark.parametrize("x_dtype", ["f32", "bf16", "f16"])
def test_quantize_dequantize_16_bit_scales_and_inputs(scale_dtype, quantizer, x_dtype):
    """quantize_blocks of an f32 / bf16 / f16 input with 16-bit block scales:
    the codes come from the f32 scale, the stored scales are it rounded
    (bit patterns compared), dequantize reads f32(stored) and writes any of
    the three dtypes."""
    import torch

    rf = _rf()
    rng = np.random.default_rng(31)
    n = 2048 * 6 + 300
    x = _values(rng, n, x_dtype, 1.0)
    xf = orc.to_f32(x, DT[x_dtype]) * np.float32(np.exp(rng.uniform(-12, 8)))
    x = orc.from_f32(xf, DT[x_dtype])
    xf = orc.to_f32(x, DT[x_dtype])
    if quantizer == "dynamic_unsigned":
        xf = np.abs(xf)
        x = orc.from_f32(xf, DT[x_dtype])
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[scale_dtype]
    qb = rf.quantize_blocks(to_device(x, x_dtype), block_size=2048, quantizer=quantizer, scale_dtype=tdt)
    q = {"dynamic_signed": orc.Q_SIGNED, "dynamic_unsigned": orc.Q_UNSIGNED, "symmetric_int8": orc.Q_SYMMETRIC}
    codes, scales = orc.quantize(xf, 2048, q[quantizer], scale_dtype=DT[scale_dtype])
    assert qb.scales.dtype == tdt
    np.testing.assert_array_equal(to_host(qb.values).view(np.uint8), codes.reshape(-1).view(np.uint8))
    np.testing.assert_array_equal(to_host(qb.scales), orc.from_f32(scales, DT[scale_dtype]))
    for out in ("f32", "bf16", "f16"):
        odt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[out]
        back = rf.dequantize_blocks(qb, dtype=odt)
        torch.cuda.synchronize()
        want = orc.from_f32(orc.dequantize(codes, scales, n, 2048, q[quantizer]), DT[out])
        got = to_host(back)
        if out == "f32":
            np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        else:
            np.testing.assert_array_equal(got, want)


def _tree_spec():
    """(shape, param dtype, grad dtype): full f16 blocks (the fast kernel's
    f16 instance), a partial f16 block, f16 params with bf16 grads (the
    generic kernel), a bf16 leaf and an f32 leaf, small leaves on fallback
    moments."""
    return [((6, 2048), "f16", "f16"), ((2048 + 700,), "f16", "f16"), ((4, 2048), "f16", "bf16"),
            ((3, 2048), "bf16", "bf16"), ((2, 2048), "f32", "f32"), ((900,), "f16", "f16"), ((300,), "f16", "f32")]


def _adamw8_tree_run(*, scale_dtype, fallback, exact, steps=3, psr=False, clip=None):
    import torch

    rf = _rf()
    spec = _tree_spec()
    rng = np.random.default_rng(5)
    host_p = [_values(rng, int(np.prod(s)), pd, 0.02) for s, pd, _ in spec]
    params = {f"l{i}": to_device(h, pd).reshape(s) for i, (h, (s, pd, _)) in enumerate(zip(host_p, spec))}
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, min_size=1024, exact=exact,
                   scale_dtype=tdt[scale_dtype], fallback_dtype=tdt[fallback])
    state = tx.init(params)
    leaves = []
    for i, (s, pd, gd) in enumerate(spec):
        m, v = state[0].mu[f"l{i}"], state[0].nu[f"l{i}"]
        L = {"pdtype": pd, "gdtype": gd, "size": int(np.prod(s)), "param": None}
        if isinstance(m, rf.QuantizedBlocks):
            assert m.scales.dtype == tdt[scale_dtype]
            L.update(kind="quant", block_size=2048, mu=to_host(m.values).copy(), nu=to_host(v.values).copy(),
                     mu_scales=orc.to_f32(to_host(m.scales), DT[scale_dtype]).copy(),
                     nu_scales=orc.to_f32(to_host(v.scales), DT[scale_dtype]).copy())
        else:
            assert m.dtype == tdt[fallback]
            L.update(kind=fallback, mu=to_host(m).copy(), nu=to_host(v).copy())
        leaves.append(L)
    tree = OracleTree(leaves)
    for step in range(steps):
        ghost = [_values(rng, L["size"], gd, 1e-2) for L, (_, _, gd) in zip(leaves, spec)]
        gdev = {f"l{i}": to_device(g, gd).reshape(s) for i, (g, (s, _, gd)) in enumerate(zip(ghost, spec))}
        for i, L in enumerate(leaves):
            L["param"] = to_host(params[f"l{i}"]).copy()
        pkey = rf.prng.PRNGKey(70 + step)
        p_bits = None
        if psr:
            kp = orc.split(tuple(int(k) for k in pkey), len(spec))
            p_bits = [orc.random_bits(tuple(kp[i]), L["size"]) for i, L in enumerate(leaves)]
        if clip is not None:
            f32g = [orc.to_f32(g, DT[gd]) for g, (_, _, gd) in zip(ghost, spec)]
            scale, _ = orc.global_norm_clip_scale(f32g, clip)
            ghost = [orc.clip_leaf(g, DT[gd], scale) for g, (_, _, gd) in zip(ghost, spec)]
        tree.step(ghost, weight_decay=0.01, lr=1e-3, count=step + 1, param_sr=psr, p_bits=p_bits,
                  scale_dtype=DT[scale_dtype])
        params, state = rf.adamw8_step(tx, params, gdev, state, key=pkey if psr else None, stochastic=psr,
                                       clip_global_norm=clip)
        torch.cuda.synchronize()
        for i, L in enumerate(leaves):
            m, v = state[0].mu[f"l{i}"], state[0].nu[f"l{i}"]
            what = f"step {step + 1} leaf {i} {spec[i]}"
            if L["kind"] == "quant":
                np.testing.assert_array_equal(to_host(m.values), L["mu"], err_msg=f"{what}: mu codes")
                np.testing.assert_array_equal(to_host(v.values), L["nu"], err_msg=f"{what}: nu codes")
                np.testing.assert_array_equal(to_host(m.scales), orc.from_f32(L["mu_scales"], DT[scale_dtype]))
                np.testing.assert_array_equal(to_host(v.scales), orc.from_f32(L["nu_scales"], DT[scale_dtype]))
            else:
                np.testing.assert_array_equal(to_host(m).view(L["mu"].dtype), L["mu"], err_msg=f"{what}: mu")
                np.testing.assert_array_equal(to_host(v).view(L["nu"].dtype), L["nu"], err_msg=f"{what}: nu")
            got = to_host(params[f"l{i}"])
            if spec[i][1] == "f32":
                if exact:
                    np.testing.assert_array_equal(got.view(np.uint32), L["param"].view(np.uint32), err_msg=what)
            elif exact:
                np.testing.assert_array_equal(got, L["param"], err_msg=f"{what}: params")
            else:
                assert bf16_ulp_distance(got, L["param"]).max() <= 1, what


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("scale_dtype", ["bf16", "f16"])
def test_adamw8_16_bit_scales_and_f16_params(scale_dtype, exact):
    _adamw8_tree_run(scale_dtype=scale_dtype, fallback="f32", exact=exact)


def test_adamw8_f16_fallback_moments_f32_scales():
    _adamw8_tree_run(scale_dtype="f32", fallback="f16", exact=True)


def test_adamw8_f16_tree_param_sr_and_clipping():
    """Param SR rounds the bf16 leaves only (f16 params round to nearest);
    the fused clipping scales f16 grads by f16(scale)."""
    _adamw8_tree_run(scale_dtype="f32", fallback="f32", exact=True, psr=True, clip=0.5, steps=2)


def test_full_precision_adamw_f16_params_and_moments():
    """optim/adam.py adamw with float16 params, grads and mu_dtype (moments
    stored with astype, round to nearest), against the oracle (IEEE
    direction: bit-exact)."""
    import torch

    rf = _rf()
    rng = np.random.default_rng(9)
    shapes = [(4, 2048), (1500,)]
    host_p = [_values(rng, int(np.prod(s)), "f16", 0.02) for s in shapes]
    params = {f"l{i}": to_device(h, "f16").reshape(s) for i, (h, s) in enumerate(zip(host_p, shapes))}
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, mu_dtype=torch.float16, exact=True)
    state = tx.init(params)
    leaves = [{"pdtype": "f16", "gdtype": "f16", "size": int(np.prod(s)), "kind": "f16",
               "param": None, "mu": to_host(state[0].mu[f"l{i}"]).copy(), "nu": to_host(state[0].nu[f"l{i}"]).copy()}
              for i, s in enumerate(shapes)]
    tree = OracleTree(leaves)
    for step in range(3):
        ghost = [_values(rng, L["size"], "f16", 1e-2) for L in leaves]
        gdev = {f"l{i}": to_device(g, "f16").reshape(s) for i, (g, s) in enumerate(zip(ghost, shapes))}
        for i, L in enumerate(leaves):
            L["param"] = to_host(params[f"l{i}"]).copy()
        tree.step(ghost, weight_decay=0.01, lr=1e-3, count=step + 1, ema_weight_f32=True, zero_decay=True)
        params, state = rf.adamw_step(tx, params, gdev, state, stochastic=False)
        torch.cuda.synchronize()
        for i, L in enumerate(leaves):
            np.testing.assert_array_equal(to_host(params[f"l{i}"]), L["param"])
            np.testing.assert_array_equal(to_host(state[0].mu[f"l{i}"]), L["mu"])
            np.testing.assert_array_equal(to_host(state[0].nu[f"l{i}"]), L["nu"])


def test_apply_updates_and_clip_f16_leaves():
    """apply_updates of f32 updates to f16 params (nearest even, no
    stochastic rounding below bf16) and clip_by_global_norm of f16 grads
    (times f16(scale), one rounding), against the oracle."""
    import torch

    rf = _rf()
    rng = np.random.default_rng(4)
    p = _values(rng, 5000, "f16", 1.0)
    u = (rng.standard_normal(5000) * 1e-3).astype(np.float32)
    params = {"a": to_device(p, "f16")}
    out = rf.apply_updates(params, {"a": to_device(u, "f32")}, key=rf.prng.PRNGKey(1), stochastic=True)
    torch.cuda.synchronize()
    want = p.copy()
    orc.apply_updates(want, orc.F16, u)
    np.testing.assert_array_equal(to_host(out["a"]), want)
    g = _values(rng, 7000, "f16", 3.0)
    tx = rf.clip_by_global_norm(1.0)
    clipped, _ = tx.update({"g": to_device(g, "f16")}, tx.init(None))
    torch.cuda.synchronize()
    scale, _ = orc.global_norm_clip_scale([orc.f16_bits_to_f32(g)], 1.0)
    np.testing.assert_array_equal(to_host(clipped["g"]), orc.clip_leaf(g, orc.F16, scale))
