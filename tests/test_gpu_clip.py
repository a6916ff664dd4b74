"""GPU parity of the fused global-norm clipping (rollfast
finetune/transforms.py:20-82 clip_by_global_norm before the optimizer step,
``adamw8_step(..., clip_global_norm=...)``) against the oracle: the oracle
computes (scale, norm), clips the grads with the leaf-dtype semantics, then
runs the step.

Bar: scale and norm bit-exact (both round each leaf's sum of squares once
from a float64 sum and add the leaf sums in f32 in leaf order); codes,
scales and moments bit-exact; params bit-exact with ``exact=True``.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import OracleTree, bf16_bits, bf16_to_f32, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu

SPEC = [((16, 2048), "bf16", "bf16"), ((3, 3000), "f32", "f32"), ((768,), "bf16", "bf16"), ((5, 4099), "f32", "bf16"),
        ((40000,), "bf16", "bf16")]


def _trees(seed, gscale):
    rng = np.random.default_rng(seed)
    hp, dp, hg, dg = {}, {}, [], {}
    for i, (shape, pd, gd) in enumerate(SPEC):
        n = int(np.prod(shape))
        p = gaussian(rng, (n,), 0.02)
        p = bf16_bits(p) if pd == "bf16" else p
        g = gaussian(rng, (n,), gscale)
        g = bf16_bits(g) if gd == "bf16" else g
        hp[f"l{i}"] = p
        dp[f"l{i}"] = to_device(p, pd).reshape(shape)
        hg.append(g)
        dg[f"l{i}"] = to_device(g, gd).reshape(shape)
    return hp, dp, hg, dg


def _f32_values(g, gd):
    return bf16_to_f32(g) if gd == "bf16" else g


def _oracle_tree(params, adam_state, rf):
    leaves = []
    for i, (shape, pd, gd) in enumerate(SPEC):
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        L = {"pdtype": pd, "gdtype": gd, "size": int(np.prod(shape)), "param": to_host(params[f"l{i}"]).copy()}
        if isinstance(m, rf.QuantizedBlocks):
            L.update(kind="quant", block_size=m.block_size, mu=to_host(m.values).copy(),
                     mu_scales=to_host(m.scales).copy(), nu=to_host(v.values).copy(), nu_scales=to_host(v.scales).copy())
        else:
            L.update(kind="f32", mu=to_host(m).copy(), nu=to_host(v).copy())
        leaves.append(L)
    return OracleTree(leaves)


def _check(tree, params, adam_state, rf, what):
    for i, (shape, pd, _gd) in enumerate(SPEC):
        L = tree.leaves[i]
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        if isinstance(m, rf.QuantizedBlocks):
            np.testing.assert_array_equal(to_host(m.values), L["mu"], err_msg=f"{what} leaf {i} mu codes")
            np.testing.assert_array_equal(to_host(v.values), L["nu"], err_msg=f"{what} leaf {i} nu codes")
            np.testing.assert_array_equal(to_host(m.scales).view(np.uint32), L["mu_scales"].view(np.uint32))
            np.testing.assert_array_equal(to_host(v.scales).view(np.uint32), L["nu_scales"].view(np.uint32))
        else:
            np.testing.assert_array_equal(to_host(m).view(np.uint32), L["mu"].view(np.uint32))
            np.testing.assert_array_equal(to_host(v).view(np.uint32), L["nu"].view(np.uint32))
        got = to_host(params[f"l{i}"])
        np.testing.assert_array_equal(got.view(np.uint16 if pd == "bf16" else np.uint32),
                                      L["param"].view(np.uint16 if pd == "bf16" else np.uint32),
                                      err_msg=f"{what} leaf {i} params")


@pytest.mark.parametrize("gscale,max_norm", [(1e-2, 1.0), (1e-2, 1e6), (3.0, 0.5)])
def test_fused_clip_matches_oracle(gscale, max_norm):
    import torch

    import rollfast_amd as rf

    hp, params, hg, dg = _trees(7, gscale)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=True)
    state = tx.init(params)
    stats = torch.empty(2, dtype=torch.float32, device="cuda")
    for step in range(2):
        if step:
            _, _, hg, dg = _trees(100 + step, gscale)
        scale, norm = orc.global_norm_clip_scale([_f32_values(g, gd) for g, (_s, _p, gd) in zip(hg, SPEC)], max_norm)
        clipped = [orc.clip_leaf(g, orc.BF16 if gd == "bf16" else orc.F32, scale) for g, (_s, _p, gd) in zip(hg, SPEC)]
        tree = _oracle_tree(params, state[0], rf)
        tree.step(clipped, weight_decay=0.01, lr=1e-3, count=step + 1)
        params, state = rf.adamw8_step(tx, params, dg, state, stochastic=False, clip_global_norm=max_norm,
                                       clip_stats=stats)
        torch.cuda.synchronize()
        got = stats.cpu().numpy()
        assert got[1].view(np.uint32) == np.float32(norm).view(np.uint32), (got[1], norm)
        assert got[0].view(np.uint32) == np.float32(scale).view(np.uint32), (got[0], scale)
        if max_norm == 1e6:
            assert got[0] == 1.0
        else:
            assert got[0] < 1.0
        _check(tree, params, state[0], rf, f"step {step + 1}")
        # the grads themselves are left as they were
        for i, (_s, _p, gd) in enumerate(SPEC):
            np.testing.assert_array_equal(to_host(dg[f"l{i}"]), hg[i])


def test_inactive_clip_equals_no_clip():
    import torch

    import rollfast_amd as rf

    _, pa, _, g = _trees(8, 1e-3)
    _, pb, _, _ = _trees(8, 1e-3)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01)
    sa, sb = tx.init(pa), tx.init(pb)
    pa, sa = rf.adamw8_step(tx, pa, g, sa, stochastic=False, clip_global_norm=1e9)
    pb, sb = rf.adamw8_step(tx, pb, g, sb, stochastic=False)
    torch.cuda.synchronize()
    for k in pa:
        np.testing.assert_array_equal(to_host(pa[k]), to_host(pb[k]))


def test_clip_with_full_precision_adamw():
    import torch

    import rollfast_amd as rf

    hp, params, hg, dg = _trees(9, 0.1)
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, exact=True)
    state = tx.init(params)
    scale, _norm = orc.global_norm_clip_scale([_f32_values(g, gd) for g, (_s, _p, gd) in zip(hg, SPEC)], 1.0)
    clipped = [orc.clip_leaf(g, orc.BF16 if gd == "bf16" else orc.F32, scale) for g, (_s, _p, gd) in zip(hg, SPEC)]
    leaves = []
    for i, (shape, pd, gd) in enumerate(SPEC):
        leaves.append({"pdtype": pd, "gdtype": gd, "size": int(np.prod(shape)), "kind": "f32",
                       "param": hp[f"l{i}"].copy(), "mu": to_host(state[0].mu[f"l{i}"]).copy(),
                       "nu": to_host(state[0].nu[f"l{i}"]).copy()})
    tree = OracleTree(leaves)
    tree.step(clipped, weight_decay=0.01, lr=1e-3, count=1, ema_weight_f32=True)
    params, state = rf.adamw_step(tx, params, dg, state, stochastic=False, clip_global_norm=1.0)
    torch.cuda.synchronize()
    for i, (shape, pd, _gd) in enumerate(SPEC):
        L = tree.leaves[i]
        np.testing.assert_array_equal(to_host(state[0].mu[f"l{i}"]).view(np.uint32), L["mu"].view(np.uint32))
        np.testing.assert_array_equal(to_host(params[f"l{i}"]).view(np.uint16 if pd == "bf16" else np.uint32),
                                      L["param"].view(np.uint16 if pd == "bf16" else np.uint32))


def test_nan_gradient_gives_nan_scale_like_the_reference():
    """A NaN anywhere makes the norm and the scale NaN (jnp.minimum
    propagates it), so every clipped gradient is NaN: codes follow the
    oracle's NaN rules, params become NaN."""
    import torch

    import rollfast_amd as rf

    hp, params, hg, dg = _trees(10, 1e-2)
    hg[1] = hg[1].copy()
    hg[1][5] = np.nan
    dg["l1"] = to_device(hg[1], "f32").reshape(SPEC[1][0])
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=True)
    state = tx.init(params)
    scale, norm = orc.global_norm_clip_scale([_f32_values(g, gd) for g, (_s, _p, gd) in zip(hg, SPEC)], 1.0)
    assert np.isnan(scale) and np.isnan(norm)
    clipped = [orc.clip_leaf(g, orc.BF16 if gd == "bf16" else orc.F32, scale) for g, (_s, _p, gd) in zip(hg, SPEC)]
    tree = _oracle_tree(params, state[0], rf)
    tree.step(clipped, weight_decay=0.01, lr=1e-3, count=1)
    stats = torch.empty(2, dtype=torch.float32, device="cuda")
    params, state = rf.adamw8_step(tx, params, dg, state, stochastic=False, clip_global_norm=1.0, clip_stats=stats)
    torch.cuda.synchronize()
    assert np.isnan(stats.cpu().numpy()).all()
    for i, (_shape, pd, _gd) in enumerate(SPEC):
        L = tree.leaves[i]
        m = state[0].mu[f"l{i}"]
        if isinstance(m, rf.QuantizedBlocks):
            np.testing.assert_array_equal(to_host(m.values), L["mu"])
            np.testing.assert_array_equal(to_host(m.scales).view(np.uint32), L["mu_scales"].view(np.uint32))
        got = to_host(params[f"l{i}"])
        vals = bf16_to_f32(got) if pd == "bf16" else got
        assert np.isnan(vals).all()


def test_clip_argument_errors():
    import torch

    import rollfast_amd as rf

    _, params, _, g = _trees(11, 1e-2)
    tx = rf.adamw8(learning_rate=1e-3)
    state = tx.init(params)
    for bad in (0.0, -1.0, float("nan"), float("inf")):
        with pytest.raises(ValueError):
            rf.adamw8_step(tx, params, g, state, stochastic=False, clip_global_norm=bad)
    with pytest.raises(ValueError):
        rf.adamw8_step(tx, params, g, state, stochastic=False, clip_global_norm=1.0,
                       clip_stats=torch.empty(1, device="cuda"))


def test_clip_transform_matches_oracle_and_passes_none():
    """rollfast_amd.clip_by_global_norm (transforms.py:20-82): every leaf is
    leaf * scale in its dtype; None leaves pass through; the count advances."""
    import torch

    import rollfast_amd as rf

    _, _, hg, dg = _trees(12, 0.05)
    tree = dict(dg)
    tree["none"] = None
    tx = rf.clip_by_global_norm(1.0)
    state = tx.init(tree)
    stats = torch.empty(2, dtype=torch.float32, device="cuda")
    out, state = tx.update(tree, state, None, stats=stats)
    torch.cuda.synchronize()
    scale, norm = orc.global_norm_clip_scale([_f32_values(g, gd) for g, (_s, _p, gd) in zip(hg, SPEC)], 1.0)
    got = stats.cpu().numpy()
    assert got[0] == scale and got[1] == norm and scale < 1.0
    for i, (shape, _pd, gd) in enumerate(SPEC):
        want = orc.clip_leaf(hg[i], orc.BF16 if gd == "bf16" else orc.F32, scale)
        o = out[f"l{i}"]
        assert tuple(o.shape) == shape
        np.testing.assert_array_equal(to_host(o).view(np.uint16 if gd == "bf16" else np.uint32),
                                      want.view(np.uint16 if gd == "bf16" else np.uint32))
        np.testing.assert_array_equal(to_host(dg[f"l{i}"]), hg[i])  # inputs untouched
    assert out["none"] is None
    assert int(state.count) == 1 and isinstance(state, rf.GlobalNormClipState)


def test_clip_transform_then_update_equals_fused_clip():
    """clip -> tx.update -> apply_updates (the reference's chain) gives the
    same bits as the fused adamw8_step(..., clip_global_norm=...)."""
    import torch

    import rollfast_amd as rf

    _, pa, _, g = _trees(13, 0.05)
    _, pb, _, _ = _trees(13, 0.05)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=True)
    clip = rf.clip_by_global_norm(1.0)
    sa, sb, cs = tx.init(pa), tx.init(pb), clip.init(pb)
    for _ in range(2):
        pa, sa = rf.adamw8_step(tx, pa, g, sa, stochastic=False, clip_global_norm=1.0)
        gc, cs = clip.update(g, cs)
        u, sb = tx.update(gc, sb, pb)
        pb = rf.apply_updates(pb, u, stochastic=False)
        torch.cuda.synchronize()
        for k in pa:
            np.testing.assert_array_equal(to_host(pa[k]), to_host(pb[k]))
            ma, mb = sa[0].mu[k], sb[0].mu[k]
            if isinstance(ma, rf.QuantizedBlocks):
                np.testing.assert_array_equal(to_host(ma.values), to_host(mb.values))
