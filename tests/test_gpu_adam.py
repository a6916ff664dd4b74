"""GPU parity of the full-precision AdamW path (rollfast optim/adam.py:
scale_by_adam / adamw with f32 or bf16 moments) against the CPU oracle.

Bar: f32 moments bit-exact; bf16 moments (stochastically rounded storage)
bit-exact for the same bits; params bit-exact with ``exact=True`` and within
one bf16 ulp otherwise; update-only f32 updates bit-exact (exact) or within
8 f32 ulps.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import OracleTree, bf16_bits, bf16_ulp_distance, f32_params_close, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu

SPEC = [((8, 2048), "bf16", "bf16"), ((3, 1000), "f32", "f32"), ((700,), "bf16", "f32"), ((5,), "f32", "bf16")]
# Every leaf a whole number of 2048-element chunks: the launch's generic list
# holds full-chunk fallback units only and takes the kernel instance built
# for that case alone.
VEC_SPEC = [((8, 2048), "bf16", "bf16"), ((2, 4096), "f32", "f32"), ((2048,), "bf16", "f32"), ((3, 2048), "f32", "bf16")]


def _build(spec, seed):
    rng = np.random.default_rng(seed)
    host, dev = {}, {}
    for i, (shape, pd, _gd) in enumerate(spec):
        p = gaussian(rng, (int(np.prod(shape)),), 0.02)
        p = bf16_bits(p) if pd == "bf16" else p
        host[f"l{i}"] = p
        dev[f"l{i}"] = to_device(p, pd).reshape(shape)
    return host, dev


def _grads(spec, seed):
    rng = np.random.default_rng(seed)
    host, dev = [], {}
    for i, (shape, _pd, gd) in enumerate(spec):
        g = gaussian(rng, (int(np.prod(shape)),), 1e-2)
        g = bf16_bits(g) if gd == "bf16" else g
        host.append(g)
        dev[f"l{i}"] = to_device(g, gd).reshape(shape)
    return host, dev


def _oracle_tree(spec, params, adam_state):
    import torch

    leaves = []
    for i, (shape, pd, gd) in enumerate(spec):
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        leaves.append({"pdtype": pd, "gdtype": gd, "size": int(np.prod(shape)),
                       "kind": "bf16" if m.dtype == torch.bfloat16 else "f32",
                       "param": to_host(params[f"l{i}"]).copy(), "mu": to_host(m).copy(), "nu": to_host(v).copy()})
    return OracleTree(leaves)


def _store_bits(state_key, n_leaves, sizes):
    """Per-leaf storage bits of optim/adam.py: next, sr = split(key, 2);
    k1, k2 = split(sr); leaf i uses split(k1 | k2, n_leaves)[i]."""
    _next, sr = orc.split(tuple(int(k) for k in state_key), 2)
    k1, k2 = orc.split(tuple(sr), 2)
    s1 = orc.split(tuple(k1), n_leaves)
    s2 = orc.split(tuple(k2), n_leaves)
    return ([orc.random_bits(tuple(s1[i]), sizes[i]) for i in range(n_leaves)],
            [orc.random_bits(tuple(s2[i]), sizes[i]) for i in range(n_leaves)])


def _compare(spec, tree, params, adam_state, exact, what, before=None):
    import torch

    for i, (shape, pd, _gd) in enumerate(spec):
        L = tree.leaves[i]
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        gm, gv = to_host(m), to_host(v)
        if m.dtype == torch.float32:
            gm, gv = gm.view(np.uint32), gv.view(np.uint32)
            wm, wv = L["mu"].view(np.uint32), L["nu"].view(np.uint32)
        else:
            wm, wv = L["mu"], L["nu"]
        np.testing.assert_array_equal(gm, wm, err_msg=f"{what} leaf {i} mu")
        np.testing.assert_array_equal(gv, wv, err_msg=f"{what} leaf {i} nu")
        if params is None:
            continue
        got = to_host(params[f"l{i}"])
        want = L["param"]
        if exact:
            np.testing.assert_array_equal(got.view(np.uint16 if pd == "bf16" else np.uint32),
                                          want.view(np.uint16 if pd == "bf16" else np.uint32),
                                          err_msg=f"{what} leaf {i} params")
        elif pd == "bf16":
            assert bf16_ulp_distance(got, want).max() <= 1, f"{what} leaf {i}"
        else:
            assert f32_params_close(got, want, before[i]).all(), f"{what} leaf {i}"


def _run_adamw(*, mu_dtype, exact, nesterov=False, psr=False, fed=False, steps=3, wd=0.01, spec=SPEC):
    import torch

    import rollfast_amd as rf

    SPEC = spec
    host, params = _build(SPEC, 1)
    tx = rf.adamw(learning_rate=1e-3, weight_decay=wd, mu_dtype=mu_dtype, nesterov=nesterov, exact=exact,
                  key=rf.prng.PRNGKey(3))
    state = tx.init(params)
    sizes = [int(np.prod(s)) for s, _, _ in SPEC]
    for step in range(steps):
        ghost, gdev = _grads(SPEC, 100 + step)
        tree = _oracle_tree(SPEC, params, state[0])
        mb = vb = None
        store = mu_dtype is not None
        if store:
            mb, vb = _store_bits(state[0].key, len(SPEC), sizes)
        pkey = rf.prng.PRNGKey(50 + step)
        pb = None
        if psr:
            kp = orc.split(tuple(int(k) for k in pkey), len(SPEC))
            pb = [orc.random_bits(tuple(kp[i]), sizes[i]) for i in range(len(SPEC))]
        before = [L["param"].copy() for L in tree.leaves]
        tree.step(ghost, weight_decay=wd, lr=1e-3, count=step + 1, nesterov=nesterov, param_sr=psr, mu_bits=mb,
                  nu_bits=vb, p_bits=pb, ema_weight_f32=True, store_sr=store, zero_decay=True)
        bits = None
        if fed:
            bits = {}
            for i in range(len(SPEC)):
                z = np.zeros(sizes[i], np.uint32)
                bits[i] = (to_device(mb[i] if store else z, "u32"), to_device(vb[i] if store else z, "u32"),
                           to_device(pb[i] if psr else z, "u32"))
        params, state = rf.adamw_step(tx, params, gdev, state, key=pkey if psr else None, stochastic=psr,
                                      random_bits=bits)
        torch.cuda.synchronize()
        _compare(SPEC, tree, params, state[0], exact, f"step {step + 1}", before)
    return state


@pytest.mark.parametrize("exact", [True, False])
def test_adamw_f32_moments(exact):
    _run_adamw(mu_dtype=None, exact=exact)


@pytest.mark.parametrize("exact", [True, False])
def test_adamw_bf16_moments_stochastic_storage_in_kernel_bits(exact):
    import torch

    _run_adamw(mu_dtype=torch.bfloat16, exact=exact)


def test_adamw_bf16_moments_fed_bits_and_param_sr():
    import torch

    _run_adamw(mu_dtype=torch.bfloat16, exact=True, psr=True, fed=True)


def test_adamw_nesterov_uses_double_weight():
    """Nesterov: EMA weighted by 1 - f32(b1) (f32), the combination by the
    double 1.0 - b1 (adam.py:146-160); bit-exact in exact mode."""
    _run_adamw(mu_dtype=None, exact=True, nesterov=True)


def test_adamw_param_sr_in_kernel_bits():
    _run_adamw(mu_dtype=None, exact=True, psr=True)


@pytest.mark.parametrize("case", ["f32", "f32_fast", "bf16_sr", "bf16_fed_psr", "nesterov", "psr"])
def test_adamw_tree_of_whole_chunks(case):
    """The instance for lists of full-chunk fallback units only, against the
    oracle at the same bars as the mixed tree."""
    import torch

    kw = {"f32": dict(mu_dtype=None, exact=True), "f32_fast": dict(mu_dtype=None, exact=False),
          "bf16_sr": dict(mu_dtype=torch.bfloat16, exact=False),
          "bf16_fed_psr": dict(mu_dtype=torch.bfloat16, exact=True, psr=True, fed=True),
          "nesterov": dict(mu_dtype=None, exact=True, nesterov=True),
          "psr": dict(mu_dtype=None, exact=True, psr=True)}[case]
    _run_adamw(spec=VEC_SPEC, **kw)


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("tree", ["mixed", "whole_chunks"])
def test_scale_by_adam_update_only_with_masked_weight_decay(exact, tree):
    """scale_by_adam(weight_decay=..., weight_decay_mask=...) adds
    wd * f32(param) to the direction (utils.py:79-90: an f32 product, not the
    weak bf16 one of optax add_decayed_weights) and returns f32 updates."""
    import torch

    import rollfast_amd as rf

    SPEC = VEC_SPEC if tree == "whole_chunks" else globals()["SPEC"]
    host, params = _build(SPEC, 2)
    mask = {f"l{i}": (i % 2 == 0) for i in range(len(SPEC))}
    tx = rf.scale_by_adam(weight_decay=0.05, weight_decay_mask=mask, exact=exact)
    state = tx.init(params)
    for step in range(2):
        ghost, gdev = _grads(SPEC, 200 + step)
        tree = _oracle_tree(SPEC, params, state)
        outs = tree.step(ghost, weight_decay=0.05, decay_mask=[mask[f"l{i}"] for i in range(len(SPEC))],
                         count=step + 1, apply=False, lr_scale=False, decay_weak=False, ema_weight_f32=True)
        updates, state = tx.update(gdev, state, params)
        torch.cuda.synchronize()
        _compare(SPEC, tree, None, state, exact, f"step {step + 1}")
        for i in range(len(SPEC)):
            got = to_host(updates[f"l{i}"])
            if exact:
                np.testing.assert_array_equal(got.view(np.uint32), outs[i].view(np.uint32))
            else:
                rel = np.abs(got.astype(np.float64) - outs[i]) / np.maximum(np.abs(outs[i]), 1e-30)
                assert rel.max() <= 8 * 2.0 ** -23
        assert isinstance(state, rf.ScaleByAdamState) and int(state.count) == step + 1
    with pytest.raises(ValueError, match="params"):
        tx.update(gdev, state, None)


def test_adamw_fused_equals_update_plus_apply():
    import torch

    import rollfast_amd as rf

    _, pa = _build(SPEC, 4)
    _, pb = _build(SPEC, 4)
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, mu_dtype=torch.bfloat16, exact=True)
    sa, sb = tx.init(pa), tx.init(pb)
    for step in range(3):
        _, g = _grads(SPEC, 300 + step)
        pa, sa = rf.adamw_step(tx, pa, g, sa, stochastic=False)
        u, sb = tx.update(g, sb, pb)
        pb = rf.apply_updates(pb, u, stochastic=False)
        torch.cuda.synchronize()
        for k in pa:
            np.testing.assert_array_equal(to_host(pa[k]), to_host(pb[k]))
            np.testing.assert_array_equal(to_host(sa[0].mu[k]), to_host(sb[0].mu[k]))
            np.testing.assert_array_equal(to_host(sa[0].nu[k]), to_host(sb[0].nu[k]))


def _nan_equal(got, want, what):
    """Equal values, NaN where the oracle has NaN (payload bits aside)."""
    gn, wn = np.isnan(got), np.isnan(want)
    np.testing.assert_array_equal(gn, wn, err_msg=f"{what}: NaN positions")
    np.testing.assert_array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32), err_msg=what)


def test_zero_weight_decay_terms_propagate_nonfinite_params():
    """optim/adam.py's scale_by_adam adds ``update + wd_step * param`` on every
    leaf its mask covers whenever it is given params, with wd_step = 0.0
    inside adamw (adam.py:185-201, :380-404); 0 * Inf and 0 * NaN are NaN.
    So a non-finite param on a leaf outside adamw's add_decayed_weights mask
    gets a NaN update, and so does every leaf of scale_by_adam(weight_decay=0)
    given params; finite params keep their updates (exact mode, against the
    oracle's weight-0 term)."""
    import torch

    import rollfast_amd as rf

    spec = [((2, 2048), "f32", "f32"), ((1000,), "f32", "f32"), ((3, 2048), "bf16", "bf16")]
    host, params = _build(spec, 9)
    host["l1"][[3, 10, 77]] = [np.inf, -np.inf, np.nan]
    host["l2"][[5]] = bf16_bits(np.float32([np.inf]))
    params["l1"].copy_(to_device(host["l1"], "f32"))
    params["l2"].copy_(to_device(host["l2"], "bf16").reshape(3, 2048))
    mask = {"l0": True, "l1": False, "l2": False}
    ghost, gdev = _grads(spec, 17)
    # adamw update-only: the weight-0 term on every leaf, the optax decay on l0
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, weight_decay_mask=mask, exact=True)
    state = tx.init(params)
    tree = _oracle_tree(spec, params, state[0])
    outs = tree.step(ghost, weight_decay=0.01, decay_mask=[True, False, False], lr=1e-3, count=1, apply=False,
                     ema_weight_f32=True, zero_decay=True)
    updates, _ = tx.update(gdev, state, params)
    torch.cuda.synchronize()
    for i in range(3):
        _nan_equal(to_host(updates[f"l{i}"]), outs[i], f"adamw leaf {i}")
    assert np.isnan(to_host(updates["l1"])[[3, 10, 77]]).all() and np.isnan(to_host(updates["l2"])[5])
    assert np.isfinite(to_host(updates["l0"])).all()
    # scale_by_adam(weight_decay=0) given params: the f32 weight-0 term on every leaf
    tx = rf.scale_by_adam(weight_decay=0.0, exact=True)
    state = tx.init(params)
    tree = _oracle_tree(spec, params, state)
    outs = tree.step(ghost, count=1, apply=False, lr_scale=False, decay_weak=False, ema_weight_f32=True,
                     zero_decay=True)
    updates, _ = tx.update(gdev, state, params)
    torch.cuda.synchronize()
    for i in range(3):
        _nan_equal(to_host(updates[f"l{i}"]), outs[i], f"scale_by_adam leaf {i}")
    assert np.isnan(to_host(updates["l1"])[[3, 10, 77]]).all()
    # without params there is no such term: finite updates throughout
    updates, _ = tx.update(gdev, state, None)
    torch.cuda.synchronize()
    assert all(np.isfinite(to_host(updates[f"l{i}"])).all() for i in range(3))
