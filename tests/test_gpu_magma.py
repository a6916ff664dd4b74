"""GPU parity of Magma in the full-precision AdamW path (rollfast
optim/adam.py:127-131, :203-217 with optim/magma.py:15-132):
``scale_by_adam(use_magma=True)`` and ``adamw(use_magma=True)``.

Bar: moments bit-exact (the step is unchanged); the keep/drop decision of
every leaf exact (the Bernoulli bits of split(magma_key, n_leaves)); the
scores within 4 f32 ulps of the oracle (its reductions are float64 sums
rounded once, as the kernels' are, in another order; its sigmoid is float64);
dropped leaves' updates exactly zero, kept ones within 1e-6 relative (the
score's few ulps) in exact mode; params within one bf16 ulp.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import OracleTree, bf16_bits, bf16_ulp_distance, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu

# (shape, param dtype, grad dtype): a whole 16384-element unit, two units and
# a tail, and small leaves on the element-wise path
SPEC = [((4, 4096), "f32", "bf16"), ((2 * 16384 + 5,), "bf16", "bf16"), ((3, 1000), "f32", "f32"),
        ((700,), "bf16", "f32"), ((5,), "f32", "bf16")]
B1 = 0.9


def _tree(seed, std, as_grads=False):
    rng = np.random.default_rng(seed)
    host, dev = [], {}
    for i, (shape, pd, gd) in enumerate(SPEC):
        x = gaussian(rng, (int(np.prod(shape)),), std)
        dt = gd if as_grads else pd
        x = bf16_bits(x) if dt == "bf16" else x
        host.append(x)
        dev[f"l{i}"] = to_device(x, dt).reshape(shape)
    return host, dev


def _f32(x, dt):
    return orc.bf16_bits_to_f32(x) if dt == "bf16" else np.asarray(x, np.float32)


def _oracle_step(params, adam_state, ghost, count, *, wd, p, tau, neg_lr, exact_store_bits=None):
    """The oracle's scale_by_adam step (decay inside, f32 product) and Magma
    on each leaf; returns (tree, finals, scores, keeps)."""
    import torch

    leaves, mu_old, gd = [], [], []
    for i, (shape, pd, g_dt) in enumerate(SPEC):
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        kind = "bf16" if m.dtype == torch.bfloat16 else "f32"
        leaves.append({"pdtype": pd, "gdtype": g_dt, "size": int(np.prod(shape)), "kind": kind,
                       "param": to_host(params[f"l{i}"]).copy(), "mu": to_host(m).copy(), "nu": to_host(v).copy()})
        mu_old.append(_f32(leaves[-1]["mu"], kind).copy())  # tree.step overwrites its moments in place
        gd.append(g_dt)
    tree = OracleTree(leaves)
    mb = vb = None
    if exact_store_bits is not None:
        mb, vb = exact_store_bits
    deltas = tree.step(ghost, weight_decay=wd, count=count, apply=False, lr_scale=False, decay_weak=False,
                       ema_weight_f32=True, store_sr=mb is not None, mu_bits=mb, nu_bits=vb)
    keys_all = orc.split(tuple(int(k) for k in adam_state.key), 3)
    leaf_keys = orc.split(tuple(keys_all[2]), len(SPEC))
    b1 = np.float32(B1)
    omb1 = np.float32(1.0) - b1
    finals, scores, keeps = [], [], []
    for i in range(len(SPEC)):
        g = _f32(ghost[i], gd[i])
        mu_new = (b1 * mu_old[i] + omb1 * g).astype(np.float32)
        s_prev = float(adam_state.magma_s[f"l{i}"].item())
        s, keep = orc.magma_leaf(g, mu_new, s_prev, leaf_keys[i], p, tau)
        finals.append(orc.magma_apply(deltas[i], s, keep, neg_lr))
        scores.append(s)
        keeps.append(keep)
    return tree, finals, scores, keeps


def _check(updates, state, tree, finals, scores, keeps, what):
    import torch

    for i in range(len(SPEC)):
        L = tree.leaves[i]
        m, v = state.mu[f"l{i}"], state.nu[f"l{i}"]
        view = np.uint32 if m.dtype == torch.float32 else np.uint16
        np.testing.assert_array_equal(to_host(m).view(view), L["mu"].view(view), err_msg=f"{what} leaf {i} mu")
        np.testing.assert_array_equal(to_host(v).view(view), L["nu"].view(view), err_msg=f"{what} leaf {i} nu")
        s = float(state.magma_s[f"l{i}"].item())
        assert abs(s - float(scores[i])) <= 4 * np.spacing(np.float32(scores[i])), (what, i, s, scores[i])
        got = to_host(updates[f"l{i}"]).reshape(-1)
        if not keeps[i]:
            assert (got == 0.0).all(), f"{what} leaf {i}: a dropped leaf must give zero updates"
        else:
            want = finals[i].astype(np.float64)
            rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), 1e-30)
            assert rel.max() <= 1e-6, (what, i, rel.max())


@pytest.mark.parametrize("p", [0.5, 1.0])
def test_scale_by_adam_magma_matches_oracle(p):
    import torch

    import rollfast_amd as rf

    _, params = _tree(1, 0.02)
    tx = rf.scale_by_adam(weight_decay=0.05, use_magma=True, magma_p=p, magma_tau=2.0, exact=True,
                          key=rf.prng.PRNGKey(4))
    state = tx.init(params)
    for i in range(len(SPEC)):
        assert float(state.magma_s[f"l{i}"].item()) == 0.5
    kept_any = dropped_any = False
    for step in range(4):
        ghost, gdev = _tree(100 + step, 1e-2, as_grads=True)
        tree, finals, scores, keeps = _oracle_step(params, state, ghost, step + 1, wd=0.05, p=p, tau=2.0,
                                                   neg_lr=None)
        old_key = state.key
        updates, state = tx.update(gdev, state, params)
        torch.cuda.synchronize()
        _check(updates, state, tree, finals, scores, keeps, f"p={p} step {step + 1}")
        # adam.py:127-128: next_state_key, sr_key, magma_key = split(key, 3)
        np.testing.assert_array_equal(np.asarray(state.key), orc.split(tuple(int(k) for k in old_key), 3)[0])
        kept_any |= any(keeps)
        dropped_any |= not all(keeps)
    assert kept_any and (dropped_any or p == 1.0)


def test_scale_by_adam_magma_bf16_moments():
    """bf16 moment storage: the Magma sums use the f32 moment before its
    stochastic rounding; the storage keys come from the middle key of the
    three-way split."""
    import torch

    import rollfast_amd as rf

    _, params = _tree(2, 0.02)
    tx = rf.scale_by_adam(use_magma=True, mu_dtype=torch.bfloat16, exact=True, key=rf.prng.PRNGKey(6))
    state = tx.init(params)
    sizes = [int(np.prod(s)) for s, _, _ in SPEC]
    for step in range(3):
        ghost, gdev = _tree(200 + step, 1e-2, as_grads=True)
        _next, sr, _magma = orc.split(tuple(int(k) for k in state.key), 3)
        k1, k2 = orc.split(tuple(sr), 2)
        s1, s2 = orc.split(tuple(k1), len(SPEC)), orc.split(tuple(k2), len(SPEC))
        bits = ([orc.random_bits(tuple(s1[i]), sizes[i]) for i in range(len(SPEC))],
                [orc.random_bits(tuple(s2[i]), sizes[i]) for i in range(len(SPEC))])
        tree, finals, scores, keeps = _oracle_step(params, state, ghost, step + 1, wd=0.0, p=0.5, tau=2.0,
                                                   neg_lr=None, exact_store_bits=bits)
        updates, state = tx.update(gdev, state, params)
        torch.cuda.synchronize()
        _check(updates, state, tree, finals, scores, keeps, f"bf16 step {step + 1}")


def test_adamw_magma_step_matches_oracle():
    """adamw(use_magma=True): decay inside scale_by_adam (f32), Magma, then
    -lr; adamw_step applies the updates (round to nearest even)."""
    import torch

    import rollfast_amd as rf

    _, params = _tree(3, 0.02)
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, use_magma=True, magma_p=0.7, exact=True,
                  key=rf.prng.PRNGKey(8))
    state = tx.init(params)
    assert len(state) == 2 and isinstance(state[0], rf.ScaleByAdamState)  # no add_decayed_weights state
    for step in range(3):
        ghost, gdev = _tree(300 + step, 1e-2, as_grads=True)
        tree, finals, scores, keeps = _oracle_step(params, state[0], ghost, step + 1, wd=0.01, p=0.7, tau=2.0,
                                                   neg_lr=np.float32(-1e-3))
        want_params = []
        for i, (_shape, pd, _gd) in enumerate(SPEC):
            p = tree.leaves[i]["param"].copy()
            orc.apply_updates(p, orc.BF16 if pd == "bf16" else orc.F32, finals[i])
            want_params.append(p)
        params, state = rf.adamw_step(tx, params, gdev, state, stochastic=False)
        torch.cuda.synchronize()
        for i, (_shape, pd, _gd) in enumerate(SPEC):
            got = to_host(params[f"l{i}"]).reshape(-1)
            if pd == "bf16":
                assert bf16_ulp_distance(got, want_params[i]).max() <= 1, (step, i)
            else:
                np.testing.assert_allclose(got, want_params[i], rtol=1e-6, atol=1e-12)
            s = float(state[0].magma_s[f"l{i}"].item())
            assert abs(s - float(scores[i])) <= 4 * np.spacing(np.float32(scores[i]))


def test_adamw_magma_applies_weight_decay_before_masking():
    """rollfast tests/test_adam.py:120-131: zero grads, weight decay 0.2,
    lr 1, magma_p = 0: every leaf is dropped, so the updates are zero."""
    import torch

    import rollfast_amd as rf

    params = {"w": torch.ones((2, 2), dtype=torch.float32, device="cuda")}
    grads = {"w": torch.zeros((2, 2), dtype=torch.float32, device="cuda")}
    tx = rf.adamw(learning_rate=1.0, weight_decay=0.2, use_magma=True, magma_p=0.0)
    updates, _ = tx.update(grads, tx.init(params), params)
    torch.cuda.synchronize()
    assert (to_host(updates["w"]) == 0.0).all()


def test_magma_in_multi_transform_runs_its_group_separately():
    """A Magma group cannot join the grouped launch: multi_transform runs
    the groups one after the other, and the Magma group's update equals
    its own transform applied to its leaves."""
    import torch

    import rollfast_amd as rf

    _, params = _tree(5, 0.02)
    labels = {f"l{i}": ("magma" if i % 2 == 0 else "plain") for i in range(len(SPEC))}

    def make():
        return rf.multi_transform({"magma": rf.adamw(1e-3, use_magma=True, key=rf.prng.PRNGKey(1)),
                                   "plain": rf.adamw(1e-3, key=rf.prng.PRNGKey(2))}, labels)

    from rollfast_amd._base import MaskedNode

    tx = make()
    state = tx.init(params)
    _, gdev = _tree(500, 1e-2, as_grads=True)
    updates, state = tx.update(gdev, state, params)
    # the group's transform sees the other group's leaves as MaskedNode
    # placeholders (they still count in split(magma_key, n_leaves))
    solo = rf.adamw(1e-3, use_magma=True, key=rf.prng.PRNGKey(1))
    sub_p = {k: (v if labels[k] == "magma" else MaskedNode()) for k, v in params.items()}
    sub_g = {k: (v if labels[k] == "magma" else MaskedNode()) for k, v in gdev.items()}
    solo_updates, _ = solo.update(sub_g, solo.init(sub_p), sub_p)
    torch.cuda.synchronize()
    for k in params:
        if labels[k] == "magma":
            np.testing.assert_array_equal(to_host(updates[k]).view(np.uint32),
                                          to_host(solo_updates[k]).view(np.uint32))


@pytest.mark.parametrize("stochastic", [False, True])
def test_adamw_step_magma_fused_apply_equals_update_plus_apply(stochastic):
    """adamw_step folds Magma's per-leaf scaling into apply_updates: the
    params, moments and scores equal tx.update + apply_updates bit for bit
    (same arithmetic: neg_lr * ((m * s) * u), then f32(p) + u rounded)."""
    import torch

    import rollfast_amd as rf

    _, pa = _tree(7, 0.02)
    _, pb = _tree(7, 0.02)
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, use_magma=True, key=rf.prng.PRNGKey(9))
    sa, sb = tx.init(pa), tx.init(pb)
    for step in range(3):
        _, g = _tree(700 + step, 1e-2, as_grads=True)
        key = rf.prng.PRNGKey(70 + step) if stochastic else None
        pa, sa = rf.adamw_step(tx, pa, g, sa, key=key, stochastic=stochastic)
        upd, sb = tx.update(g, sb, pb)
        pb = rf.apply_updates(pb, upd, key=key, stochastic=stochastic)
        torch.cuda.synchronize()
        for i, (_shape, pd, _gd) in enumerate(SPEC):
            view = np.uint16 if pd == "bf16" else np.uint32
            np.testing.assert_array_equal(to_host(pa[f"l{i}"]).view(view), to_host(pb[f"l{i}"]).view(view))
            np.testing.assert_array_equal(to_host(sa[0].mu[f"l{i}"]).view(np.uint32),
                                          to_host(sb[0].mu[f"l{i}"]).view(np.uint32))
            assert float(sa[0].magma_s[f"l{i}"].item()) == float(sb[0].magma_s[f"l{i}"].item())


def _float64_sums(g, mu_new):
    """The three Magma sums of one leaf in float64 and the sums of the
    terms' magnitudes (the scale of any reordering error)."""
    g64, m64 = g.astype(np.float64), mu_new.astype(np.float64)
    terms = (g64 * m64, g64 * g64, m64 * m64)
    return np.array([t.sum() for t in terms]), np.array([np.abs(t).sum() for t in terms])


@pytest.mark.parametrize("mu_dtype", [None, "bf16"])
def test_step_magma_sums_match_reduce_and_float64(mu_dtype):
    """The step's own Magma sums (the plan's magma_sums output, which
    scale_by_adam(use_magma=True) reads) equal rf_magma_reduce's standalone
    pass and a float64 sum over the oracle's new first moment, to the
    reordering error of float64 sums (1e-12 of the terms' magnitudes)."""
    import torch

    import rollfast_amd as rf
    from rollfast_amd import _lib

    _, params = _tree(3, 0.02)
    tx = rf.scale_by_adam(mu_dtype=torch.bfloat16 if mu_dtype else None, key=rf.prng.PRNGKey(2))
    state = tx.init(params)
    engine = tx.update.engine
    b1 = np.float32(B1)
    omb1 = np.float32(engine.ema_weight(B1))
    for step in range(2):
        ghost, gdev = _tree(200 + step, 1e-2, as_grads=True)
        gl = [gdev[f"l{i}"] for i in range(len(SPEC))]
        ml = [state.mu[f"l{i}"] for i in range(len(SPEC))]
        mu_old = [to_host(m).copy() for m in ml]
        table = (_lib.MagmaLeaf * len(SPEC))()
        for i, (g, m) in enumerate(zip(gl, ml)):
            r = table[i]
            r.grad, r.mu, r.size = g.data_ptr(), m.data_ptr(), g.numel()
            r.grad_dtype = _lib.RF_BF16 if g.dtype == torch.bfloat16 else _lib.RF_F32
            r.mu_dtype = _lib.RF_BF16 if m.dtype == torch.bfloat16 else _lib.RF_F32
            r.key_index = i
        alone = torch.empty(3 * len(SPEC), dtype=torch.float64, device="cuda")
        _lib.check(_lib.lib().rf_magma_reduce(table, len(SPEC), float(b1), float(omb1), alone.data_ptr(),
                                              _lib.stream_ptr()), "rf_magma_reduce")
        fused = torch.empty(3 * len(SPEC), dtype=torch.float64, device="cuda")
        _, state = engine.run(gdev, state, None, apply=False, decay_mask=None, weight_decay=None, neg_lr=None,
                              magma_sums=fused)
        torch.cuda.synchronize()
        alone_h, fused_h = to_host(alone).reshape(-1, 3), to_host(fused).reshape(-1, 3)
        for i, (_, _, g_dt) in enumerate(SPEC):
            mdt = "bf16" if mu_dtype else "f32"
            g = _f32(ghost[i], g_dt)
            mu_new = (b1 * _f32(mu_old[i], mdt) + omb1 * g).astype(np.float32)
            want, scale = _float64_sums(g, mu_new)
            tol = 1e-12 * scale + 1e-300
            assert (np.abs(fused_h[i] - want) <= tol).all(), (step, i, fused_h[i], want)
            assert (np.abs(alone_h[i] - want) <= tol).all(), (step, i, alone_h[i], want)


def test_step_magma_sums_refused_for_quantized_moments():
    """Only plans whose every leaf has unquantized moments produce the Magma
    sums; an adamw8 plan (quantized moments) refuses them."""
    import torch

    import rollfast_amd as rf

    params = {"w": torch.zeros(8192, dtype=torch.float32, device="cuda")}
    tx = rf.adamw8(learning_rate=1e-3)
    state = tx.init(params)
    grads = {"w": torch.full((8192,), 1e-3, dtype=torch.float32, device="cuda")}
    engine = tx.update.engine
    sums = torch.empty(3, dtype=torch.float64, device="cuda")
    with pytest.raises(NotImplementedError, match="unquantized moments"):
        engine.run(grads, state[0], None, apply=False, decay_mask=None, weight_decay=None, neg_lr=None,
                   magma_sums=sums)


def test_step_magma_sums_refused_for_fused_plans():
    """The Magma sums come from update-only launches only: a fused step
    (params written) refuses them."""
    import torch

    import rollfast_amd as rf

    params = {"w": torch.zeros(4096, dtype=torch.float32, device="cuda")}
    tx = rf.adamw(learning_rate=1e-3)
    state = tx.init(params)
    grads = {"w": torch.full((4096,), 1e-3, dtype=torch.float32, device="cuda")}
    sums = torch.empty(3, dtype=torch.float64, device="cuda")
    with pytest.raises(NotImplementedError, match="update-only"):
        tx.update.engine.run(grads, state[0], params, apply=True, decay_mask=None, weight_decay=None,
                             neg_lr=np.float32(-1e-3), magma_sums=sums)


@pytest.mark.parametrize("only_empty", [False, True])
def test_magma_zero_size_leaf(only_empty):
    """A leaf without elements (the step has no work units for it) sums to
    zero: cosine 0, score 0.9 * s + 0.1 * sigmoid(0), its Bernoulli draw
    still taken from its own key; a tree of only such leaves runs no step
    kernel at all and still gets its sums."""
    import torch

    import rollfast_amd as rf

    params = {"e": torch.zeros(0, dtype=torch.float32, device="cuda")}
    if not only_empty:
        params["w"] = torch.full((3000,), 0.01, dtype=torch.float32, device="cuda")
    tx = rf.scale_by_adam(use_magma=True, magma_p=0.5, magma_tau=2.0, key=rf.prng.PRNGKey(9))
    state = tx.init(params)
    grads = {k: torch.full_like(v, 1e-3) for k, v in params.items()}
    names = sorted(params)  # the flattening order of a dict tree
    leaf_keys = orc.split(tuple(orc.split(tuple(int(k) for k in state.key), 3)[2]), len(names))
    updates, new_state = tx.update(grads, state, params)
    torch.cuda.synchronize()
    i = names.index("e")
    s_want, _ = orc.magma_leaf(np.zeros(0, np.float32), np.zeros(0, np.float32), 0.5, leaf_keys[i], 0.5, 2.0)
    assert float(new_state.magma_s["e"].item()) == float(s_want)
    assert updates["e"].numel() == 0
