"""GPU parity of grouped launches: ``multi_transform`` over adamw8 / adamw
groups (the fine-tune builders' ``_build_grouped_transform``,
finetune/builders.py:1529-1621) runs as one launch whose leaves carry a
group index.  It must equal the groups run one by one (``masked`` inner
transforms, separate launches) bit for bit, including the per-group keys of
moment stochastic rounding and bf16 moment storage, and equal the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests._helpers import OracleTree, bf16_bits, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu

LEAVES = [("emb", (4, 2048), "bf16", "base"), ("w1", (3, 3000), "f32", "base"), ("lora_a", (8, 600), "bf16", "lora"),
          ("lora_b", (600, 8), "bf16", "lora"), ("head", (5000,), "f32", "head"), ("norm", (100,), "bf16", "head")]
LABELS = {name: lab for name, _s, _d, lab in LEAVES}


def _tree(seed, std):
    rng = np.random.default_rng(seed)
    host, dev = {}, {}
    for name, shape, dt, _lab in LEAVES:
        x = gaussian(rng, (int(np.prod(shape)),), std)
        x = bf16_bits(x) if dt == "bf16" else x
        host[name] = x
        dev[name] = to_device(x, dt).reshape(shape)
    return host, dev


def _transforms(rf, *, msr=False, exact=True, bf16_head=False):
    import torch

    return {
        "base": rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=msr, exact=exact,
                          key=rf.prng.PRNGKey(1)),
        "lora": rf.adamw8(learning_rate=lambda c: 5e-3 / (1.0 + float(c)), weight_decay=0.0, quantize=False,
                          stochastic_rounding=msr, exact=exact, key=rf.prng.PRNGKey(2)),
        "head": rf.adamw(learning_rate=2e-3, weight_decay=0.05, exact=exact, key=rf.prng.PRNGKey(3),
                         mu_dtype=torch.bfloat16 if bf16_head else None),
    }


def _moment_bits(m):
    import rollfast_amd as rf

    if isinstance(m, rf.QuantizedBlocks):
        return [to_host(m.values), to_host(m.scales).view(np.uint32)]
    if isinstance(m, rf.MaskedNode):
        return []
    return [to_host(m).view(np.uint16 if to_host(m).dtype == np.uint16 else np.uint32)]


def _assert_same(pa, pb, sa_groups, sb_groups, what):
    for name, _s, dt, lab in LEAVES:
        u = np.uint16 if dt == "bf16" else np.uint32
        np.testing.assert_array_equal(to_host(pa[name]).view(u), to_host(pb[name]).view(u), err_msg=f"{what} {name}")
        for field in ("mu", "nu"):
            ma = getattr(sa_groups[lab][0], field)[name]
            mb = getattr(sb_groups[lab][0], field)[name]
            for x, y in zip(_moment_bits(ma), _moment_bits(mb)):
                np.testing.assert_array_equal(x, y, err_msg=f"{what} {name} {field}")


@pytest.mark.parametrize("msr,bf16_head,psr,exact", [(False, False, False, True), (True, True, True, True),
                                                     (False, False, False, False), (False, True, True, False)])
def test_grouped_step_equals_groups_one_by_one(msr, bf16_head, psr, exact):
    """exact=False: the hardware direction with the learning rate folded in,
    whose constants a grouped launch derives per group on the device, must
    give the separate launches' bits too."""
    import torch

    import rollfast_amd as rf

    _, pa = _tree(1, 0.02)
    _, pb = _tree(1, 0.02)
    txa = rf.multi_transform(_transforms(rf, msr=msr, exact=exact, bf16_head=bf16_head), LABELS)
    sa = txa.init(pa)
    singles = _transforms(rf, msr=msr, exact=exact, bf16_head=bf16_head)
    masks = {lab: {name: LABELS[name] == lab for name in LABELS} for lab in singles}
    txb = {lab: rf.masked(tx, masks[lab]) for lab, tx in singles.items()}
    sb = {lab: tx.init(pb) for lab, tx in txb.items()}
    for step in range(3):
        _, g = _tree(100 + step, 1e-2)
        key = rf.prng.PRNGKey(40 + step)
        pa, sa = rf.adamw8_step(txa, pa, g, sa, key=key if psr else None, stochastic=psr)
        for lab, tx in txb.items():
            pb, sb[lab] = rf.adamw8_step(tx, pb, g, sb[lab], key=key if psr else None, stochastic=psr)
        torch.cuda.synchronize()
        ga = {lab: s.inner_state for lab, s in sa.inner_states.items()}
        gb = {lab: s.inner_state for lab, s in sb.items()}
        _assert_same(pa, pb, ga, gb, f"step {step + 1}")
        for lab in singles:
            assert int(ga[lab][0].count) == step + 1
            np.testing.assert_array_equal(np.asarray(ga[lab][0].key), np.asarray(gb[lab][0].key))
            if isinstance(ga[lab][-1], rf.ScaleByScheduleState):  # the lora group's learning-rate schedule
                assert int(ga[lab][-1].count) == int(gb[lab][-1].count) == step + 1
    # the three groups went through one launch per dtype combination, not one per group
    runner = txa.update._runner
    assert runner is not None and len(runner._plans) == 1


def test_grouped_step_matches_oracle():
    """Each group's leaves follow the oracle with that group's learning rate,
    weight decay and EMA convention (adamw8: f32(1 - b1); adamw: 1 - f32(b1))."""
    import torch

    import rollfast_amd as rf

    hp, params = _tree(2, 0.02)
    tx = rf.multi_transform(_transforms(rf), LABELS)
    state = tx.init(params)
    for step in range(2):
        hg, g = _tree(200 + step, 1e-2)
        trees = {}
        for lab in ("base", "lora", "head"):
            leaves = []
            for name, shape, dt, lb in LEAVES:
                if lb != lab:
                    continue
                adam = state.inner_states[lab].inner_state[0]
                m, v = adam.mu[name], adam.nu[name]
                L = {"pdtype": dt, "gdtype": dt, "size": int(np.prod(shape)), "param": to_host(params[name]).copy()}
                if isinstance(m, rf.QuantizedBlocks):
                    L.update(kind="quant", block_size=m.block_size, mu=to_host(m.values).copy(),
                             mu_scales=to_host(m.scales).copy(), nu=to_host(v.values).copy(),
                             nu_scales=to_host(v.scales).copy())
                else:
                    L.update(kind="f32", mu=to_host(m).copy(), nu=to_host(v).copy())
                leaves.append((name, L))
            t = OracleTree([L for _n, L in leaves])
            grads = [hg[n] for n, _L in leaves]
            if lab == "base":
                t.step(grads, weight_decay=0.01, lr=1e-3, count=step + 1)
            elif lab == "lora":
                t.step(grads, weight_decay=0.0, lr=float(np.float32(5e-3 / (1.0 + step))), count=step + 1)
            else:
                t.step(grads, weight_decay=0.05, lr=2e-3, count=step + 1, ema_weight_f32=True)
            trees[lab] = (leaves, t)
        params, state = rf.adamw8_step(tx, params, g, state, stochastic=False)
        torch.cuda.synchronize()
        for lab, (leaves, t) in trees.items():
            adam = state.inner_states[lab].inner_state[0]
            for (name, _L), L in zip(leaves, t.leaves):
                dt = L["pdtype"]
                u = np.uint16 if dt == "bf16" else np.uint32
                np.testing.assert_array_equal(to_host(params[name]).view(u), L["param"].view(u),
                                              err_msg=f"step {step + 1} {name}")
                m = adam.mu[name]
                if isinstance(m, rf.QuantizedBlocks):
                    np.testing.assert_array_equal(to_host(m.values), L["mu"])
                    np.testing.assert_array_equal(to_host(adam.nu[name].values), L["nu"])
                else:
                    np.testing.assert_array_equal(to_host(m).view(np.uint32), L["mu"].view(np.uint32))


def test_guarded_clipped_grouped_step_equals_separate_passes():
    """apply_if_finite(chain(clip_by_global_norm(1), multi_transform(...))),
    the fine-tune chain, as one fused step equals the standalone clip
    followed by the groups one by one; a non-finite step is rejected."""
    import torch

    import rollfast_amd as rf

    _, pa = _tree(3, 0.02)
    _, pb = _tree(3, 0.02)
    txa = rf.apply_if_finite(rf.chain(rf.clip_by_global_norm(1.0), rf.multi_transform(_transforms(rf), LABELS)), 1)
    sa = txa.init(pa)
    clip = rf.clip_by_global_norm(1.0)
    cs = clip.init(pb)
    singles = _transforms(rf)
    txb = {lab: rf.masked(tx, {n: LABELS[n] == lab for n in LABELS}) for lab, tx in singles.items()}
    sb = {lab: tx.init(pb) for lab, tx in txb.items()}
    for step in range(3):
        _, g = _tree(300 + step, 3.0)  # large grads: the clip is active
        pa, sa = rf.adamw8_step(txa, pa, g, sa, stochastic=False)
        gc, cs = clip.update(g, cs)
        for lab, tx in txb.items():
            pb, sb[lab] = rf.adamw8_step(tx, pb, gc, sb[lab], stochastic=False)
        torch.cuda.synchronize()
        inner = sa.inner_state
        assert int(inner[0].count) == step + 1  # the chained clip state advances
        ga = {lab: s.inner_state for lab, s in inner[1].inner_states.items()}
        _assert_same(pa, pb, ga, {lab: s.inner_state for lab, s in sb.items()}, f"step {step + 1}")
    before = {n: to_host(pa[n]).copy() for n in LABELS}
    _, g = _tree(400, 1e-2)
    g["head"].view(-1)[7] = float("nan")
    pa, sa2 = rf.adamw8_step(txa, pa, g, sa, stochastic=False)
    torch.cuda.synchronize()
    assert int(sa2.notfinite_count) == 1 and sa2.inner_state is sa.inner_state
    for n in LABELS:
        np.testing.assert_array_equal(to_host(pa[n]), before[n])


def test_grouped_update_only_mode_and_fallback():
    """tx.update of a grouped multi_transform equals the masked groups one by
    one; groups that cannot share a launch (different b1) run one by one in
    update-only mode and refuse the fused step."""
    import torch

    import rollfast_amd as rf

    _, p = _tree(4, 0.02)
    txa = rf.multi_transform(_transforms(rf), LABELS)
    sa = txa.init(p)
    singles = _transforms(rf)
    _, g = _tree(500, 1e-2)
    ua, sa = txa.update(g, sa, p)
    ub = dict(g)
    for lab, tx in singles.items():
        mtx = rf.masked(tx, {n: LABELS[n] == lab for n in LABELS})
        ub, _ = mtx.update(ub, mtx.init(p), p)
    torch.cuda.synchronize()
    for n in LABELS:
        assert ua[n].dtype == torch.float32
        np.testing.assert_array_equal(to_host(ua[n]).view(np.uint32), to_host(ub[n]).view(np.uint32))

    mixed = {"base": rf.adamw8(learning_rate=1e-3, b1=0.8), "lora": rf.adamw8(learning_rate=1e-3),
             "head": rf.adamw(learning_rate=1e-3)}
    txm = rf.multi_transform(mixed, LABELS)
    sm = txm.init(p)
    um, sm = txm.update(g, sm, p)
    torch.cuda.synchronize()
    assert all(int(s.inner_state[0].count) == 1 for s in sm.inner_states.values())
    assert all(um[n].dtype == torch.float32 for n in LABELS)
    with pytest.raises(NotImplementedError, match="share b1"):
        rf.adamw8_step(txm, p, g, sm, stochastic=False)


def test_group_table_abi_checks():
    """The C ABI refuses a grouped run whose group count differs from the
    plan's (1 + the largest leaf.group)."""
    import ctypes

    import torch

    from rollfast_amd import _lib

    lib = _lib.lib()
    n = 4096
    g = torch.zeros(n, device="cuda")
    p = torch.zeros(n, device="cuda")
    m = torch.zeros(n, device="cuda")
    v = torch.zeros(n, device="cuda")
    rows = (_lib.Adam8Leaf * 2)()
    for i in range(2):
        r = rows[i]
        r.param, r.grad, r.mu, r.nu = p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr()
        r.size, r.param_dtype, r.grad_dtype, r.moment_kind = n // 2, _lib.RF_F32, _lib.RF_F32, _lib.RF_MOMENT_F32
        r.state_index = r.param_index = i
        r.group = i
    rows[1].param, rows[1].grad = p.data_ptr() + 2 * n, g.data_ptr() + 2 * n
    rows[1].mu, rows[1].nu = m.data_ptr() + 2 * n, v.data_ptr() + 2 * n
    plan = ctypes.c_void_p()
    assert lib.rf_adam8_plan_create(rows, 2, 1, ctypes.byref(plan)) == 0
    try:
        hp = _lib.Adam8Hparams()
        hp.b1, hp.b2, hp.one_minus_b1, hp.one_minus_b2 = 0.9, 0.999, 0.1, 0.001
        hp.bc1, hp.bc2, hp.bc1_next, hp.eps = 0.1, 0.001, 0.19, 1e-8
        hp.flags = _lib.RF_LR
        grp = (_lib.Adam8Group * 2)()
        grp[0].neg_lr, grp[1].neg_lr = -1e-3, -2e-3
        grp[0].one_minus_b1 = grp[1].one_minus_b1 = 0.1
        hp.groups = ctypes.cast(grp, ctypes.c_void_p)
        hp.n_groups = 1
        assert lib.rf_adam8_plan_run(plan, ctypes.byref(hp), None) == _lib.RF_ERR_INVALID
        assert b"group" in lib.rf_last_error()
        hp.n_groups = 2
        hp.groups = None
        assert lib.rf_adam8_plan_run(plan, ctypes.byref(hp), None) == _lib.RF_ERR_INVALID
        hp.groups = ctypes.cast(grp, ctypes.c_void_p)
        g.fill_(1.0)
        torch.cuda.synchronize()
        assert lib.rf_adam8_plan_run(plan, ctypes.byref(hp), None) == 0
        torch.cuda.synchronize()
        # first step from zero moments: u = 1 / (1 + eps'), so p = -lr of each group
        got = p.cpu().numpy()
        assert np.allclose(got[: n // 2], -1e-3, rtol=1e-5) and np.allclose(got[n // 2:], -2e-3, rtol=1e-5)
    finally:
        lib.rf_adam8_plan_destroy(plan)


def test_grouped_cached_table_follows_changes():
    """From the second call the grouped step rewrites only grad pointers of
    its cached table; a replaced param tensor, a storage swap or new labels
    must send it back to a full rebuild (results equal to the groups one by
    one throughout)."""
    import torch

    import rollfast_amd as rf

    _, pa = _tree(6, 0.02)
    _, pb = _tree(6, 0.02)
    labels_a = dict(LABELS)
    txa = rf.multi_transform(_transforms(rf), lambda _: labels_a)
    sa = txa.init(pa)
    singles = _transforms(rf)
    txb = {lab: rf.masked(tx, {n: LABELS[n] == lab for n in LABELS}) for lab, tx in singles.items()}
    sb = {lab: tx.init(pb) for lab, tx in txb.items()}
    for step in range(6):
        if step == 2:  # a new param tensor object for one leaf, in both trees
            pa["w1"] = pa["w1"].clone()
            pb["w1"] = pb["w1"].clone()
        if step == 3:  # a storage swap behind the same object
            pa["head"].data = pa["head"].data.clone()
            pb["head"].data = pb["head"].data.clone()
        if step == 4:  # an equal labels tree, but a new object
            labels_a = dict(LABELS)
        _, g = _tree(600 + step, 1e-2)
        pa, sa = rf.adamw8_step(txa, pa, g, sa, stochastic=False)
        for lab, tx in txb.items():
            pb, sb[lab] = rf.adamw8_step(tx, pb, g, sb[lab], stochastic=False)
        torch.cuda.synchronize()
        ga = {lab: s.inner_state for lab, s in sa.inner_states.items()}
        gb = {lab: s.inner_state for lab, s in sb.items()}
        _assert_same(pa, pb, ga, gb, f"step {step + 1}")
