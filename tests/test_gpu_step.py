"""GPU parity of the fused adamw8 step and the Optax-mode update against the
CPU oracle, through the public API (rollfast_amd.adamw8 / adamw8_step) and
the C ABI underneath.

Bar (stated per assertion):
* moment codes and block scales: bit-exact;
* params: bit-exact with ``exact=True`` (IEEE div/sqrt), within one bf16
  ulp otherwise (bf16 and f32 params alike);
* Optax-mode f32 updates: bit-exact with ``exact=True``, relative error
  <= 8 f32 ulps (hardware rcp/sqrt) otherwise.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import (
    OracleTree,
    bf16_bits,
    bf16_to_f32,
    bf16_ulp_distance,
    f32_params_close,
    gaussian,
    to_device,
    to_host,
)

pytestmark = pytest.mark.gpu


def _rf():
    import rollfast_amd as rf

    return rf


def _leaf_np(rng, size, pdtype, std=0.02):
    p = gaussian(rng, (size,), std)
    return bf16_bits(p) if pdtype == "bf16" else p


def _build(spec, seed):
    """spec: list of (shape, pdtype, gdtype).  Returns host params and device
    params (dict with sorted keys so flatten order == list order)."""
    rng = np.random.default_rng(seed)
    host, dev = {}, {}
    for i, (shape, pd, _gd) in enumerate(spec):
        size = int(np.prod(shape))
        p = _leaf_np(rng, size, pd)
        host[f"l{i:03d}"] = p
        dev[f"l{i:03d}"] = to_device(p, pd).reshape(shape)
    return host, dev


def _grads(spec, seed, std=1e-2):
    rng = np.random.default_rng(seed)
    host, dev = [], {}
    for i, (shape, _pd, gd) in enumerate(spec):
        size = int(np.prod(shape))
        g = gaussian(rng, (size,), std)
        g = bf16_bits(g) if gd == "bf16" else g
        host.append(g)
        dev[f"l{i:03d}"] = to_device(g, gd).reshape(shape)
    return host, dev


def _oracle_from_state(spec, host_params, state_adam):
    import rollfast_amd as rf

    leaves = []
    for i, (shape, pd, gd) in enumerate(spec):
        name = f"l{i:03d}"
        m = state_adam.mu[name]
        v = state_adam.nu[name]
        L = {"pdtype": pd, "gdtype": gd, "size": int(np.prod(shape)), "param": host_params[name].copy()}
        if isinstance(m, rf.QuantizedBlocks):
            L.update(kind="quant", block_size=m.block_size, mu=to_host(m.values).copy(),
                     mu_scales=to_host(m.scales).copy(), nu=to_host(v.values).copy(),
                     nu_scales=to_host(v.scales).copy())
        else:
            import torch

            kind = "bf16" if m.dtype == torch.bfloat16 else "f32"
            L.update(kind=kind, mu=to_host(m).copy(), nu=to_host(v).copy())
        leaves.append(L)
    return OracleTree(leaves)


def _compare_state(spec, tree, state_adam, what):
    import torch

    import rollfast_amd as rf

    for i, L in enumerate(tree.leaves):
        name = f"l{i:03d}"
        m, v = state_adam.mu[name], state_adam.nu[name]
        if isinstance(m, rf.QuantizedBlocks):
            np.testing.assert_array_equal(to_host(m.values), L["mu"], err_msg=f"{what} leaf {i} mu codes")
            np.testing.assert_array_equal(to_host(v.values), L["nu"], err_msg=f"{what} leaf {i} nu codes")
            np.testing.assert_array_equal(to_host(m.scales).view(np.uint32), L["mu_scales"].view(np.uint32),
                                          err_msg=f"{what} leaf {i} mu scales")
            np.testing.assert_array_equal(to_host(v.scales).view(np.uint32), L["nu_scales"].view(np.uint32),
                                          err_msg=f"{what} leaf {i} nu scales")
        else:
            a, b = to_host(m), L["mu"]
            if m.dtype == torch.float32:
                a, b = a.view(np.uint32), b.view(np.uint32)
            np.testing.assert_array_equal(a, b, err_msg=f"{what} leaf {i} fallback mu")
            a, b = to_host(v), L["nu"]
            if v.dtype == torch.float32:
                a, b = a.view(np.uint32), b.view(np.uint32)
            np.testing.assert_array_equal(a, b, err_msg=f"{what} leaf {i} fallback nu")


def _compare_params(spec, tree, dev_params, exact, what, before):
    for i, ((shape, pd, _gd), L) in enumerate(zip(spec, tree.leaves)):
        got = to_host(dev_params[f"l{i:03d}"])
        want = L["param"]
        if exact:
            np.testing.assert_array_equal(got.view(np.uint16 if pd == "bf16" else np.uint32),
                                          want.view(np.uint16 if pd == "bf16" else np.uint32),
                                          err_msg=f"{what} leaf {i} params (bit-exact)")
        elif pd == "bf16":
            d = bf16_ulp_distance(got, want)
            assert d.max() <= 1, f"{what} leaf {i}: bf16 params differ by {d.max()} ulp"
        else:
            ok = f32_params_close(got, want, before[i])
            assert ok.all(), f"{what} leaf {i}: f32 params beyond 8 ulps of the update"


def _run(spec, *, steps=3, exact=False, block_size=2048, min_size=4096, wd=0.01, lr=1e-3, msr=False,
         psr=False, nesterov=False, fallback=None, seed=0, eps_root=0.0, key=None):
    import torch

    rf = _rf()
    host_params, params = _build(spec, seed)
    tx = rf.adamw8(learning_rate=lr, weight_decay=wd, block_size=block_size, min_size=min_size,
                   stochastic_rounding=msr, nesterov=nesterov, exact=exact, eps_root=eps_root,
                   fallback_dtype=fallback, key=rf.prng.PRNGKey(7) if key is None else key)
    state = tx.init(params)
    for step in range(steps):
        ghost, gdev = _grads(spec, seed + 1000 + step)
        # Oracle starts from the device state (params too): one step compared.
        for i, (_shape, pd, _gd) in enumerate(spec):
            host_params[f"l{i:03d}"] = to_host(params[f"l{i:03d}"]).copy()
        tree = _oracle_from_state(spec, host_params, state[0])
        before = [L["param"].copy() for L in tree.leaves]
        count_inc = int(state[0].count) + 1
        key_mu, key_nu, _ = orc.split(state[0].key, 3)
        n = len(spec)
        mu_bits = nu_bits = p_bits = None
        pkey = rf.prng.PRNGKey(100 + step)
        if msr:
            kmu = orc.split(key_mu, n)
            knu = orc.split(key_nu, n)
            mu_bits, nu_bits = [], []
            for i, L in enumerate(tree.leaves):
                padded = (len(L["mu"]) if L["kind"] == "quant" else L["size"])
                mu_bits.append(orc.random_bits(kmu[i], padded))
                nu_bits.append(orc.random_bits(knu[i], padded))
        if psr:
            kp = orc.split(pkey, n)
            p_bits = [orc.random_bits(kp[i], L["size"]) for i, L in enumerate(tree.leaves)]
        # a decay schedule is read at the link's count (0, 1, ...) and is an
        # f32 array scalar: the f32 product, not the weak-typed one
        wd_step = float(np.float32(wd(np.int32(step)))) if callable(wd) else wd
        tree.step(ghost, weight_decay=wd_step, lr=lr, count=count_inc, nesterov=nesterov, moment_sr=msr,
                  param_sr=psr, mu_bits=mu_bits, nu_bits=nu_bits, p_bits=p_bits, eps_root=eps_root,
                  decay_weak=not callable(wd))
        params, state = rf.adamw8_step(tx, params, gdev, state, key=pkey if psr else None, stochastic=psr)
        torch.cuda.synchronize()
        _compare_state(spec, tree, state[0], f"step {step + 1}")
        _compare_params(spec, tree, params, exact, f"step {step + 1}", before)


C1 = [((1024, 1024), "f32", "f32")]


@pytest.mark.parametrize("exact", [True, False])
def test_c1_fp32_1024x1024_three_steps(exact):
    """The single-step CPU-reference configuration (1024x1024 f32, block 2048,
    lr 1e-3, wd 0.01), steps 1..3."""
    _run(C1, steps=3, exact=exact)


MIXED = [
    ((64, 2048), "bf16", "bf16"),   # full 2048 blocks, vectorised path
    ((3, 3000), "bf16", "f32"),     # 9000: 4 full blocks + partial block
    ((768,), "bf16", "bf16"),       # below min_size: f32 fallback moments
    ((4096,), "f32", "bf16"),       # exactly min_size: quantized
    ((5, 1111), "f32", "f32"),      # odd size, partial block
    ((1,), "bf16", "bf16"),         # single element fallback
]


@pytest.mark.parametrize("exact", [True, False])
def test_mixed_tree_bf16_f32(exact):
    _run(MIXED, steps=3, exact=exact)


def test_generic_block_size_256_and_nesterov():
    spec = [((40, 256), "bf16", "bf16"), ((1000,), "f32", "f32"), ((33, 7), "bf16", "f32")]
    _run(spec, steps=2, block_size=256, min_size=16, nesterov=True, exact=True)


@pytest.mark.parametrize("msr,psr", [(False, False), (True, True)])
def test_block_size_4096_partial_blocks_by_workgroup(msr, psr):
    """Blocks of 4096 (every block a generic unit, taken by a workgroup's
    four waves, 1024 elements each): whole blocks and partial last ones
    (15000 = 3 x 4096 + 2712, 9000 = 2 x 4096 + 808), with moment and param
    stochastic rounding."""
    spec = [((3, 5000), "bf16", "bf16"), ((9000,), "bf16", "f32")]
    _run(spec, steps=2, block_size=4096, min_size=4096, msr=msr, psr=psr, exact=True)


def test_odd_block_size_and_eps_root():
    spec = [((10, 300), "bf16", "bf16"), ((7000,), "f32", "bf16")]
    _run(spec, steps=2, block_size=1000, min_size=100, eps_root=1e-12, exact=True)


def test_bf16_fallback_moments():
    spec = [((100,), "bf16", "bf16"), ((2048,), "f32", "f32")]
    import torch

    _run(spec, steps=2, min_size=1 << 20, fallback=torch.bfloat16, exact=True)


def test_moment_stochastic_rounding_matches_threefry_bits():
    """In-kernel Threefry bits == the oracle's jax.random.bits layout."""
    _run(MIXED, steps=2, msr=True, exact=True)


def test_param_stochastic_rounding_matches_threefry_bits():
    spec = [((64, 2048), "bf16", "bf16"), ((3, 3000), "bf16", "f32"), ((768,), "bf16", "bf16")]
    _run(spec, steps=2, psr=True, exact=True)


def test_weight_decay_schedule():
    """adamw8(weight_decay=schedule) (adam8.py:400, :435-440): the decay link
    evaluates the schedule at its own count, 0 on the first step, and the f32
    value multiplies the params in f32 (bf16 params included)."""
    sched = lambda c: 0.05 / (1.0 + np.float32(c))  # noqa: E731
    _run(MIXED, steps=3, wd=sched, exact=True)


def test_fold_in_group_key_drives_moment_sr():
    """adamw8(key=jax.random.fold_in(root, index)), the fine-tune builders'
    per-group key (finetune/builders.py:1582), with moment and param
    stochastic rounding: the in-kernel bits follow that key's stream."""
    rf = _rf()
    _run(MIXED, steps=2, msr=True, psr=True, exact=True, key=rf.prng.fold_in(rf.prng.PRNGKey(1234), 3))


def test_fast_direction_over_twenty_steps():
    spec = [((128, 2048), "bf16", "bf16"), ((777,), "bf16", "bf16")]
    _run(spec, steps=20, exact=False)


@pytest.mark.parametrize("lr_ulps", [0, 3, -3, 6])
def test_folded_step_where_updates_cancel_params(lr_ulps):
    """The default direction folds -lr into the reciprocal and the decay
    into the param (s = fma(m, rcp(D'), fma(wdl, p, p))).  On the first step
    u ~ sign(g), so params of magnitude lr nearly cancel: with
    lr = 2^-7 (1 - k 2^-11) and |p| = 2^-7, |p + U| / |p| is about k 2^-11,
    on either side of the 2^-10 bound past which the kernel recomputes an
    element with IEEE arithmetic (k = 0: about 1e-4, recomputed; k = 3, 6:
    kept, where the folded form's error is largest relative to the sum;
    k = -3: the sum changes sign).  Half the params are ordinary.  Codes and
    scales bit-exact, params within one bf16 ulp."""
    import torch

    rf = _rf()
    spec = [((64, 2048), "bf16", "bf16")]
    lr = float(np.float32(2.0 ** -7 * (1.0 - lr_ulps * 2.0 ** -11)))
    ghost, gdev = _grads(spec, 4242)
    g = bf16_to_f32(ghost[0])
    rng = np.random.default_rng(11)
    p = gaussian(rng, g.shape, 0.02)
    half = np.arange(g.size) % 2 == 0
    p[half] = np.where(g[half] >= 0, 2.0 ** -7, -(2.0 ** -7))
    host = {"l000": bf16_bits(p)}
    params = {"l000": to_device(host["l000"], "bf16").reshape(spec[0][0])}
    tx = rf.adamw8(learning_rate=lr, weight_decay=0.01, key=rf.prng.PRNGKey(7))
    state = tx.init(params)
    tree = _oracle_from_state(spec, host, state[0])
    before = [L["param"].copy() for L in tree.leaves]
    tree.step(ghost, weight_decay=0.01, lr=lr, count=1)
    want = bf16_to_f32(tree.leaves[0]["param"])
    ratio = np.abs(want[half]) / 2.0 ** -7
    assert np.median(ratio) < 2.0 ** -8, "the constructed params must nearly cancel"
    params, state = rf.adamw8_step(tx, params, gdev, state, stochastic=False)
    torch.cuda.synchronize()
    _compare_state(spec, tree, state[0], f"lr_ulps {lr_ulps}")
    _compare_params(spec, tree, params, False, f"lr_ulps {lr_ulps}", before)


@pytest.mark.parametrize("lr,wd", [(1e-1, 1e-3), (3e-2, 2e-3), (1e-2, 0.0), (1.0, 1e-5), (1e-6, 0.1), (-1e-3, 0.01)])
def test_folded_direction_wide_hyperparameters(lr, wd):
    """The learning-rate-folded direction over learning rates and decays
    either side of its |lr * wd| <= 2^-14 range (3e-2 * bf16(2e-3) is just
    inside, 1e-1 * 1e-3 outside), without decay, with a negative learning
    rate, and params whose magnitudes span 1e-6 .. 10 with Student-t grads:
    codes and scales bit-exact, params within one bf16 ulp, three steps each
    from the device state."""
    import torch

    rf = _rf()
    spec = [((32, 2048), "bf16", "bf16"), ((5000,), "bf16", "bf16")]
    rng = np.random.default_rng(77)
    host, params = {}, {}
    for i, (shape, _pd, _gd) in enumerate(spec):
        n = int(np.prod(shape))
        mag = np.exp(rng.uniform(np.log(1e-6), np.log(10.0), n))
        p = (mag * rng.choice([-1.0, 1.0], n)).astype(np.float32)
        host[f"l{i:03d}"] = bf16_bits(p)
        params[f"l{i:03d}"] = to_device(host[f"l{i:03d}"], "bf16").reshape(shape)
    tx = rf.adamw8(learning_rate=lr, weight_decay=wd, key=rf.prng.PRNGKey(7))
    state = tx.init(params)
    for step in range(3):
        ghost, gdev = [], {}
        for i, (shape, _pd, _gd) in enumerate(spec):
            n = int(np.prod(shape))
            g = bf16_bits((rng.standard_t(3, n) * 1e-3).astype(np.float32))
            ghost.append(g)
            gdev[f"l{i:03d}"] = to_device(g, "bf16").reshape(shape)
        for i in range(len(spec)):
            host[f"l{i:03d}"] = to_host(params[f"l{i:03d}"]).copy()
        tree = _oracle_from_state(spec, host, state[0])
        before = [L["param"].copy() for L in tree.leaves]
        tree.step(ghost, weight_decay=wd, lr=lr, count=int(state[0].count) + 1)
        params, state = rf.adamw8_step(tx, params, gdev, state, stochastic=False)
        torch.cuda.synchronize()
        _compare_state(spec, tree, state[0], f"lr {lr} wd {wd} step {step + 1}")
        _compare_params(spec, tree, params, False, f"lr {lr} wd {wd} step {step + 1}", before)


# ---------------------------------------------------------- Optax mode --
def _optax_mode(spec, *, adamw, exact, seed=3):
    import torch

    rf = _rf()
    host_params, params = _build(spec, seed)
    if adamw:
        tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, min_size=1024, exact=exact)
    else:
        tx = rf.scale_by_adam8(min_size=1024, exact=exact)
    state = tx.init(params)
    for step in range(2):
        ghost, gdev = _grads(spec, seed + 10 + step)
        adam_state = state[0] if adamw else state
        tree = _oracle_from_state(spec, host_params, adam_state)
        count_inc = int(adam_state.count) + 1
        outs = tree.step(ghost, weight_decay=0.01 if adamw else 0.0, lr=1e-3, count=count_inc, apply=False,
                         lr_scale=adamw)
        updates, state = tx.update(gdev, state, params)
        torch.cuda.synchronize()
        _compare_state(spec, tree, state[0] if adamw else state, f"optax step {step + 1}")
        for i in range(len(spec)):
            got = to_host(updates[f"l{i:03d}"])
            want = outs[i]
            if exact:
                np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
            else:
                rel = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want), 1e-30)
                assert rel.max() <= 8 * 2.0**-23, f"leaf {i}: relative error {rel.max()}"
        # Params untouched by the Optax-mode update.
        for i, (_s, pd, _g) in enumerate(spec):
            got = to_host(params[f"l{i:03d}"])
            np.testing.assert_array_equal(got, host_params[f"l{i:03d}"])


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("adamw", [True, False])
def test_optax_mode_updates(adamw, exact):
    spec = [((8, 2048), "bf16", "bf16"), ((3000,), "f32", "f32"), ((100,), "bf16", "f32")]
    _optax_mode(spec, adamw=adamw, exact=exact)


def test_fused_equals_update_plus_apply_updates():
    """adamw8_step == tx.update + apply_updates (RNE), bit for bit."""
    import torch

    rf = _rf()
    spec = [((16, 2048), "bf16", "bf16"), ((500,), "f32", "bf16")]
    host, pa = _build(spec, 11)
    _, pb = _build(spec, 11)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=True)
    sa = tx.init(pa)
    sb = tx.init(pb)
    for step in range(3):
        _, g = _grads(spec, 50 + step)
        pa, sa = rf.adamw8_step(tx, pa, g, sa, stochastic=False)
        u, sb = tx.update(g, sb, pb)
        pb = rf.apply_updates(pb, u, stochastic=False)
        torch.cuda.synchronize()
        for k in pa:
            np.testing.assert_array_equal(to_host(pa[k]), to_host(pb[k]))
            ma, mb = sa[0].mu[k], sb[0].mu[k]
            if isinstance(ma, rf.QuantizedBlocks):
                np.testing.assert_array_equal(to_host(ma.values), to_host(mb.values))
                np.testing.assert_array_equal(to_host(ma.scales), to_host(mb.scales))


def test_fed_bits_equal_in_kernel_bits():
    """RF_FED_BITS with the oracle's bits gives the in-kernel-bits result."""
    import torch

    rf = _rf()
    spec = [((8, 2048), "bf16", "bf16"), ((1500,), "bf16", "bf16")]
    _, pa = _build(spec, 5)
    _, pb = _build(spec, 5)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=True, min_size=1024, exact=True)
    sa, sb = tx.init(pa), tx.init(pb)
    _, g = _grads(spec, 77)
    pkey = rf.prng.PRNGKey(3)
    key_mu, key_nu, _ = orc.split(sa[0].key, 3)
    kmu, knu, kp = orc.split(key_mu, 2), orc.split(key_nu, 2), orc.split(pkey, 2)
    bits = {}
    for i, name in enumerate(sorted(pa)):
        m = sa[0].mu[name]
        padded = m.values.numel()
        size = pa[name].numel()
        bits[i] = (to_device(orc.random_bits(kmu[i], padded), "u32"),
                   to_device(orc.random_bits(knu[i], padded), "u32"),
                   to_device(orc.random_bits(kp[i], size), "u32"))
    pa, sa = rf.adamw8_step(tx, pa, g, sa, key=pkey, stochastic=True)
    pb, sb = rf.adamw8_step(tx, pb, g, sb, key=pkey, stochastic=True, random_bits=bits)
    torch.cuda.synchronize()
    for k in pa:
        np.testing.assert_array_equal(to_host(pa[k]), to_host(pb[k]))
        np.testing.assert_array_equal(to_host(sa[0].mu[k].values), to_host(sb[0].mu[k].values))
        np.testing.assert_array_equal(to_host(sa[0].nu[k].values), to_host(sb[0].nu[k].values))


def test_state_key_and_count_evolve_like_reference():
    rf = _rf()
    import torch

    params = {"w": torch.zeros((4096,), dtype=torch.bfloat16, device="cuda")}
    tx = rf.adamw8(learning_rate=1e-3)
    st = tx.init(params)
    # init: split(PRNGKey(42), 3)[2] (adam8.py:274, utils.py:73-76)
    np.testing.assert_array_equal(st[0].key, orc.split((0, 42), 3)[2])
    k = st[0].key
    for t in range(1, 4):
        _, st = rf.adamw8_step(tx, params, {"w": torch.zeros_like(params["w"])}, st, stochastic=False)
        k = orc.split(k, 3)[2]
        np.testing.assert_array_equal(st[0].key, k)
        assert int(st[0].count) == t


def test_cached_leaf_table_follows_changes():
    """The host reuses the previous step's leaf table when the same param and
    moment objects come back; every kind of change must still reach the
    kernel: a grad dtype change, params rebuilt as new tensors, a moment leaf
    replaced by a copy, a param's storage swapped with ``.data``.  Each step
    is compared with the oracle (bit-exact: exact mode)."""
    import dataclasses

    import torch

    rf = _rf()
    spec = [((8, 2048), "bf16", "bf16"), ((3, 3000), "f32", "bf16"), ((700,), "bf16", "bf16")]
    host_params, params = _build(spec, 5)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=True)
    state = tx.init(params)

    def change_grad_dtype(params, state):
        return params, state, [((8, 2048), "bf16", "f32"), spec[1], spec[2]]

    def new_param_tensors(params, state):
        return {k: v.clone() for k, v in params.items()}, state, spec

    def copy_moment_leaf(params, state):
        adam = state[0]
        m = adam.mu["l000"]
        mu = dict(adam.mu)
        mu["l000"] = dataclasses.replace(m, values=m.values.clone(), scales=m.scales.clone())
        return params, (adam._replace(mu=mu),) + tuple(state[1:]), spec

    def swap_param_storage(params, state):
        params["l001"].data = params["l001"].clone()
        return params, state, spec

    plan = [None, None, change_grad_dtype, None, new_param_tensors, copy_moment_leaf, None, swap_param_storage,
            None]
    for step, mutate in enumerate(plan):
        gspec = spec
        if mutate is not None:
            params, state, gspec = mutate(params, state)
        ghost, gdev = _grads(gspec, 77 + step)
        for i in range(len(spec)):
            host_params[f"l{i:03d}"] = to_host(params[f"l{i:03d}"]).copy()
        tree = _oracle_from_state(gspec, host_params, state[0])
        before = [L["param"].copy() for L in tree.leaves]
        tree.step(ghost, weight_decay=0.01, lr=1e-3, count=int(state[0].count) + 1)
        params, state = rf.adamw8_step(tx, params, gdev, state, stochastic=False)
        torch.cuda.synchronize()
        _compare_state(gspec, tree, state[0], f"step {step + 1}")
        _compare_params(gspec, tree, params, True, f"step {step + 1}", before)


@pytest.mark.parametrize("exact", [True, False])
def test_non_finite_and_extreme_gradient_blocks(exact):
    """Blocks whose gradients hold a NaN, a +Inf, values whose square
    overflows, all zeros, f32 denormals or values so small that the block
    scale falls below the fast path's exact-division range.  Such blocks take
    the literal requantization (the reference's NaN-propagating absmax gives
    scale 1 for a NaN block); codes and scales must still match the oracle
    bit for bit and params where finite, over two steps."""
    import torch

    rf = _rf()
    rng = np.random.default_rng(3)
    n = 8 * 2048
    host_p = {"a": (rng.standard_normal(n) * 0.02).astype(np.float32),
              "b": bf16_bits((rng.standard_normal(n) * 0.02).astype(np.float32))}
    params = {"a": to_device(host_p["a"], "f32"), "b": to_device(host_p["b"], "bf16")}
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=exact)
    state = tx.init(params)

    def grads_for(step):
        g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
        g[1 * 2048 + 17] = np.nan
        g[2 * 2048 + 5] = np.inf
        g[3 * 2048:4 * 2048] *= np.float32(1e22)        # g*g overflows to +Inf
        g[4 * 2048:5 * 2048] = 0.0
        g[5 * 2048:6 * 2048] = np.float32(1e-40) * np.sign(g[5 * 2048:6 * 2048])
        g[6 * 2048:7 * 2048] *= np.float32(1e-24)       # block scale < 2^-70
        if step == 1:
            g[7 * 2048 + 100] = -np.inf
        return g

    for step in range(2):
        ga = grads_for(step)
        gb = bf16_bits(grads_for(step))
        leaves = []
        for name, pd in (("a", "f32"), ("b", "bf16")):
            m, v = state[0].mu[name], state[0].nu[name]
            leaves.append({"pdtype": pd, "gdtype": pd, "kind": "quant", "size": n, "block_size": 2048,
                           "param": to_host(params[name]).copy(), "mu": to_host(m.values).copy(),
                           "mu_scales": to_host(m.scales).copy(), "nu": to_host(v.values).copy(),
                           "nu_scales": to_host(v.scales).copy()})
        tree = OracleTree(leaves)
        before_a = leaves[0]["param"].copy()
        tree.step([ga, gb], weight_decay=0.01, lr=1e-3, count=step + 1)
        params, state = rf.adamw8_step(tx, params, {"a": to_device(ga, "f32"), "b": to_device(gb, "bf16")},
                                       state, stochastic=False)
        torch.cuda.synchronize()
        for name, L in zip(("a", "b"), tree.leaves):
            m, v = state[0].mu[name], state[0].nu[name]
            np.testing.assert_array_equal(to_host(m.values), L["mu"], err_msg=f"step {step + 1} {name} mu codes")
            np.testing.assert_array_equal(to_host(v.values), L["nu"], err_msg=f"step {step + 1} {name} nu codes")
            np.testing.assert_array_equal(to_host(m.scales).view(np.uint32), L["mu_scales"].view(np.uint32))
            np.testing.assert_array_equal(to_host(v.scales).view(np.uint32), L["nu_scales"].view(np.uint32))
            got = to_host(params[name])
            want = L["param"]
            if name == "a":
                gf, wf = got, want
            else:
                gf, wf = bf16_to_f32(got), bf16_to_f32(want)
            np.testing.assert_array_equal(np.isnan(gf), np.isnan(wf), err_msg=f"step {step + 1} {name} NaN positions")
            fin = np.isfinite(wf)
            np.testing.assert_array_equal(gf[~fin & ~np.isnan(wf)], wf[~fin & ~np.isnan(wf)])
            if exact:
                np.testing.assert_array_equal(gf[fin].view(np.uint32), wf[fin].view(np.uint32))
            elif name == "a":
                assert f32_params_close(gf[fin], wf[fin], before_a[fin]).all()
            else:
                assert bf16_ulp_distance(got[fin], want[fin]).max() <= 1
