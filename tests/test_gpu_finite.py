"""GPU parity of the non-finite guard (optax.apply_if_finite around the
optimizer, as finetune/builders.py:1605-1609 wraps the fine-tune chain)
against the oracle's restatement: the finite test over the raw grads, the
counters, the reject branch (moments untouched, params given the zero update
so -0 turns +0, update-only mode returns zeros like the grads) and the
accepted steps, which equal the unguarded step.

Bar: codes, scales, moments and params bit-exact with ``exact=True`` (NaN
payloads excepted once a non-finite step has been let through); counters
equal.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import OracleTree, bf16_bits, bf16_to_f32, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu

# quantized bf16 and f32 leaves, a partial-block leaf, fallback leaves below min_size
SPEC = [((8, 2048), "bf16", "bf16"), ((3, 3000), "f32", "f32"), ((700,), "bf16", "bf16"), ((5, 4099), "f32", "bf16"),
        ((37,), "f32", "f32")]


def _dt(name):
    return orc.BF16 if name == "bf16" else orc.F32


def _params(seed):
    rng = np.random.default_rng(seed)
    host, dev = [], {}
    for i, (shape, pd, _gd) in enumerate(SPEC):
        n = int(np.prod(shape))
        p = gaussian(rng, (n,), 0.02)
        p[::97] = -0.0  # signed zeros: the reject branch turns them into +0
        p = bf16_bits(p) if pd == "bf16" else p
        host.append(p)
        dev[f"l{i}"] = to_device(p, pd).reshape(shape)
    return host, dev


def _grads(seed, poison=None):
    """Gaussian grads; ``poison`` = (leaf, value) plants one non-finite (or
    huge) element."""
    rng = np.random.default_rng(seed)
    host, dev = [], {}
    for i, (shape, _pd, gd) in enumerate(SPEC):
        n = int(np.prod(shape))
        g = gaussian(rng, (n,), 1e-2)
        if poison is not None and poison[0] == i:
            g[n // 3] = poison[1]
        g = bf16_bits(g) if gd == "bf16" else g
        host.append(g)
        dev[f"l{i}"] = to_device(g, gd).reshape(shape)
    return host, dev


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


def _same_float(got_bits, want_bits, nbytes, what):
    """Bitwise equality, NaN payloads aside."""
    utype, ftype = (np.uint16, None) if nbytes == 2 else (np.uint32, np.float32)
    got_bits, want_bits = got_bits.view(utype), want_bits.view(utype)
    if ftype is None:
        gf, wf = bf16_to_f32(got_bits), bf16_to_f32(want_bits)
    else:
        gf, wf = got_bits.view(ftype), want_bits.view(ftype)
    both_nan = np.isnan(gf) & np.isnan(wf)
    bad = (got_bits != want_bits) & ~both_nan
    assert not bad.any(), f"{what}: {int(bad.sum())} elements differ, first at {int(np.argmax(bad))}"


def _check(tree, params, adam_state, rf, what):
    for i, (_shape, pd, _gd) in enumerate(SPEC):
        L = tree.leaves[i]
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        if isinstance(m, rf.QuantizedBlocks):
            np.testing.assert_array_equal(to_host(m.values), L["mu"], err_msg=f"{what} leaf {i} mu codes")
            np.testing.assert_array_equal(to_host(v.values), L["nu"], err_msg=f"{what} leaf {i} nu codes")
            _same_float(to_host(m.scales), L["mu_scales"], 4, f"{what} leaf {i} mu scales")
            _same_float(to_host(v.scales), L["nu_scales"], 4, f"{what} leaf {i} nu scales")
        else:
            _same_float(to_host(m), L["mu"], 4, f"{what} leaf {i} mu")
            _same_float(to_host(v), L["nu"], 4, f"{what} leaf {i} nu")
        _same_float(to_host(params[f"l{i}"]), L["param"], 2 if pd == "bf16" else 4, f"{what} leaf {i} params")


# (grad poison per step): None = finite.  With max_consecutive_errors=1 the
# first non-finite step of a run is rejected and the second is let through.
SEQUENCE = [None, (1, np.nan), (3, np.inf), None, (0, -np.inf), None]


@pytest.mark.parametrize("clip", [None, 1.0])
@pytest.mark.parametrize("stochastic", [False, True])
def test_guarded_fused_step_matches_oracle(clip, stochastic):
    import torch

    import rollfast_amd as rf

    _, params = _params(1)
    tx = rf.apply_if_finite(rf.adamw8(learning_rate=1e-3, weight_decay=0.01, min_size=4096, exact=True), 1)
    state = tx.init(params)
    assert isinstance(state, rf.ApplyIfFiniteState)
    nf, total, applied = 0, 0, 0
    for step, poison in enumerate(SEQUENCE):
        hg, dg = _grads(10 + step, poison)
        isfinite = orc.all_finite(hg, [_dt(gd) for _s, _p, gd in SPEC])
        assert isfinite == (poison is None)
        do_apply, nf, total = orc.apply_if_finite_decision(nf, total, isfinite, 1)
        tree = _oracle_tree(params, state.inner_state[0], rf)
        if do_apply:
            grads = hg
            if clip is not None:
                scale, _norm = orc.global_norm_clip_scale(
                    [bf16_to_f32(g) if gd == "bf16" else g for g, (_s, _p, gd) in zip(hg, SPEC)], clip)
                grads = [orc.clip_leaf(g, _dt(gd), scale) for g, (_s, _p, gd) in zip(hg, SPEC)]
            # no param SR in the oracle: with stochastic=True only rejected steps are compared
            tree.step(grads, weight_decay=0.01, lr=1e-3, count=applied + 1)
            applied += 1
        else:
            for i, (_s, pd, _gd) in enumerate(SPEC):
                orc.reject_params(tree.leaves[i]["param"], _dt(pd))
        key = rf.prng.PRNGKey(step) if stochastic else None
        prev_inner = state.inner_state
        params, state = rf.adamw8_step(tx, params, dg, state, key=key, stochastic=stochastic,
                                       clip_global_norm=clip)
        torch.cuda.synchronize()
        what = f"step {step + 1} ({'applied' if do_apply else 'rejected'})"
        assert int(state.notfinite_count) == nf, what
        assert int(state.total_notfinite) == total, what
        assert bool(state.last_finite) == isfinite, what
        assert int(state.inner_state[0].count) == applied, what
        if not do_apply:
            assert state.inner_state is prev_inner, what
            np.testing.assert_array_equal(np.asarray(state.inner_state[0].key), np.asarray(prev_inner[0].key))
        if do_apply and stochastic:
            continue
        _check(tree, params, state.inner_state[0], rf, what)


def test_rejected_step_leaves_state_and_clears_negative_zero():
    import torch

    import rollfast_amd as rf

    hp, params = _params(2)
    tx = rf.apply_if_finite(rf.adamw8(learning_rate=1e-3, weight_decay=0.01), 3)
    state = tx.init(params)
    _, g = _grads(5)
    params, state = rf.adamw8_step(tx, params, g, state, stochastic=False)
    torch.cuda.synchronize()
    for i, (_s, pd, _gd) in enumerate(SPEC):  # signed zeros back in (the applied step moved them)
        if pd == "bf16":
            params[f"l{i}"].view(torch.int16).view(-1)[::97] = -32768
        else:
            params[f"l{i}"].view(torch.int32).view(-1)[::97] = -2147483648
    torch.cuda.synchronize()
    before = [to_host(params[f"l{i}"]).copy() for i in range(len(SPEC))]
    mu_before = {k: to_host(v.values if isinstance(v, rf.QuantizedBlocks) else v).copy()
                 for k, v in state.inner_state[0].mu.items()}
    for step in range(3):  # three rejections in a row are allowed with max_consecutive_errors=3
        _, g = _grads(6 + step, (step % len(SPEC), np.nan))
        params, state = rf.adamw8_step(tx, params, g, state, stochastic=False)
        torch.cuda.synchronize()
        assert int(state.notfinite_count) == step + 1 and int(state.inner_state[0].count) == 1
    for i, (_s, pd, _gd) in enumerate(SPEC):
        want = before[i].copy()
        orc.reject_params(want, _dt(pd))
        got = to_host(params[f"l{i}"])
        u = np.uint16 if pd == "bf16" else np.uint32
        np.testing.assert_array_equal(got.view(u), want.view(u))
        neg_zero = 0x8000 if pd == "bf16" else 0x80000000
        assert not (got.view(u) == neg_zero).any()
        assert (before[i].view(u) == neg_zero).any()
    for k, v in state.inner_state[0].mu.items():
        np.testing.assert_array_equal(to_host(v.values if isinstance(v, rf.QuantizedBlocks) else v), mu_before[k])


def test_huge_finite_grads_are_finite():
    """Grads near the f32 maximum make the f32 global norm overflow, but they
    are finite: the step is applied (the finite test uses the f64 sums)."""
    import torch

    import rollfast_amd as rf

    _, params = _params(3)
    tx = rf.apply_if_finite(rf.adamw8(learning_rate=1e-3, weight_decay=0.0), 1)
    state = tx.init(params)
    _, g = _grads(20, (1, 3.0e38))
    stats = torch.zeros(2, dtype=torch.float32, device="cuda")
    params, state = rf.adamw8_step(tx, params, g, state, stochastic=False, clip_global_norm=1.0, clip_stats=stats)
    torch.cuda.synchronize()
    assert bool(state.last_finite) and int(state.notfinite_count) == 0
    assert int(state.inner_state[0].count) == 1
    assert np.isinf(stats.cpu().numpy()[1])


@pytest.mark.parametrize("builder", ["adamw", "scale_by_adam8"])
def test_guarded_update_only_mode(builder):
    """tx.update of the guarded transformation: accepted steps equal the
    unguarded update; a rejected step returns zeros like the grads (their
    dtype) and the old inner state."""
    import torch

    import rollfast_amd as rf

    _, pa = _params(4)
    _, pb = _params(4)
    if builder == "adamw":
        inner_a = rf.adamw(learning_rate=1e-3, weight_decay=0.01, exact=True)
        inner_b = rf.adamw(learning_rate=1e-3, weight_decay=0.01, exact=True)
    else:
        inner_a = rf.scale_by_adam8(exact=True)
        inner_b = rf.scale_by_adam8(exact=True)
    tx = rf.apply_if_finite(inner_a, 1)
    sa, sb = tx.init(pa), inner_b.init(pb)
    for step, poison in enumerate([None, (2, np.nan), None]):
        _, g = _grads(30 + step, poison)
        ua, sa_new = tx.update(g, sa, pa)
        torch.cuda.synchronize()
        if poison is None:
            ub, sb = inner_b.update(g, sb, pb)
            torch.cuda.synchronize()
            for k in ua:
                np.testing.assert_array_equal(to_host(ua[k]).view(np.uint32), to_host(ub[k]).view(np.uint32))
            assert int(sa_new.notfinite_count) == 0
        else:
            assert sa_new.inner_state is sa.inner_state
            assert int(sa_new.notfinite_count) == 1 and int(sa_new.total_notfinite) == 1
            for k in ua:
                assert ua[k].dtype == g[k].dtype and ua[k].shape == g[k].shape
                assert not to_host(ua[k]).any()
        sa = sa_new
    # moments after [finite, rejected, finite] equal two unguarded steps
    inner_state_a = sa.inner_state if hasattr(sa.inner_state, "mu") else sa.inner_state[0]
    inner_state_b = sb if hasattr(sb, "mu") else sb[0]
    for k in inner_state_a.mu:
        ma, mb = inner_state_a.mu[k], inner_state_b.mu[k]
        ta = ma.values if isinstance(ma, rf.QuantizedBlocks) else ma
        tb = mb.values if isinstance(mb, rf.QuantizedBlocks) else mb
        np.testing.assert_array_equal(to_host(ta), to_host(tb))


def test_guarded_full_precision_fused_step():
    """adamw (f32 moments) in the guard, fused: a rejected step leaves the
    f32 moments bit-identical."""
    import torch

    import rollfast_amd as rf

    _, params = _params(5)
    tx = rf.apply_if_finite(rf.adamw(learning_rate=1e-3, weight_decay=0.01, exact=True), 1)
    state = tx.init(params)
    _, g = _grads(40)
    params, state = rf.adamw_step(tx, params, g, state, stochastic=False)
    torch.cuda.synchronize()
    mu = {k: to_host(v).copy() for k, v in state.inner_state[0].mu.items()}
    _, g = _grads(41, (4, np.nan))
    params, state = rf.adamw_step(tx, params, g, state, stochastic=False)
    torch.cuda.synchronize()
    assert int(state.notfinite_count) == 1 and int(state.inner_state[0].count) == 1
    for k, v in state.inner_state[0].mu.items():
        np.testing.assert_array_equal(to_host(v).view(np.uint32), mu[k].view(np.uint32))
