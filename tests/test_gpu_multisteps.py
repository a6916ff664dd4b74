"""GPU parity of gradient accumulation: optax.MultiSteps, the wrapper the
fine-tune builders put around their whole transformation
(finetune/builders.py:1614-1620), against the oracle's restatement.

- ``rf_accumulate`` (mean, sum, reset) over ragged, misaligned leaves of
  every dtype pair, special values included: bit-exact, NaN payloads aside.
- ``adamw8_step(MultiSteps(apply_if_finite(adamw8(exact=True))))`` over
  three windows with a non-finite micro-batch: accumulator, params, moments
  and every counter bit-exact against the oracle at each micro-step.
- Update-only mode: zero updates between emits, the inner's updates on the
  accumulator at the emit.
- Properties at a larger size: k = 1 equals the inner step, and a window of
  identical grads equals one inner step, for the builders' composition
  apply_if_finite(chain(clip_by_global_norm, multi_transform)) too.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import OracleTree, bf16_bits, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu

_DT = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}


def _same_float(got, want, dtype, what):
    """Bitwise equality of F32 values or 16-bit patterns, NaN payloads aside."""
    if dtype == orc.F32:
        gf, wf = np.asarray(got, np.float32), np.asarray(want, np.float32)
        gb, wb = gf.view(np.uint32), wf.view(np.uint32)
    else:
        gb, wb = np.asarray(got, np.uint16), np.asarray(want, np.uint16)
        gf, wf = orc.to_f32(gb, dtype), orc.to_f32(wb, dtype)
    bad = (gb != wb) & ~(np.isnan(gf) & np.isnan(wf))
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} differ, first at {int(np.argmax(bad))}"


def _with_specials(rng, n, std):
    x = gaussian(rng, (n,), std)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-40, 3e38, -3e38], np.float32)
    if n >= 64:
        idx = rng.choice(n, size=min(n // 16, 64), replace=False)
        x[idx] = specials[rng.integers(0, specials.size, idx.size)]
    return x


# (grad dtype, accumulator dtype): the promoted-dtype cases MultiSteps
# accepts, and two the C ABI computes in f32 and rounds into the accumulator
PAIRS = [("f32", "f32"), ("bf16", "f32"), ("f16", "f32"), ("bf16", "bf16"), ("f16", "f16"), ("f32", "bf16"),
         ("bf16", "f16")]
SIZES = [1, 7, 8, 9, 8191, 8192, 8193, 70001]


def test_accumulate_kernel_matches_oracle():
    import torch

    from rollfast_amd import _lib

    rng = np.random.default_rng(11)
    leaves = []  # (gd, ad, size, misaligned)
    for gd, ad in PAIRS:
        for n in SIZES:
            leaves.append((gd, ad, n, False))
        leaves.append((gd, ad, 4099, True))
    acc_host, acc_dev = [], []
    for gd, ad, n, mis in leaves:
        a0 = _with_specials(rng, n, 0.5)
        a0 = orc.from_f32(a0, _DT[ad]).copy()
        buf = to_device(np.concatenate([orc.from_f32(np.zeros(1, np.float32), _DT[ad]), a0]) if mis else a0, ad)
        acc_dev.append(buf[1:] if mis else buf)
        acc_host.append(a0)
    steps = [(orc.ACC_MEAN, 0), (orc.ACC_MEAN, 1), (orc.ACC_MEAN, 2), (orc.ACC_ZERO, 0), (orc.ACC_SUM, 0),
             (orc.ACC_MEAN, 5), (orc.ACC_SUM, 0)]
    for si, (mode, n_acc) in enumerate(steps):
        rows, keep = [], []
        for li, (gd, ad, n, mis) in enumerate(leaves):
            g = orc.from_f32(_with_specials(rng, n, 1.0), _DT[gd]).copy()
            if mis:
                gbuf = to_device(np.concatenate([orc.from_f32(np.zeros(1, np.float32), _DT[gd]), g]), gd)[1:]
            else:
                gbuf = to_device(g, gd)
            keep.append(gbuf)
            orc.accumulate(mode, n_acc, g, _DT[gd], acc_host[li], _DT[ad])
            row = _lib.AccumLeaf()
            row.grad = gbuf.data_ptr()
            row.acc = acc_dev[li].data_ptr()
            row.size = n
            row.grad_dtype = _DT[gd]
            row.acc_dtype = _DT[ad]
            rows.append(row)
        table = (_lib.AccumLeaf * len(rows))(*rows)
        print(f"accumulate step {si} mode {mode} n_acc {n_acc}", flush=True)
        _lib.check(_lib.lib().rf_accumulate(table, len(rows), mode, n_acc, _lib.stream_ptr()), "rf_accumulate")
        torch.cuda.synchronize()
        for li, (gd, ad, n, mis) in enumerate(leaves):
            _same_float(to_host(acc_dev[li]), acc_host[li], _DT[ad], f"step {si} leaf {li} ({gd}->{ad}, n={n}, "
                                                                      f"misaligned={mis})")


def test_accumulate_rejects_bad_arguments():
    import torch

    from rollfast_amd import _lib

    a = torch.zeros(16, device="cuda")
    row = _lib.AccumLeaf()
    row.grad = a.data_ptr()
    row.acc = a.data_ptr()
    row.size = 16
    row.grad_dtype = _lib.RF_F32
    row.acc_dtype = _lib.RF_F32
    table = (_lib.AccumLeaf * 1)(row)
    with pytest.raises(ValueError, match="unknown mode"):
        _lib.check(_lib.lib().rf_accumulate(table, 1, 7, 0, _lib.stream_ptr()), "rf_accumulate")
    with pytest.raises(ValueError, match="negative n_acc"):
        _lib.check(_lib.lib().rf_accumulate(table, 1, _lib.RF_ACC_MEAN, -1, _lib.stream_ptr()), "rf_accumulate")
    row.grad_dtype = 9
    table = (_lib.AccumLeaf * 1)(row)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.lib().rf_accumulate(table, 1, _lib.RF_ACC_SUM, 0, _lib.stream_ptr()), "rf_accumulate")
    _lib.check(_lib.lib().rf_accumulate(table, 0, _lib.RF_ACC_SUM, 0, _lib.stream_ptr()), "empty table")


# ------------------------------------------------ the guarded fused step --
# quantized bf16 and f32 leaves, a partial-block leaf, fallback leaves
SPEC = [((8, 2048), "bf16", "bf16"), ((3, 3000), "f32", "f32"), ((700,), "bf16", "bf16"), ((5, 4099), "f32", "bf16"),
        ((37,), "f32", "f32")]
K = 3
POISON = {4: (1, np.nan)}  # micro-step -> (leaf, value)


def _params(seed):
    rng = np.random.default_rng(seed)
    dev = {}
    for i, (shape, pd, _gd) in enumerate(SPEC):
        p = gaussian(rng, (int(np.prod(shape)),), 0.02)
        dev[f"l{i}"] = to_device(bf16_bits(p) if pd == "bf16" else p, pd).reshape(shape)
    return dev


def _grads(seed, poison=None):
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
    for i, (shape, pd, _gd) in enumerate(SPEC):
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        L = {"pdtype": pd, "gdtype": "f32", "size": int(np.prod(shape)), "param": to_host(params[f"l{i}"]).copy()}
        if isinstance(m, rf.QuantizedBlocks):
            L.update(kind="quant", block_size=m.block_size, mu=to_host(m.values).copy(),
                     mu_scales=to_host(m.scales).copy(), nu=to_host(v.values).copy(), nu_scales=to_host(v.scales).copy())
        else:
            L.update(kind="f32", mu=to_host(m).copy(), nu=to_host(v).copy())
        leaves.append(L)
    return OracleTree(leaves)


def _check_tree(tree, params, adam_state, rf, what):
    for i, (_shape, pd, _gd) in enumerate(SPEC):
        L = tree.leaves[i]
        m, v = adam_state.mu[f"l{i}"], adam_state.nu[f"l{i}"]
        if isinstance(m, rf.QuantizedBlocks):
            np.testing.assert_array_equal(to_host(m.values), L["mu"], err_msg=f"{what} leaf {i} mu codes")
            np.testing.assert_array_equal(to_host(v.values), L["nu"], err_msg=f"{what} leaf {i} nu codes")
            _same_float(to_host(m.scales), L["mu_scales"], orc.F32, f"{what} leaf {i} mu scales")
            _same_float(to_host(v.scales), L["nu_scales"], orc.F32, f"{what} leaf {i} nu scales")
        else:
            _same_float(to_host(m), L["mu"], orc.F32, f"{what} leaf {i} mu")
            _same_float(to_host(v), L["nu"], orc.F32, f"{what} leaf {i} nu")
        _same_float(to_host(params[f"l{i}"]), L["param"], _DT[pd], f"{what} leaf {i} params")


@pytest.mark.parametrize("use_grad_mean", [True, False])
def test_guarded_multisteps_fused_step_matches_oracle(use_grad_mean):
    """Three windows of k = 3 with a NaN in the second: its emit is rejected
    by the guard, the reset keeps the NaN (0 * NaN), and the third window's
    emit, non-finite again, is let through (max_consecutive_errors = 1)."""
    import torch

    import rollfast_amd as rf

    params = _params(1)
    inner = rf.apply_if_finite(rf.adamw8(learning_rate=1e-3, weight_decay=0.01, min_size=4096, exact=True), 1)
    tx = rf.MultiSteps(inner, every_k_schedule=K, use_grad_mean=use_grad_mean, accumulator_dtype="float32")
    state = tx.init(params)
    assert isinstance(state, rf.MultiStepsState)
    mode = orc.ACC_MEAN if use_grad_mean else orc.ACC_SUM
    acc = [np.zeros(int(np.prod(s)), np.float32) for s, _p, _g in SPEC]
    mini = gstep = nf = total = applied = 0
    for step in range(3 * K):
        hg, dg = _grads(20 + step, POISON.get(step))
        for i, (_s, _p, gd) in enumerate(SPEC):
            orc.accumulate(mode, mini, hg[i], _DT[gd], acc[i], orc.F32)
        emit, mini, gstep = orc.multisteps_counters(mini, gstep, K)
        tree = _oracle_tree(params, state.inner_opt_state.inner_state[0], rf)
        if emit:
            isfinite = orc.all_finite(acc, [orc.F32] * len(acc))
            do_apply, nf, total = orc.apply_if_finite_decision(nf, total, isfinite, 1)
            if do_apply:
                tree.step([a.copy() for a in acc], weight_decay=0.01, lr=1e-3, count=applied + 1)
                applied += 1
            else:
                for i, (_s, pd, _gd) in enumerate(SPEC):
                    orc.reject_params(tree.leaves[i]["param"], _DT[pd])
            for a in acc:
                orc.accumulate(orc.ACC_ZERO, 0, None, orc.F32, a, orc.F32)
        print(f"multisteps mean={use_grad_mean} micro-step {step} emit={emit}", flush=True)
        params, state = rf.adamw8_step(tx, params, dg, state, stochastic=False)
        torch.cuda.synchronize()
        what = f"micro-step {step}"
        assert int(state.mini_step) == mini and int(state.gradient_step) == gstep, what
        guard = state.inner_opt_state
        assert int(guard.notfinite_count) == nf and int(guard.total_notfinite) == total, what
        assert int(np.asarray(guard.inner_state[0].count)) == applied, what
        assert tx.has_updated(state) == emit
        for i, a in enumerate(acc):
            _same_float(to_host(state.acc_grads[f"l{i}"]), a, orc.F32, f"{what} accumulator leaf {i}")
        _check_tree(tree, params, guard.inner_state[0], rf, what)
    assert applied == 2 and total == 2


def test_multisteps_update_only_mode():
    """tx.update: zeros on the micro-steps that do not emit, the inner
    update of the accumulator on the one that does."""
    import torch

    import rollfast_amd as rf

    params = _params(2)
    tx = rf.MultiSteps(rf.adamw8(learning_rate=1e-3, weight_decay=0.01, min_size=4096, exact=True), 2,
                       accumulator_dtype=torch.float32)
    state = tx.init(params)
    acc = [np.zeros(int(np.prod(s)), np.float32) for s, _p, _g in SPEC]
    for step in range(4):
        hg, dg = _grads(40 + step)
        for i, (_s, _p, gd) in enumerate(SPEC):
            orc.accumulate(orc.ACC_MEAN, step % 2, hg[i], _DT[gd], acc[i], orc.F32)
        tree = _oracle_tree(params, state.inner_opt_state[0], rf)
        updates, state = tx.update(dg, state, params)
        torch.cuda.synchronize()
        if step % 2 == 0:
            for i, (shape, _p, _g) in enumerate(SPEC):
                u = updates[f"l{i}"]
                assert u.dtype == torch.float32 and tuple(u.shape) == shape
                assert not torch.any(u != 0).item() and not torch.any(torch.signbit(u)).item()
            continue
        want = tree.step([a.copy() for a in acc], weight_decay=0.01, lr=1e-3, count=step // 2 + 1, apply=False)
        for i in range(len(SPEC)):
            _same_float(to_host(updates[f"l{i}"]), want[i], orc.F32, f"micro-step {step} updates leaf {i}")
        _check_tree(tree, params, state.inner_opt_state[0], rf, f"micro-step {step}")
        for a in acc:
            orc.accumulate(orc.ACC_ZERO, 0, None, orc.F32, a, orc.F32)
        params = rf.apply_updates(params, updates, stochastic=False)


# ---------------------------------------------------- properties at size --
def _big(seed, std, dt):
    rng = np.random.default_rng(seed)
    shapes = {"emb": (4096, 512), "w": (1024, 1536), "b": (1536,), "odd": (3, 50001)}
    return {k: to_device(bf16_bits(gaussian(rng, (int(np.prod(s)),), std)) if dt == "bf16" else
                         gaussian(rng, (int(np.prod(s)),), std), dt).reshape(s) for k, s in shapes.items()}


def _assert_trees_equal(a, b, what):
    for k in a:
        np.testing.assert_array_equal(to_host(a[k]), to_host(b[k]), err_msg=f"{what} {k}")


def _moments(state):
    import rollfast_amd as rf

    out = []
    for leaf in (list(state.mu.values()) + list(state.nu.values())):
        if isinstance(leaf, rf.MaskedNode):
            continue
        if isinstance(leaf, rf.QuantizedBlocks):
            out += [to_host(leaf.values), to_host(leaf.scales)]
        else:
            out.append(to_host(leaf))
    return out


@pytest.mark.parametrize("acc_dtype", [None, "float32"])
def test_k1_equals_the_inner_step(acc_dtype):
    """k = 1: the accumulator is 0 + (g - 0) / 1 = g (exactly, also widened
    to f32), so every micro-step is the inner step, param SR included."""
    import torch

    import rollfast_amd as rf

    pa, pb = _big(5, 0.02, "bf16"), _big(5, 0.02, "bf16")
    txa = rf.MultiSteps(rf.adamw8(learning_rate=1e-3, weight_decay=0.01), 1, accumulator_dtype=acc_dtype)
    txb = rf.adamw8(learning_rate=1e-3, weight_decay=0.01)
    sa, sb = txa.init(pa), txb.init(pb)
    for step in range(3):
        g = _big(60 + step, 1e-2, "bf16")
        key = rf.prng.PRNGKey(step)
        pa, sa = rf.adamw8_step(txa, pa, g, sa, key=key)
        pb, sb = rf.adamw8_step(txb, pb, g, sb, key=key)
        torch.cuda.synchronize()
        _assert_trees_equal(pa, pb, f"step {step} params")
        for x, y in zip(_moments(sa.inner_opt_state[0]), _moments(sb[0])):
            np.testing.assert_array_equal(x, y)
        assert int(sa.gradient_step) == step + 1 and int(sa.mini_step) == 0


def test_window_of_identical_grads_equals_one_step_of_the_builders_chain():
    """The builders' composition MultiSteps(apply_if_finite(chain(
    clip_by_global_norm, multi_transform(...)))) fed the same grads k times:
    the running mean of a constant is that constant, so each emit equals one
    step of the composition without MultiSteps, and the params do not move
    in between."""
    import torch

    import rollfast_amd as rf

    labels = {"emb": "base", "w": "base", "b": "head", "odd": "lora"}

    def composition():
        groups = {
            "base": rf.adamw8(learning_rate=1e-3, weight_decay=0.01, key=rf.prng.PRNGKey(1)),
            "lora": rf.adamw8(learning_rate=5e-3, weight_decay=0.0, quantize=False, key=rf.prng.PRNGKey(2)),
            "head": rf.adamw(learning_rate=2e-3, weight_decay=0.05, key=rf.prng.PRNGKey(3)),
        }
        return rf.apply_if_finite(rf.chain(rf.clip_by_global_norm(1.0), rf.multi_transform(groups, labels)), 1)

    k = 4
    pa, pb = _big(7, 0.02, "bf16"), _big(7, 0.02, "bf16")
    txa = rf.MultiSteps(composition(), k)  # accumulator in the params' dtype (bf16)
    txb = composition()
    sa, sb = txa.init(pa), txb.init(pb)
    for window in range(2):
        g = _big(80 + window, 3.0, "bf16")  # large: the clip is active
        key = rf.prng.PRNGKey(100 + window)
        for micro in range(k):
            before = {n: to_host(pa[n]).copy() for n in pa}
            pa, sa = rf.adamw8_step(txa, pa, g, sa, key=key)
            torch.cuda.synchronize()
            if micro < k - 1:
                for n in pa:
                    np.testing.assert_array_equal(to_host(pa[n]), before[n], err_msg=f"window {window} micro {micro}")
        pb, sb = rf.adamw8_step(txb, pb, g, sb, key=key)
        torch.cuda.synchronize()
        _assert_trees_equal(pa, pb, f"window {window} params")
        ga = sa.inner_opt_state.inner_state[1].inner_states
        gb = sb.inner_state[1].inner_states
        for lab in ga:
            for x, y in zip(_moments(ga[lab].inner_state[0]), _moments(gb[lab].inner_state[0])):
                np.testing.assert_array_equal(x, y, err_msg=f"window {window} group {lab}")
        assert int(sa.gradient_step) == window + 1
        for n in pa:
            acc = sa.acc_grads[n]
            assert acc.dtype == torch.bfloat16 and not torch.any(acc != 0).item()


def test_skip_function_schedule_and_errors():
    import torch

    import rollfast_amd as rf

    params = _big(9, 0.02, "bf16")
    calls = []

    def skip_fn(updates, gradient_step, params):
        del updates, params
        calls.append(int(gradient_step))
        return np.asarray(len(calls) == 3), {"seen": len(calls)}

    tx = rf.MultiSteps(rf.adamw8(learning_rate=1e-3), every_k_schedule=lambda s: 2 if int(s) < 1 else 3,
                       should_skip_update_fn=skip_fn)
    state = tx.init(params)
    assert state.skip_state == {"seen": 1}
    g = _big(90, 1e-2, "bf16")
    minis, gsteps = [], []
    for _ in range(6):
        before = [to_host(a).copy() for a in state.acc_grads.values()]
        params, state = rf.adamw8_step(tx, params, g, state, key=rf.prng.PRNGKey(0))
        torch.cuda.synchronize()
        minis.append(int(state.mini_step))
        gsteps.append(int(state.gradient_step))
        if len(calls) == 3:  # the skipped micro-step: accumulator and counters kept
            for a, b in zip(state.acc_grads.values(), before):
                np.testing.assert_array_equal(to_host(a), b)
    # k = 2 for gradient step 0, then 3; the third call (init's is the first)
    # is skipped
    assert minis == [1, 1, 0, 1, 2, 0] and gsteps == [0, 0, 1, 1, 1, 2]
    assert calls == [0, 0, 0, 0, 1, 1, 1]
    assert state.skip_state == {"seen": 7}
    zeros, s2 = tx.update(g, state, params)  # a skipped update-only call: zeros like the accumulator
    torch.cuda.synchronize()
    assert len(calls) == 8 and int(s2.mini_step) == 1

    bad = rf.MultiSteps(rf.adamw8(learning_rate=1e-3), 2, should_skip_update_fn=lambda u, s, p: (np.int32(0), ()))
    with pytest.raises(ValueError, match="boolean scalar"):
        bad.update(g, bad.init(params), params)

    f32_grads = {n: v.float() for n, v in g.items()}
    tx16 = rf.MultiSteps(rf.adamw8(learning_rate=1e-3), 2)  # bf16 accumulator: f32 grads would promote it
    with pytest.raises(TypeError, match="promote"):
        tx16.update(f32_grads, tx16.init(params), params)
    tx32 = rf.MultiSteps(rf.adamw8(learning_rate=1e-3), 2, accumulator_dtype=torch.float32)
    s32 = tx32.init(params)
    u, s32 = tx32.update(f32_grads, s32, params)
    torch.cuda.synchronize()
    assert int(s32.mini_step) == 1
    with pytest.raises(ValueError, match="PRNG"):
        rf.adamw8_step(tx32, params, g, s32, key=None)
