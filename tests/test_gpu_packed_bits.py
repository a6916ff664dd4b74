"""GPU parity and statistics of the packed bit source (``sr_bits="packed"``,
``RF_PACKED_BITS``; no reference counterpart).

The packed source keeps the reference's per-leaf keys but spends one
Threefry-2x32-20 block on four param roundings (element e: half e & 1 of word
e & 2 ? y1 : y0 of the block at counter e >> 2) and one main block on both
moments of a pair of elements (element e: half e & 1 of y0 for the first
moment, of y1 for the second, of the block at counter e >> 1 under the
first-moment key).  A moment code's draw is the word (main << 16) | fill,
with the fill half from the block at counter 2^63 + (e >> 1), which the
kernel computes only when the main half leaves the decision open; bf16
moment storage takes the main half alone.

Bars:
* every packed result is bitwise the oracle's result on the packed stream
  fed as bits (``oracle.packed_param_bits`` / ``packed_moment_bits``): codes,
  scales, stored bf16 moments and params (``exact=True``);
* param rounding is unbiased: over 64 keys the mean relative rounding error
  per magnitude decade is zero within 5 standard errors;
* moment rounding takes the upper code with probability (n - cb_l) /
  (cb_u - cb_l), within 5 sigma, and the draws that share a main block
  (both moments, a pair of elements) are uncorrelated;
* on a leaf of 2^22 elements, where some 120 draws per moment and step need
  their fill block, every code is the oracle's;
* the four roundings that share a block are independent: the up/down
  decisions of elements e and e + k (k = 1, 2, 3) are uncorrelated within
  5 standard errors.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import bf16_bits, gaussian, to_device, to_host
from tests.test_gpu_step import MIXED, _build, _compare_params, _compare_state, _grads, _oracle_from_state

pytestmark = pytest.mark.gpu


def _key(k):
    return tuple(int(v) for v in k)


def _run_packed(spec, *, steps, msr, psr, seed=0, wd=0.01, lr=1e-3):
    import torch

    import rollfast_amd as rf

    host_params, params = _build(spec, seed)
    tx = rf.adamw8(learning_rate=lr, weight_decay=wd, stochastic_rounding=msr, exact=True, key=rf.prng.PRNGKey(7),
                   sr_bits="packed")
    state = tx.init(params)
    n = len(spec)
    for step in range(steps):
        ghost, gdev = _grads(spec, seed + 1000 + step)
        for i, (_shape, _pd, _gd) in enumerate(spec):
            host_params[f"l{i:03d}"] = to_host(params[f"l{i:03d}"]).copy()
        tree = _oracle_from_state(spec, host_params, state[0])
        before = [L["param"].copy() for L in tree.leaves]
        key_mu, _key_nu, _ = orc.split(state[0].key, 3)
        mu_bits = nu_bits = p_bits = None
        pkey = rf.prng.PRNGKey(300 + step)
        if msr:
            kmu = orc.split(key_mu, n)
            mu_bits, nu_bits = [], []
            for i, L in enumerate(tree.leaves):
                padded = len(L["mu"]) if L["kind"] == "quant" else L["size"]
                bm, bv = orc.packed_moment_bits(kmu[i], padded)
                mu_bits.append(bm)
                nu_bits.append(bv)
        if psr:
            kp = orc.split(_key(pkey), n)
            p_bits = [orc.packed_param_bits(kp[i], L["size"]) for i, L in enumerate(tree.leaves)]
        tree.step(ghost, weight_decay=wd, lr=lr, count=int(state[0].count) + 1, moment_sr=msr, param_sr=psr,
                  mu_bits=mu_bits, nu_bits=nu_bits, p_bits=p_bits)
        params, state = rf.adamw8_step(tx, params, gdev, state, key=pkey if psr else None, stochastic=psr)
        torch.cuda.synchronize()
        _compare_state(spec, tree, state[0], f"packed step {step + 1}")
        _compare_params(spec, tree, params, True, f"packed step {step + 1}", before)


def test_packed_param_sr_fused_step():
    """Fast blocks, partial blocks, fallback leaves and f32 params (which take
    no stochastic rounding) of one fused launch."""
    _run_packed(MIXED, steps=2, msr=False, psr=True)


def test_packed_moment_sr_fused_step():
    _run_packed(MIXED, steps=2, msr=True, psr=False)


def test_packed_moment_sr_fill_blocks_one_big_leaf():
    """One 2^22-element leaf (2048 fast blocks): about one draw in 2^16 per
    moment is left open by its main half and decided with the fill block
    (some 120 per moment and step), so a fill path that decided wrongly, or
    read the wrong half or block, would change codes the oracle checks."""
    _run_packed([((2048, 2048), "bf16", "bf16")], steps=2, msr=True, psr=True)


def test_packed_both_roundings_block_4096():
    """Blocks of 4096 (the generic kernel, a workgroup per block, literal
    coding) with both roundings from the packed source."""
    import rollfast_amd as rf  # noqa: F401

    spec = [((3, 5000), "bf16", "bf16"), ((9000,), "bf16", "f32"), ((64, 2048), "bf16", "bf16")]
    _run_packed(spec, steps=2, msr=True, psr=True)


def test_packed_optax_form_equals_fused():
    """tx.update + apply_updates(sr_bits="packed") == adamw8_step with the
    packed tx, bit for bit (the same per-leaf keys and stream)."""
    import torch

    import rollfast_amd as rf

    spec = [((16, 2048), "bf16", "bf16"), ((500,), "bf16", "bf16"), ((3, 3000), "bf16", "f32")]
    _, pa = _build(spec, 11)
    _, pb = _build(spec, 11)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=True, exact=True, sr_bits="packed")
    sa, sb = tx.init(pa), tx.init(pb)
    for step in range(2):
        _, g = _grads(spec, 60 + step)
        key = rf.prng.PRNGKey(40 + step)
        pa, sa = rf.adamw8_step(tx, pa, g, sa, key=key, stochastic=True)
        u, sb = tx.update(g, sb, pb)
        pb = rf.apply_updates(pb, u, key=key, stochastic=True, sr_bits="packed")
        torch.cuda.synchronize()
        for k in pa:
            np.testing.assert_array_equal(to_host(pa[k]), to_host(pb[k]), err_msg=f"step {step} {k}")


def test_packed_full_precision_adamw_bf16_moments():
    """optim/adam.py's bf16 moment storage (RF_LEAF_STORE_SR) on the packed
    source: leaf i's first- and second-moment noise from the main halves of
    the block at counter e >> 1 under its first-moment storage key."""
    import torch

    import rollfast_amd as rf
    from tests.test_gpu_adam import SPEC, _build as abuild, _compare, _grads as agrads, _oracle_tree

    host, params = abuild(SPEC, 1)
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, mu_dtype=torch.bfloat16, exact=True,
                  key=rf.prng.PRNGKey(3), sr_bits="packed")
    state = tx.init(params)
    sizes = [int(np.prod(s)) for s, _, _ in SPEC]
    for step in range(2):
        ghost, gdev = agrads(SPEC, 100 + step)
        tree = _oracle_tree(SPEC, params, state[0])
        _next, sr = orc.split(_key(state[0].key), 2)
        k1, _k2 = orc.split(tuple(sr), 2)
        s1 = orc.split(tuple(k1), len(SPEC))
        pairs = [orc.packed_store_bits(s1[i], sizes[i]) for i in range(len(SPEC))]
        pkey = rf.prng.PRNGKey(50 + step)
        kp = orc.split(_key(pkey), len(SPEC))
        pb = [orc.packed_param_bits(kp[i], sizes[i]) for i in range(len(SPEC))]
        tree.step(ghost, weight_decay=0.01, lr=1e-3, count=step + 1, param_sr=True, mu_bits=[p[0] for p in pairs],
                  nu_bits=[p[1] for p in pairs], p_bits=pb, ema_weight_f32=True, store_sr=True, zero_decay=True)
        params, state = rf.adamw_step(tx, params, gdev, state, key=pkey, stochastic=True)
        torch.cuda.synchronize()
        _compare(SPEC, tree, params, state[0], True, f"packed adamw step {step + 1}")


def test_packed_apply_updates_and_sr_bf16_bitwise():
    """apply_updates (a work list over ragged leaves, vector and scalar
    tails) and _stochastic_round_bf16 on the packed source against the
    oracle's rounding of the packed stream."""
    import torch

    import rollfast_amd as rf
    from rollfast_amd.utils import _stochastic_round_bf16

    rng = np.random.default_rng(5)
    sizes = [8192 * 3 + 5, 777, 16, 1]
    params, updates, host_p, host_u = {}, {}, [], []
    for i, n in enumerate(sizes):
        p = bf16_bits(gaussian(rng, (n,), 0.5))
        u = gaussian(rng, (n,), 1e-3)
        host_p.append(p)
        host_u.append(u)
        params[f"l{i}"] = to_device(p, "bf16")
        updates[f"l{i}"] = to_device(u, "f32")
    key = rf.prng.PRNGKey(21)
    out = rf.apply_updates(params, updates, key=key, stochastic=True, sr_bits="packed")
    torch.cuda.synchronize()
    kp = orc.split(_key(key), len(sizes))
    for i, n in enumerate(sizes):
        want = host_p[i].copy()
        orc.apply_updates(want, orc.BF16, host_u[i], bits=orc.packed_param_bits(kp[i], n))
        np.testing.assert_array_equal(to_host(out[f"l{i}"]), want, err_msg=f"leaf {i}")

    for n in (1 << 20, 1003):
        x = to_device(gaussian(rng, (n,), 3.0), "f32")
        k = rf.prng.PRNGKey(n)
        got = to_host(_stochastic_round_bf16(x, k, sr_bits="packed"))
        want = orc.sr_bf16(to_host(x), orc.packed_param_bits(_key(k), n))
        assert np.count_nonzero(got != want) == 0, f"n={n}"


def test_packed_param_sr_unbiased_and_independent():
    """Unbiasedness over 64 keys per magnitude decade (the statistic of the
    standalone 2^30 test), and independence of the four roundings that share
    a block: on inputs a quarter, a half and three quarters of a bf16 ulp
    above a bf16 value, the up decisions of e and e + k are uncorrelated."""
    import torch

    import rollfast_amd as rf
    from rollfast_amd.utils import _stochastic_round_bf16

    m = 1 << 20
    rng = np.random.default_rng(8)
    mag = np.exp(rng.uniform(np.log(1e-6), np.log(1e2), m)).astype(np.float32)
    xh = (mag * rng.choice([-1.0, 1.0], m)).astype(np.float32)
    x = to_device(xh, "f32")
    xd = x.to(torch.float64)
    acc = torch.zeros(m, dtype=torch.float64, device="cuda")
    for s in range(64):
        r = _stochastic_round_bf16(x, rf.prng.PRNGKey(1000 + s), sr_bits="packed").to(torch.float64)
        acc += (r - xd) / xd.abs()
    rel = (acc / 64).cpu().numpy()
    dec = np.floor(np.log10(np.abs(xh)))
    for d in np.unique(dec):
        sel = rel[dec == d]
        if sel.size < 1000:
            continue
        assert abs(sel.mean()) < 5 * (2.0 ** -7 / 8) / np.sqrt(sel.size), (d, sel.mean())

    # independence: x = 1 + f * 2^-7 (f in {1/4, 1/2, 3/4}) rounds up with
    # probability f; 1 << 20 elements per key, decisions of pairs (e, e + k)
    n = 1 << 20
    for f in (0.25, 0.5, 0.75):
        xv = torch.full((n,), 1.0 + f * 2.0 ** -7, dtype=torch.float32, device="cuda")
        up = (_stochastic_round_bf16(xv, rf.prng.PRNGKey(int(f * 100)), sr_bits="packed").to(torch.float32)
              > 1.0).to(torch.float64).cpu().numpy()
        assert abs(up.mean() - f) < 5 * np.sqrt(f * (1 - f) / n), (f, up.mean())
        z = up - f
        for k in (1, 2, 3):
            for r in range(4):  # every position of the pair inside a block
                a, b = z[r::4], z[r + k::4]
                a, b = a[: b.size], b[: a.size]
                cov = float((a * b).mean())
                assert abs(cov) < 5 * f * (1 - f) / np.sqrt(a.size), (f, k, r, cov)


def test_packed_moment_sr_probability():
    """Moment stochastic rounding on the packed source: a block whose values
    sit between two codebook entries takes the upper code with probability
    (n - cb_l) / (cb_u - cb_l) (adam8.py:557-564), within 5 sigma, for the
    first and the second moment (which draw y0 and y1 of the same block)."""
    import torch

    import rollfast_amd as rf

    bs = 2048
    nb = 256
    size = nb * bs
    tx = rf.scale_by_adam8(b1=0.0, b2=0.0, stochastic_rounding=True, key=rf.prng.PRNGKey(2), sr_bits="packed")
    # b1 = b2 = 0: m = g and v = g*g exactly (EMA weights 1), so the codes
    # quantize g and g*g over blocks whose absmax is pinned to 1.
    cbs = orc.codebook(True).astype(np.float64)
    cbu = orc.codebook(False).astype(np.float64)
    lo_s, hi_s = cbs[200], cbs[201]
    t = 0.3
    g = np.full(size, lo_s + t * (hi_s - lo_s), np.float32)
    g[::bs] = 1.0  # absmax 1 -> scale 1 for both moments (1*1 = 1)
    params = {"w": torch.zeros(size, dtype=torch.float32, device="cuda")}
    state = tx.init(params)
    grads = {"w": to_device(g, "f32")}
    _, state = tx.update(grads, state, params)
    torch.cuda.synchronize()
    mc = to_host(state.mu["w"].values).reshape(-1)
    vc = to_host(state.nu["w"].values).reshape(-1)
    inner = np.ones(size, bool)
    inner[::bs] = False
    gm = np.float32(g[1])
    pm = (np.float64(gm) - lo_s) / (hi_s - lo_s)
    up_m = np.mean(mc[inner] == 201)
    assert set(np.unique(mc[inner]).tolist()) <= {200, 201}
    cnt = int(inner.sum())
    assert abs(up_m - pm) < 5 * np.sqrt(pm * (1 - pm) / cnt), (up_m, pm)
    v = np.float64(np.float32(gm * gm))
    ui = int(np.searchsorted(cbu, v, side="left"))
    pv = (v - cbu[ui - 1]) / (cbu[ui] - cbu[ui - 1])
    up_v = np.mean(vc[inner] == ui)
    assert set(np.unique(vc[inner]).tolist()) <= {ui - 1, ui}
    assert abs(up_v - pv) < 5 * np.sqrt(pv * (1 - pv) / cnt), (up_v, pv)

    # draws that share a main block: the two moments of an element (y0, y1)
    # and the two elements of a pair (the halves of a word); and across
    # neighbouring pairs.  Element 0 of each block holds its absmax; the
    # columns from 2 keep the pairs aligned.
    zm = (mc.reshape(nb, bs)[:, 2:bs - 2] == 201).astype(np.float64) - pm
    zv = (vc.reshape(nb, bs)[:, 2:bs - 2] == ui).astype(np.float64) - pv
    sd_mv = np.sqrt(pm * (1 - pm) * pv * (1 - pv) / zm.size)
    assert abs(float((zm * zv).mean())) < 5 * sd_mv
    for z, pp in ((zm, pm), (zv, pv)):
        for k in (1, 2):
            for r in (0, 1):  # r = 0, k = 1: the two halves of one word
                a, b = z[:, r::2], z[:, r + k::2]
                a, b = a[:, : b.shape[1]], b[:, : a.shape[1]]
                cov = float((a * b).mean())
                assert abs(cov) < 5 * pp * (1 - pp) / np.sqrt(a.size), (k, r, cov)
