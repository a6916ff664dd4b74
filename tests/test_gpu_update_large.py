"""Update-only launches (``tx.update``, the reference's Optax form) over many
blocks: each chunk's f32 updates pass through the wave's LDS region and are
stored on whole cache lines, nontemporally from 768 fast blocks per CU on.
A leaf of 2^29 bf16 elements (262,144 blocks) is above that on MI355X
(256 CUs).

Blocks are independent (adam8.py:137-187), so the first, the last and 14
random blocks are checked against the oracle run on each block alone, over
two steps: codes and scales bit-exact, f32 updates bit-exact (``exact=True``,
the IEEE direction), params untouched.  Moment rounding: nearest, the packed
source and the jax.random.bits stream of the leaf keys (the oracle gets
``orc.packed_moment_bits`` / ``orc.random_bits`` at each block's offset).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

BS = 2048
N = 1 << 29


def _rows(t, idx, dtype):
    import torch

    flat = t.reshape(-1)
    sel = torch.as_tensor(idx, device=flat.device, dtype=torch.int64)
    rows = flat.view(-1, BS).index_select(0, sel)
    if rows.dtype == torch.bfloat16:
        rows = rows.view(torch.int16)
    return rows.cpu().numpy().view(dtype)


@pytest.mark.parametrize("source", ["nearest", "packed", "jax"])
def test_large_update_only_blocks_match_oracle(source):
    import torch

    import rollfast_amd as rf

    ncu = torch.cuda.get_device_properties(0).multi_processor_count
    nb = N // BS
    assert nb >= 768 * ncu, "the leaf must be large enough for nontemporal update stores"
    msr = source != "nearest"
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    print(f"[update-large] {source}: allocating", flush=True)
    params = {"w": (torch.randn(N, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)}
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=msr, exact=True,
                   sr_bits="packed" if source == "packed" else "jax")
    state = tx.init(params)
    rng = np.random.default_rng(9)
    idx = np.unique(np.concatenate([[0, nb - 1], rng.choice(nb, size=14, replace=False)]))
    m0, v0 = state[0].mu["w"], state[0].nu["w"]
    mc, vc = _rows(m0.values, idx, np.uint8).copy(), _rows(v0.values, idx, np.uint8).copy()
    ms = m0.scales.reshape(-1).cpu().numpy()[idx].copy()
    vs = v0.scales.reshape(-1).cpu().numpy()[idx].copy()
    p_rows = _rows(params["w"], idx, np.uint16).copy()
    for step in range(2):
        print(f"[update-large] {source}: step {step + 1}", flush=True)
        grads = {"w": (torch.randn(N, generator=gen, device="cuda") * 1e-3).to(torch.bfloat16)}
        g_rows = _rows(grads["w"], idx, np.uint16)
        key_mu, key_nu, _ = orc.split(tuple(int(k) for k in state[0].key), 3)
        kmu = orc.split(tuple(key_mu), 1)[0]
        knu = orc.split(tuple(key_nu), 1)[0]
        count = int(state[0].count) + 1
        updates, state = tx.update(grads, state, params)
        torch.cuda.synchronize()
        got_u = _rows(updates["w"], idx, np.float32)
        got_mc = _rows(state[0].mu["w"].values, idx, np.uint8)
        got_vc = _rows(state[0].nu["w"].values, idx, np.uint8)
        got_ms = state[0].mu["w"].scales.reshape(-1).cpu().numpy()[idx]
        got_vs = state[0].nu["w"].scales.reshape(-1).cpu().numpy()[idx]
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=count, decay=True, apply=False, moment_sr=msr)
        for r, b in enumerate(idx):
            off = int(b) * BS
            kw = {}
            if source == "packed":
                kw = dict(zip(("mu_bits", "nu_bits"), orc.packed_moment_bits(kmu, BS, off)))
            elif source == "jax":
                kw = dict(mu_bits=orc.random_bits(kmu, BS, off), nu_bits=orc.random_bits(knu, BS, off))
            want_u = np.empty(BS, np.float32)
            s_m, s_v = ms[r:r + 1], vs[r:r + 1]
            orc.adam8_leaf(hp, p_rows[r].copy(), orc.BF16, g_rows[r].copy(), orc.BF16, orc.MOM_QUANT, mc[r], s_m,
                           vc[r], s_v, BS, updates_out=want_u, **kw)
            where = f"{source} step {step + 1} block {b}"
            np.testing.assert_array_equal(got_mc[r], mc[r], err_msg=f"{where}: mu codes")
            np.testing.assert_array_equal(got_vc[r], vc[r], err_msg=f"{where}: nu codes")
            np.testing.assert_array_equal(got_ms[r], s_m[0], err_msg=f"{where}: mu scale")
            np.testing.assert_array_equal(got_vs[r], s_v[0], err_msg=f"{where}: nu scale")
            np.testing.assert_array_equal(got_u[r].view(np.uint32), want_u.view(np.uint32), err_msg=f"{where}: updates")
        np.testing.assert_array_equal(_rows(params["w"], idx, np.uint16), p_rows)
        del grads, updates
