"""The whole Llama-7B tree (291 leaves, 6,738,415,616 bf16 params, all
quantized) through ``adamw8_step``: the benchmark's launch shape (one fused
launch over every leaf, runs of 4 blocks, whole chip-fulls of workgroups)
and default mode (hardware rcp/sqrt direction), for 3 steps with fresh
grads ~N(0, 1e-3) each step.

Blocks are independent (adam8.py:137-187: absmax, scale and codes are per
2048-element block; the update is elementwise), so each leaf's first block,
last block and 8 random blocks are checked against the oracle run on that
block alone.  The oracle keeps its own codes and scales across the steps
(bar: bit-exact) and takes the device's params before each step (bar: within
one bf16 ulp after it).

The other tests turn on param and moment stochastic rounding with three bit
sources: fed random bits (arbitrary uint32 words on the device, the same
words given to the oracle), the in-kernel jax.random.bits stream of the
per-leaf keys (291 leaves' key derivation; the oracle gets
``orc.random_bits`` of the same keys at each sampled block's offset) and the
packed source (``orc.packed_param_bits`` / ``packed_moment_bits`` at the
block's offset).  The moment codes stay bit-exact and the params within one
bf16 ulp (the direction's hardware rcp/sqrt can move the f32 sum by a few
ulps before it is rounded).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import bf16_ulp_distance

pytestmark = pytest.mark.gpu

BS = 2048


def _rows(t, idx):
    """Rows idx of a flat device tensor viewed as [nblocks, BS], on the host
    (bf16 as uint16 patterns, uint32 as uint32)."""
    import torch

    as_view = {torch.bfloat16: (torch.int16, np.uint16), torch.uint32: (torch.int32, np.uint32)}
    tv, hv = as_view.get(t.dtype, (None, None))
    if tv is not None:
        t = t.view(tv)
    v = t.reshape(-1, BS)[torch.as_tensor(idx, device=t.device)].cpu().numpy()
    return v.view(hv) if hv is not None else v


def _random_words(n, gen):
    """n arbitrary uint32 words on the device (every bit random)."""
    import torch

    return torch.randint(0, 256, (4 * n,), dtype=torch.uint8, device="cuda", generator=gen).view(torch.uint32)


def _key(k):
    return tuple(int(v) for v in k)


def _llama_tree_run(sr: bool, steps: int, source: str = "fed"):
    """``source``: the SR bits -- "fed", "jax" (in-kernel jax.random.bits)
    or "packed" (in-kernel packed source)."""
    import torch

    import bench
    import rollfast_amd as rf

    shapes = [s for _, s in bench.llama7b_shapes()]
    names = [f"l{i:03d}" for i in range(len(shapes))]  # dict flatten order = leaf index
    sizes = [int(np.prod(s)) for s in shapes]
    assert len(shapes) == 291 and sum(sizes) == 6_738_415_616
    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    print(f"[llama7b] sr={sr}: allocating params", flush=True)
    params = {nm: (torch.randn(s, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
              for nm, s in zip(names, shapes)}
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=sr,
                   sr_bits="packed" if source == "packed" else "jax")
    state = tx.init(params)
    rng = np.random.default_rng(3)
    picks = []
    for n in sizes:
        nb = n // BS
        assert nb * BS == n
        picks.append(np.unique(np.concatenate([[0, nb - 1], rng.choice(nb, size=min(8, nb), replace=False)])))
    # the oracle's copy of the sampled blocks' moments
    orc_m = []
    for nm, idx in zip(names, picks):
        m, v = state[0].mu[nm], state[0].nu[nm]
        orc_m.append({"mc": _rows(m.values, idx).copy(), "vc": _rows(v.values, idx).copy(),
                      "ms": m.scales.cpu().numpy()[idx].copy(), "vs": v.scales.cpu().numpy()[idx].copy()})
    checked = 0
    for step in range(steps):
        print(f"[llama7b] sr={sr}: step {step + 1}", flush=True)
        grads = {nm: (torch.randn(s, generator=gen, device="cuda") * 1e-3).to(torch.bfloat16)
                 for nm, s in zip(names, shapes)}
        bits = fed = None
        pkey = rf.prng.PRNGKey(100 + step)
        if sr and source == "fed":
            bits = {i: (_random_words(sizes[i], gen), _random_words(sizes[i], gen), _random_words(sizes[i], gen))
                    for i in range(len(names))}
            fed = [tuple(_rows(b, idx) for b in bits[i]) for i, idx in enumerate(picks)]
        elif sr:
            # the words the in-kernel source draws for each sampled block:
            # leaf i's keys are split(key_mu | key_nu | param key, 291)[i]
            key_mu, key_nu, _ = orc.split(_key(state[0].key), 3)
            kmu, knu = orc.split(tuple(key_mu), len(names)), orc.split(tuple(key_nu), len(names))
            kp = orc.split(_key(pkey), len(names))
            fed = []
            for i, idx in enumerate(picks):
                rows = ([], [], [])
                for b in idx:
                    off = int(b) * BS
                    if source == "packed":
                        bm, bv = orc.packed_moment_bits(kmu[i], BS, off)
                        bp = orc.packed_param_bits(kp[i], BS, off)
                    else:
                        bm, bv = orc.random_bits(kmu[i], BS, off), orc.random_bits(knu[i], BS, off)
                        bp = orc.random_bits(kp[i], BS, off)
                    for lst, w in zip(rows, (bm, bv, bp)):
                        lst.append(w)
                fed.append(tuple(np.stack(r) for r in rows))
        before = [(_rows(params[nm], idx), _rows(grads[nm], idx)) for nm, idx in zip(names, picks)]
        params, state = rf.adamw8_step(tx, params, grads, state, key=pkey, stochastic=sr, random_bits=bits)
        torch.cuda.synchronize()
        del grads, bits
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=step + 1, decay=True, apply=True,
                              moment_sr=sr, param_sr=sr)
        worst = 0
        for i, (nm, idx) in enumerate(zip(names, picks)):
            p0, g0 = before[i]
            got_p = _rows(params[nm], idx)
            m, v = state[0].mu[nm], state[0].nu[nm]
            got_mc, got_vc = _rows(m.values, idx), _rows(v.values, idx)
            got_ms, got_vs = m.scales.cpu().numpy()[idx], v.scales.cpu().numpy()[idx]
            om = orc_m[i]
            for r in range(idx.size):
                p = p0[r].copy()
                mc, vc = om["mc"][r], om["vc"][r]
                ms, vs = om["ms"][r:r + 1], om["vs"][r:r + 1]
                kw = {}
                if sr:
                    kw = dict(mu_bits=fed[i][0][r], nu_bits=fed[i][1][r], p_bits=fed[i][2][r])
                orc.adam8_leaf(hp, p, orc.BF16, g0[r], orc.BF16, orc.MOM_QUANT, mc, ms, vc, vs, BS, **kw)
                where = f"step {step + 1} leaf {i} {shapes[i]} block {idx[r]}"
                np.testing.assert_array_equal(got_mc[r], mc, err_msg=f"{where}: mu codes")
                np.testing.assert_array_equal(got_vc[r], vc, err_msg=f"{where}: nu codes")
                assert got_ms[r].view(np.uint32) == ms.view(np.uint32)[0], f"{where}: mu scale"
                assert got_vs[r].view(np.uint32) == vs.view(np.uint32)[0], f"{where}: nu scale"
                worst = max(worst, int(bf16_ulp_distance(got_p[r], p).max()))
                checked += 1
        assert worst <= 1, f"step {step + 1}: params differ by {worst} bf16 ulp"
    del params, state
    torch.cuda.empty_cache()
    assert checked == steps * sum(p.size for p in picks)
    # 226 matrices x 10 blocks + 65 norm vectors x 2 blocks
    assert sum(p.size for p in picks) == 226 * 10 + 65 * 2


def test_llama7b_whole_tree_three_steps_default_mode():
    _llama_tree_run(sr=False, steps=3)


def test_llama7b_whole_tree_param_and_moment_sr_fed_bits():
    _llama_tree_run(sr=True, steps=2)


def test_llama7b_whole_tree_param_and_moment_sr_jax_stream():
    _llama_tree_run(sr=True, steps=2, source="jax")


def test_llama7b_whole_tree_param_and_moment_sr_packed():
    _llama_tree_run(sr=True, steps=2, source="packed")
