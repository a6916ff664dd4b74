"""One bf16 leaf of 2^32 + 10,240 + 777 elements (2,097,158 blocks, the last
one partial) through ``adamw8_step`` with param and moment stochastic
rounding drawn in the kernel, for 2 steps.

The leaf's element index passes 2^31 and 2^32: the Threefry counter of
jax.random.bits (``jax_threefry_partitionable``: the element index as the
(high, low) 32-bit counter words) takes a non-zero high word there, and
every offset into the params, grads, codes and scales needs 64 bits.  Blocks
are independent (adam8.py:137-187), so the blocks on both sides of 2^31 and
2^32 elements, the first, the last full and the partial last block and 6
random ones are checked against the oracle run on that block alone, its
bits drawn with ``orc.random_bits(key, n, offset=block * 2048)`` from the
leaf's keys (adam8.py:306 for the moment keys, utils.py:648-708 for the
param key).  Bar: codes and scales bit-exact; params within one bf16 ulp
(default hardware rcp/sqrt direction).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import bf16_ulp_distance

pytestmark = pytest.mark.gpu

BS = 2048
N = (1 << 32) + 5 * BS + 777
NB = (N + BS - 1) // BS


def _block(t, b, n):
    """Elements [b*BS, min((b+1)*BS, n)) of a flat device tensor, on the host
    (bf16 as uint16 patterns)."""
    import torch

    lo, hi = b * BS, min((b + 1) * BS, n)
    v = t.reshape(-1)[lo:hi]
    if v.dtype == torch.bfloat16:
        v = v.view(torch.int16)
        return v.cpu().numpy().view(np.uint16)
    return v.cpu().numpy()


def _fill_normal(t, std, gen):
    """t (flat bf16, device) <- N(0, std^2), 2^28 elements at a time."""
    import torch

    flat = t.reshape(-1)
    step = 1 << 28
    for lo in range(0, flat.numel(), step):
        hi = min(lo + step, flat.numel())
        flat[lo:hi] = (torch.randn(hi - lo, generator=gen, device="cuda") * std).to(torch.bfloat16)


def test_leaf_beyond_2p32_elements_sr_in_kernel_bits():
    import torch

    import rollfast_amd as rf

    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    print(f"[bigleaf] allocating a {N}-element bf16 leaf ({NB} blocks)", flush=True)
    params = {"w": torch.empty(N, dtype=torch.bfloat16, device="cuda")}
    _fill_normal(params["w"], 0.02, gen)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=True, key=rf.prng.PRNGKey(5))
    state = tx.init(params)
    m, v = state[0].mu["w"], state[0].nu["w"]
    assert tuple(m.values.shape) == (NB, BS)
    rng = np.random.default_rng(4)
    edges = [0, (1 << 31) // BS - 1, (1 << 31) // BS, (1 << 32) // BS - 1, (1 << 32) // BS, NB - 2, NB - 1]
    idx = np.unique(np.concatenate([edges, rng.choice(NB, size=6, replace=False)]))
    orc_m = {int(b): {"mc": m.values[b].cpu().numpy().copy(), "vc": v.values[b].cpu().numpy().copy(),
                      "ms": m.scales[b:b + 1].cpu().numpy().copy(), "vs": v.scales[b:b + 1].cpu().numpy().copy()}
             for b in idx}
    grads = {"w": torch.empty(N, dtype=torch.bfloat16, device="cuda")}
    for step in range(2):
        print(f"[bigleaf] step {step + 1}", flush=True)
        _fill_normal(grads["w"], 1e-3, gen)
        before = {int(b): (_block(params["w"], b, N), _block(grads["w"], b, N)) for b in idx}
        key_mu, key_nu, _ = orc.split(state[0].key, 3)
        kmu, knu = orc.split(key_mu, 1)[0], orc.split(key_nu, 1)[0]
        pkey = rf.prng.PRNGKey(200 + step)
        kp = orc.split(pkey, 1)[0]
        params, state = rf.adamw8_step(tx, params, grads, state, key=pkey, stochastic=True)
        torch.cuda.synchronize()
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=step + 1, decay=True, apply=True,
                              moment_sr=True, param_sr=True)
        m, v = state[0].mu["w"], state[0].nu["w"]
        worst = 0
        for b in idx:
            b = int(b)
            p, g = before[b]
            p = p.copy()
            o = orc_m[b]
            orc.adam8_leaf(hp, p, orc.BF16, g, orc.BF16, orc.MOM_QUANT, o["mc"], o["ms"], o["vc"], o["vs"], BS,
                           mu_bits=orc.random_bits(kmu, BS, offset=b * BS),
                           nu_bits=orc.random_bits(knu, BS, offset=b * BS),
                           p_bits=orc.random_bits(kp, g.size, offset=b * BS))
            where = f"step {step + 1} block {b} (elements from {b * BS})"
            np.testing.assert_array_equal(m.values[b].cpu().numpy(), o["mc"], err_msg=f"{where}: mu codes")
            np.testing.assert_array_equal(v.values[b].cpu().numpy(), o["vc"], err_msg=f"{where}: nu codes")
            assert m.scales[b:b + 1].cpu().numpy().view(np.uint32)[0] == o["ms"].view(np.uint32)[0], where
            assert v.scales[b:b + 1].cpu().numpy().view(np.uint32)[0] == o["vs"].view(np.uint32)[0], where
            worst = max(worst, int(bf16_ulp_distance(_block(params["w"], b, N), p).max()))
        assert worst <= 1, f"step {step + 1}: params differ by {worst} bf16 ulp"
    del params, grads, state
    torch.cuda.empty_cache()
