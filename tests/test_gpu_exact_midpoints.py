"""Exact mode where the bf16 rounding is decided by the last f32 ulps.

With bf16 params of zero the fused step's f32 sum is the update itself,
s = -lr * u.  At step 1 |u| is about 1 - 55 * 2^-24 - k * 2^-24 for
|g| = eps * 2^23 / k (the f32 bias corrections put sqrt(v') about 6.4e-6
above |g'|, eps adds k ulps), so with lr = (1 + 2^-8)(1 + 63 * 2^-23) and k
in [0.5, 16] every sum lies within about 8 f32 ulps of 1 + 2^-8, the bf16
midpoint between 1 and 1 + 2^-7, on either side (adam8.py:304-389,
utils.py:648-708).  Which side it ends on is decided by the last ulps of
the quotient, so the hardware rcp/sqrt direction disagrees with the
reference on many elements, and exact mode
(rounding settled from the hardware direction where the bound allows, the
IEEE direction elsewhere) must agree on every one.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

BS = 2048
LR = (1.0 + 2.0 ** -8) * (1.0 + 63 * 2.0 ** -23)


def _case(seed):
    rng = np.random.default_rng(seed)
    n = 4 * BS
    k = rng.uniform(0.5, 16.0, n)
    g = (1e-8 * 2.0 ** 23 / k) * rng.choice([-1.0, 1.0], n)
    return np.zeros(n, np.uint16), orc.f32_to_bf16_bits(g.astype(np.float32))


def _run(p_bits, g_bits, exact, sr_bits=None):
    import torch

    import rollfast_amd as rf

    def dev(bits):
        return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).cuda()

    params, grads = {"w": dev(p_bits)}, {"w": dev(g_bits)}
    tx = rf.adamw8(learning_rate=LR, weight_decay=0.0, exact=exact)
    state = tx.init(params)
    if sr_bits is None:
        params, state = rf.adamw8_step(tx, params, grads, state, stochastic=False)
    else:
        fed = torch.from_numpy(sr_bits.view(np.int32).copy()).view(torch.uint32).cuda()
        params, state = rf.adamw8_step(tx, params, grads, state, key=rf.prng.PRNGKey(0), stochastic=True,
                                       random_bits={0: (None, None, fed)})
    torch.cuda.synchronize()
    m, v = state[0].mu["w"], state[0].nu["w"]
    return (params["w"].view(torch.int16).cpu().numpy().view(np.uint16), m.values.cpu().numpy().reshape(-1),
            m.scales.cpu().numpy(), v.values.cpu().numpy().reshape(-1), v.scales.cpu().numpy())


def _oracle(p_bits, g_bits, sr_bits=None):
    n = p_bits.size
    p = p_bits.copy()
    mu = np.full(n, 127, np.uint8)
    nu = np.zeros(n, np.uint8)
    mus = np.ones(n // BS, np.float32)
    nus = np.ones(n // BS, np.float32)
    hp = orc.make_hparams(weight_decay=0.0, lr=LR, count=1, decay=False, apply=True, param_sr=sr_bits is not None)
    orc.adam8_leaf(hp, p, orc.BF16, g_bits, orc.BF16, orc.MOM_QUANT, mu, mus, nu, nus, BS, p_bits=sr_bits)
    return p, mu, mus, nu, nus


@pytest.mark.parametrize("seed,rounding", [(1, "rne"), (2, "rne"), (3, "sr_fed")])
def test_exact_mode_at_bf16_midpoints(seed, rounding):
    """rounding "sr_fed": param stochastic rounding with fed bits whose low
    halves are all 0x8000, which puts the step of every element's rounding
    at that same midpoint (utils.py:365-371)."""
    p_bits, g_bits = _case(seed)
    sr_bits = np.full(p_bits.size, 0x8000, np.uint32) if rounding == "sr_fed" else None
    want = _oracle(p_bits, g_bits, sr_bits)
    # the sums sit at the midpoint: the reference itself rounds both ways
    rounded_up = np.count_nonzero((want[0] & 0x7FFF) == 0x3F81)
    assert 0 < rounded_up < p_bits.size
    got = _run(p_bits, g_bits, exact=True, sr_bits=sr_bits)
    for name, a, b in zip(("params", "mu codes", "mu scales", "nu codes", "nu scales"), got, want):
        np.testing.assert_array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8),
                                      err_msg=f"exact mode: {name}")
    # the same inputs through the hardware direction: params off by one bf16
    # ulp where the last ulps decide (codes and scales stay exact)
    fast = _run(p_bits, g_bits, exact=False, sr_bits=sr_bits)
    off = np.count_nonzero(fast[0] != want[0])
    print(f"[midpoints] seed {seed} {rounding}: {rounded_up} of {p_bits.size} rounded up by the reference, "
          f"{off} params differ in the default mode", flush=True)
    assert off > 0
    np.testing.assert_array_equal(fast[1], want[1])
    np.testing.assert_array_equal(fast[3], want[3])
