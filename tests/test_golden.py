"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the oracle).

CPU: the oracle still reproduces every fixture bit for bit.
GPU: the HIP path reproduces them through the public API -- codes and
scales bit-exact; params bit-exact with ``exact=True``; f32 params within
one bf16 ulp with the hardware reciprocal path; bf16 params with fed
stochastic-rounding bits bit-exact.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import f32_params_close, to_device, to_host

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BS = 2048


def _load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# --------------------------------------------------------------- CPU ------
def test_oracle_reproduces_step_f32():
    z = _load("step_f32")
    n = z["p0"].size
    p = z["p0"].copy()
    mu = np.full(n, 127, np.uint8)
    nu = np.zeros(n, np.uint8)
    ms = np.ones(n // BS, np.float32)
    vs = np.ones(n // BS, np.float32)
    for t in range(1, 4):
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=t, decay=True, apply=True)
        orc.adam8_leaf(hp, p, orc.F32, z["grads"][t - 1], orc.F32, orc.MOM_QUANT, mu, ms, nu, vs, BS)
        np.testing.assert_array_equal(p.view(np.uint32), z[f"p{t}"].view(np.uint32))
        np.testing.assert_array_equal(mu, z[f"mu{t}"])
        np.testing.assert_array_equal(nu, z[f"nu{t}"])
        np.testing.assert_array_equal(ms.view(np.uint32), z[f"ms{t}"].view(np.uint32))
        np.testing.assert_array_equal(vs.view(np.uint32), z[f"vs{t}"].view(np.uint32))
    # the zero-gradient block of step 2 really exercised a decaying block
    assert np.all(z["grads"][1, BS:2 * BS] == 0)


def test_oracle_reproduces_step_bf16_sr():
    z = _load("step_bf16_sr")
    n = z["p0"].size
    nb = -(-n // BS)
    p = z["p0"].copy()
    mu = np.full(nb * BS, 127, np.uint8)
    nu = np.zeros(nb * BS, np.uint8)
    ms = np.ones(nb, np.float32)
    vs = np.ones(nb, np.float32)
    for t in range(1, 3):
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=t, decay=True, apply=True, moment_sr=True,
                              param_sr=True)
        orc.adam8_leaf(hp, p, orc.BF16, z["grads"][t - 1], orc.BF16, orc.MOM_QUANT, mu, ms, nu, vs, BS,
                       mu_bits=z["mbits"][t - 1], nu_bits=z["vbits"][t - 1], p_bits=z["pbits"][t - 1])
        np.testing.assert_array_equal(p, z[f"p{t}"])
        np.testing.assert_array_equal(mu, z[f"mu{t}"])
        np.testing.assert_array_equal(nu, z[f"nu{t}"])
        np.testing.assert_array_equal(ms, z[f"ms{t}"])
        np.testing.assert_array_equal(vs, z[f"vs{t}"])


def test_oracle_reproduces_quantize_and_sr():
    z = _load("quantize")
    for name, q, src in (("s", orc.Q_SIGNED, "x"), ("u", orc.Q_UNSIGNED, "xu"), ("y", orc.Q_SYMMETRIC, "x"),
                         ("e", orc.Q_SIGNED, "edge")):
        codes, scales = orc.quantize(z[src], 256, q)
        np.testing.assert_array_equal(codes.reshape(-1).view(np.uint8), z[f"codes_{name}"])
        np.testing.assert_array_equal(scales.view(np.uint32), z[f"scales_{name}"].view(np.uint32))
    s = _load("sr_bf16")
    np.testing.assert_array_equal(orc.sr_bf16(s["x"], s["bits"]), s["out"])


# --------------------------------------------------------------- GPU ------
def _zero_state(tx, params):
    return tx.init(params)


@pytest.mark.gpu
@pytest.mark.parametrize("exact", [True, False])
def test_gpu_step_f32_matches_golden(exact):
    import rollfast_amd as rf

    z = _load("step_f32")
    params = {"w": to_device(z["p0"], "f32")}
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=exact)
    state = tx.init(params)
    for t in range(1, 4):
        grads = {"w": to_device(z["grads"][t - 1], "f32")}
        params, state = rf.adamw8_step(tx, params, grads, state, stochastic=False)
        got_p = to_host(params["w"])
        if exact:
            np.testing.assert_array_equal(got_p.view(np.uint32), z[f"p{t}"].view(np.uint32))
        else:
            before = z[f"p{t - 1}"] if t > 1 else z["p0"]
            assert np.all(f32_params_close(got_p, z[f"p{t}"], before, steps=t))
        adam = state[0]
        np.testing.assert_array_equal(to_host(adam.mu["w"].values), z[f"mu{t}"])
        np.testing.assert_array_equal(to_host(adam.nu["w"].values), z[f"nu{t}"])
        np.testing.assert_array_equal(to_host(adam.mu["w"].scales).view(np.uint32), z[f"ms{t}"].view(np.uint32))
        np.testing.assert_array_equal(to_host(adam.nu["w"].scales).view(np.uint32), z[f"vs{t}"].view(np.uint32))
        if not exact:
            # keep the chain on the golden trajectory: the next step reads the params
            params = {"w": to_device(z[f"p{t}"], "f32")}


@pytest.mark.gpu
def test_gpu_step_bf16_fed_bits_matches_golden():
    import rollfast_amd as rf

    z = _load("step_bf16_sr")
    params = {"w": to_device(z["p0"], "bf16")}
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=True, exact=True)
    state = tx.init(params)
    for t in range(1, 3):
        grads = {"w": to_device(z["grads"][t - 1], "bf16")}
        bits = {0: (to_device(z["mbits"][t - 1], "u32"), to_device(z["vbits"][t - 1], "u32"),
                    to_device(z["pbits"][t - 1], "u32"))}
        params, state = rf.adamw8_step(tx, params, grads, state, key=rf.prng.PRNGKey(0), stochastic=True,
                                       random_bits=bits)
        np.testing.assert_array_equal(to_host(params["w"]), z[f"p{t}"])
        adam = state[0]
        np.testing.assert_array_equal(to_host(adam.mu["w"].values), z[f"mu{t}"])
        np.testing.assert_array_equal(to_host(adam.nu["w"].values), z[f"nu{t}"])
        np.testing.assert_array_equal(to_host(adam.mu["w"].scales), z[f"ms{t}"])
        np.testing.assert_array_equal(to_host(adam.nu["w"].scales), z[f"vs{t}"])


@pytest.mark.gpu
def test_gpu_quantize_and_sr_match_golden():
    import rollfast_amd as rf
    from rollfast_amd.utils import _stochastic_round_bf16

    z = _load("quantize")
    for name, quantizer, src in (("s", "dynamic_signed", "x"), ("u", "dynamic_unsigned", "xu"),
                                 ("y", "symmetric_int8", "x"), ("e", "dynamic_signed", "edge")):
        qb = rf.quantize_blocks(to_device(z[src], "f32"), block_size=256, quantizer=quantizer)
        np.testing.assert_array_equal(to_host(qb.values).view(np.uint8), z[f"codes_{name}"])
        np.testing.assert_array_equal(to_host(qb.scales).view(np.uint32), z[f"scales_{name}"].view(np.uint32))
    s = _load("sr_bf16")
    out = _stochastic_round_bf16(to_device(s["x"], "f32"), rf.prng.PRNGKey(0),
                                 random_bits=to_device(s["bits"], "u32"))
    np.testing.assert_array_equal(to_host(out), s["out"])
