#!/usr/bin/env python
"""Write the golden fixtures of the adam8 step from the CPU oracle.

The reference (rollfast, JAX) cannot run in this environment (jax, optax and
Python >= 3.12 are absent), so the fixtures are outputs of the oracle, whose
functions are pinned independently by tests/test_oracle.py.  They freeze the
oracle's results so that any later change to it, or to the HIP path, that
moves a bit is caught against data rather than against a re-computation.

Fixtures (numpy .npz, no pickled objects):
  step_f32.npz      f32 params [4 x 2048], 3 steps of adamw8 (lr 1e-3,
                    wd 0.01, eps 1e-8), quantized moments; inputs and the
                    params / codes / scales after each step.
  step_bf16_sr.npz  bf16 params [3 x 2048 - 300] (ragged tail), 2 steps with
                    moment and param stochastic rounding fed by raw bits.
  quantize.npz      4096 mixed-magnitude f32 values with +-0, denormals,
                    +-Inf, NaN (block 256): codes and scales of the signed,
                    unsigned and symmetric quantizers.
  sr_bf16.npz       f32 -> bf16 stochastic rounding with fed bits.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

BS = 2048


def step_f32():
    rng = np.random.default_rng(100)
    n = 4 * BS
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    grads = (rng.standard_normal((3, n)) * 1e-2).astype(np.float32)
    grads[1, BS:2 * BS] = 0.0  # a block whose gradient vanishes for one step
    p = p0.copy()
    mu = np.full(n, 127, np.uint8)
    nu = np.zeros(n, np.uint8)
    ms = np.ones(4, np.float32)
    vs = np.ones(4, np.float32)
    out = {"p0": p0, "grads": grads}
    for t in range(1, 4):
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=t, decay=True, apply=True)
        orc.adam8_leaf(hp, p, orc.F32, grads[t - 1], orc.F32, orc.MOM_QUANT, mu, ms, nu, vs, BS)
        out[f"p{t}"] = p.copy()
        out[f"mu{t}"] = mu.copy()
        out[f"ms{t}"] = ms.copy()
        out[f"nu{t}"] = nu.copy()
        out[f"vs{t}"] = vs.copy()
    return out


def step_bf16_sr():
    rng = np.random.default_rng(101)
    n = 3 * BS - 300
    nb = 3
    p0 = orc.f32_to_bf16_bits((rng.standard_normal(n) * 0.02).astype(np.float32))
    grads = np.stack([orc.f32_to_bf16_bits((rng.standard_normal(n) * 1e-3).astype(np.float32)) for _ in range(2)])
    mbits = rng.integers(0, 1 << 32, size=(2, nb * BS), dtype=np.uint32)
    vbits = rng.integers(0, 1 << 32, size=(2, nb * BS), dtype=np.uint32)
    pbits = rng.integers(0, 1 << 32, size=(2, n), dtype=np.uint32)
    p = p0.copy()
    mu = np.full(nb * BS, 127, np.uint8)
    nu = np.zeros(nb * BS, np.uint8)
    ms = np.ones(nb, np.float32)
    vs = np.ones(nb, np.float32)
    out = {"p0": p0, "grads": grads, "mbits": mbits, "vbits": vbits, "pbits": pbits}
    for t in range(1, 3):
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=t, decay=True, apply=True, moment_sr=True,
                              param_sr=True)
        orc.adam8_leaf(hp, p, orc.BF16, grads[t - 1], orc.BF16, orc.MOM_QUANT, mu, ms, nu, vs, BS,
                       mu_bits=mbits[t - 1], nu_bits=vbits[t - 1], p_bits=pbits[t - 1])
        out[f"p{t}"] = p.copy()
        out[f"mu{t}"] = mu.copy()
        out[f"ms{t}"] = ms.copy()
        out[f"nu{t}"] = nu.copy()
        out[f"vs{t}"] = vs.copy()
    return out


def quantize():
    rng = np.random.default_rng(102)
    n = 4096
    mag = np.exp(rng.uniform(np.log(1e-8), np.log(1e2), n)).astype(np.float32)
    x = (mag * rng.choice([-1.0, 1.0], n)).astype(np.float32)
    x[:8] = np.array([0.0, -0.0, 1e-40, -1e-41, 1e-45, 3.0, -3.0, 0.5], np.float32)
    x[256:512] = 0.0                                  # an all-zero block: scale 1
    x[512:768] = np.float32(1e-39) * rng.standard_normal(256).astype(np.float32)  # denormal block
    edge = x.copy()
    edge[1024] = np.inf
    edge[1300] = -np.inf
    edge[1600] = np.nan
    xu = np.abs(x)
    out = {"x": x, "edge": edge, "xu": xu}
    for name, q, src in (("s", orc.Q_SIGNED, x), ("u", orc.Q_UNSIGNED, xu), ("y", orc.Q_SYMMETRIC, x),
                         ("e", orc.Q_SIGNED, edge)):
        codes, scales = orc.quantize(src, 256, q)
        out[f"codes_{name}"] = codes.reshape(-1).view(np.uint8)
        out[f"scales_{name}"] = scales
    return out


def sr_bf16():
    rng = np.random.default_rng(103)
    n = 8192
    x = (rng.standard_normal(n) * np.exp(rng.uniform(-20, 20, n))).astype(np.float32)
    x[:6] = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 3.3895314e38], np.float32)
    bits = rng.integers(0, 1 << 32, n, dtype=np.uint32)
    return {"x": x, "bits": bits, "out": orc.sr_bf16(x, bits)}


def main():
    orc.set_threads(1)
    for name, fn in (("step_f32", step_f32), ("step_bf16_sr", step_bf16_sr), ("quantize", quantize),
                     ("sr_bf16", sr_bf16)):
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
