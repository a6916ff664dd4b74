"""The C ABI driven by compiled C++ with no Python in the loop
(tests/c_host/rf_c_host_step.cpp): device buffers from the HIP runtime, a
plan over a bf16 leaf of whole blocks, a bf16 leaf with a partial last block
and an f32 leaf with f32 fallback moments, two fused adamw8 steps with the
IEEE direction, the second over new gradient buffers
(rf_adam8_plan_run_leaves).  These are the calls an XLA FFI handler makes.

The C++ host derives the step scalars itself; they must equal the oracle's
derivation bit for bit (adam8.py:322-339).  The results must equal the
oracle's two steps on the inputs the host wrote: params, codes, scales and
fallback moments bit-exact (adam8.py:304-443 with utils.py:648-708).
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "tests", "c_host", "librf_c_host_step.so")
LEAVES = [(3 * 2048, orc.BF16, True), (5000, orc.BF16, True), (1000, orc.F32, False)]


def test_cpp_host_plan_two_steps_match_oracle(tmp_path):
    import torch

    from rollfast_amd import _lib

    torch.cuda.set_device(0)
    _lib.lib()  # the product library first: the C++ host links against the same file
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: build() compiles it")
    host = ctypes.CDLL(LIB)
    host.rf_c_host_step_run.argtypes = [ctypes.c_char_p]
    host.rf_c_host_step_run.restype = ctypes.c_int
    print("[c_host] two steps through the plan entry points", flush=True)
    rc = host.rf_c_host_step_run(str(tmp_path).encode())
    assert rc == 0, f"rf_c_host_step_run returned {rc}"

    def arr(name, dtype):
        return np.fromfile(tmp_path / name, dtype=dtype)

    for step in (1, 2):
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=step, decay=True, apply=True)
        want = np.array([hp.b1, hp.one_minus_b1, hp.b2, hp.one_minus_b2, hp.bc1, hp.bc2, hp.eps, hp.eps_root,
                         hp.weight_decay, hp.neg_lr], dtype=np.float32)
        got = arr(f"hp_step{step}.bin", np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=f"step {step} scalars")

    for i, (size, pdt, quant) in enumerate(LEAVES):
        pt = np.uint16 if pdt == orc.BF16 else np.float32
        p = arr(f"p0_{i}.bin", pt).copy()
        assert p.size == size
        if quant:
            nb = (size + 2047) // 2048
            mu = np.full(nb * 2048, 127, np.uint8)
            nu = np.zeros(nb * 2048, np.uint8)
            mus = np.ones(nb, np.float32)
            nus = np.ones(nb, np.float32)
            kind = orc.MOM_QUANT
        else:
            mu = np.zeros(size, np.float32)
            nu = np.zeros(size, np.float32)
            mus = nus = None
            kind = orc.MOM_F32
        for step in (1, 2):
            hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=step, decay=True, apply=True)
            g = arr(f"g{step}_{i}.bin", pt)
            orc.adam8_leaf(hp, p, pdt, g, pdt, kind, mu, mus, nu, nus, 2048)
        where = f"leaf {i} ({size} elements)"
        np.testing.assert_array_equal(arr(f"p_{i}.bin", pt).view(np.uint16 if pt == np.uint16 else np.uint32),
                                      p.view(np.uint16 if pt == np.uint16 else np.uint32),
                                      err_msg=f"{where}: params")
        if quant:
            np.testing.assert_array_equal(arr(f"mu_{i}.bin", np.uint8), mu, err_msg=f"{where}: mu codes")
            np.testing.assert_array_equal(arr(f"nu_{i}.bin", np.uint8), nu, err_msg=f"{where}: nu codes")
            np.testing.assert_array_equal(arr(f"mus_{i}.bin", np.float32).view(np.uint32), mus.view(np.uint32),
                                          err_msg=f"{where}: mu scales")
            np.testing.assert_array_equal(arr(f"nus_{i}.bin", np.float32).view(np.uint32), nus.view(np.uint32),
                                          err_msg=f"{where}: nu scales")
        else:
            np.testing.assert_array_equal(arr(f"mu_{i}.bin", np.float32).view(np.uint32), mu.view(np.uint32),
                                          err_msg=f"{where}: mu")
            np.testing.assert_array_equal(arr(f"nu_{i}.bin", np.float32).view(np.uint32), nu.view(np.uint32),
                                          err_msg=f"{where}: nu")
