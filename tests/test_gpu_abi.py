"""The C ABI driven directly with raw device pointers, as a foreign binding
(XLA FFI handler, cgo, a C++ trainer) would call it: the one-shot
rf_adam8_step, and a plan run on its creation-time table with
rf_adam8_plan_run, checked against the oracle; rf_adam8_plan_info reports the
launch grouping."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import bf16_bits, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu


def _leaf_and_buffers(n, seed):
    import torch

    from rollfast_amd import _lib

    rng = np.random.default_rng(seed)
    nb = -(-n // 2048)
    p = bf16_bits(gaussian(rng, (n,), 0.02))
    g = bf16_bits(gaussian(rng, (n,), 1e-2))
    bufs = {"p": to_device(p, "bf16"), "g": to_device(g, "bf16"),
            "mc": torch.full((nb * 2048,), 127, dtype=torch.uint8, device="cuda"),
            "ms": torch.ones(nb, dtype=torch.float32, device="cuda"),
            "vc": torch.zeros(nb * 2048, dtype=torch.uint8, device="cuda"),
            "vs": torch.ones(nb, dtype=torch.float32, device="cuda")}
    L = _lib.Adam8Leaf()
    L.param = bufs["p"].data_ptr()
    L.grad = bufs["g"].data_ptr()
    L.mu = bufs["mc"].data_ptr()
    L.mu_scales = bufs["ms"].data_ptr()
    L.nu = bufs["vc"].data_ptr()
    L.nu_scales = bufs["vs"].data_ptr()
    L.size = n
    L.block_size = 2048
    L.param_dtype = _lib.RF_BF16
    L.grad_dtype = _lib.RF_BF16
    L.moment_kind = _lib.RF_MOMENT_QUANTIZED
    L.flags = _lib.RF_LEAF_DECAY
    host = {"p": p.copy(), "g": g, "mc": np.full(nb * 2048, 127, np.uint8), "ms": np.ones(nb, np.float32),
            "vc": np.zeros(nb * 2048, np.uint8), "vs": np.ones(nb, np.float32)}
    return L, bufs, host


def _hparams(count):
    from rollfast_amd import _lib

    o = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=count, decay=True, apply=True)
    hp = _lib.Adam8Hparams()
    for f in ("b1", "one_minus_b1", "b2", "one_minus_b2", "bc1", "bc2", "bc1_next", "eps", "eps_root",
              "weight_decay"):
        setattr(hp, f, getattr(o, f))
    hp.nesterov_one_minus_b1 = o.nest_one_minus_b1
    hp.neg_lr = o.neg_lr
    hp.flags = _lib.RF_LR | _lib.RF_DECAY_WEAK | 128  # RF_EXACT: bit-exact params
    return hp, o


def _oracle_step(host, o, n):
    orc.adam8_leaf(o, host["p"], orc.BF16, host["g"], orc.BF16, orc.MOM_QUANT, host["mc"], host["ms"], host["vc"],
                   host["vs"], 2048)


def _compare(bufs, host):
    np.testing.assert_array_equal(to_host(bufs["p"]), host["p"])
    np.testing.assert_array_equal(to_host(bufs["mc"]), host["mc"])
    np.testing.assert_array_equal(to_host(bufs["vc"]), host["vc"])
    np.testing.assert_array_equal(to_host(bufs["ms"]).view(np.uint32), host["ms"].view(np.uint32))
    np.testing.assert_array_equal(to_host(bufs["vs"]).view(np.uint32), host["vs"].view(np.uint32))


def test_one_shot_step_through_the_abi():
    import torch

    from rollfast_amd import _lib

    n = 5 * 2048 + 77
    L, bufs, host = _leaf_and_buffers(n, 1)
    table = (_lib.Adam8Leaf * 1)(L)
    hp, o = _hparams(1)
    st = _lib.lib().rf_adam8_step(table, 1, 1, ctypes.byref(hp), _lib.stream_ptr())
    assert st == _lib.RF_OK, _lib.lib().rf_last_error()
    torch.cuda.synchronize()
    _oracle_step(host, o, n)
    _compare(bufs, host)


def test_plan_run_on_creation_table_and_info():
    import torch

    from rollfast_amd import _lib

    n = 7 * 2048
    L1, b1, h1 = _leaf_and_buffers(n, 2)
    L2, b2, h2 = _leaf_and_buffers(1000, 3)   # partial block: generic kernel
    table = (_lib.Adam8Leaf * 2)(L1, L2)
    table[1].state_index = table[1].param_index = 1
    plan = ctypes.c_void_p()
    lib = _lib.lib()
    assert lib.rf_adam8_plan_create(table, 2, 1, ctypes.byref(plan)) == _lib.RF_OK
    try:
        launches, leaves, units = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        assert lib.rf_adam8_plan_info(plan, ctypes.byref(launches), ctypes.byref(leaves), ctypes.byref(units)) == 0
        # the partial block's generic unit rides in the bf16 fast launch
        assert leaves.value == 2 and launches.value == 1 and units.value == 7 + 1
        for step in range(1, 3):
            hp, o = _hparams(step)
            assert lib.rf_adam8_plan_run(plan, ctypes.byref(hp), _lib.stream_ptr()) == _lib.RF_OK
            torch.cuda.synchronize()
            for h, n_ in ((h1, n), (h2, 1000)):
                _oracle_step(h, o, n_)
            _compare(b1, h1)
            _compare(b2, h2)
    finally:
        assert lib.rf_adam8_plan_destroy(plan) == _lib.RF_OK


@pytest.mark.parametrize("n", [1, 7, 8, 2047, 2 * 2048 + 512, 3 * 2048 + 1, 5 * 2048 + 77])
def test_partial_last_block_ignores_old_padding_codes(n):
    """A leaf's partial last block: the padding's old codes do not enter the
    new moments (quantize_blocks pads the new moments with zeros,
    adam8.py:137-141), so garbage padding codes give the oracle's codes,
    scales and params bit for bit, and the padding comes back as zero codes.
    Sizes from one element to several whole blocks plus a tail."""
    import torch

    from rollfast_amd import _lib

    L, bufs, host = _leaf_and_buffers(n, 11)
    nb = -(-n // 2048)
    rng = np.random.default_rng(5)
    pad = np.arange(n, nb * 2048)
    for key in ("mc", "vc"):
        junk = rng.integers(0, 256, pad.size, dtype=np.uint8)
        host[key][pad] = junk
        bufs[key][torch.as_tensor(pad, device="cuda")] = torch.as_tensor(junk, device="cuda")
    table = (_lib.Adam8Leaf * 1)(L)
    for step in range(1, 4):
        hp, o = _hparams(step)
        st = _lib.lib().rf_adam8_step(table, 1, 1, ctypes.byref(hp), _lib.stream_ptr())
        assert st == _lib.RF_OK, _lib.lib().rf_last_error()
        torch.cuda.synchronize()
        _oracle_step(host, o, n)
        _compare(bufs, host)
        assert (to_host(bufs["mc"])[pad] == 127).all() and (to_host(bufs["vc"])[pad] == 0).all()
