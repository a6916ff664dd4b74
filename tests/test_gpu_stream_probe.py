"""The fused step's stream probe (rf_adam8_plan_stream_probe, diagnostics):
it moves the step's bytes over the plan's full-block work lists and leaves
every buffer as it found it -- params, grads, codes and scales byte for byte,
f32 and 16-bit stored scales alike -- and counts the blocks it moved."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_stream_probe_leaves_state_unchanged_and_counts_blocks():
    import torch

    import rollfast_amd as rf
    from rollfast_amd import _lib

    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    shapes = {"a": (64, 2048), "b": (3, 4096), "c": (5000,), "d": (100,), "e": (8, 2048)}
    dtypes = {"a": torch.bfloat16, "b": torch.float32, "c": torch.bfloat16, "d": torch.bfloat16, "e": torch.bfloat16}
    params = {k: (torch.randn(s, generator=gen, device="cuda") * 0.02).to(dtypes[k]) for k, s in shapes.items()}
    grads = {k: (torch.randn(s, generator=gen, device="cuda") * 1e-3).to(dtypes[k]) for k, s in shapes.items()}
    probes = {}
    for scale_dtype in (None, torch.bfloat16):
        tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, scale_dtype=scale_dtype)
        state = tx.init(params)
        params, state = rf.adamw8_step(tx, params, grads, state, stochastic=False)  # builds the plan
        torch.cuda.synchronize()

        def snap():
            out = [t.clone() for t in params.values()] + [t.clone() for t in grads.values()]
            for tree in (state[0].mu, state[0].nu):
                for k in sorted(tree):
                    q = tree[k]
                    out += [q.values.clone(), q.scales.clone()] if isinstance(q, rf.QuantizedBlocks) else [q.clone()]
            return out

        before = snap()
        plan = tx.update.engine._last["plan"]
        print(f"[probe] scale dtype {scale_dtype}", flush=True)
        blocks = plan.stream_probe(_lib.stream_ptr())
        blocks2 = plan.stream_probe(_lib.stream_ptr())
        torch.cuda.synchronize()
        after = snap()
        for i, (x, y) in enumerate(zip(before, after)):
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), f"buffer {i} changed by the probe"
        # full 2048-blocks of the quantized leaves: a 64, b 6, c 2 (5000 =
        # 2 blocks + a partial one, left to the generic kernel), e 8; d has
        # fallback moments
        assert blocks == blocks2 == 64 + 6 + 2 + 8
        probes[scale_dtype] = blocks
    assert len(probes) == 2


def test_stream_probe_refuses_update_only_plans():
    import ctypes

    import torch

    from rollfast_amd import _lib

    lib = _lib.lib()
    p = torch.zeros(4096, device="cuda")
    g = torch.zeros(4096, device="cuda")
    u = torch.zeros(4096, device="cuda")
    mc = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    vc = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    ms = torch.ones(2, device="cuda")
    vs = torch.ones(2, device="cuda")
    t = (_lib.Adam8Leaf * 1)()
    L = t[0]
    L.param, L.grad, L.updates = p.data_ptr(), g.data_ptr(), u.data_ptr()
    L.mu, L.nu, L.mu_scales, L.nu_scales = mc.data_ptr(), vc.data_ptr(), ms.data_ptr(), vs.data_ptr()
    L.size, L.block_size = 4096, 2048
    L.param_dtype = L.grad_dtype = _lib.RF_F32
    L.moment_kind = _lib.RF_MOMENT_QUANTIZED
    h = ctypes.c_void_p()
    assert lib.rf_adam8_plan_create(t, 1, 0, ctypes.byref(h)) == _lib.RF_OK, lib.rf_last_error()
    try:
        n = ctypes.c_int64(-1)
        assert lib.rf_adam8_plan_stream_probe(h, _lib.stream_ptr(), ctypes.byref(n)) == _lib.RF_ERR_UNSUPPORTED
        assert n.value == -1
    finally:
        assert lib.rf_adam8_plan_destroy(h) == _lib.RF_OK
    assert np.isfinite(float(p.sum()))
