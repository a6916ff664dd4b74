"""Empty (zero-size) leaves beside real ones, through every mode of the step.

JAX arrays of size 0 are ordinary pytree leaves for rollfast's optimizers
(adam8.py:572-630 gives them fallback moments, since size < min_size; the
update of an empty array is empty).  Their torch tensors may carry null data
pointers; the plan must accept them, launch nothing for them and leave the
other leaves' results bit for bit what they are without the empty leaf
(round-to-nearest-even params and moments: no per-leaf keys involved)."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _trees(with_empty: bool):
    import torch

    g = torch.Generator(device="cpu").manual_seed(5)
    w = (torch.randn(5000, generator=g) * 0.02).to("cuda", torch.bfloat16)
    gw = (torch.randn(5000, generator=g) * 1e-3).to("cuda", torch.bfloat16)
    params, grads = {"w": w}, {"w": gw}
    if with_empty:
        params["a_empty"] = torch.zeros(0, dtype=torch.bfloat16, device="cuda")
        grads["a_empty"] = torch.zeros(0, dtype=torch.bfloat16, device="cuda")
    return params, grads


@pytest.mark.parametrize("opt", ["adamw8", "adamw"])
def test_empty_leaf_fused_and_update_only(opt):
    import torch

    import rollfast_amd as rf
    from tests._helpers import to_host

    results = {}
    for with_empty in (False, True):
        params, grads = _trees(with_empty)
        tx = (rf.adamw8(learning_rate=1e-3, stochastic_rounding=False) if opt == "adamw8"
              else rf.adamw(learning_rate=1e-3))
        step = rf.adamw8_step if opt == "adamw8" else rf.adamw_step
        state = tx.init(params)
        for _ in range(3):
            params, state = step(tx, params, grads, state, key=rf.prng.PRNGKey(1), stochastic=False)
        updates, _ = tx.update(grads, state, params)
        applied = rf.apply_updates(params, updates, stochastic=False)
        torch.cuda.synchronize()
        if with_empty:
            assert params["a_empty"].numel() == 0 and updates["a_empty"].numel() == 0
            assert applied["a_empty"].numel() == 0
        results[with_empty] = (to_host(params["w"].view(torch.int16)).tobytes(),
                               to_host(updates["w"]).tobytes(),
                               to_host(applied["w"].view(torch.int16)).tobytes())
    assert results[True] == results[False]
    assert np.frombuffer(results[True][1], np.float32).any()
