"""GPU parity of the moment-format conversions (state migration between
adamw8 and full-precision adamw states): every quantized leaf dequantizes to
the oracle's ``cb[code] * scale`` (adam8.py:190-204) and quantizes to the
oracle's codes and scales (adam8.py:113-187) bit for bit; the round trip
8-bit -> f32 -> 8-bit repeats every block whose largest element holds the
code of +1.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import bf16_bits, gaussian, to_device, to_host

pytestmark = pytest.mark.gpu

SPEC = [("a", (8, 2048), "bf16"), ("b", (3, 3000), "f32"), ("c", (700,), "bf16"), ("d", (5, 4099), "bf16")]


def _tree(seed, std):
    rng = np.random.default_rng(seed)
    dev = {}
    for name, shape, dt in SPEC:
        x = gaussian(rng, (int(np.prod(shape)),), std)
        dev[name] = to_device(bf16_bits(x) if dt == "bf16" else x, dt).reshape(shape)
    return dev


def _trained_adam8(rf, steps=3):
    import torch

    params = _tree(1, 0.02)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01)
    state = tx.init(params)
    for s in range(steps):
        params, state = rf.adamw8_step(tx, params, _tree(10 + s, 1e-2), state, stochastic=False)
    torch.cuda.synchronize()
    return params, state[0]


def test_dequantize_state_tree_matches_oracle_and_round_trips():
    import torch

    import rollfast_amd as rf

    _, st = _trained_adam8(rf)
    for field, q in (("mu", orc.Q_SIGNED), ("nu", orc.Q_UNSIGNED)):
        tree = getattr(st, field)
        f32 = rf.dequantize_state_tree(tree)
        torch.cuda.synchronize()
        for name, shape, _dt in SPEC:
            leaf = tree[name]
            got = to_host(f32[name])
            assert got.dtype == np.float32 and f32[name].shape == torch.Size(shape)
            if isinstance(leaf, rf.QuantizedBlocks):
                want = orc.dequantize(to_host(leaf.values), to_host(leaf.scales), leaf.size, leaf.block_size, q)
                np.testing.assert_array_equal(got.reshape(-1).view(np.uint32), want.view(np.uint32))
            else:
                np.testing.assert_array_equal(got.reshape(-1), to_host(leaf).reshape(-1))
        # back to 8 bits: the oracle's quantization of the dequantized values.
        # Not the identity in general: the signed codebook has +1 but no -1,
        # so a block whose absmax element is negative comes back with a
        # smaller scale.  Blocks whose absmax element is positive do repeat.
        back = rf.quantize_state_tree(f32, tree)
        torch.cuda.synchronize()
        for name, _shape, _dt in SPEC:
            a, b = tree[name], back[name]
            if isinstance(a, rf.QuantizedBlocks):
                assert isinstance(b, rf.QuantizedBlocks) and b.codebook_id == a.codebook_id
                assert (b.shape, b.size, b.block_size, b.block_layout) == (a.shape, a.size, a.block_size,
                                                                           a.block_layout)
                codes, scales = orc.quantize(to_host(f32[name]).reshape(-1), a.block_size, q)
                va = to_host(a.values).reshape(-1, a.block_size)
                vb = to_host(b.values).reshape(-1, a.block_size)
                np.testing.assert_array_equal(vb, codes.reshape(vb.shape), err_msg=f"{field} {name}")
                np.testing.assert_array_equal(to_host(b.scales).view(np.uint32), scales.view(np.uint32))
                cb = orc.codebook(q == orc.Q_SIGNED)
                top = cb[va].max(axis=1) == 1.0  # blocks holding the code of +1
                np.testing.assert_array_equal(vb[top], va[top])
                np.testing.assert_array_equal(to_host(b.scales)[top], to_host(a.scales)[top])
                if q == orc.Q_UNSIGNED:  # v >= 0: only all-zero blocks lack the code of +1
                    assert (va[~top] == 0).all()
            else:
                np.testing.assert_array_equal(to_host(b), to_host(a))


def test_state_conversions_both_ways():
    """adamw8 state -> adamw state (f32 moments) -> training continues with
    adamw; then back into the 8-bit format, equal to the oracle's
    quantization of the f32 moments."""
    import torch

    import rollfast_amd as rf

    params, st8 = _trained_adam8(rf)
    st = rf.adam_state_from_adam8(st8)
    assert isinstance(st, rf.ScaleByAdamState) and int(st.count) == 3
    np.testing.assert_array_equal(np.asarray(st.key), np.asarray(st8.key))
    tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01)
    chain_state = (st,) + tuple(tx.init(params)[1:])
    params, chain_state = rf.adamw_step(tx, params, _tree(50, 1e-2), chain_state, stochastic=False)
    torch.cuda.synchronize()
    st = chain_state[0]
    assert int(st.count) == 4
    template = rf.adamw8(learning_rate=1e-3).init(params)[0]
    back = rf.adam8_state_from_adam(st, template)
    torch.cuda.synchronize()
    assert isinstance(back, rf.ScaleByAdam8State) and int(back.count) == 4
    for field, q in (("mu", orc.Q_SIGNED), ("nu", orc.Q_UNSIGNED)):
        for name, _shape, _dt in SPEC:
            leaf = getattr(back, field)[name]
            src = to_host(getattr(st, field)[name]).reshape(-1)
            if isinstance(leaf, rf.QuantizedBlocks):
                codes, scales = orc.quantize(src, leaf.block_size, q)
                np.testing.assert_array_equal(to_host(leaf.values).reshape(-1), codes.reshape(-1),
                                              err_msg=f"{field} {name}")
                np.testing.assert_array_equal(to_host(leaf.scales).view(np.uint32), scales.view(np.uint32))
            else:
                np.testing.assert_array_equal(to_host(leaf).reshape(-1), src)
    # the converted state drives the 8-bit optimizer again
    tx8 = rf.adamw8(learning_rate=1e-3, weight_decay=0.01)
    s8 = (back,) + tuple(tx8.init(params)[1:])
    params, s8 = rf.adamw8_step(tx8, params, _tree(60, 1e-2), s8, stochastic=False)
    torch.cuda.synchronize()
    assert int(s8[0].count) == 5


def test_quantize_state_tree_stochastic_rounding_keys():
    """With stochastic rounding, leaf i uses split(key, n)[i] like the
    optimizer's store (adam8.py:644-646): equal to quantize_blocks with that
    key."""
    import torch

    import rollfast_amd as rf

    _, st8 = _trained_adam8(rf, steps=1)
    f32 = rf.dequantize_state_tree(st8.mu)
    key = rf.prng.PRNGKey(9)
    sr = rf.quantize_state_tree(f32, st8.mu, stochastic_rounding=True, key=key)
    keys = rf.prng.split(key, len(SPEC))
    for i, (name, _shape, _dt) in enumerate(SPEC):
        t = st8.mu[name]
        if not isinstance(t, rf.QuantizedBlocks):
            continue
        want = rf.quantize_blocks(f32[name], block_size=t.block_size, stochastic_rounding=True, key=keys[i])
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_host(sr[name].values), to_host(want.values))
    with pytest.raises(ValueError, match="PRNG key"):
        rf.quantize_state_tree(f32, st8.mu, stochastic_rounding=True)
