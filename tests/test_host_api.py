"""Host side of the adam8 API (no GPU): pytree order, PRNG key streams,
state construction and metadata, byte accounting, signatures and the
reference's error behaviour.  Anything that would run a kernel is checked
to refuse host tensors instead of falling back to a CPU path."""

from __future__ import annotations

import inspect
from typing import NamedTuple

import numpy as np
import pytest
import torch

import rollfast_amd as rf
from oracle import oracle as orc
from rollfast_amd import _tree, prng
from rollfast_amd.optim import adam8 as A


# ------------------------------------------------------------------ trees --
class Pair(NamedTuple):
    a: object
    b: object


def test_tree_flatten_order_matches_jax_conventions():
    """dict keys sorted, sequences in order, None has no leaves, namedtuples
    by field order (jax.tree_util flatten order)."""
    tree = {"z": 1, "a": [2, (3, None)], "m": Pair(b=5, a=4), "n": None}
    leaves, td = _tree.flatten(tree)
    assert leaves == [2, 3, 4, 5, 1]
    back = _tree.unflatten(td, [10 * x for x in leaves])
    assert back == {"z": 10, "a": [20, (30, None)], "m": Pair(a=40, b=50), "n": None}
    assert td.num_leaves == 5


def test_tree_flatten_up_to_and_map():
    params = {"w": 1, "b": 2}
    _, td = _tree.flatten(params)
    assert _tree.flatten_up_to(td, {"w": [1, 2], "b": (3,)}) == [(3,), [1, 2]]
    assert _tree.tree_map(lambda x, y: x + y, params, {"w": 10, "b": 20}) == {"w": 11, "b": 22}


def test_quantized_blocks_is_a_node_with_static_aux():
    qb = A.QuantizedBlocks(values="V", scales="S", shape=(3,), size=3, block_size=2)
    leaves, td = _tree.flatten({"m": qb})
    assert leaves == ["V", "S"]
    back = _tree.unflatten(td, ["V2", "S2"])["m"]
    assert isinstance(back, A.QuantizedBlocks)
    assert (back.values, back.scales, back.shape, back.size, back.block_size) == ("V2", "S2", (3,), 3, 2)


# ------------------------------------------------------------------- PRNG --
def test_prng_key_and_streams_match_oracle():
    assert prng.PRNGKey(0).tolist() == [0, 0]
    assert prng.PRNGKey(42).tolist() == [0, 42]
    assert prng.PRNGKey(-1).tolist() == [0, 0xFFFFFFFF]
    key = np.array([0x13198A2E, 0x03707344], np.uint32)
    np.testing.assert_array_equal(prng.split(key, 7), orc.split(tuple(key), 7))
    np.testing.assert_array_equal(prng.bits(key, 1000, offset=(1 << 32) - 500),
                                  orc.random_bits(tuple(key), 1000, offset=(1 << 32) - 500))
    y = prng.threefry2x32(np.array([0, 0], np.uint32), np.uint32(0), np.uint32(0))
    assert (int(y[0]), int(y[1])) == (0x6B200159, 0x99BA4EFE)
    assert prng.fresh_key(None).tolist() == [0, 42]
    # JAX's printed split(PRNGKey(0)) in the partitionable layout
    assert prng.split(prng.PRNGKey(0), 2).tolist() == [[1797259609, 2579123966], [928981903, 3453687069]]


def test_fold_in_group_keys():
    """jax.random.fold_in (the fine-tune builders' per-group adamw8 keys,
    finetune/builders.py:1582): the seed pair [0, data] hashed as one
    Threefry counter.  fold_in(PRNGKey(0), 0) is therefore the Random123 zero
    vector, and fold_in(k, i) is row i of the partitionable split(k, n) (the
    published split(PRNGKey(0)) rows for i = 0, 1).  A seed pair in the other
    order ([data, 0]) or the legacy split layout fails these."""
    assert prng.fold_in(prng.PRNGKey(0), 0).tolist() == [0x6B200159, 0x99BA4EFE]
    assert prng.fold_in(prng.PRNGKey(0), 1).tolist() == [928981903, 3453687069]
    key = np.array([0x13198A2E, 0x03707344], np.uint32)
    rows = orc.split(tuple(key), 40)
    for i in (0, 1, 7, 39):
        assert prng.fold_in(key, i).tolist() == rows[i].tolist()
    big = (1 << 32) - 1
    assert prng.fold_in(key, big).tolist() == list(orc.threefry2x32(tuple(int(k) for k in key), (0, big)))
    for bad in (-1, 1 << 32):
        with pytest.raises(OverflowError):
            prng.fold_in(key, bad)
    # a group key feeds adamw8(key=...) like any other key
    tx = rf.adamw8(learning_rate=1e-3, key=prng.fold_in(prng.PRNGKey(7), 2))
    assert tx is not None


# ------------------------------------------------------- state / metadata --
def _cpu_params():
    return {
        "w": torch.linspace(-1.0, 1.0, 4096).reshape(64, 64),
        "b": torch.zeros(100),
        "h": torch.zeros(3000, dtype=torch.bfloat16),
        "i": torch.zeros(5000, dtype=torch.int32),
        "none": None,
    }


def test_scale_by_adam8_init_structure():
    """tests/test_adam8.py:87-118 plus _init_moment_leaf (adam8.py:605-630):
    signed mu / unsigned nu codebooks, uint8 codes at the zero code, unit
    scales, fallback zeros for small or integer leaves, None passes through."""
    tx = rf.scale_by_adam8(block_size=256, min_size=1, stochastic_rounding=False)
    st = tx.init(_cpu_params())
    assert isinstance(st, rf.ScaleByAdam8State)
    assert int(st.count) == 0 and st.count.dtype == np.int32
    assert st.key.dtype == np.uint32 and st.key.shape == (2,)
    # next key of split(PRNGKey(42), 3) (adam8.py:274)
    np.testing.assert_array_equal(st.key, prng.split(prng.PRNGKey(42), 3)[2])
    for tree, cid, zero in ((st.mu, rf.DYNAMIC_SIGNED_CODEBOOK_ID, 127), (st.nu, rf.DYNAMIC_UNSIGNED_CODEBOOK_ID, 0)):
        q = tree["w"]
        assert isinstance(q, rf.QuantizedBlocks)
        assert q.codebook_id == cid and q.zero_point == zero and (q.qmin, q.qmax) == (0, 255)
        assert q.values.dtype == torch.uint8 and tuple(q.values.shape) == (16, 256)
        assert bool(torch.all(q.values == zero)) and bool(torch.all(q.scales == 1.0))
        assert q.shape == (64, 64) and q.size == 4096 and q.block_size == 256
        assert isinstance(tree["h"], rf.QuantizedBlocks) and tuple(tree["h"].values.shape) == (12, 256)
        assert tree["i"].dtype == torch.float32 and tree["i"].shape == (5000,)  # not inexact: fallback
        assert tree["none"] is None
    md = st.mu["w"].metadata()
    assert md["quantizer"] == "blockwise_dynamic_signed_8bit"
    assert md["block_layout"] == "shard_local"
    assert md["values_dtype"] == "uint8" and md["scale_dtype"] == "float32"


def test_min_size_and_fallback_dtype():
    tx = rf.scale_by_adam8(min_size=4096, fallback_dtype=torch.bfloat16)
    st = tx.init({"small": torch.zeros(4095), "big": torch.zeros(4096)})
    assert st.mu["small"].dtype == torch.bfloat16
    assert isinstance(st.mu["big"], rf.QuantizedBlocks)
    st = rf.scale_by_adam8(quantize=False).init({"big": torch.zeros(8192)})
    assert st.mu["big"].dtype == torch.float32


def test_weight_decay_schedule_state():
    """A weight-decay schedule gives the chain's decay link a step count
    (0 at init, masked when a mask is given); a scalar keeps it empty."""
    sched = lambda c: 0.01 * (c + 1)  # noqa: E731
    p = _cpu_params()
    st = rf.adamw8(learning_rate=1e-3, weight_decay=sched).init(p)
    assert len(st) == 3 and int(st[1].count) == 0 and type(st[1]).__name__ == "ScaleByScheduleState"
    st = rf.adamw8(learning_rate=1e-3, weight_decay=sched, weight_decay_mask={k: True for k in p}).init(p)
    assert type(st[1]).__name__ == "MaskedState" and int(st[1].inner_state.count) == 0
    st = rf.adamw(learning_rate=1e-3, weight_decay=sched).init({"w": torch.zeros(8, 8)})
    assert int(st[1].count) == 0
    st = rf.adamw8(learning_rate=1e-3, weight_decay=0.01).init(p)
    assert type(st[1]).__name__ == "EmptyState"


def test_adamw8_state_tuple_layout():
    """optax chain state: (ScaleByAdam8State, add_decayed_weights?, lr)."""
    st = rf.adamw8(1e-3).init({"w": torch.zeros(8)})
    assert len(st) == 3 and isinstance(st[0], rf.ScaleByAdam8State)
    st = rf.adamw8(1e-3, weight_decay=0.0).init({"w": torch.zeros(8)})
    assert len(st) == 2
    st = rf.adamw8(lambda c: 1e-3, weight_decay=0.01, weight_decay_mask={"w": True}).init({"w": torch.zeros(8)})
    assert len(st) == 3 and int(st[2].count) == 0


def test_byte_accounting_known_answers():
    """benchmarks/optimizer_state/adamw8.py:15-19 shapes (w0, w1 4096x64 f32,
    bias 1024 f32): adamw8 state 1,058,828 B; unquantized 4,202,508 B
    (adam8.py:207-240)."""
    params = {"w0": torch.zeros(4096, 64), "w1": torch.zeros(4096, 64), "bias": torch.zeros(1024)}
    st = rf.adamw8(1e-3, weight_decay=0.01).init(params)
    assert rf.tree_state_nbytes(st) == 1_058_828
    st = rf.adamw8(1e-3, weight_decay=0.01, quantize=False).init(params)
    assert rf.tree_state_nbytes(st) == 4_202_508
    assert rf.estimate_quantized_moment_bytes(4096 * 64) == 262_144 + 128 * 4
    assert rf.estimate_quantized_moment_bytes(0) == 0
    assert rf.estimate_quantized_moment_bytes(1) == 2048 + 4


# ------------------------------------------------------------- signatures --
def test_adamw8_signature_exposes_quantized_state_controls():
    """tests/compat/test_optimizer_signatures.py:68-83."""
    sig = inspect.signature(rf.adamw8)
    for name in ("learning_rate", "b1", "b2", "eps", "weight_decay", "block_size", "min_size", "scale_dtype",
                 "fallback_dtype", "stochastic_rounding"):
        assert name in sig.parameters
    defaults = {k: v.default for k, v in sig.parameters.items()}
    assert defaults["b1"] == 0.9 and defaults["b2"] == 0.999 and defaults["eps"] == 1e-8
    assert defaults["weight_decay"] == 1e-4 and defaults["block_size"] == 2048 and defaults["min_size"] == 4096
    sig = inspect.signature(rf.apply_updates)
    assert list(sig.parameters)[:4] == ["params", "updates", "key", "stochastic"]
    assert sig.parameters["stochastic"].default is True


# ----------------------------------------------------------------- errors --
def test_reference_errors():
    with pytest.raises(NotImplementedError, match="Magma"):
        rf.adamw8(1e-3, use_magma=True)
    with pytest.raises(ValueError, match="block_size"):
        rf.scale_by_adam8(block_size=0)
    with pytest.raises(ValueError, match="block_layout"):
        rf.scale_by_adam8(block_layout="global")
    with pytest.raises(ValueError, match="PRNG `key`"):
        rf.apply_updates({"w": torch.zeros(2)}, {"w": torch.zeros(2)}, key=None, stochastic=True)
    with pytest.raises(ValueError, match="quantizer"):
        rf.quantize_blocks(torch.zeros(4), quantizer="int4")
    with pytest.raises(ValueError, match="key"):
        rf.quantize_blocks(torch.zeros(4), stochastic_rounding=True)


def test_product_path_refuses_host_tensors():
    """No CPU fallback: every kernel entry refuses tensors off the GPU."""
    with pytest.raises(ValueError, match="ROCm device"):
        rf.quantize_blocks(torch.zeros(4096))
    with pytest.raises(ValueError, match="ROCm device"):
        rf.apply_updates({"w": torch.zeros(2)}, {"w": torch.zeros(2)}, stochastic=False)
    tx = rf.adamw8(1e-3)
    params = {"w": torch.zeros(4096)}
    st = tx.init(params)
    with pytest.raises(ValueError, match="ROCm device"):
        tx.update({"w": torch.zeros(4096)}, st, params)
    with pytest.raises(ValueError, match="ROCm device"):
        rf.adamw8_step(tx, params, {"w": torch.zeros(4096)}, st, stochastic=False)


def test_tree_ordered_dict_keeps_insertion_order():
    from collections import OrderedDict

    tree = OrderedDict([("z", 1), ("a", 2)])
    leaves, td = _tree.flatten(tree)
    assert leaves == [1, 2]
    back = _tree.unflatten(td, [3, 4])
    assert isinstance(back, OrderedDict) and list(back.items()) == [("z", 3), ("a", 4)]
    assert _tree.flatten_up_to(td, OrderedDict([("z", "x"), ("a", "y")])) == ["x", "y"]
    with pytest.raises(ValueError):
        _tree.flatten_up_to(td, OrderedDict([("a", "y"), ("z", "x")]))


def test_clip_by_global_norm_construction():
    with pytest.raises(ValueError, match="max_norm must be positive"):
        rf.clip_by_global_norm(0.0)
    st = rf.clip_by_global_norm(1.0).init({"w": torch.zeros(2)})
    assert int(st.count) == 0
    with pytest.raises(ValueError, match="ROCm device"):
        rf.clip_by_global_norm(1.0).update({"w": torch.zeros(2)}, st)


def test_apply_if_finite_construction_and_state():
    tx = rf.apply_if_finite(rf.adamw8(1e-3, weight_decay=0.01), 2)
    st = tx.init({"w": torch.zeros(8)})
    assert isinstance(st, rf.ApplyIfFiniteState)
    assert st._fields == ("notfinite_count", "last_finite", "total_notfinite", "inner_state")
    assert int(st.notfinite_count) == 0 and bool(st.last_finite) and int(st.total_notfinite) == 0
    assert st.notfinite_count.dtype == np.int32 and st.last_finite.dtype == np.bool_
    assert isinstance(st.inner_state, tuple) and isinstance(st.inner_state[0], rf.ScaleByAdam8State)
    with pytest.raises(NotImplementedError, match="apply_if_finite wraps"):
        rf.apply_if_finite(rf.clip_by_global_norm(1.0), 1)
    # no CPU fallback behind the guard either
    with pytest.raises(ValueError, match="ROCm device"):
        tx.update({"w": torch.zeros(8)}, st, {"w": torch.zeros(8)})
    txg = rf.apply_if_finite(rf.scale_by_adam8(), 1)
    with pytest.raises(TypeError, match="adamw8"):
        rf.adamw8_step(txg, {"w": torch.zeros(8)}, {"w": torch.zeros(8)}, txg.init({"w": torch.zeros(8)}),
                       stochastic=False)


def test_optax_combinators_state_layout():
    params = {"a": torch.zeros(8192), "b": torch.zeros(16), "c": torch.zeros(4)}
    labels = {"a": "q", "b": "f", "c": "f"}
    tx = rf.multi_transform({"q": rf.adamw8(1e-3), "f": rf.adamw(1e-3)}, labels)
    st = tx.init(params)
    assert isinstance(st, rf.MultiTransformState) and list(st.inner_states) == ["q", "f"]
    q = st.inner_states["q"]
    assert isinstance(q, rf.MaskedState)
    assert isinstance(q.inner_state[0].mu["a"], rf.QuantizedBlocks)
    assert isinstance(q.inner_state[0].mu["b"], rf.MaskedNode) and isinstance(q.inner_state[0].mu["c"], rf.MaskedNode)
    f = st.inner_states["f"].inner_state[0]
    assert isinstance(f, rf.ScaleByAdamState) and isinstance(f.mu["a"], rf.MaskedNode) and f.mu["b"].dtype == torch.float32
    with pytest.raises(ValueError, match="no corresponding transformation"):
        rf.multi_transform({"q": rf.adamw8(1e-3)}, labels).init(params)
    # labels may be a callable of the params
    st2 = rf.multi_transform({"q": rf.adamw8(1e-3), "f": rf.adamw(1e-3)}, lambda p: labels).init(params)
    assert list(st2.inner_states) == ["q", "f"]
    ch = rf.chain(rf.clip_by_global_norm(1.0), tx)
    cst = ch.init(params)
    assert isinstance(cst, tuple) and len(cst) == 2 and int(cst[0].count) == 0
    m = rf.masked(rf.adamw8(1e-3), {"a": True, "b": False, "c": False}).init(params)
    assert isinstance(m, rf.MaskedState) and isinstance(m.inner_state[0].mu["b"], rf.MaskedNode)
    # no CPU fallback behind the combinators
    with pytest.raises(ValueError, match="ROCm device"):
        tx.update(params, st, params)
    with pytest.raises(ValueError, match="ROCm device"):
        rf.adamw8_step(rf.apply_if_finite(ch, 1), params, params, rf.apply_if_finite(ch, 1).init(params),
                       stochastic=False)


def test_state_conversions_refuse_host_tensors():
    st = rf.adamw8(1e-3).init({"w": torch.zeros(8192), "b": torch.zeros(4)})[0]
    with pytest.raises(ValueError, match="ROCm device"):
        rf.dequantize_state_tree(st.mu)
    with pytest.raises(ValueError, match="PRNG key"):
        rf.quantize_state_tree({"w": torch.zeros(8192), "b": torch.zeros(4)}, st.mu, stochastic_rounding=True)
    with pytest.raises(ValueError, match="ROCm device"):
        rf.quantize_state_tree({"w": torch.zeros(8192), "b": torch.zeros(4)}, st.mu)


def test_native_host_walk_matches_python_flatten():
    """The native fast path walks (grads, mu, nu, params) in the order of
    rollfast_amd._tree: dicts by sorted keys, lists and tuples in order,
    None and MaskedNode as grads leaves; anything else is left to Python."""
    from rollfast_amd import _lib

    host = _lib.pyhost()
    t = [torch.zeros(i + 1) for i in range(6)]
    g = {"b": [t[0], (t[1], None)], "a": {"y": t[2], "x": rf.MaskedNode()}, "c": t[3]}
    m = {"b": ["m0", ("m1", "m2")], "a": {"y": "m3", "x": "m4"}, "c": "m5"}
    v = {"b": ["v0", ("v1", "v2")], "a": {"y": "v3", "x": "v4"}, "c": "v5"}
    p = {"b": ["p0", ("p1", "p2")], "a": {"y": "p3", "x": "p4"}, "c": "p5"}
    lg, lm, lv, lp = host.gather(g, m, v, p)
    want_g, td = _tree.flatten(g, is_leaf=lambda x: x is None or isinstance(x, rf.MaskedNode))
    assert [id(x) for x in lg] == [id(x) for x in want_g]
    assert lm == _tree.flatten_up_to(td, m) and lv == _tree.flatten_up_to(td, v) and lp == _tree.flatten_up_to(td, p)
    assert host.gather(g, m, v, None)[3] is None
    # structure mismatches and containers left to the Python walk
    assert host.gather(g, {**m, "d": 1}, v, p) is None
    assert host.gather({"k": (t[0],)}, {"k": ["x"]}, {"k": ["y"]}, None) is None

    class NT(NamedTuple):
        a: object

    assert host.gather(NT(t[0]), NT(1), NT(2), None) is None
    assert host.gather({1: t[0], "a": t[1]}, {1: 0, "a": 0}, {1: 0, "a": 0}, None) is None  # keys do not sort
    # refresh refuses host tensors (the caller then rebuilds the table)
    assert host.refresh([t[0]], ["m"], ["v"], None, [], 0, 0) is False


# ----------------------------------------------------------------- Magma --
def test_magma_construction_and_state():
    """scale_by_adam / adamw with use_magma=True (optim/adam.py:95-119,
    :380-404): argument checks of magma.py:8-13, a 0.5 f32 score per array
    leaf (utils.py:65-70; None and MaskedNode leaves kept), and adamw's chain
    state without an add_decayed_weights entry."""
    with pytest.raises(ValueError, match="magma_p"):
        rf.scale_by_adam(use_magma=True, magma_p=1.1)
    with pytest.raises(ValueError, match="magma_tau"):
        rf.scale_by_adam(use_magma=True, magma_tau=0.0)
    with pytest.raises(ValueError, match="magma_p"):
        rf.adamw(1e-3, use_magma=True, magma_p=-0.1)
    params = {"w": torch.zeros(3, 2), "b": None, "m": rf.MaskedNode()}
    st = rf.scale_by_adam(use_magma=True).init(params)
    assert st.magma_s["b"] is None and isinstance(st.magma_s["m"], rf.MaskedNode)
    s = st.magma_s["w"]
    assert s.shape == () and s.dtype == torch.float32 and float(s) == 0.5
    assert rf.scale_by_adam().init(params).magma_s == ()
    ast = rf.adamw(1e-3, weight_decay=0.1, use_magma=True).init(params)
    assert len(ast) == 2 and isinstance(ast[0], rf.ScaleByAdamState) and isinstance(ast[1], rf.EmptyState)
    assert len(rf.adamw(1e-3, weight_decay=0.1).init(params)) == 3


def test_magma_refuses_host_tensors():
    tx = rf.scale_by_adam(use_magma=True)
    params = {"w": torch.zeros(4)}
    with pytest.raises((TypeError, ValueError)):
        tx.update({"w": torch.ones(4)}, tx.init(params), params)
