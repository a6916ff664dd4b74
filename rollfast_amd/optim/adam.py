"""AdamW with full-precision (f32) or stochastically rounded bf16 moments, on
the MI355X step kernels.

Host-side mirror of ``src/rollfast/optim/adam.py`` (rollfast): ``scale_by_adam``,
``adamw`` and ``ScaleByAdamState`` with the reference's names, argument
meanings, state pytree and errors.  The update runs in ``librfadam8.so``
through the same multi-tensor launch as ``adamw8`` with every leaf on the
unquantized ("fallback") moment path:

* first-moment EMA ``(1 - f32(b1)) * g + f32(b1) * m`` with the gradient
  weight computed in f32 (reference utils.py:327-335, :437-467); second
  moment ``(1.0 - b2) * g^2 + b2 * v`` (utils.py:470-494);
* Nesterov combination with the double-precision ``1.0 - b1``
  (adam.py:146-160);
* ``mu_dtype=bfloat16``: moments stored with stochastic rounding, keys
  ``k1, k2 = split(sr_key)`` split again per leaf (adam.py:219-222,
  utils.py:374-409);
* ``adamw`` = ``chain(scale_by_adam, add_decayed_weights, scale_by_learning_rate)``
  (adam.py:381-406), fused into the same launch.

Magma (``use_magma=True``, optim/magma.py:15-132 as adam.py:127-131,
:203-217 call it): the step runs in update-only mode (decay inside, f32
product) and also sums ``g * m'``, ``g * g`` and ``m' * m'`` per leaf over
its new first moment ``m'`` (the plan's ``magma_sums`` output); after it,
``rf_magma_scale`` turns the sums into the leaf's cosine, score and
Bernoulli mask and scales the update in place (times ``-lr`` for ``adamw``),
or ``adamw_step`` folds that factor into ``apply_updates``.
The PRNG key splits three ways (next, SR, Magma).  Magma runs without the
fused clipping, the non-finite guard and the grouped launch: those raise
``NotImplementedError`` (a ``chain``/``multi_transform`` around it still
works, one transform after the other).
"""

from __future__ import annotations

from typing import Any, Callable, NamedTuple, Optional, Union

import numpy as np

from .. import _lib, _tree, prng
from .._base import (
    EmptyState,
    GradientTransformation,
    GradientTransformationExtraArgs,
    MaskedState,
    ScaleByScheduleState,
    is_passthrough_leaf as _is_passthrough_leaf,
)
from .adam8 import (
    _Adamw8Update,
    _as_f32,
    _Config,
    _decay_mask_leaves,
    _Engine,
    _require_device_tensor,
    _torch,
    _check_sr_bits,
    canonicalize_dtype,
    decay_link_state,
)


class ScaleByAdamState(NamedTuple):
    """State for the Adam algorithm (adam.py:28-35)."""

    count: Any
    mu: Any
    nu: Any
    magma_s: Any
    key: Any


class _AdamEngine(_Engine):
    """The adam8 engine with optim/adam.py's scalars, keys and state."""

    store_sr = False  # set per instance for mu_dtype=bfloat16
    # scale_by_adam's own decay, update + wd * param, applies whenever params
    # are given, with weight 0 inside adamw (adam.py:185-201, :380-404)
    own_zero_decay = True

    @staticmethod
    def ema_weight(b1) -> np.float32:
        """``1.0 - decay32`` in f32 (utils.py:327-335)."""
        return np.float32(1.0) - _as_f32(b1)

    @staticmethod
    def split_keys(state_key):
        """``next_state_key, sr_key = split(key, 2)`` (adam.py:128-133) and
        ``k1, k2 = split(sr_key)`` for the two moment trees (adam.py:219-221)."""
        next_key, sr_key = prng.split(state_key, 2)
        k1, k2 = prng.split(sr_key, 2)
        return k1, k2, next_key

    @staticmethod
    def new_state(state, count_inc, next_key):
        return ScaleByAdamState(count=np.asarray(count_inc, dtype=np.int32), mu=state.mu, nu=state.nu,
                                magma_s=state.magma_s, key=next_key)


class _MagmaAdamEngine(_AdamEngine):
    """The adam engine with Magma's three-way key split."""

    @staticmethod
    def split_keys(state_key):
        """``next_state_key, sr_key, magma_key = split(key, 3)`` (adam.py:127-128)
        and ``k1, k2 = split(sr_key)`` for the two moment trees."""
        next_key, sr_key, _magma_key = prng.split(state_key, 3)
        k1, k2 = prng.split(sr_key, 2)
        return k1, k2, next_key


def _validate_magma_args(p: float, tau: float) -> None:
    """magma.py:8-13."""
    if not 0.0 <= p <= 1.0:
        raise ValueError(f"magma_p must be in [0, 1], got {p!r}.")
    if tau <= 0.0:
        raise ValueError(f"magma_tau must be positive, got {tau!r}.")


def _init_magma_state(params):
    """utils.py:65-70: an f32 scalar 0.5 per array leaf, on the leaf's device."""
    torch = _torch()

    def leaf(x):
        if _is_passthrough_leaf(x):
            return x
        return torch.full((), 0.5, dtype=torch.float32, device=x.device)

    return _tree.tree_map(leaf, params, is_leaf=_is_passthrough_leaf)


def _dtype_code(t) -> int:
    torch = _torch()
    code = {torch.bfloat16: _lib.RF_BF16, torch.float32: _lib.RF_F32, torch.float16: _lib.RF_F16}.get(t.dtype)
    if code is None:
        raise NotImplementedError(f"dtype {t.dtype} is not supported (float32, bfloat16 or float16)")
    return code


def _magma_step(engine, magma_p, magma_tau, updates, state, params, *, decay_mask, weight_decay, neg_lr,
                fuse_apply=None):
    """One scale_by_adam(use_magma=True) update (adam.py:123-235 with
    magma.py:15-132): the step in update-only mode, which also writes each
    leaf's Magma sums (of the raw update and the new first moment), then the
    per-leaf scaling of its f32 updates by ``neg_lr * (mask * score)``.
    ``fuse_apply=(params, key, stochastic)``: instead of scaling the
    updates, apply them to the params with the scaling folded in (the
    fused step's ``apply_updates``); returns (None, new state)."""
    torch = _torch()
    g_leaves, g_td = _tree.flatten(updates, is_leaf=_is_passthrough_leaf)
    mu_leaves = _tree.flatten_up_to(g_td, state.mu) if g_leaves else []
    s_leaves = _tree.flatten_up_to(g_td, state.magma_s) if g_leaves else []
    picked = [i for i, (g, m) in enumerate(zip(g_leaves, mu_leaves))
              if not (_is_passthrough_leaf(g) or _is_passthrough_leaf(m))]
    if not picked:
        out, new_state = engine.run(updates, state, params, apply=False, decay_mask=decay_mask,
                                    weight_decay=weight_decay, neg_lr=None)
        return out, new_state
    hold = []  # contiguous operands, alive until the launches are enqueued
    table = (_lib.MagmaLeaf * len(picked))()
    device = None
    for k, i in enumerate(picked):
        g = _require_device_tensor(g_leaves[i], "gradient").contiguous()
        m = _require_device_tensor(mu_leaves[i], "first moment").contiguous()
        if device is None:
            device = g.device
        if g.device != device or m.device != device:
            raise ValueError("all leaves of one Magma step must live on one device")
        if g.numel() != m.numel():
            raise ValueError("updates and optimizer state have different tree structures")
        hold += [g, m]
        r = table[k]
        r.grad, r.mu, r.size = g.data_ptr(), m.data_ptr(), g.numel()
        r.grad_dtype, r.mu_dtype, r.key_index = _dtype_code(g), _dtype_code(m), i
    lib = _lib.lib()
    magma_key = prng.split(prng.as_key(state.key), 3)[2]
    with torch.cuda.device(device):
        stream = _lib.stream_ptr()
        # The step's rows are the picked leaves, in order (both skip the
        # leaves whose update or first moment is None / MaskedNode).
        sums = torch.empty(3 * len(picked), dtype=torch.float64, device=device)
        out, new_state = engine.run(updates, state, params, apply=False, decay_mask=decay_mask,
                                    weight_decay=weight_decay, neg_lr=None, magma_sums=sums)
        out_leaves = _tree.flatten_up_to(g_td, out)
        for k, i in enumerate(picked):
            u = out_leaves[i]
            if not u.is_contiguous():
                raise RuntimeError("the step's updates are expected contiguous")
            table[k].updates = u.data_ptr()
        scores = torch.stack([_require_device_tensor(s_leaves[i], "magma score").reshape(()).to(
            device=device, dtype=torch.float32) for i in picked])
        lr = 1.0 if neg_lr is None else float(np.float32(neg_lr))
        factor = torch.empty(len(picked), dtype=torch.float32, device=device) if fuse_apply else None
        _lib.check(lib.rf_magma_scale(table, len(picked), sums.data_ptr(), scores.data_ptr(), float(magma_p),
                                      float(magma_tau), int(magma_key[0]), int(magma_key[1]), len(g_leaves), lr,
                                      None if factor is None else factor.data_ptr(), stream), "rf_magma_scale")
        if fuse_apply:
            _magma_apply(fuse_apply, g_td, picked, out_leaves, factor, lr, stream)
            out = None
    new_s = list(s_leaves)
    for k, i in enumerate(picked):
        new_s[i] = scores[k]
    del hold
    return out, new_state._replace(magma_s=_tree.unflatten(g_td, new_s))


def _magma_apply(fuse_apply, g_td, picked, out_leaves, factor, neg_lr, stream) -> None:
    """apply_updates (utils.py:648-708) of the unscaled updates with
    ``neg_lr * (factor[k] * u)`` per leaf (``rf_magma_apply_updates``); the
    param key of leaf i is split(key)[i], as apply_updates keys it."""
    params, key, stochastic = fuse_apply
    if stochastic and key is None:
        raise ValueError("apply_updates requires a PRNG `key` when stochastic=True. "
                         "Pass stochastic=False for deterministic rounding.")
    p_leaves = _tree.flatten_up_to(g_td, params)
    rows = (_lib.ApplyLeaf * len(picked))()
    for k, i in enumerate(picked):
        p = _require_device_tensor(p_leaves[i], "param")
        if not p.is_contiguous():
            raise ValueError("params must be contiguous (they are updated in place)")
        if p.numel() != out_leaves[i].numel():
            raise ValueError("param and update sizes differ")
        r = rows[k]
        r.param, r.updates, r.bits = p.data_ptr(), out_leaves[i].data_ptr(), None
        r.size, r.param_dtype, r.param_index = p.numel(), _dtype_code(p), i
    k0, k1 = (prng.as_key(key) if key is not None else np.zeros(2, np.uint32))[:2]
    _lib.check(_lib.lib().rf_magma_apply_updates(rows, len(picked), factor.data_ptr(), neg_lr,
                                                 1 if stochastic else 0, int(k0), int(k1), stream),
               "rf_magma_apply_updates")


def _has_nonzero_or_scheduled(value) -> bool:
    """utils.py:105-111."""
    if isinstance(value, (int, float)):
        if value < 0.0:
            raise ValueError("Scalar optimizer coefficients must be nonnegative.")
        return value != 0.0
    return True


def _zeros_like_tree(params, dtype):
    """utils.py:25-43: zeros of ``dtype`` for every array leaf (complex leaves
    would keep complex64; they are not supported by the kernels)."""
    torch = _torch()

    def zeros(x):
        if _is_passthrough_leaf(x):
            return x
        if x.dtype.is_complex:
            raise NotImplementedError("complex parameters are not supported")
        return torch.zeros(x.shape, dtype=dtype, device=x.device)

    return _tree.tree_map(zeros, params, is_leaf=_is_passthrough_leaf)


def _make_engine(b1, b2, eps, eps_root, mu_dtype, nesterov, key, exact, magma: bool = False,
                 sr_bits: str = "jax") -> _AdamEngine:
    torch = _torch()
    cfg = _Config(b1, b2, eps, eps_root, 2048, 1 << 62, torch.float32, mu_dtype, False, "shard_local", False,
                  bool(nesterov), key, bool(exact), _check_sr_bits(sr_bits))
    eng = (_MagmaAdamEngine if magma else _AdamEngine)(cfg)
    eng.store_sr = mu_dtype == torch.bfloat16
    return eng


def _canonical_mu_dtype(mu_dtype):
    torch = _torch()
    d = torch.float32 if mu_dtype is None else canonicalize_dtype(mu_dtype)
    if d not in (torch.float32, torch.bfloat16, torch.float16):
        raise NotImplementedError("mu_dtype must be float32, bfloat16 or float16")
    return d


def _adam_decay(weight_decay, weight_decay_mask, updates, state, params):
    """scale_by_adam's own decoupled decay (adam.py:185-202): (leaf mask,
    f32 decay) whenever params are given -- a zero weight included, since
    the reference adds ``0 * param`` too (NaN for a non-finite param) -- or
    (None, None) without params."""
    decays = _has_nonzero_or_scheduled(weight_decay)
    if decays and params is None:
        raise ValueError(
            "`params` must be provided to `scale_by_adam.update` when "
            "`weight_decay` is nonzero or scheduled."
        )
    if params is None:
        return None, None
    n = len(_tree.leaves(updates, is_leaf=_is_passthrough_leaf))
    decay_mask = _decay_mask_leaves(weight_decay_mask, params, n)
    # _resolve_scalar(weight_decay, state.count): a schedule sees the count
    # before the increment (adam.py:196).
    wd = weight_decay
    if callable(wd):
        wd = wd(np.asarray(state.count, dtype=np.int32))
    # update + wd * param.astype(f32) (utils.py:79-90): f32 product, so the
    # decay is passed as an array scalar (no weak bf16 typing).
    return decay_mask, np.float32(_as_f32(wd))


_MAGMA_FUSED_MSG = ("Magma is not supported with the fused global-norm clipping, the non-finite guard "
                    "or the grouped launch")


class _ScaleByAdamUpdate:
    """``scale_by_adam(...).update`` (adam.py:123-235)."""

    def __init__(self, engine: _AdamEngine, weight_decay, weight_decay_mask, magma=None):
        self.engine = engine
        self.weight_decay = weight_decay
        self.weight_decay_mask = weight_decay_mask
        self.magma = magma  # (p, tau) with use_magma=True, else None

    def __call__(self, updates, state, params=None):
        return self._step(updates, state, params, apply=False)

    def _step(self, updates, state, params, *, apply: bool, skip_nonfinite=False, finite_out=None,
              finite_host=None, clip_global_norm=None, clip_stats=None, **fused_only):
        del fused_only  # param_key, param_sr, random_bits: fused-step arguments
        if apply:
            raise TypeError("scale_by_adam has no learning rate: the fused step needs adamw(...)")
        decay_mask, wd = _adam_decay(self.weight_decay, self.weight_decay_mask, updates, state, params)
        if self.magma is not None:
            if skip_nonfinite or finite_out is not None or finite_host is not None or clip_global_norm:
                raise NotImplementedError(_MAGMA_FUSED_MSG)
            return _magma_step(self.engine, *self.magma, updates, state, params, decay_mask=decay_mask,
                               weight_decay=wd, neg_lr=None)
        return self.engine.run(updates, state, params, apply=False, decay_mask=decay_mask, weight_decay=wd,
                               neg_lr=None, skip_nonfinite=skip_nonfinite, finite_out=finite_out,
                               finite_host=finite_host, clip_global_norm=clip_global_norm, clip_stats=clip_stats)


class _AdamwMagmaUpdate:
    """``adamw(..., use_magma=True).update``: the chain scale_by_adam (decay
    inside, then Magma) -> scale_by_learning_rate (adam.py:380-404); the
    learning rate multiplies the masked update."""

    def __init__(self, engine: _AdamEngine, learning_rate, weight_decay, weight_decay_mask, magma):
        self.engine = engine
        self.learning_rate = learning_rate
        self.weight_decay = weight_decay
        self.weight_decay_mask = weight_decay_mask
        self.magma = magma
        self._lr = _Adamw8Update(engine, learning_rate, 0.0, None, False)._lr

    def __call__(self, updates, state, params=None, **extra_args):
        del extra_args
        return self._step(updates, state, params, apply=False)

    def _step(self, updates, state, params, *, apply: bool, skip_nonfinite=False, finite_out=None,
              finite_host=None, clip_global_norm=None, clip_stats=None, param_key=None, param_sr=False,
              random_bits=None):
        """``apply=True``: the step applied to the params in place with the
        Magma scaling folded into apply_updates (``param_key`` /
        ``param_sr`` are apply_updates' ``key`` / ``stochastic``)."""
        del clip_stats
        if random_bits is not None:
            raise NotImplementedError("fed random bits are not supported with Magma")
        if skip_nonfinite or finite_out is not None or finite_host is not None or clip_global_norm:
            raise NotImplementedError(_MAGMA_FUSED_MSG)
        adam_state, lr_state = state[0], state[-1]
        neg_lr, new_lr_state = self._lr(lr_state)
        decay_mask, wd = _adam_decay(self.weight_decay, self.weight_decay_mask, updates, adam_state, params)
        out, new_adam = _magma_step(self.engine, *self.magma, updates, adam_state, params, decay_mask=decay_mask,
                                    weight_decay=wd, neg_lr=neg_lr,
                                    fuse_apply=(params, param_key, param_sr) if apply else None)
        return out, (new_adam,) + tuple(state[1:-1]) + (new_lr_state,)


def scale_by_adam(
    b1=0.9,
    b2=0.999,
    eps=1e-8,
    eps_root=0.0,
    mu_dtype=None,
    *,
    weight_decay=0.0,
    weight_decay_mask: Optional[Union[Any, Callable[[Any], Any]]] = None,
    nesterov: bool = False,
    use_magma: bool = False,
    magma_p: float = 0.5,
    magma_tau: float = 2.0,
    axis_name: Optional[str] = None,
    key=None,
    exact: bool = False,
    sr_bits: str = "jax",
) -> GradientTransformation:
    """Rescale updates according to the Adam algorithm (adam.py:38-235).
    ``exact`` (extension): IEEE division and square root in the direction.
    ``sr_bits`` (extension): the bit source of bf16 moment storage and of
    the fused step's param rounding, "jax" or "packed" (as for
    scale_by_adam8); Magma keeps "jax".  ``axis_name`` names a collective
    axis of the reference's sharded runs and has no effect on one device."""
    del axis_name
    if use_magma:
        _validate_magma_args(magma_p, magma_tau)
        if _check_sr_bits(sr_bits) != "jax":
            raise NotImplementedError("Magma draws its stochastic rounding from the jax stream only")
    _has_nonzero_or_scheduled(weight_decay)
    mu = _canonical_mu_dtype(mu_dtype)
    engine = _make_engine(b1, b2, eps, eps_root, mu, nesterov, key, exact, magma=use_magma, sr_bits=sr_bits)

    def init_fn(params):
        return ScaleByAdamState(count=np.zeros((), dtype=np.int32), mu=_zeros_like_tree(params, mu),
                                nu=_zeros_like_tree(params, mu),
                                magma_s=_init_magma_state(params) if use_magma else (), key=prng.fresh_key(key))

    magma = (float(magma_p), float(magma_tau)) if use_magma else None
    return GradientTransformation(init_fn, _ScaleByAdamUpdate(engine, weight_decay, weight_decay_mask, magma))


def adamw(
    learning_rate,
    b1=0.9,
    b2=0.999,
    eps=1e-8,
    eps_root=0.0,
    mu_dtype=None,
    weight_decay=1e-4,
    weight_decay_mask: Optional[Union[Any, Callable[[Any], Any]]] = None,
    *,
    nesterov: bool = False,
    use_magma: bool = False,
    magma_p: float = 0.5,
    magma_tau: float = 2.0,
    axis_name: Optional[str] = None,
    key=None,
    exact: bool = False,
    sr_bits: str = "jax",
) -> GradientTransformationExtraArgs:
    """Adam with decoupled weight decay (adam.py:238-406): the optax chain
    ``scale_by_adam -> add_decayed_weights -> scale_by_learning_rate`` in one
    launch.  The state is the chain's tuple ``(ScaleByAdamState,
    add_decayed_weights state?, lr state)``."""
    if use_magma:
        # scale_by_adam(weight_decay, use_magma) -> scale_by_learning_rate
        inner = scale_by_adam(b1=b1, b2=b2, eps=eps, eps_root=eps_root, mu_dtype=mu_dtype,
                              weight_decay=weight_decay, weight_decay_mask=weight_decay_mask, nesterov=nesterov,
                              use_magma=True, magma_p=magma_p, magma_tau=magma_tau, axis_name=axis_name, key=key,
                              exact=exact, sr_bits=sr_bits)

        def magma_init(params):
            lr_state = (ScaleByScheduleState(count=np.zeros((), dtype=np.int32)) if callable(learning_rate)
                        else EmptyState())
            return (inner.init(params), lr_state)

        return GradientTransformationExtraArgs(
            magma_init, _AdamwMagmaUpdate(inner.update.engine, learning_rate, weight_decay, weight_decay_mask,
                                          inner.update.magma))
    inner = scale_by_adam(b1=b1, b2=b2, eps=eps, eps_root=eps_root, mu_dtype=mu_dtype, nesterov=nesterov,
                          axis_name=axis_name, key=key, exact=exact, magma_p=magma_p, magma_tau=magma_tau,
                          sr_bits=sr_bits)
    wd_nonzero = _has_nonzero_or_scheduled(weight_decay)
    engine = inner.update.engine

    def init_fn(params):
        states = [inner.init(params)]
        if wd_nonzero:
            states.append(decay_link_state(weight_decay, weight_decay_mask))
        if callable(learning_rate):
            states.append(ScaleByScheduleState(count=np.zeros((), dtype=np.int32)))
        else:
            states.append(EmptyState())
        return tuple(states)

    return GradientTransformationExtraArgs(
        init_fn, _Adamw8Update(engine, learning_rate, weight_decay, weight_decay_mask, wd_nonzero))


def adamw_step(tx, params, grads, state, key=None, stochastic: bool = True, *, random_bits=None,
               clip_global_norm=None, clip_stats=None):
    """Fused ``tx.update`` + ``rollfast.apply_updates`` for ``tx = adamw(...)``
    (one HBM pass; no reference counterpart).  ``random_bits`` (testing):
    ``{leaf_index: (mu_bits, nu_bits, param_bits)}`` raw uint32 words that
    replace the in-kernel bits of the bf16 moment storage and the param SR.
    ``clip_global_norm`` / ``clip_stats``: fused global-norm clipping, as for
    ``adamw8_step``."""
    from .adam8 import adamw8_step

    if isinstance(tx.update, _AdamwMagmaUpdate):
        # tx.update then apply_updates (utils.py:648-708), with Magma's
        # per-leaf scaling folded into the apply pass
        if random_bits is not None or clip_global_norm is not None:
            raise NotImplementedError(_MAGMA_FUSED_MSG)
        if stochastic and key is None:
            raise ValueError("apply_updates requires a PRNG `key` when stochastic=True. "
                             "Pass stochastic=False for deterministic rounding.")
        _out, new_state = tx.update._step(grads, state, params, apply=True, param_key=key, param_sr=stochastic)
        return params, new_state
    if isinstance(tx.update, _ScaleByAdamUpdate) or (isinstance(tx.update, _Adamw8Update)
                                                     and not isinstance(tx.update.engine, _AdamEngine)):
        raise TypeError("adamw_step needs a transformation built by adamw(...) or a composition of them "
                        "(apply_if_finite, chain with clip_by_global_norm, multi_transform)")
    return adamw8_step(tx, params, grads, state, key=key, stochastic=stochastic, random_bits=random_bits,
                       clip_global_norm=clip_global_norm, clip_stats=clip_stats)


__all__ = ("ScaleByAdamState", "adamw", "adamw_step", "scale_by_adam")
