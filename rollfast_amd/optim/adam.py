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

Magma (``use_magma=True``) is not implemented in rollfast_amd and raises
``NotImplementedError``.
"""

from __future__ import annotations

from typing import Any, Callable, NamedTuple, Optional, Union

import numpy as np

from .. import _tree, prng
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
    _torch,
    canonicalize_dtype,
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


def _make_engine(b1, b2, eps, eps_root, mu_dtype, nesterov, key, exact) -> _AdamEngine:
    torch = _torch()
    cfg = _Config(b1, b2, eps, eps_root, 2048, 1 << 62, torch.float32, mu_dtype, False, "shard_local", False,
                  bool(nesterov), key, bool(exact))
    eng = _AdamEngine(cfg)
    eng.store_sr = mu_dtype == torch.bfloat16
    return eng


def _canonical_mu_dtype(mu_dtype):
    torch = _torch()
    d = torch.float32 if mu_dtype is None else canonicalize_dtype(mu_dtype)
    if d not in (torch.float32, torch.bfloat16):
        raise NotImplementedError("mu_dtype must be float32 or bfloat16")
    return d


class _ScaleByAdamUpdate:
    """``scale_by_adam(...).update`` (adam.py:123-235)."""

    def __init__(self, engine: _AdamEngine, weight_decay, weight_decay_mask):
        self.engine = engine
        self.weight_decay = weight_decay
        self.weight_decay_mask = weight_decay_mask

    def __call__(self, updates, state, params=None):
        return self._step(updates, state, params, apply=False)

    def _step(self, updates, state, params, *, apply: bool, skip_nonfinite=False, finite_out=None,
              finite_host=None, clip_global_norm=None, clip_stats=None, **fused_only):
        del fused_only  # param_key, param_sr, random_bits: fused-step arguments
        if apply:
            raise TypeError("scale_by_adam has no learning rate: the fused step needs adamw(...)")
        decays = _has_nonzero_or_scheduled(self.weight_decay)
        if decays and params is None:
            raise ValueError(
                "`params` must be provided to `scale_by_adam.update` when "
                "`weight_decay` is nonzero or scheduled."
            )
        decay_mask = None
        wd = None
        if params is not None and decays:
            n = len(_tree.leaves(updates, is_leaf=_is_passthrough_leaf))
            decay_mask = _decay_mask_leaves(self.weight_decay_mask, params, n)
            # _resolve_scalar(weight_decay, state.count): a schedule sees the
            # count before the increment (adam.py:196).
            wd = self.weight_decay
            if callable(wd):
                wd = wd(np.asarray(state.count, dtype=np.int32))
            # update + wd * param.astype(f32) (utils.py:79-90): f32 product, so
            # the decay is passed as an array scalar (no weak bf16 typing).
            wd = np.float32(_as_f32(wd))
        return self.engine.run(updates, state, params, apply=False, decay_mask=decay_mask, weight_decay=wd,
                               neg_lr=None, skip_nonfinite=skip_nonfinite, finite_out=finite_out,
                               finite_host=finite_host, clip_global_norm=clip_global_norm, clip_stats=clip_stats)


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
) -> GradientTransformation:
    """Rescale updates according to the Adam algorithm (adam.py:38-235).
    ``exact`` (extension): IEEE division and square root in the direction."""
    del magma_p, magma_tau, axis_name
    if use_magma:
        raise NotImplementedError("Magma is not supported by rollfast_amd.")
    _has_nonzero_or_scheduled(weight_decay)
    mu = _canonical_mu_dtype(mu_dtype)
    engine = _make_engine(b1, b2, eps, eps_root, mu, nesterov, key, exact)

    def init_fn(params):
        return ScaleByAdamState(count=np.zeros((), dtype=np.int32), mu=_zeros_like_tree(params, mu),
                                nu=_zeros_like_tree(params, mu), magma_s=(), key=prng.fresh_key(key))

    return GradientTransformation(init_fn, _ScaleByAdamUpdate(engine, weight_decay, weight_decay_mask))


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
) -> GradientTransformationExtraArgs:
    """Adam with decoupled weight decay (adam.py:238-406): the optax chain
    ``scale_by_adam -> add_decayed_weights -> scale_by_learning_rate`` in one
    launch.  The state is the chain's tuple ``(ScaleByAdamState,
    add_decayed_weights state?, lr state)``."""
    if use_magma:
        raise NotImplementedError("Magma is not supported by rollfast_amd.")
    if callable(weight_decay):
        raise NotImplementedError("weight-decay schedules are not supported by adamw; pass a scalar")
    inner = scale_by_adam(b1=b1, b2=b2, eps=eps, eps_root=eps_root, mu_dtype=mu_dtype, nesterov=nesterov,
                          axis_name=axis_name, key=key, exact=exact, magma_p=magma_p, magma_tau=magma_tau)
    wd_nonzero = _has_nonzero_or_scheduled(weight_decay)
    engine = inner.update.engine

    def init_fn(params):
        states = [inner.init(params)]
        if wd_nonzero:
            states.append(MaskedState(EmptyState()) if weight_decay_mask is not None else EmptyState())
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

    if isinstance(tx.update, _ScaleByAdamUpdate) or (isinstance(tx.update, _Adamw8Update)
                                                     and not isinstance(tx.update.engine, _AdamEngine)):
        raise TypeError("adamw_step needs a transformation built by adamw(...) or a composition of them "
                        "(apply_if_finite, chain with clip_by_global_norm, multi_transform)")
    return adamw8_step(tx, params, grads, state, key=key, stochastic=stochastic, random_bits=random_bits,
                       clip_global_norm=clip_global_norm, clip_stats=clip_stats)


__all__ = ("ScaleByAdamState", "adamw", "adamw_step", "scale_by_adam")
