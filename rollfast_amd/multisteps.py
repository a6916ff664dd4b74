"""Gradient accumulation over micro-steps: ``optax.MultiSteps`` on MI355X kernels.

The fine-tune builders wrap their whole transformation in
``optax.MultiSteps(tx, every_k_schedule=steps, use_grad_mean=...,
accumulator_dtype=...)`` when ``AccumulationConfig.steps > 1``
(finetune/builders.py:1614-1620, :1340-1344).  optax is a dependency of the
reference (``optax>=0.2.8,<0.3.0``, pyproject.toml:32), not vendored; this
module restates its published ``MultiSteps.update`` for the transformations
of this package:

- every micro-step folds the incoming grads into the accumulator, in place,
  with one multi-tensor launch (``rf_accumulate``): Welford's running mean
  ``acc + (g - acc) / (mini_step + 1)`` or the sum ``g + acc``;
- the k-th micro-step (``mini_step == k - 1``) runs the inner update on the
  accumulator as its grads -- for ``adamw8_step`` / ``adamw_step`` that is
  the inner's fused, grouped and guarded launch -- then resets the
  accumulator to ``0 * acc`` (optax's ``(1 - emit) * acc``: a signed zero,
  NaN where the accumulator held Inf or NaN);
- the other micro-steps return zero updates and leave the inner state as it
  was; the fused step leaves the params untouched on them.

optax also runs the inner update on the partial accumulator of a
non-emitting micro-step and multiplies its result by zero.  That work is
skipped here: its updates are zeros either way, except for two cases this
module does not reproduce: the sign of those zeros (a param of -0.0 plus a
+0.0 update becomes +0.0 in the reference's ``apply_updates``), and an inner
update that is not finite on a partial accumulator (possible only without
the ``apply_if_finite`` guard, which the builders put inside MultiSteps),
whose zero multiple is NaN.
"""

from __future__ import annotations

from typing import Any, Callable, NamedTuple, Optional

import numpy as np

from . import _lib, _tree
from ._base import GradientTransformationExtraArgs, is_passthrough_leaf as _is_passthrough_leaf, safe_int32_increment


class MultiStepsState(NamedTuple):
    """optax.MultiStepsState: the micro-step counter within the window, the
    count of emitted (inner) steps, the inner state, the accumulator (one
    tensor per param leaf) and the skip function's state."""

    mini_step: Any
    gradient_step: Any
    inner_opt_state: Any
    acc_grads: Any
    skip_state: Any = ()


def _default_skip(updates, gradient_step, params):
    del updates, gradient_step, params
    return np.asarray(False, dtype=np.bool_), ()


def _dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: _lib.RF_F32, torch.bfloat16: _lib.RF_BF16, torch.float16: _lib.RF_F16}
    if dtype not in codes:
        raise NotImplementedError(f"dtype {dtype} is not supported (float32, bfloat16 or float16)")
    return codes[dtype]


def _promoted(a, b):
    """JAX's promotion of two float dtypes among f32 / bf16 / f16."""
    import torch

    return a if a == b else torch.float32


def _skip_flag(x) -> bool:
    """The boolean scalar of ``should_skip_update_fn`` (numpy, Python or a
    torch tensor), rejected like optax rejects any other dtype or shape."""
    import torch

    if isinstance(x, torch.Tensor):
        ok = x.dtype == torch.bool and x.dim() == 0
        dtype, shape = x.dtype, tuple(x.shape)
    else:
        arr = np.asarray(x)
        ok = arr.dtype == np.bool_ and arr.shape == ()
        dtype, shape = arr.dtype, arr.shape
    if not ok:
        raise ValueError("The `should_skip_update_fn` function should return a boolean scalar array, but it "
                         f"returned an array of dtype {dtype} and shape {shape}")
    return bool(x.item()) if isinstance(x, torch.Tensor) else bool(np.asarray(x))


class _MultiStepsUpdate:
    """``MultiSteps(...).update``.  ``_step`` is the form the fused steps
    (``adamw8_step``, ``adamw_step``) call: ``apply=True`` writes the params
    on the emitting micro-step and leaves them on the others."""

    def __init__(self, ms: "MultiSteps"):
        self.ms = ms

    def _accumulate(self, grads, acc_grads, mode: int, n_acc: int):
        import torch

        a_leaves = _tree.leaves(acc_grads, is_leaf=_is_passthrough_leaf)
        if mode == _lib.RF_ACC_ZERO:
            g_leaves = [None] * len(a_leaves)
        else:
            g_leaves = _tree.leaves(grads, is_leaf=_is_passthrough_leaf)
        if len(g_leaves) != len(a_leaves):
            raise ValueError(f"updates have {len(g_leaves)} leaves but the accumulator has {len(a_leaves)}")
        rows = []
        device = None
        for g, a in zip(g_leaves, a_leaves):
            if _is_passthrough_leaf(a) or not isinstance(a, torch.Tensor):
                continue
            if not a.is_cuda or not a.is_contiguous():
                raise ValueError("the accumulator must hold contiguous tensors on a ROCm device")
            if device is None:
                device = a.device
            if a.device != device:
                raise ValueError("all leaves must live on the same device")
            row = _lib.AccumLeaf()
            row.acc = a.data_ptr()
            row.size = int(a.numel())
            row.acc_dtype = _dtype_code(a.dtype)
            if mode == _lib.RF_ACC_ZERO:
                row.grad = None
                row.grad_dtype = row.acc_dtype
            else:
                if not isinstance(g, torch.Tensor) or not g.is_cuda or g.device != device:
                    raise ValueError("updates must be torch tensors on the accumulator's device")
                if g.shape != a.shape:
                    raise ValueError(f"update of shape {tuple(g.shape)} for an accumulator of shape "
                                     f"{tuple(a.shape)}")
                if _promoted(g.dtype, a.dtype) != a.dtype:
                    # optax keeps the promoted dtype, which changes the state's
                    # type between the branches of its lax.cond: JAX rejects it
                    raise TypeError(f"MultiSteps: {g.dtype} updates promote a {a.dtype} accumulator to "
                                    f"{_promoted(g.dtype, a.dtype)}; use accumulator_dtype=float32 or "
                                    f"updates of the accumulator's dtype")
                if not g.is_contiguous():
                    g = g.contiguous()
                row.grad = g.data_ptr()
                row.grad_dtype = _dtype_code(g.dtype)
            rows.append((row, g))
        if not rows:
            return
        table = (_lib.AccumLeaf * len(rows))(*[r for r, _ in rows])
        with torch.cuda.device(device):
            _lib.check(_lib.lib().rf_accumulate(table, len(rows), int(mode), int(n_acc), _lib.stream_ptr()),
                       "MultiSteps accumulate")

    def _step(self, updates, state, params, *, apply: bool, **kwargs):
        import torch

        ms = self.ms
        gradient_step = int(np.asarray(state.gradient_step))
        mini_step = int(np.asarray(state.mini_step))
        k_steps = int(np.asarray(ms._every_k_schedule(np.asarray(gradient_step, dtype=np.int32))))
        if k_steps < 1:
            raise ValueError(f"every_k_schedule returned {k_steps}; it must be at least 1")
        skip, skip_state = ms._should_skip_update_fn(updates, np.asarray(gradient_step, dtype=np.int32), params)
        if _skip_flag(skip):
            new_state = state._replace(skip_state=skip_state)
            if apply:
                return None, new_state
            zeros = _tree.tree_map(lambda a: a if _is_passthrough_leaf(a) else torch.zeros_like(a),
                                   state.acc_grads, is_leaf=_is_passthrough_leaf)
            return zeros, new_state

        mode = _lib.RF_ACC_MEAN if ms._use_grad_mean else _lib.RF_ACC_SUM
        self._accumulate(updates, state.acc_grads, mode, mini_step)
        emit = mini_step == k_steps - 1
        if emit:
            inner_upd = ms._opt.update
            if hasattr(inner_upd, "_step"):
                out, inner_state = inner_upd._step(state.acc_grads, state.inner_opt_state, params, apply=apply,
                                                   **kwargs)
            elif apply:
                raise TypeError("the fused step needs an inner transformation built by this package")
            else:
                out, inner_state = inner_upd(state.acc_grads, state.inner_opt_state, params)
            if not apply:
                out = _detach_from(out, state.acc_grads)
            self._accumulate(None, state.acc_grads, _lib.RF_ACC_ZERO, 0)
        else:
            inner_state = state.inner_opt_state
            out = None
            if not apply:
                out = _tree.tree_map(
                    lambda g: g if _is_passthrough_leaf(g) else torch.zeros(g.shape, dtype=torch.float32,
                                                                            device=g.device),
                    updates, is_leaf=_is_passthrough_leaf)
        new_state = MultiStepsState(
            mini_step=np.asarray(safe_int32_increment(mini_step) % k_steps, dtype=np.int32),
            gradient_step=np.asarray(safe_int32_increment(gradient_step) if emit else gradient_step,
                                     dtype=np.int32),
            inner_opt_state=inner_state,
            acc_grads=state.acc_grads,
            skip_state=skip_state,
        )
        return out, new_state

    def __call__(self, updates, state, params=None, **extra_args):
        del extra_args
        return self._step(updates, state, params, apply=False)


def _detach_from(out, acc_grads):
    """Updates the inner transformation returned that share memory with the
    accumulator (a pass-through leaf) are copied before the reset."""
    import torch

    ptrs = {a.untyped_storage().data_ptr() for a in _tree.leaves(acc_grads, is_leaf=_is_passthrough_leaf)
            if isinstance(a, torch.Tensor)}

    def fix(u):
        if isinstance(u, torch.Tensor) and u.untyped_storage().data_ptr() in ptrs:
            return u.clone()
        return u

    return _tree.tree_map(fix, out, is_leaf=_is_passthrough_leaf)


class MultiSteps:
    """optax.MultiSteps(opt, every_k_schedule, use_grad_mean=True,
    should_skip_update_fn=None, accumulator_dtype=None), the wrapper of
    finetune/builders.py:1614-1620.

    ``every_k_schedule``: an int, or a function of the gradient step (an
    int32 scalar) returning the window length.  ``accumulator_dtype``: the
    accumulator's dtype (None: each param's dtype).  ``should_skip_update_fn
    (updates, gradient_step, params) -> (bool scalar, skip_state)``: a
    skipped micro-step returns zero updates and leaves the counters and the
    accumulator as they were.
    """

    def __init__(self, opt, every_k_schedule, use_grad_mean: bool = True,
                 should_skip_update_fn: Optional[Callable] = None, accumulator_dtype=None):
        self._opt = opt
        if isinstance(every_k_schedule, (int, np.integer)):
            k = int(every_k_schedule)
            self._every_k_schedule = lambda step: k
        else:
            self._every_k_schedule = every_k_schedule
        self._use_grad_mean = bool(use_grad_mean)
        self._should_skip_update_fn = should_skip_update_fn or _default_skip
        self._accumulator_dtype = None
        if accumulator_dtype is not None:
            from .optim.adam8 import canonicalize_dtype

            self._accumulator_dtype = canonicalize_dtype(accumulator_dtype)
        self.update = _MultiStepsUpdate(self)

    @property
    def inner_opt(self):
        return self._opt

    def init(self, params) -> MultiStepsState:
        import torch

        def zeros(p):
            if _is_passthrough_leaf(p) or not isinstance(p, torch.Tensor):
                return p
            dt = self._accumulator_dtype if self._accumulator_dtype is not None else p.dtype
            _dtype_code(dt)
            return torch.zeros(p.shape, dtype=dt, device=p.device)

        acc = _tree.tree_map(zeros, params, is_leaf=_is_passthrough_leaf)
        gradient_step = np.zeros((), dtype=np.int32)
        _, skip_state = self._should_skip_update_fn(acc, gradient_step, params)
        return MultiStepsState(
            mini_step=np.zeros((), dtype=np.int32),
            gradient_step=gradient_step,
            inner_opt_state=self._opt.init(params),
            acc_grads=acc,
            skip_state=skip_state,
        )

    def has_updated(self, state) -> bool:
        """True right after an emitting micro-step: ``mini_step == 0 and
        gradient_step > 0``."""
        return int(np.asarray(state.mini_step)) == 0 and int(np.asarray(state.gradient_step)) > 0

    def gradient_transformation(self) -> GradientTransformationExtraArgs:
        return GradientTransformationExtraArgs(self.init, self.update)


__all__ = ("MultiSteps", "MultiStepsState")
