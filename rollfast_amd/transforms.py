"""Gradient transforms of rollfast's fine-tuning builders, on MI355X kernels.

Mirror of ``src/rollfast/finetune/transforms.py``: ``clip_by_global_norm``
and ``GlobalNormClipState``.  The norm and the scaling run in
``librfadam8.so`` (``rf_clip_by_global_norm``: a multi-tensor norm pre-pass
and one multi-tensor scaling launch).  The optimizer steps also take the
same clipping fused (``adamw8_step(..., clip_global_norm=...)``), which
reads the grads once instead of reading and writing them.

``apply_if_finite`` restates ``optax.apply_if_finite``, the non-finite guard
the fine-tune builders wrap around their chain (finetune/builders.py:
1605-1609, ``GradientPolicy(nonfinite="skip", max_consecutive_nonfinite=1)``
by default, finetune/config.py:226-233), for the optimizers of this package:
the step's norm pre-pass tests every grad for Inf/NaN and the step units
apply the reject branch on the device.
"""

from __future__ import annotations

import ctypes
from typing import Any, NamedTuple

import numpy as np

from . import _lib, _tree
from ._base import (
    ApplyIfFiniteState,
    GradientTransformation,
    GradientTransformationExtraArgs,
    is_passthrough_leaf as _is_passthrough_leaf,
    safe_int32_increment,
)


class GlobalNormClipState(NamedTuple):
    """State for the global-norm clipping transform (transforms.py:14-17)."""

    count: Any


def _next_clip_state(state) -> GlobalNormClipState:
    """transforms.py:54: ``GlobalNormClipState(count=state.count + 1)``."""
    return GlobalNormClipState(count=np.asarray(np.int32(int(np.asarray(state.count)) + 1), dtype=np.int32))


class _ClipUpdate:
    """``clip_by_global_norm(max_norm).update`` (transforms.py:36-54) as one
    norm pre-pass and one scaling launch.  ``max_norm`` also lets the fused
    optimizer steps recognise ``chain(clip_by_global_norm(m), tx)``."""

    def __init__(self, max_norm: float):
        self.max_norm = max_norm

    def __call__(self, updates, state, params=None, stats=None):
        """``stats`` (extension): optional float32 device tensor of 2 elements
        receiving (scale, norm)."""
        import torch

        del params
        leaves, td = _tree.flatten(updates, is_leaf=lambda x: x is None)
        rows = []
        out = []
        device = None
        for leaf in leaves:
            if leaf is None or _is_passthrough_leaf(leaf) or not hasattr(leaf, "dtype"):
                out.append(leaf)
                continue
            if not isinstance(leaf, torch.Tensor) or not leaf.is_cuda:
                raise ValueError("updates must be torch tensors on a ROCm device")
            if device is None:
                device = leaf.device
            if leaf.device != device:
                raise ValueError("all leaves must live on the same device")
            if leaf.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                raise NotImplementedError(f"dtype {leaf.dtype} is not supported (float32, bfloat16 or float16)")
            src = leaf.contiguous()
            dst = torch.empty_like(src)
            row = _lib.ClipLeaf()
            row.grad = src.data_ptr()
            row.out = dst.data_ptr()
            row.size = int(src.numel())
            row.dtype = {torch.bfloat16: _lib.RF_BF16, torch.float16: _lib.RF_F16}.get(src.dtype, _lib.RF_F32)
            rows.append((row, src))
            out.append(dst.view(leaf.shape))
        if rows:
            table = (_lib.ClipLeaf * len(rows))(*[r for r, _ in rows])
            stats_ptr = None
            if stats is not None:
                if stats.dtype != torch.float32 or stats.numel() < 2 or not stats.is_cuda:
                    raise ValueError("stats must be a float32 device tensor of 2 elements")
                stats_ptr = stats.data_ptr()
            with torch.cuda.device(device):
                _lib.check(_lib.lib().rf_clip_by_global_norm(table, len(rows), ctypes.c_float(self.max_norm),
                                                             ctypes.c_void_p(stats_ptr), _lib.stream_ptr()),
                           "clip_by_global_norm")
        return _tree.unflatten(td, out), _next_clip_state(state)


def clip_by_global_norm(max_norm: float, *, axis_name=None, partition_axis_names=None,
                        replicated_axis_names=None) -> GradientTransformation:
    """Clip by global norm over the leaves (transforms.py:20-54): scale every
    leaf by ``min(1, max_norm / (norm + 1e-6))`` in the leaf dtype.  The axis
    arguments name collective axes of a multi-device reduction, which
    rollfast_amd (one device) does not perform; they must be None."""
    if max_norm <= 0.0:
        raise ValueError("max_norm must be positive.")
    if axis_name is not None or partition_axis_names is not None or replicated_axis_names is not None:
        raise NotImplementedError("cross-device norm reduction is not implemented: rollfast_amd runs on one device")

    def init_fn(params):
        del params
        return GlobalNormClipState(count=np.zeros((), dtype=np.int32))

    return GradientTransformation(init_fn, _ClipUpdate(float(max_norm)))


class _ApplyIfFiniteUpdate:
    """``optax.apply_if_finite(inner, max_consecutive_errors).update``.

    optax semantics: ``isfinite`` = every element of every incoming update
    (the grads, before any clipping of the inner chain) is finite;
    ``notfinite_count`` = 0 if finite else the saturating increment of the
    previous count; the inner update is applied when ``isfinite or
    notfinite_count > max_consecutive_errors``, otherwise the result is zero
    updates (zeros like the grads) and the unchanged inner state;
    ``total_notfinite`` counts every non-finite step.

    Here the inner update runs as one launch with RF_SKIP_NONFINITE (when a
    rejection is possible) and its finite flag: the kernels leave the moments
    untouched on a rejected step and the fused step applies the zero update to
    the params (``f32(p) + 0``).  The next state's counters depend on the
    flag, so the host reads it back every step: the launch copies it to
    pinned host memory right after the norm pre-pass, and the call waits for
    that copy only, not for the step, which keeps running.
    """

    def __init__(self, inner, max_consecutive_errors: int):
        self.inner = inner
        self.max_consecutive_errors = int(max_consecutive_errors)
        self._flag = None  # pinned host int32 the launch copies the finite flag into

    def _step(self, updates, state, params, *, apply: bool, **kwargs):
        import torch

        notfinite_next = safe_int32_increment(int(np.asarray(state.notfinite_count)))
        may_reject = not notfinite_next > self.max_consecutive_errors
        device = None
        for leaf in _tree.leaves(updates, is_leaf=_is_passthrough_leaf):
            if isinstance(leaf, torch.Tensor) and leaf.is_cuda:
                device = leaf.device
                break
        flag = None
        if device is not None:
            if self._flag is None:
                self._flag = torch.ones(1, dtype=torch.int32, pin_memory=True)
            flag = self._flag
            flag[0] = 1  # a run with no elements leaves it: vacuously finite
        out, new_inner = self.inner.update._step(updates, state.inner_state, params, apply=apply,
                                                 skip_nonfinite=may_reject, finite_host=flag, **kwargs)
        isfinite = True if flag is None else bool(int(flag[0]))
        if isfinite or not may_reject:
            inner_state = new_inner
        else:
            inner_state = state.inner_state
            if not apply:
                out = _tree.tree_map(lambda x: x if _is_passthrough_leaf(x) else torch.zeros_like(x), updates,
                                     is_leaf=_is_passthrough_leaf)
        total = int(np.asarray(state.total_notfinite))
        new_state = ApplyIfFiniteState(
            notfinite_count=np.asarray(0 if isfinite else notfinite_next, dtype=np.int32),
            last_finite=np.asarray(isfinite, dtype=np.bool_),
            total_notfinite=np.asarray(total if isfinite else safe_int32_increment(total), dtype=np.int32),
            inner_state=inner_state,
        )
        return out, new_state

    def __call__(self, updates, state, params=None, **extra_args):
        del extra_args
        return self._step(updates, state, params, apply=False)


def apply_if_finite(inner: GradientTransformation, max_consecutive_errors: int) -> GradientTransformationExtraArgs:
    """Skip steps whose grads hold an Inf or NaN, up to
    ``max_consecutive_errors`` in a row (optax.apply_if_finite, as wrapped by
    finetune/builders.py:1605-1609).  ``inner`` is a transformation built by
    ``adamw8``, ``scale_by_adam8``, ``adamw`` or ``scale_by_adam``; the guarded
    step stays one launch (``adamw8_step`` / ``adamw_step`` accept the
    wrapped transformation too)."""
    if not hasattr(inner.update, "_step"):
        raise NotImplementedError(
            "apply_if_finite wraps the transformations built by adamw8, scale_by_adam8, adamw or scale_by_adam")

    def init_fn(params):
        return ApplyIfFiniteState(
            notfinite_count=np.zeros((), dtype=np.int32),
            last_finite=np.asarray(True, dtype=np.bool_),
            total_notfinite=np.zeros((), dtype=np.int32),
            inner_state=inner.init(params),
        )

    return GradientTransformationExtraArgs(init_fn, _ApplyIfFiniteUpdate(inner, max_consecutive_errors))


__all__ = ("ApplyIfFiniteState", "GlobalNormClipState", "apply_if_finite", "clip_by_global_norm")
