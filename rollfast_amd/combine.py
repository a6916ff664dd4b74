"""The optax combinators the fine-tune builders assemble their optimizer
from (finetune/builders.py:1529-1621): ``chain``, ``masked`` and
``multi_transform`` (through ``_multi_transform``, builders.py:234-244).
Optax is a third-party dependency of the reference (``optax>=0.2.8,<0.3.0``)
and is absent here; these restate its semantics and state pytrees.

They also carry the fused paths of this package:

* ``multi_transform`` over ``adamw8`` / ``adamw`` transforms that share
  betas, eps and the step count (the fine-tune groups differ in learning
  rate, weight decay, quantization and key) runs as ONE launch: every leaf
  row carries its group index and the group table carries the per-group
  scalars.  Other combinations run group by group, as optax does.
* ``chain(clip_by_global_norm(m), tx)`` fuses the clipping into ``tx``'s
  launch (a norm pre-pass instead of a read-and-write scaling pass).
* ``adamw8_step`` / ``adamw_step`` accept these compositions (and
  ``apply_if_finite`` around them) and keep them one launch.
"""

from __future__ import annotations

from typing import Any, Hashable, Mapping, NamedTuple

from . import _tree
from ._base import (
    GradientTransformationExtraArgs,
    MaskedNode,
    MaskedState,
    is_passthrough_leaf as _is_passthrough_leaf,
)


class MultiTransformState(NamedTuple):
    """State of optax.multi_transform: one (masked) inner state per label."""

    inner_states: Any


def _mask_flags(mask, tree) -> list:
    """Per-leaf booleans of an optax mask (a tree of bools with the structure
    of ``tree``, or a callable returning one), aligned with ``tree``'s
    flattened leaves (None and MaskedNode count as leaves)."""
    mask_tree = mask(tree) if callable(mask) else mask
    leaves, td = _tree.flatten(tree, is_leaf=_is_passthrough_leaf)
    flags = _tree.flatten_up_to(td, mask_tree)
    return [bool(f) for f in flags]


def _apply_mask(tree, flags: list):
    leaves, td = _tree.flatten(tree, is_leaf=_is_passthrough_leaf)
    return _tree.unflatten(td, [x if f else MaskedNode() for x, f in zip(leaves, flags)])


def _inner_step(tx):
    step = getattr(tx.update, "_step", None)
    if step is None:
        raise NotImplementedError(
            "the fused step composes adamw8, adamw, scale_by_adam8, scale_by_adam, chain(clip_by_global_norm, "
            "...), multi_transform and apply_if_finite")
    return step


class _MaskedUpdate:
    """optax.masked(inner, mask).update: the inner transformation sees
    MaskedNode in place of the leaves whose mask is False; those leaves keep
    their incoming updates."""

    def __init__(self, inner, mask):
        self.inner = inner
        self.mask = mask

    def _split(self, updates, params):
        flags = _mask_flags(self.mask, updates)
        mu = _apply_mask(updates, flags)
        mp = None if params is None else _apply_mask(params, flags)
        return flags, mu, mp

    @staticmethod
    def _merge(flags, new_updates, updates):
        new_leaves, td = _tree.flatten(new_updates, is_leaf=_is_passthrough_leaf)
        old_leaves = _tree.flatten_up_to(td, updates)
        return _tree.unflatten(td, [n if f else o for n, o, f in zip(new_leaves, old_leaves, flags)])

    def __call__(self, updates, state, params=None, **extra_args):
        del extra_args
        flags, mu, mp = self._split(updates, params)
        new_u, new_inner = self.inner.update(mu, state.inner_state, mp)
        return self._merge(flags, new_u, updates), MaskedState(inner_state=new_inner)

    def _step(self, updates, state, params, *, apply: bool, **kwargs):
        flags, mu, mp = self._split(updates, params)
        new_u, new_inner = _inner_step(self.inner)(mu, state.inner_state, mp, apply=apply, **kwargs)
        out = None if apply else self._merge(flags, new_u, updates)
        return out, MaskedState(inner_state=new_inner)


def masked(inner, mask) -> GradientTransformationExtraArgs:
    """optax.masked: apply ``inner`` to the leaves where ``mask`` is True."""

    def init_fn(params):
        return MaskedState(inner_state=inner.init(_apply_mask(params, _mask_flags(mask, params))))

    return GradientTransformationExtraArgs(init_fn, _MaskedUpdate(inner, mask))


class _ChainUpdate:
    """optax.chain(*transforms).update: the transforms in order, the state a
    tuple of theirs."""

    def __init__(self, transforms):
        self.transforms = tuple(transforms)

    def __call__(self, updates, state, params=None, **extra_args):
        del extra_args
        new_states = []
        for tx, s in zip(self.transforms, state):
            updates, s = tx.update(updates, s, params)
            new_states.append(s)
        return updates, tuple(new_states)

    def _step(self, updates, state, params, *, apply: bool, clip_global_norm=None, **kwargs):
        from .transforms import _ClipUpdate, _next_clip_state

        txs = self.transforms
        if len(txs) == 1:
            out, s = _inner_step(txs[0])(updates, state[0], params, apply=apply, clip_global_norm=clip_global_norm,
                                         **kwargs)
            return out, (s,)
        if len(txs) == 2 and isinstance(txs[0].update, _ClipUpdate):
            if clip_global_norm is not None:
                raise ValueError("clip_global_norm given twice (argument and chained clip_by_global_norm)")
            out, s = _inner_step(txs[1])(updates, state[1], params, apply=apply,
                                         clip_global_norm=txs[0].update.max_norm, **kwargs)
            return out, (_next_clip_state(state[0]), s)
        raise NotImplementedError("a fused step takes chain(clip_by_global_norm(m), tx) or chain(tx)")


def chain(*transforms) -> GradientTransformationExtraArgs:
    """optax.chain: apply the transformations in sequence."""

    def init_fn(params):
        return tuple(tx.init(params) for tx in transforms)

    return GradientTransformationExtraArgs(init_fn, _ChainUpdate(transforms))


class _MultiTransformUpdate:
    """optax.multi_transform(transforms, param_labels).update."""

    def __init__(self, transforms: Mapping[Hashable, Any], param_labels):
        self.transforms = transforms
        self.param_labels = param_labels
        self._runner = None

    def _labels_obj(self, tree):
        return self.param_labels(tree) if callable(self.param_labels) else self.param_labels

    def _labels(self, tree, labels_obj=None) -> list:
        labels = self._labels_obj(tree) if labels_obj is None else labels_obj
        _leaves, td = _tree.flatten(tree, is_leaf=_is_passthrough_leaf)
        return _tree.flatten_up_to(td, labels)

    def _members(self, updates, state, labels_obj=None):
        """(group update object, its chain state, membership flags) per label
        whose transformation can join a grouped launch, else None."""
        from .optim.adam8 import _Adamw8Update, _GroupedRunner

        labels = self._labels(updates, labels_obj)
        members = []
        for group, tx in self.transforms.items():
            if not isinstance(tx.update, _Adamw8Update):
                return None
            members.append((tx.update, state.inner_states[group].inner_state, [lab == group for lab in labels]))
        if not _GroupedRunner.compatible([m[0] for m in members], [m[1][0] for m in members]):
            return None
        return members

    def __call__(self, updates, state, params=None, **extra_args):
        del extra_args
        members = self._members(updates, state)
        if members is not None:
            return self._grouped(updates, state, params, members, apply=False)
        labels = self._labels(updates)
        new_inner = {}
        for group, tx in self.transforms.items():
            flags = [lab == group for lab in labels]
            mp = None if params is None else _apply_mask(params, flags)
            new_u, s = tx.update(_apply_mask(updates, flags), state.inner_states[group].inner_state, mp)
            updates = _MaskedUpdate._merge(flags, new_u, updates)
            new_inner[group] = MaskedState(inner_state=s)
        return updates, MultiTransformState(inner_states=new_inner)

    def _grouped(self, updates, state, params, members, *, apply: bool, **kwargs):
        from .optim.adam8 import _GroupedRunner

        if self._runner is None:
            self._runner = _GroupedRunner()
        out_leaves, td, new_states = self._runner.run(members, updates, params, apply=apply, **kwargs)
        new_inner = {group: MaskedState(inner_state=s) for group, s in zip(self.transforms, new_states)}
        out = None if apply else _tree.unflatten(td, out_leaves)
        return out, MultiTransformState(inner_states=new_inner)

    def _step(self, updates, state, params, *, apply: bool, **kwargs):
        from .optim.adam8 import _Adamw8Update

        labels_obj = self._labels_obj(updates)
        if apply and self._runner is not None:
            # steady state: the same labels and state objects as the previous call
            groups_in = [(tx.update, state.inner_states[g].inner_state) for g, tx in self.transforms.items()]
            if all(isinstance(u, _Adamw8Update) for u, _ in groups_in):
                new_states = self._runner.run_cached(groups_in, labels_obj, updates, params, **kwargs)
                if new_states is not None:
                    return None, MultiTransformState(
                        inner_states={g: MaskedState(inner_state=s) for g, s in zip(self.transforms, new_states)})
        members = self._members(updates, state, labels_obj)
        if members is None:
            raise NotImplementedError(
                "a fused multi_transform step needs adamw8 / adamw groups that share b1, b2, eps, eps_root, "
                "nesterov, exact, stochastic_rounding and the step count")
        return self._grouped(updates, state, params, members, apply=apply, labels_obj=labels_obj, **kwargs)


def multi_transform(transforms: Mapping[Hashable, Any], param_labels) -> GradientTransformationExtraArgs:
    """optax.multi_transform: each leaf is updated by the transformation of
    its label (``param_labels``: a tree of labels like the params, or a
    callable returning one)."""

    def init_fn(params):
        labels = param_labels(params) if callable(param_labels) else param_labels
        _leaves, td = _tree.flatten(params, is_leaf=_is_passthrough_leaf)
        flat = _tree.flatten_up_to(td, labels)
        label_set = set(flat)
        if not label_set.issubset(transforms.keys()):
            raise ValueError(
                "Some parameters have no corresponding transformation.\n"
                f"Parameter labels: {sorted(map(str, label_set))} \n"
                f"Transforms keys: {sorted(map(str, transforms.keys()))} \n")
        inner = {}
        for group, tx in transforms.items():
            flags = [lab == group for lab in flat]
            inner[group] = MaskedState(inner_state=tx.init(_apply_mask(params, flags)))
        return MultiTransformState(inner_states=inner)

    return GradientTransformationExtraArgs(init_fn, _MultiTransformUpdate(transforms, param_labels))


__all__ = ("MultiTransformState", "chain", "masked", "multi_transform")
