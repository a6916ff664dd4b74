"""The Optax types the reference's adam8 API is built from.

rollfast's ``adamw8`` returns ``optax.chain(scale_by_adam8, add_decayed_weights,
scale_by_learning_rate)`` (``src/rollfast/optim/adam8.py:418-443``); its state
is the chain's tuple of component states.  Optax is a third-party dependency
of the reference (``optax>=0.2.8,<0.3.0``) and is not available here, so
the few types that shape the API and the state pytree are restated with the
same names, fields and flattening order.
"""

from __future__ import annotations

from typing import Any, Callable, NamedTuple

NO_PARAMS_MSG = (
    "You are using a transformation that requires the current value of "
    "parameters, but you are not passing `params` when calling `update`."
)


class MaskedNode(NamedTuple):
    """Placeholder for a masked-out leaf (optax.transforms._masking.MaskedNode)."""


class EmptyState(NamedTuple):
    """State of a stateless transformation (optax.EmptyState)."""


class ScaleByScheduleState(NamedTuple):
    """State of scale_by_schedule: the step counter fed to the schedule."""

    count: Any


class MaskedState(NamedTuple):
    """State of optax.masked (wraps add_decayed_weights when a mask is given)."""

    inner_state: Any


class ApplyIfFiniteState(NamedTuple):
    """State of optax.apply_if_finite (the non-finite guard of the fine-tune
    builders, finetune/builders.py:1605-1609): consecutive and total counts of
    steps whose grads held an Inf or NaN, whether the last one was finite, and
    the wrapped transformation's state."""

    notfinite_count: Any
    last_finite: Any
    total_notfinite: Any
    inner_state: Any


class GradientTransformation(NamedTuple):
    init: Callable
    update: Callable


class GradientTransformationExtraArgs(GradientTransformation):
    """optax.GradientTransformationExtraArgs: ``update`` accepts extra kwargs."""


def is_passthrough_leaf(x: Any) -> bool:
    """adam8.py:705-706 and utils.py:13-14: None or MaskedNode."""
    return x is None or isinstance(x, MaskedNode)


def safe_int32_increment(count: int) -> int:
    """optax.numerics.safe_increment for int32 counters: saturates at 2^31-1."""
    count = int(count)
    return count + 1 if count < 2**31 - 1 else count
