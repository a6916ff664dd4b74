"""Moment-format conversion between the 8-bit and the full-precision AdamW
states, for state migration and checkpoint tools.

The reference's migration (``finetune/state_migration.py:474-495``
``_compatible_leaf``) keeps a moment leaf only when old and new have the same
format and re-initialises it otherwise; a quantized moment is read through
``_dequantize_state_leaf`` (``optim/adam8.py:691-696``) and written through
``_store_moment_tree`` (``optim/adam8.py:633-688``).  These functions apply
those two over whole state trees on the device kernels (one dequantize or
quantize launch per leaf), so a state can change format instead of being
reset:

* ``dequantize_state_tree`` / ``quantize_state_tree``: moment trees;
* ``adam_state_from_adam8`` / ``adam8_state_from_adam``: whole
  ``ScaleByAdam8State`` <-> ``ScaleByAdamState`` (optim/adam.py:28-35).
"""

from __future__ import annotations

from typing import Any

import numpy as np

from .. import _tree, prng
from .._base import is_passthrough_leaf as _is_passthrough_leaf
from .adam import ScaleByAdamState
from .adam8 import (
    QuantizedBlocks,
    ScaleByAdam8State,
    _is_state_leaf,
    _quantizer_from_codebook_id,
    _require_device_tensor,
    _torch,
    dequantize_blocks,
    quantize_blocks,
)


def _dequantize_state_leaf(leaf):
    """adam8.py:691-696: QuantizedBlocks -> f32 (padding removed); other
    arrays -> f32; None / MaskedNode pass through."""
    torch = _torch()
    if isinstance(leaf, QuantizedBlocks):
        return dequantize_blocks(leaf, dtype=torch.float32)
    if _is_passthrough_leaf(leaf):
        return leaf
    _require_device_tensor(leaf, "moment")
    return leaf.to(torch.float32)


def dequantize_state_tree(tree) -> Any:
    """Every moment leaf of ``tree`` as a float32 array of its param's shape."""
    return _tree.tree_map(_dequantize_state_leaf, tree, is_leaf=_is_state_leaf)


def quantize_state_tree(tree, template, *, stochastic_rounding: bool = False, key=None) -> Any:
    """adam8.py:633-688 ``_store_moment_tree``: leaf i of ``tree`` is
    quantized like ``template``'s leaf i (quantizer, block size, layout) when
    that is a ``QuantizedBlocks``, else cast to the template leaf's dtype;
    passthrough template leaves stay.  Stochastic rounding draws leaf i's
    bits from ``split(key, n_leaves)[i]``, as the optimizer does."""
    if stochastic_rounding and key is None:
        raise ValueError("stochastic rounding requires a PRNG key.")
    t_leaves, t_td = _tree.flatten(template, is_leaf=_is_state_leaf)
    m_leaves = _tree.flatten_up_to(t_td, tree)
    keys = prng.split(prng.as_key(key), len(t_leaves)) if (stochastic_rounding and t_leaves) else None
    out = []
    for i, (m, t) in enumerate(zip(m_leaves, t_leaves)):
        if isinstance(t, QuantizedBlocks):
            _require_device_tensor(m, "moment")
            if int(m.numel()) != t.size:
                raise ValueError(f"leaf {i}: {m.numel()} elements, the template holds {t.size}")
            out.append(quantize_blocks(
                m, block_size=t.block_size, scale_dtype=t.scales.dtype, stochastic_rounding=stochastic_rounding,
                key=None if keys is None else keys[i], block_layout=t.block_layout,
                quantizer=_quantizer_from_codebook_id(t.codebook_id)))
        elif _is_passthrough_leaf(t):
            out.append(t)
        else:
            _require_device_tensor(m, "moment")
            out.append(m.to(t.dtype).reshape(t.shape))
    return _tree.unflatten(t_td, out)


def adam_state_from_adam8(state: ScaleByAdam8State) -> ScaleByAdamState:
    """An adamw8 state as the full-precision ``scale_by_adam`` state: f32
    moments (dequantized), the same count and key, no Magma state."""
    return ScaleByAdamState(count=np.asarray(state.count, dtype=np.int32), mu=dequantize_state_tree(state.mu),
                            nu=dequantize_state_tree(state.nu), magma_s=(), key=state.key)


def adam8_state_from_adam(state: ScaleByAdamState, template: ScaleByAdam8State, *,
                          stochastic_rounding: bool = False, key=None) -> ScaleByAdam8State:
    """A full-precision ``scale_by_adam`` state in ``template``'s 8-bit
    format (the state ``adamw8(...).init`` gives for the same params): the
    moments are quantized leaf by leaf as the optimizer stores them; count
    and key carry over.  With stochastic rounding, the first and second
    moments draw from ``split(key)``'s two halves."""
    key_mu = key_nu = None
    if stochastic_rounding:
        if key is None:
            raise ValueError("stochastic rounding requires a PRNG key.")
        key_mu, key_nu = prng.split(prng.as_key(key), 2)
    return ScaleByAdam8State(
        count=np.asarray(state.count, dtype=np.int32),
        mu=quantize_state_tree(state.mu, template.mu, stochastic_rounding=stochastic_rounding, key=key_mu),
        nu=quantize_state_tree(state.nu, template.nu, stochastic_rounding=stochastic_rounding, key=key_nu),
        key=state.key,
    )


__all__ = ("adam8_state_from_adam", "adam_state_from_adam8", "dequantize_state_tree", "quantize_state_tree")
