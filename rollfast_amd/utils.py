"""Parameter application and bf16 stochastic rounding on HIP kernels.

Mirror of the hot-path helpers of ``src/rollfast/utils.py`` (rollfast):
``apply_updates`` (:648-708), ``apply_updates_prefix`` (:711-769),
``_stochastic_round_bf16`` (:342-371) and ``_tree_stochastic_cast``
(:374-409).  Arrays are torch tensors on a ROCm device; the arithmetic runs
in ``librfadam8.so`` (``rf_apply_updates``, ``rf_sr_bf16``).  Parameters are
updated in place and returned (JAX donation semantics).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, _tree, prng
from ._base import MaskedNode, is_passthrough_leaf

_KEY_MSG = (
    "apply_updates requires a PRNG `key` when stochastic=True. "
    "Pass stochastic=False for deterministic rounding."
)


def _is_aux_leaf(x) -> bool:
    """utils.py:13-14."""
    return x is None or isinstance(x, MaskedNode)


def _torch():
    import torch

    return torch


_SR_BITS = ("jax", "packed")


def _check_sr_bits(sr_bits) -> bool:
    """True for the packed bit source (no reference counterpart: one
    Threefry-2x32-20 block per four roundings, element e taking the 16-bit
    half (e & 1) of word (e & 2 ? y1 : y0) of the block at counter e >> 2
    under the leaf's key); False for jax.random.bits' stream."""
    if sr_bits not in _SR_BITS:
        raise ValueError(f"sr_bits must be one of {_SR_BITS}, got {sr_bits!r}")
    return sr_bits == "packed"


def _apply_call(table, n: int, stochastic: bool, k, packed: bool) -> None:
    lib = _lib.lib()
    if stochastic and packed:
        _lib.check(lib.rf_apply_updates_packed(table, n, int(k[0]), int(k[1]), _lib.stream_ptr()), "apply_updates")
    else:
        _lib.check(lib.rf_apply_updates(table, n, 1 if stochastic else 0, int(k[0]), int(k[1]), _lib.stream_ptr()),
                   "apply_updates")


def _launch_apply(pairs, stochastic: bool, key, packed: bool = False) -> None:
    """pairs: [(param_tensor, update_tensor, param_index)]."""
    torch = _torch()
    if not pairs:
        return
    rows = []
    keep = []
    device = pairs[0][0].device
    for p, u, idx in pairs:
        if not isinstance(p, torch.Tensor) or not p.is_cuda:
            raise ValueError("params must be torch tensors on a ROCm device")
        if p.device != device or u.device != device:
            raise ValueError("all leaves must live on the same device")
        if not p.is_contiguous():
            raise ValueError("params must be contiguous (they are updated in place)")
        if p.numel() != u.numel():
            raise ValueError(f"param and update sizes differ ({p.numel()} vs {u.numel()})")
        pdt = {torch.bfloat16: _lib.RF_BF16, torch.float32: _lib.RF_F32, torch.float16: _lib.RF_F16}.get(p.dtype)
        if pdt is None:
            raise NotImplementedError(f"param dtype {p.dtype} is not supported (float32, bfloat16 or float16)")
        # The reference adds the update in f32 (utils.py:694-700).
        uf = u if (u.dtype == torch.float32 and u.is_contiguous()) else u.to(torch.float32).contiguous()
        keep.append(uf)
        row = _lib.ApplyLeaf()
        row.param = p.data_ptr()
        row.updates = uf.data_ptr()
        row.bits = None
        row.size = int(p.numel())
        row.param_dtype = pdt
        row.param_index = int(idx)
        rows.append(row)
    k = prng.as_key(key) if key is not None else np.zeros(2, np.uint32)
    table = (_lib.ApplyLeaf * len(rows))(*rows)
    with torch.cuda.device(device):
        _apply_call(table, len(rows), stochastic, k, packed)
    # The kernel is stream-ordered after any producer of `keep`; dropping the
    # references here is safe with torch's stream-ordered caching allocator.
    del keep


def _launch_rows(rows: bytes, n: int, device: int, stochastic: bool, key, packed: bool = False) -> None:
    """rf_apply_updates over ``n`` rf_apply_leaf records laid out in ``rows``."""
    torch = _torch()
    k = prng.as_key(key) if key is not None else np.zeros(2, np.uint32)
    buf = ctypes.create_string_buffer(rows, len(rows))
    table = ctypes.cast(buf, ctypes.POINTER(_lib.ApplyLeaf))
    with torch.cuda.device(device):
        _apply_call(table, n, stochastic, k, packed)


def apply_updates(params, updates, key=None, stochastic: bool = True, *, sr_bits: str = "jax"):
    """Apply updates with optional stochastic rounding for bf16 params
    (utils.py:648-708): bf16 leaves take ``f32(p) + f32(u)`` then SR (per-leaf
    key ``split(key, n_leaves)[i]``) or round-to-nearest-even; f32 leaves
    take ``p + u``.  None / MaskedNode leaves are left unchanged.
    ``sr_bits`` (extension): "jax" (jax.random.bits' stream) or "packed"."""
    packed = _check_sr_bits(sr_bits)
    if stochastic and key is None:
        raise ValueError(_KEY_MSG)
    # Native walk (contiguous f32/bf16 params, f32 updates, dict/list/tuple
    # containers); anything else takes the Python walk below.
    fast = _lib.pyhost().apply_rows(params, updates)
    if fast is not None:
        rows, n, device, tree = fast
        if n:
            _launch_rows(rows, n, device, stochastic, key, packed)
        return tree
    leaves, td = _tree.flatten(params, is_leaf=_is_aux_leaf)
    u_leaves = _tree.flatten_up_to(td, updates)
    pairs = []
    for i, (p, u) in enumerate(zip(leaves, u_leaves)):
        if _is_aux_leaf(p) or _is_aux_leaf(u):
            continue
        pairs.append((p, u, i))
    _launch_apply(pairs, stochastic, key, packed)
    return _tree.unflatten(td, leaves)


def apply_updates_prefix(model, updates, key=None, stochastic: bool = True, *, sr_bits: str = "jax"):
    """Equinox-compatible apply_updates where ``updates`` may be a prefix of
    ``model`` (utils.py:711-769): a None / MaskedNode update leaves the whole
    model subtree unchanged; keys are split over the update leaves."""
    packed = _check_sr_bits(sr_bits)
    if stochastic and key is None:
        raise ValueError(_KEY_MSG)
    u_leaves, u_td = _tree.flatten(updates, is_leaf=_is_aux_leaf)
    m_sub = _tree.flatten_up_to(u_td, model)
    pairs = []
    for i, (u, p) in enumerate(zip(u_leaves, m_sub)):
        if _is_aux_leaf(u) or _is_aux_leaf(p):
            continue
        pairs.append((p, u, i))
    _launch_apply(pairs, stochastic, key, packed)
    return _tree.unflatten(u_td, m_sub)


def _stochastic_round_bf16(x, key, random_bits=None, *, sr_bits: str = "jax"):
    """FP32 -> BF16 stochastic rounding by integer bit-add (utils.py:342-371).
    ``random_bits`` (testing): raw uint32 words replacing the in-kernel
    ``jax.random.bits(key, x.shape)``.  ``sr_bits`` (extension): "jax" or
    "packed" (a Threefry block per four elements)."""
    torch = _torch()
    packed = _check_sr_bits(sr_bits)
    if x.dtype == torch.bfloat16:
        return x
    if not isinstance(x, torch.Tensor) or not x.is_cuda:
        raise ValueError("x must be a torch tensor on a ROCm device")
    xf = x.to(torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    k = prng.as_key(key) if key is not None else np.zeros(2, np.uint32)
    bits = None
    if random_bits is not None:
        bits = random_bits.contiguous()
        if bits.dtype != torch.uint32 or bits.numel() != xf.numel():
            raise ValueError("random_bits must be uint32 with one word per element")
        if packed:
            raise ValueError("random_bits replace the in-kernel bits: sr_bits must stay 'jax'")
    elif key is None:
        raise ValueError("stochastic rounding requires a PRNG key.")
    with torch.cuda.device(x.device):
        if packed:
            st = _lib.lib().rf_sr_bf16_packed(xf.data_ptr(), int(xf.numel()), int(k[0]), int(k[1]), out.data_ptr(),
                                              _lib.stream_ptr())
        else:
            st = _lib.lib().rf_sr_bf16(xf.data_ptr(), int(xf.numel()), int(k[0]), int(k[1]),
                                       None if bits is None else bits.data_ptr(), out.data_ptr(), _lib.stream_ptr())
        _lib.check(st, "_stochastic_round_bf16")
    return out


def _tree_stochastic_cast(tree, target_dtype, key, *, sr_bits: str = "jax"):
    """Cast a pytree, stochastically rounding to bf16 (utils.py:374-409):
    per-leaf keys ``split(key, n_leaves)``; MaskedNode / None / non-array
    leaves pass through.  ``sr_bits``: as for _stochastic_round_bf16."""
    _check_sr_bits(sr_bits)
    torch = _torch()
    leaves, td = _tree.flatten(tree, is_leaf=_is_aux_leaf)
    keys = prng.split(key, len(leaves))
    out = []
    for leaf, k in zip(leaves, keys):
        if _is_aux_leaf(leaf) or not hasattr(leaf, "dtype"):
            out.append(leaf)
        elif leaf.dtype.is_complex and not target_dtype.is_complex:
            out.append(leaf.to(torch.complex64))
        elif target_dtype == torch.bfloat16:
            out.append(_stochastic_round_bf16(leaf, k, sr_bits=sr_bits))
        else:
            out.append(leaf.to(target_dtype))
    return _tree.unflatten(td, out)


__all__ = (
    "apply_updates",
    "apply_updates_prefix",
    "is_passthrough_leaf",
)
