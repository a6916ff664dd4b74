"""Gradient transforms of rollfast's fine-tuning builders, on MI355X kernels.

Mirror of ``src/rollfast/finetune/transforms.py``: ``clip_by_global_norm``
and ``GlobalNormClipState``.  The norm and the scaling run in
``librfadam8.so`` (``rf_clip_by_global_norm``: a multi-tensor norm pre-pass
and one multi-tensor scaling launch).  The optimizer steps also take the
same clipping fused (``adamw8_step(..., clip_global_norm=...)``), which
reads the grads once instead of reading and writing them.
"""

from __future__ import annotations

import ctypes
from typing import Any, NamedTuple

import numpy as np

from . import _lib, _tree
from ._base import GradientTransformation, is_passthrough_leaf as _is_passthrough_leaf


class GlobalNormClipState(NamedTuple):
    """State for the global-norm clipping transform (transforms.py:14-17)."""

    count: Any


def clip_by_global_norm(max_norm: float, *, axis_name=None, partition_axis_names=None,
                        replicated_axis_names=None) -> GradientTransformation:
    """Clip by global norm over the leaves (transforms.py:20-54): scale every
    leaf by ``min(1, max_norm / (norm + 1e-6))`` in the leaf dtype.  The axis
    arguments name collective axes of a multi-device reduction, which this
    single-device build does not perform; they must be None."""
    import torch

    if max_norm <= 0.0:
        raise ValueError("max_norm must be positive.")
    if axis_name is not None or partition_axis_names is not None or replicated_axis_names is not None:
        raise NotImplementedError("cross-device norm reduction is not part of this single-device build")

    def init_fn(params):
        del params
        return GlobalNormClipState(count=np.zeros((), dtype=np.int32))

    def update_fn(updates, state, params=None, stats=None):
        """``stats`` (extension): optional float32 device tensor of 2 elements
        receiving (scale, norm)."""
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
            if leaf.dtype not in (torch.float32, torch.bfloat16):
                raise NotImplementedError(f"dtype {leaf.dtype} is not supported (float32 or bfloat16)")
            src = leaf.contiguous()
            dst = torch.empty_like(src)
            row = _lib.ClipLeaf()
            row.grad = src.data_ptr()
            row.out = dst.data_ptr()
            row.size = int(src.numel())
            row.dtype = _lib.RF_BF16 if src.dtype == torch.bfloat16 else _lib.RF_F32
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
                _lib.check(_lib.lib().rf_clip_by_global_norm(table, len(rows), ctypes.c_float(float(max_norm)),
                                                             ctypes.c_void_p(stats_ptr), _lib.stream_ptr()),
                           "clip_by_global_norm")
        count = np.asarray(np.int32(int(np.asarray(state.count)) + 1), dtype=np.int32)
        return _tree.unflatten(td, out), GlobalNormClipState(count=count)

    return GradientTransformation(init_fn, update_fn)


__all__ = ("GlobalNormClipState", "clip_by_global_norm")
