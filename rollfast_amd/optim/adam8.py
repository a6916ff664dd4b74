"""AdamW with blockwise 8-bit optimizer-state moments, on MI355X HIP kernels.

Host-side mirror of ``src/rollfast/optim/adam8.py`` (rollfast): the same
public names, argument meanings, state pytree and errors.  Arrays are
``torch`` tensors on a ROCm device (torch is used for device memory and
streams only); every computation on them runs in ``librfadam8.so``:

* ``quantize_blocks`` / ``dequantize_blocks`` -> ``rf_blockwise_quantize`` /
  ``rf_blockwise_dequantize`` (reference ``adam8.py:113-204``);
* ``scale_by_adam8().update`` and ``adamw8().update`` -> one multi-tensor
  launch of the fused step kernel in update-only mode (reference
  ``adam8.py:304-389`` and the ``optax.chain`` of ``:418-443``);
* ``adamw8_step`` (new, no reference counterpart) -> the same kernel with the
  parameter write of ``rollfast.apply_updates`` fused in: one HBM pass.

Updates are in place (JAX donation semantics): the returned state shares its
tensors with the input state.  The step counter and PRNG key are host NumPy
scalars/arrays, so deriving the bias correction and the per-leaf keys never
waits on the device.
"""

from __future__ import annotations

import ctypes
import dataclasses
import math
import weakref
from typing import Any, Callable, Literal, NamedTuple, Optional, Union

import numpy as np

from .. import _lib, _tree, prng
from .._base import (
    NO_PARAMS_MSG,
    EmptyState,
    GradientTransformation,
    GradientTransformationExtraArgs,
    MaskedNode,
    MaskedState,
    ScaleByScheduleState,
    is_passthrough_leaf as _is_passthrough_leaf,
    safe_int32_increment,
)

SYMMETRIC_INT8_CODEBOOK_ID = "rollfast.symmetric_int8.neg127_pos127.v1"
DYNAMIC_SIGNED_CODEBOOK_ID = "bitsandbytes.dynamic.signed.8bit.v1"
DYNAMIC_UNSIGNED_CODEBOOK_ID = "bitsandbytes.dynamic.unsigned.8bit.v1"
BlockLayout = Literal["shard_local", "logical_global"]
CodebookQuantizer = Literal["dynamic_signed", "dynamic_unsigned", "symmetric_int8"]


def _torch():
    import torch

    return torch


# ------------------------------------------------------------- dtypes ------
def canonicalize_dtype(dtype):
    """Accept torch dtypes, NumPy dtypes or names ("float32", "bfloat16")."""
    torch = _torch()
    if isinstance(dtype, torch.dtype):
        return dtype
    name = getattr(dtype, "name", None) or getattr(dtype, "__name__", None) or str(dtype)
    name = name.replace("torch.", "").replace("jnp.", "")
    table = {
        "float32": torch.float32,
        "bfloat16": torch.bfloat16,
        "float16": torch.float16,
        "float64": torch.float64,
        "uint8": torch.uint8,
        "int8": torch.int8,
        "int32": torch.int32,
    }
    if name not in table:
        raise ValueError(f"unknown dtype {dtype!r}")
    return table[name]


def dtype_name(dtype) -> str:
    """NumPy-style dtype name ("float32", "uint8", "bfloat16")."""
    return str(dtype).replace("torch.", "")


def _is_inexact(dtype) -> bool:
    return dtype.is_floating_point or dtype.is_complex


def _rf_dtype(dtype, what: str) -> int:
    torch = _torch()
    if dtype == torch.float32:
        return _lib.RF_F32
    if dtype == torch.bfloat16:
        return _lib.RF_BF16
    if dtype == torch.float16:
        return _lib.RF_F16
    raise NotImplementedError(f"{what} dtype {dtype} is not supported (float32, bfloat16 or float16)")


def _scale_flag(dtype) -> int:
    """RF_LEAF_SCALE_* flag of a block-scale dtype (scale_dtype, adam8.py:186)."""
    torch = _torch()
    if dtype == torch.float32:
        return 0
    if dtype == torch.bfloat16:
        return _lib.RF_LEAF_SCALE_BF16
    if dtype == torch.float16:
        return _lib.RF_LEAF_SCALE_F16
    raise NotImplementedError(f"scale dtype {dtype} is not supported (float32, bfloat16 or float16)")


def _check_scale_dtype(dtype):
    _scale_flag(dtype)
    return dtype


# ------------------------------------------------------ QuantizedBlocks ----
@dataclasses.dataclass(frozen=True, eq=False)
class QuantizedBlocks:
    """Blockwise fixed-codebook 8-bit representation for one state leaf
    (adam8.py:28-101): ``values`` [nblocks, block_size] codes (uint8, or int8
    for the symmetric quantizer, padding included) and ``scales`` [nblocks]."""

    values: Any
    scales: Any
    shape: tuple
    size: int
    block_size: int
    quantizer: str = "blockwise_dynamic_signed_8bit"
    codebook_id: str = DYNAMIC_SIGNED_CODEBOOK_ID
    qmin: int = 0
    qmax: int = 255
    zero_point: int = 0
    block_layout: BlockLayout = "shard_local"

    def tree_flatten(self):
        return (self.values, self.scales), (
            self.shape,
            self.size,
            self.block_size,
            self.quantizer,
            self.codebook_id,
            self.qmin,
            self.qmax,
            self.zero_point,
            self.block_layout,
        )

    @classmethod
    def tree_unflatten(cls, aux_data, children):
        shape, size, block_size, quantizer, codebook_id, qmin, qmax, zero_point, block_layout = aux_data
        values, scales = children
        return cls(
            values=values,
            scales=scales,
            shape=shape,
            size=size,
            block_size=block_size,
            quantizer=quantizer,
            codebook_id=codebook_id,
            qmin=qmin,
            qmax=qmax,
            zero_point=zero_point,
            block_layout=block_layout,
        )

    def metadata(self) -> dict[str, Any]:
        """Exact checkpoint metadata for this quantized state leaf."""
        return {
            "quantizer": self.quantizer,
            "codebook_id": self.codebook_id,
            "qmin": self.qmin,
            "qmax": self.qmax,
            "zero_point": self.zero_point,
            "shape": self.shape,
            "size": self.size,
            "block_size": self.block_size,
            "block_layout": self.block_layout,
            "scale_dtype": dtype_name(self.scales.dtype),
            "values_dtype": dtype_name(self.values.dtype),
        }


_tree.register_node(QuantizedBlocks, lambda q: q.tree_flatten(), QuantizedBlocks.tree_unflatten)


class ScaleByAdam8State(NamedTuple):
    """State for Adam with quantized first and second moments (adam8.py:104-110)."""

    count: Any
    mu: Any
    nu: Any
    key: Any


def _is_state_leaf(x: Any) -> bool:
    return isinstance(x, QuantizedBlocks) or _is_passthrough_leaf(x)


_QUANTIZER_CODE = {
    "dynamic_signed": _lib.RF_Q_DYNAMIC_SIGNED,
    "dynamic_unsigned": _lib.RF_Q_DYNAMIC_UNSIGNED,
    "symmetric_int8": _lib.RF_Q_SYMMETRIC_INT8,
}


def _codebook_id_for_quantizer(quantizer: str) -> str:
    if quantizer == "dynamic_signed":
        return DYNAMIC_SIGNED_CODEBOOK_ID
    if quantizer == "dynamic_unsigned":
        return DYNAMIC_UNSIGNED_CODEBOOK_ID
    if quantizer == "symmetric_int8":
        return SYMMETRIC_INT8_CODEBOOK_ID
    raise ValueError(f"Unknown quantizer: {quantizer!r}.")


def _zero_code_for_quantizer(quantizer: str) -> int:
    """adam8.py:532-539: index of the codebook entry nearest zero."""
    if quantizer == "dynamic_signed":
        return 127
    return 0


def _quantizer_from_codebook_id(codebook_id: str) -> str:
    if codebook_id == DYNAMIC_SIGNED_CODEBOOK_ID:
        return "dynamic_signed"
    if codebook_id == DYNAMIC_UNSIGNED_CODEBOOK_ID:
        return "dynamic_unsigned"
    if codebook_id == SYMMETRIC_INT8_CODEBOOK_ID:
        return "symmetric_int8"
    raise ValueError(f"Unknown codebook_id: {codebook_id!r}.")


def _require_device_tensor(x, what: str):
    torch = _torch()
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{what} must be a torch.Tensor on a ROCm device, got {type(x)}")
    if not x.is_cuda:
        raise ValueError(f"{what} must live on a ROCm device (got {x.device})")
    return x


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _device_ctx(t):
    return _torch().cuda.device(t.device)


# ------------------------------------------------ quantize / dequantize ----
def quantize_blocks(
    x,
    *,
    block_size: int = 2048,
    scale_dtype=None,
    stochastic_rounding: bool = False,
    key=None,
    block_layout: BlockLayout = "shard_local",
    quantizer: CodebookQuantizer = "dynamic_signed",
    random_bits=None,
) -> QuantizedBlocks:
    """Quantize one array with fixed-codebook blockwise dynamic scales
    (adam8.py:113-187).  ``random_bits`` (extension): raw ``uint32`` words
    [nblocks*block_size] consumed by stochastic rounding instead of bits
    generated from ``key`` in the kernel."""
    torch = _torch()
    if block_size <= 0:
        raise ValueError("block_size must be positive.")
    if block_layout not in {"shard_local", "logical_global"}:
        raise ValueError("block_layout must be 'shard_local' or 'logical_global'.")
    if quantizer not in {"dynamic_signed", "dynamic_unsigned", "symmetric_int8"}:
        raise ValueError(
            "quantizer must be 'dynamic_signed', 'dynamic_unsigned', or "
            "'symmetric_int8'."
        )
    scale_dtype = _check_scale_dtype(torch.float32 if scale_dtype is None else canonicalize_dtype(scale_dtype))
    if stochastic_rounding and key is None and random_bits is None:
        raise ValueError("stochastic rounding requires a PRNG key.")
    _require_device_tensor(x, "x")
    # jnp.asarray(x, float32): f32, bf16 and f16 inputs are widened in the kernel
    x_in = x.contiguous() if x.dtype in (torch.float32, torch.bfloat16, torch.float16) else x.to(torch.float32)
    shape = tuple(x.shape)
    size = int(x.numel())
    blocks_count = max(1, math.ceil(size / block_size))
    vdtype = torch.int8 if quantizer == "symmetric_int8" else torch.uint8
    values = torch.empty((blocks_count, block_size), dtype=vdtype, device=x.device)
    scales = torch.empty((blocks_count,), dtype=scale_dtype, device=x.device)
    k = prng.as_key(key) if key is not None else np.zeros(2, np.uint32)
    bits = None
    if random_bits is not None:
        bits = _require_device_tensor(random_bits, "random_bits").contiguous()
        if bits.dtype != torch.uint32 or bits.numel() != blocks_count * block_size:
            raise ValueError("random_bits must be uint32 [nblocks * block_size]")
    with _device_ctx(x):
        _lib.check(
            _lib.lib().rf_blockwise_quantize(
                _QUANTIZER_CODE[quantizer], _ptr(x_in), _rf_dtype(x_in.dtype, "input"), size, int(block_size),
                1 if stochastic_rounding else 0, int(k[0]), int(k[1]), _ptr(bits),
                values.data_ptr(), scales.data_ptr(), _rf_dtype(scale_dtype, "scale"), _lib.stream_ptr(),
            ),
            "quantize_blocks",
        )
    if quantizer == "symmetric_int8":
        return QuantizedBlocks(
            values=values, scales=scales, shape=shape, size=size, block_size=block_size,
            quantizer="blockwise_symmetric_int8", codebook_id=SYMMETRIC_INT8_CODEBOOK_ID,
            qmin=-127, qmax=127, zero_point=0, block_layout=block_layout,
        )
    return QuantizedBlocks(
        values=values, scales=scales, shape=shape, size=size, block_size=block_size,
        quantizer=f"blockwise_{quantizer}_8bit", codebook_id=_codebook_id_for_quantizer(quantizer),
        qmin=0, qmax=255, zero_point=_zero_code_for_quantizer(quantizer), block_layout=block_layout,
    )


def dequantize_blocks(blocks: QuantizedBlocks, *, dtype=None):
    """Dequantize a ``QuantizedBlocks`` leaf and remove deterministic padding
    (adam8.py:190-204)."""
    torch = _torch()
    dtype = torch.float32 if dtype is None else canonicalize_dtype(dtype)
    quantizer = _quantizer_from_codebook_id(blocks.codebook_id)
    values = _require_device_tensor(blocks.values, "values").contiguous()
    scales = _require_device_tensor(blocks.scales, "scales").contiguous()
    _check_scale_dtype(scales.dtype)  # values * scales.astype(float32) (adam8.py:202)
    out_dtype = dtype if dtype in (torch.float32, torch.bfloat16, torch.float16) else torch.float32
    out = torch.empty((blocks.size,), dtype=out_dtype, device=values.device)
    with _device_ctx(values):
        _lib.check(
            _lib.lib().rf_blockwise_dequantize(
                _QUANTIZER_CODE[quantizer], values.data_ptr(), scales.data_ptr(), _rf_dtype(scales.dtype, "scale"),
                int(blocks.size), int(blocks.block_size), _rf_dtype(out_dtype, "output"), out.data_ptr(),
                _lib.stream_ptr(),
            ),
            "dequantize_blocks",
        )
    out = out.reshape(blocks.shape)
    return out if out_dtype == dtype else out.to(dtype)


# ------------------------------------------------------ byte accounting ----
def quantized_nbytes(blocks: QuantizedBlocks) -> int:
    """Materialized array bytes used by one quantized state leaf (adam8.py:207-212)."""
    return int(blocks.values.numel() * blocks.values.element_size()) + int(
        blocks.scales.numel() * blocks.scales.element_size()
    )


def _leaf_nbytes(leaf) -> int:
    if hasattr(leaf, "element_size") and hasattr(leaf, "numel"):
        return int(leaf.numel() * leaf.element_size())
    if hasattr(leaf, "dtype") and hasattr(leaf, "size") and hasattr(leaf, "itemsize"):
        return int(leaf.size * leaf.itemsize)
    return 0


def tree_state_nbytes(tree: Any) -> int:
    """Array storage bytes in an optimizer-state pytree (adam8.py:215-224)."""
    total = 0
    for leaf in _tree.leaves(tree, is_leaf=_is_state_leaf):
        if isinstance(leaf, QuantizedBlocks):
            total += quantized_nbytes(leaf)
        else:
            total += _leaf_nbytes(leaf)
    return total


def estimate_quantized_moment_bytes(size: int, *, block_size: int = 2048, scale_dtype=None) -> int:
    """Bytes for one quantized moment leaf with ``size`` elements (adam8.py:227-240)."""
    torch = _torch()
    scale_dtype = torch.float32 if scale_dtype is None else canonicalize_dtype(scale_dtype)
    if size <= 0:
        return 0
    blocks_count = max(1, math.ceil(size / block_size))
    itemsize = torch.tensor([], dtype=scale_dtype).element_size()
    return int(blocks_count * block_size) + int(blocks_count * itemsize)


# ----------------------------------------------------- state construction --
@dataclasses.dataclass(frozen=True)
class _Config:
    b1: Any
    b2: Any
    eps: Any
    eps_root: Any
    block_size: int
    min_size: int
    scale_dtype: Any
    fallback_dtype: Any
    stochastic_rounding: bool
    block_layout: str
    quantize: bool
    nesterov: bool
    key: Any
    exact: bool
    sr_bits: str = "jax"


SR_BITS = ("jax", "packed")


def _check_sr_bits(sr_bits) -> str:
    """The bit source of the in-kernel stochastic roundings: "jax" (the
    default) draws jax.random.bits' stream, one Threefry-2x32-20 block per
    32-bit word (bitwise the reference's layout); "packed" (no reference
    counterpart) spends one block on four param roundings, or on both
    moments' draws of a pair of elements (16 bits each, completed to the
    uniform's 23 from a second block only when they leave the draw open),
    from the same per-leaf keys."""
    if sr_bits not in SR_BITS:
        raise ValueError(f"sr_bits must be one of {SR_BITS}, got {sr_bits!r}")
    return sr_bits


def _init_moment_leaf(param, cfg: _Config, quantizer: str):
    """adam8.py:605-630: zeros of fallback_dtype, quantized when eligible."""
    torch = _torch()
    if _is_passthrough_leaf(param):
        return param
    zeros_dtype = cfg.fallback_dtype
    if cfg.quantize and param.numel() >= cfg.min_size and _is_inexact(param.dtype):
        size = int(param.numel())
        blocks_count = max(1, math.ceil(size / cfg.block_size))
        # quantize_blocks(zeros): every block has absmax 0 -> scale 1.0 and
        # every code is the codebook's zero code.
        return QuantizedBlocks(
            values=torch.full((blocks_count, cfg.block_size), _zero_code_for_quantizer(quantizer),
                              dtype=torch.uint8, device=param.device),
            scales=torch.ones((blocks_count,), dtype=cfg.scale_dtype, device=param.device),
            shape=tuple(param.shape),
            size=size,
            block_size=cfg.block_size,
            quantizer=f"blockwise_{quantizer}_8bit",
            codebook_id=_codebook_id_for_quantizer(quantizer),
            qmin=0,
            qmax=255,
            zero_point=_zero_code_for_quantizer(quantizer),
            block_layout=cfg.block_layout,
        )
    return torch.zeros(param.shape, dtype=zeros_dtype, device=param.device)


def _init_moment_tree(params, cfg: _Config, quantizer: str):
    return _tree.tree_map(lambda p: _init_moment_leaf(p, cfg, quantizer), params, is_leaf=_is_passthrough_leaf)


def _as_f32(x) -> np.float32:
    if hasattr(x, "detach"):
        x = x.detach().cpu().item()
    return np.float32(x)


def _one_minus(b) -> np.float32:
    """``1.0 - b`` as the reference evaluates it: in double for a Python
    scalar (then f32 when it meets the f32 arrays), in f32 for an array."""
    if isinstance(b, (int, float)):
        return np.float32(1.0 - b)
    return np.float32(1.0) - _as_f32(b)


def _bias_correction(b, count: int) -> np.float32:
    """``1.0 - b**count`` in f32 (adam8.py:338-339; f32 pow)."""
    with np.errstate(all="ignore"):
        return np.float32(1.0) - np.power(_as_f32(b), np.float32(count))


# ------------------------------------------------------------ the engine ---
class _LeafPlan:
    """A cached ``rf_adam8_plan`` for one leaf-table structure."""

    def __init__(self, table, n: int, apply: bool):
        handle = ctypes.c_void_p()
        _lib.check(_lib.lib().rf_adam8_plan_create(table, n, 1 if apply else 0, ctypes.byref(handle)),
                   "rf_adam8_plan_create")
        self.handle = handle
        self.n = n

    def run(self, table, hp, stream):
        _lib.check(_lib.lib().rf_adam8_plan_run_leaves(self.handle, table, self.n, ctypes.byref(hp), stream),
                   "rf_adam8_plan_run_leaves")

    def wait_prepass(self):
        _lib.check(_lib.lib().rf_adam8_plan_wait_prepass(self.handle), "rf_adam8_plan_wait_prepass")

    def stream_probe(self, stream) -> int:
        """Enqueue the plan's stream probe (the fused step's bytes, no
        arithmetic) over its creation-time buffers; returns the 2048-element
        blocks it moves."""
        blocks = ctypes.c_int64(0)
        _lib.check(_lib.lib().rf_adam8_plan_stream_probe(self.handle, stream, ctypes.byref(blocks)),
                   "rf_adam8_plan_stream_probe")
        return int(blocks.value)

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            try:
                _lib.lib().rf_adam8_plan_destroy(h)
            except Exception:
                pass
            self.handle = None


def _aligned(t, a: int) -> bool:
    return t is None or t.data_ptr() % a == 0


class _AllLeaves:
    """Decay mask of every leaf (``weight_decay_mask=None``): it needs no
    per-leaf list, so the steady-state step does not walk the tree for it."""

    def __getitem__(self, i) -> bool:
        return True

    def __repr__(self) -> str:
        return "ALL_LEAVES"


ALL_LEAVES = _AllLeaves()


def _buffers(m, v, p) -> tuple:
    """A leaf's moment buffers and param tensors."""
    if isinstance(m, QuantizedBlocks):
        t = (m.values, m.scales, v.values, v.scales)
    else:
        t = (m, v)
    return t + ((p,) if p is not None else ())


def _buffer_ptrs(m, v, p) -> tuple:
    """Device addresses of a leaf's moment buffers and param."""
    return tuple(t.data_ptr() for t in _buffers(m, v, p))


class _Engine:
    """Builds the leaf table for a step and launches it (one launch per tree).

    The table of the previous call is kept with weak references to the
    tensors it points at.  When the next call passes the same tree structure,
    the same param and moment objects (updated in place, as this API does)
    and grads of the same dtypes and sizes, only the grad pointers are
    rewritten: the per-leaf validation of the first call is not repeated.
    """

    # optim/adam.py's scale_by_adam adds its own decay term (weight 0 inside
    # adamw) whenever it is given params; scale_by_adam8 has none
    own_zero_decay = False

    def __init__(self, cfg: _Config):
        self.cfg = cfg
        self._plans: dict = {}
        self._last = None

    @staticmethod
    def ema_weight(b1) -> np.float32:
        """Gradient weight of the first-moment EMA: ``1.0 - b1`` as adam8.py:323
        evaluates it."""
        return _one_minus(b1)

    @staticmethod
    def split_keys(state_key):
        """(moment-SR key of mu, of nu, next state key): adam8.py:306."""
        key_mu, key_nu, next_key = prng.split(state_key, 3)
        return key_mu, key_nu, next_key

    @staticmethod
    def new_state(state, count_inc, next_key):
        return ScaleByAdam8State(count=np.asarray(count_inc, dtype=np.int32), mu=state.mu, nu=state.nu,
                                 key=next_key)

    # bf16 fallback moments are stored with stochastic rounding (adamw8 rounds
    # them to nearest even, adam8.py:688).
    store_sr = False

    # -- full table build (first call, or anything changed) -----------------
    def _build_rows(self, g_leaves, mu_leaves, nu_leaves, p_leaves, *, apply, decay_mask, random_bits,
                    zero_decay=False):
        """Leaf table rows of one launch.  ``zero_decay``: every row also gets
        optim/adam.py's weight-0 decay term (``RF_LEAF_ZERO_DECAY``), so every
        row needs its param."""
        torch = _torch()
        n = len(g_leaves)
        out_leaves: list = [None] * n
        rows = []
        structure = []
        # per row: (leaf index, weakrefs of mu, nu, param, weakrefs of the
        # buffer tensors, their device pointers, grad dtype code, size,
        # 16-byte aligned) -- the record rf_pyhost.cpp's refresh() reads
        refs = []
        device = None
        for i in range(n):
            g, m, v = g_leaves[i], mu_leaves[i], nu_leaves[i]
            if _is_passthrough_leaf(m) or _is_passthrough_leaf(g):
                out_leaves[i] = m if _is_passthrough_leaf(m) else g
                continue
            _require_device_tensor(g, "gradient")
            if device is None:
                device = g.device
            if g.device != device:
                raise ValueError("all leaves must live on the same device")
            gdt = _rf_dtype(g.dtype, "gradient")
            if not g.is_contiguous():
                g = g.contiguous()
            size = int(g.numel())
            row = _lib.Adam8Leaf()
            row.grad = g.data_ptr()
            row.size = size
            row.grad_dtype = gdt
            row.state_index = i
            row.param_index = i
            decays = bool(decay_mask[i]) if decay_mask is not None else False
            p = p_leaves[i] if p_leaves is not None else None
            needs_p = apply or decays or zero_decay
            if needs_p and (p is None or _is_passthrough_leaf(p)):
                raise ValueError(NO_PARAMS_MSG)
            if needs_p:
                _require_device_tensor(p, "param")
                if p.device != device:
                    raise ValueError("all leaves must live on the same device")
                if not p.is_contiguous():
                    raise ValueError("params must be contiguous (they are updated in place)")
                if int(p.numel()) != size:
                    raise ValueError(f"param and gradient sizes differ ({p.numel()} vs {size})")
                row.param = p.data_ptr()
                row.param_dtype = _rf_dtype(p.dtype, "param")
            else:
                p = None
                row.param_dtype = _lib.RF_F32
            row.flags = (_lib.RF_LEAF_DECAY if decays else 0) | (_lib.RF_LEAF_ZERO_DECAY if zero_decay else 0)
            if isinstance(m, QuantizedBlocks):
                if not isinstance(v, QuantizedBlocks):
                    raise ValueError("first and second moment leaves differ in kind")
                if m.codebook_id != DYNAMIC_SIGNED_CODEBOOK_ID or v.codebook_id != DYNAMIC_UNSIGNED_CODEBOOK_ID:
                    raise NotImplementedError("moment leaves must use the dynamic signed/unsigned codebooks")
                if m.size != size or v.size != size or m.block_size != v.block_size:
                    raise ValueError("quantized moment leaf does not match its gradient")
                for t in (m.values, v.values, m.scales, v.scales):
                    _require_device_tensor(t, "moment")
                    if t.device != device:
                        raise ValueError("all leaves must live on the same device")
                    if not t.is_contiguous():
                        raise ValueError("moment buffers must be contiguous (they are updated in place)")
                if m.scales.dtype != v.scales.dtype:
                    raise ValueError("first and second moment scales differ in dtype")
                row.flags |= _scale_flag(m.scales.dtype)
                nb = max(1, math.ceil(size / m.block_size))
                for t, want in ((m.values, nb * m.block_size), (v.values, nb * m.block_size), (m.scales, nb),
                                (v.scales, nb)):
                    if int(t.numel()) != want:
                        raise ValueError("quantized moment buffers do not match size and block_size")
                row.moment_kind = _lib.RF_MOMENT_QUANTIZED
                row.block_size = int(m.block_size)
                row.mu = m.values.data_ptr()
                row.mu_scales = m.scales.data_ptr()
                row.nu = v.values.data_ptr()
                row.nu_scales = v.scales.data_ptr()
                align_ok = m.values.data_ptr() % 8 == 0 and v.values.data_ptr() % 8 == 0
            else:
                _require_device_tensor(m, "first moment")
                _require_device_tensor(v, "second moment")
                if m.device != device or v.device != device:
                    raise ValueError("all leaves must live on the same device")
                if m.dtype != v.dtype or int(m.numel()) != size or int(v.numel()) != size:
                    raise ValueError("fallback moment leaf does not match its gradient")
                if not (m.is_contiguous() and v.is_contiguous()):
                    raise ValueError("moment buffers must be contiguous (they are updated in place)")
                if m.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                    raise NotImplementedError(f"fallback moment dtype {m.dtype} is not supported")
                row.moment_kind = {torch.bfloat16: _lib.RF_MOMENT_BF16, torch.float16: _lib.RF_MOMENT_F16}.get(
                    m.dtype, _lib.RF_MOMENT_F32)
                if self.store_sr and m.dtype == torch.bfloat16:
                    row.flags |= _lib.RF_LEAF_STORE_SR
                row.mu = m.data_ptr()
                row.nu = v.data_ptr()
                align_ok = m.data_ptr() % 16 == 0 and v.data_ptr() % 16 == 0
            out = None
            if not apply:
                out = torch.empty(g.shape, dtype=torch.float32, device=g.device)
                row.updates = out.data_ptr()
                out_leaves[i] = out
            if random_bits is not None and i in random_bits:
                mb, vb, pb = random_bits[i]
                row.mu_bits = _ptr(mb)
                row.nu_bits = _ptr(vb)
                row.param_bits = _ptr(pb)
            align_ok = (
                align_ok
                and g.data_ptr() % 16 == 0
                and (row.param is None or row.param % 16 == 0)
                and (out is None or out.data_ptr() % 16 == 0)
            )
            rows.append(row)
            structure.append((size, row.block_size, row.param_dtype, gdt, row.moment_kind, i, row.flags, align_ok,
                              row.mu_bits is not None or row.nu_bits is not None, row.param_bits is not None))
            bufs = _buffers(m, v, p)
            refs.append((i, weakref.ref(m), weakref.ref(v), None if p is None else weakref.ref(p),
                         tuple(weakref.ref(t) for t in bufs), tuple(t.data_ptr() for t in bufs), gdt, size,
                         align_ok))
        return rows, structure, refs, out_leaves, device

    # -- cached table (same objects as the previous call) -------------------
    def _reuse_rows(self, last, g_leaves, mu_leaves, nu_leaves, p_leaves, apply):
        """Rewrites the grad (and, update-only mode, output) pointers of the
        previous table when every other buffer is the same object on the same
        storage; returns the out-leaf list, or None when anything differs."""
        torch = _torch()
        Tensor = torch.Tensor
        table = last["table"]
        dev = last["device"]
        dev_index = dev.index
        n = len(g_leaves)
        out_leaves: list = [None] * n
        refs = last["refs"]
        if len(refs) != sum(1 for i in range(n) if not (_is_passthrough_leaf(mu_leaves[i])
                                                        or _is_passthrough_leaf(g_leaves[i]))):
            return None
        gdtypes = (torch.float32, torch.bfloat16)  # by RF_F32 / RF_BF16
        for j, (i, mref, vref, pref, _bufrefs, ptrs, gdt, size, align_ok) in enumerate(refs):
            gdtype = gdtypes[gdt]
            g, m, v = g_leaves[i], mu_leaves[i], nu_leaves[i]
            if mref() is not m or vref() is not v:
                return None
            p = None
            if pref is not None:
                p = p_leaves[i] if p_leaves is not None else None
                if pref() is not p:
                    return None
            # same objects, same storage (a `.data` swap changes the pointer)
            if _buffer_ptrs(m, v, p) != ptrs:
                return None
            if not isinstance(g, Tensor) or g.dtype is not gdtype or g.get_device() != dev_index:
                return None
            if g.numel() != size or not g.is_contiguous():
                return None
            gp = g.data_ptr()
            if align_ok and gp & 15:
                return None
            row = table[j]
            row.grad = gp
            if not apply:
                out = torch.empty(g.shape, dtype=torch.float32, device=dev)
                row.updates = out.data_ptr()
                out_leaves[i] = out
        for i in range(n):
            m, g = mu_leaves[i], g_leaves[i]
            if _is_passthrough_leaf(m) or _is_passthrough_leaf(g):
                out_leaves[i] = m if _is_passthrough_leaf(m) else g
        return out_leaves

    def _launch(self, table, n_rows, device, plan, count_inc, key_mu, key_nu, *, apply, decay_mask,
                weight_decay, neg_lr, param_key, param_sr, random_bits, clip_global_norm, clip_stats,
                skip_nonfinite, finite_out, finite_host, magma_sums=None):
        """Scalars of the step (adam8.py:322-339 and the optax chain) and the
        plan launch over ``table``.  ``magma_sums``: a device f64 tensor of
        3 per table row that the launch fills with the rows' Magma sums."""
        torch = _torch()
        cfg = self.cfg
        flags = 0
        if cfg.nesterov:
            flags |= _lib.RF_NESTEROV
        if neg_lr is not None:
            flags |= _lib.RF_LR
        if decay_mask is not None and isinstance(weight_decay, (int, float)):
            flags |= _lib.RF_DECAY_WEAK
        if cfg.stochastic_rounding:
            flags |= _lib.RF_MOMENT_SR
        if apply and param_sr:
            flags |= _lib.RF_PARAM_SR
        if cfg.exact:
            flags |= _lib.RF_EXACT
        if random_bits is not None:
            flags |= _lib.RF_FED_BITS
        elif cfg.sr_bits == "packed":
            flags |= _lib.RF_PACKED_BITS
        if skip_nonfinite:
            flags |= _lib.RF_SKIP_NONFINITE

        hp = _common_hparams(cfg, count_inc, flags, param_key, clip_global_norm, clip_stats, finite_out,
                             finite_host)
        hp.one_minus_b1 = self.ema_weight(cfg.b1)
        hp.weight_decay = _as_f32(weight_decay) if weight_decay is not None else np.float32(0.0)
        hp.neg_lr = neg_lr if neg_lr is not None else np.float32(1.0)
        hp.key_mu[0], hp.key_mu[1] = int(key_mu[0]), int(key_mu[1])
        hp.key_nu[0], hp.key_nu[1] = int(key_nu[0]), int(key_nu[1])
        if magma_sums is not None:
            hp.magma_sums = magma_sums.data_ptr()

        if n_rows:
            with torch.cuda.device(device):
                plan.run(table, hp, _lib.stream_ptr())
                if finite_host is not None:
                    plan.wait_prepass()

    def run(
        self,
        updates,
        state: ScaleByAdam8State,
        params,
        *,
        apply: bool,
        decay_mask: Optional[list],
        weight_decay,
        neg_lr: Optional[np.float32],
        param_key=None,
        param_sr: bool = False,
        random_bits: Optional[dict] = None,
        clip_global_norm: Optional[float] = None,
        clip_stats=None,
        skip_nonfinite: bool = False,
        finite_out=None,
        finite_host=None,
        magma_sums=None,
        zero_decay: bool = False,
    ):
        torch = _torch()
        cfg = self.cfg
        key_mu, key_nu, next_key = self.split_keys(state.key)
        mask_key = (decay_mask if decay_mask is None or decay_mask is ALL_LEAVES else tuple(decay_mask),
                    bool(zero_decay))
        count_inc = safe_int32_increment(int(np.asarray(state.count)))

        # Steady state of the fused step (same tree, params and moment objects
        # as the previous call): the native fast path walks the four trees
        # and rewrites the grad pointers of the cached table.
        last = self._last
        if (last is not None and random_bits is None and last["apply"] == apply and last["n"]
                and last["mask"] == mask_key):
            host = _lib.pyhost()
            lists = host.gather(updates, state.mu, state.nu, params)
            addr = ctypes.addressof(last["table"])
            if lists is not None and host.refresh(*lists, last["refs"], addr, last["device"].index):
                out_tree = None
                if not apply:  # f32 outputs: one buffer, a view per leaf (reused once nothing holds it)
                    with torch.cuda.device(last["device"]):
                        out_tree = host.updates_out(updates, lists[0], lists[1], last["refs"], addr,
                                                    last.setdefault("ucache", []))
                self._launch(last["table"], last["n"], last["device"], last["plan"], count_inc, key_mu, key_nu,
                             apply=apply, decay_mask=decay_mask, weight_decay=weight_decay, neg_lr=neg_lr,
                             param_key=param_key, param_sr=param_sr, random_bits=None,
                             clip_global_norm=clip_global_norm, clip_stats=clip_stats,
                             skip_nonfinite=skip_nonfinite, finite_out=finite_out, finite_host=finite_host,
                             magma_sums=magma_sums)
                return out_tree, self.new_state(state, count_inc, next_key)

        g_leaves, g_td = _tree.flatten(updates, is_leaf=_is_passthrough_leaf)
        mu_leaves = _tree.flatten_up_to(g_td, state.mu) if g_td.num_leaves else []
        nu_leaves = _tree.flatten_up_to(g_td, state.nu) if g_td.num_leaves else []
        p_leaves = None
        if params is not None:
            p_leaves = _tree.flatten_up_to(g_td, params)

        last = self._last
        out_leaves = None
        if (last is not None and random_bits is None and last["apply"] == apply and last["mask"] == mask_key
                and last["td"] == g_td):
            out_leaves = self._reuse_rows(last, g_leaves, mu_leaves, nu_leaves, p_leaves, apply)
        if out_leaves is not None:
            table, n_rows, device, plan = last["table"], last["n"], last["device"], last["plan"]
        else:
            self._last = None
            if len(_tree.leaves(state.mu, is_leaf=_is_state_leaf)) != len(g_leaves):
                raise ValueError("updates and optimizer state have different tree structures")
            rows, structure, refs, out_leaves, device = self._build_rows(
                g_leaves, mu_leaves, nu_leaves, p_leaves, apply=apply, decay_mask=decay_mask,
                random_bits=random_bits, zero_decay=zero_decay)
            n_rows = len(rows)
            table = (_lib.Adam8Leaf * n_rows)(*rows) if rows else None
            plan = None
            if rows:
                skey = (bool(apply), device.index, tuple(structure))
                plan = self._plans.get(skey)
                if plan is None:
                    with torch.cuda.device(device):
                        plan = _LeafPlan(table, n_rows, apply)
                    if len(self._plans) > 64:
                        self._plans.clear()
                    self._plans[skey] = plan
                if random_bits is None:
                    self._last = {"apply": apply, "mask": mask_key, "td": g_td, "refs": refs, "table": table,
                                  "n": n_rows, "device": device, "plan": plan}

        self._launch(table, n_rows, device, plan, count_inc, key_mu, key_nu, apply=apply,
                     decay_mask=decay_mask, weight_decay=weight_decay, neg_lr=neg_lr, param_key=param_key,
                     param_sr=param_sr, random_bits=random_bits, clip_global_norm=clip_global_norm,
                     clip_stats=clip_stats, skip_nonfinite=skip_nonfinite, finite_out=finite_out,
                     finite_host=finite_host, magma_sums=magma_sums)

        new_state = self.new_state(state, count_inc, next_key)
        out_tree = _tree.unflatten(g_td, out_leaves) if not apply else None
        return out_tree, new_state


def _common_hparams(cfg: _Config, count_inc: int, flags: int, param_key, clip_global_norm, clip_stats, finite_out,
                    finite_host):
    """The launch scalars every leaf shares: betas, bias corrections at
    ``count_inc`` (adam8.py:336-339), eps, flags, the param-SR key, clipping
    and the finite flag outputs."""
    torch = _torch()
    hp = _lib.Adam8Hparams()
    hp.b1 = _as_f32(cfg.b1)
    hp.nesterov_one_minus_b1 = _one_minus(cfg.b1)
    hp.b2 = _as_f32(cfg.b2)
    hp.one_minus_b2 = _one_minus(cfg.b2)
    hp.bc1 = _bias_correction(cfg.b1, count_inc)
    hp.bc2 = _bias_correction(cfg.b2, count_inc)
    hp.bc1_next = _bias_correction(cfg.b1, safe_int32_increment(count_inc))
    hp.eps = _as_f32(cfg.eps)
    hp.eps_root = _as_f32(cfg.eps_root)
    hp.flags = flags
    if param_key is not None:
        pk = prng.as_key(param_key)
        hp.key_param[0], hp.key_param[1] = int(pk[0]), int(pk[1])
    if clip_global_norm is not None:
        if not (float(clip_global_norm) > 0.0) or not math.isfinite(float(clip_global_norm)):
            raise ValueError("max_norm must be positive.")
        hp.clip_max_norm = float(clip_global_norm)
        if clip_stats is not None:
            _require_device_tensor(clip_stats, "clip_stats")
            if clip_stats.dtype != torch.float32 or clip_stats.numel() < 2 or not clip_stats.is_contiguous():
                raise ValueError("clip_stats must be a contiguous float32 device tensor of 2 elements")
            hp.clip_out = clip_stats.data_ptr()
    if finite_out is not None:
        hp.finite_out = finite_out.data_ptr()
    if finite_host is not None:
        hp.finite_host = finite_host.data_ptr()
    return hp


def _validate(block_size, min_size, block_layout, fallback_dtype, scale_dtype):
    torch = _torch()
    if block_size <= 0:
        raise ValueError("block_size must be positive.")
    if min_size < 0:
        raise ValueError("min_size must be non-negative.")
    if block_layout not in {"shard_local", "logical_global"}:
        raise ValueError("block_layout must be 'shard_local' or 'logical_global'.")
    _check_scale_dtype(scale_dtype)
    if fallback_dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise NotImplementedError("fallback_dtype must be float32, bfloat16 or float16")


class _ScaleByAdam8Update:
    """``scale_by_adam8(...).update`` (adam8.py:304-389): Adam direction only."""

    def __init__(self, engine: _Engine):
        self.engine = engine

    def _step(self, updates, state, params, *, apply: bool, skip_nonfinite=False, finite_out=None,
              finite_host=None, clip_global_norm=None, clip_stats=None, **fused_only):
        del params, fused_only  # param_key, param_sr, random_bits: fused-step arguments
        if apply:
            raise TypeError("scale_by_adam8 has no learning rate: the fused step needs adamw8(...)")
        return self.engine.run(updates, state, None, apply=False, decay_mask=None, weight_decay=None, neg_lr=None,
                               skip_nonfinite=skip_nonfinite, finite_out=finite_out, finite_host=finite_host,
                               clip_global_norm=clip_global_norm, clip_stats=clip_stats)

    def __call__(self, updates, state, params=None):
        return self._step(updates, state, params, apply=False)


def scale_by_adam8(
    b1=0.9,
    b2=0.999,
    eps=1e-8,
    eps_root=0.0,
    *,
    block_size: int = 2048,
    min_size: int = 4096,
    scale_dtype=None,
    fallback_dtype=None,
    stochastic_rounding: bool = False,
    block_layout: BlockLayout = "shard_local",
    quantize: bool = True,
    nesterov: bool = False,
    key=None,
    exact: bool = False,
    sr_bits: str = "jax",
) -> GradientTransformation:
    """Rescale gradients by Adam while storing eligible moments as 8-bit
    blocks (adam8.py:243-391).  ``exact`` (extension): IEEE division and
    square root in the update direction instead of the hardware
    reciprocal/square-root (moments, codes and scales are bit-exact either
    way).  ``sr_bits`` (extension): the random-bit source of the moments'
    stochastic rounding and of the fused step's param rounding, "jax"
    (jax.random.bits' layout) or "packed" (one Threefry block per pair of
    elements for both moments, per four elements for params)."""
    torch = _torch()
    scale_dtype = torch.float32 if scale_dtype is None else canonicalize_dtype(scale_dtype)
    fallback_dtype = torch.float32 if fallback_dtype is None else canonicalize_dtype(fallback_dtype)
    _validate(block_size, min_size, block_layout, fallback_dtype, scale_dtype)
    cfg = _Config(b1, b2, eps, eps_root, int(block_size), int(min_size), scale_dtype, fallback_dtype,
                  bool(stochastic_rounding), block_layout, bool(quantize), bool(nesterov), key, bool(exact),
                  _check_sr_bits(sr_bits))
    engine = _Engine(cfg)

    def init_fn(params):
        key_mu, key_nu, next_key = prng.split(prng.fresh_key(cfg.key), 3)
        del key_mu, key_nu  # zero state: quantize_blocks(zeros) draws no random bits
        mu = _init_moment_tree(params, cfg, "dynamic_signed")
        nu = _init_moment_tree(params, cfg, "dynamic_unsigned")
        return ScaleByAdam8State(count=np.zeros((), dtype=np.int32), mu=mu, nu=nu, key=next_key)

    return GradientTransformation(init_fn, _ScaleByAdam8Update(engine))


def _decay_mask_leaves(mask, params, n_leaves: int) -> list:
    """Per-leaf booleans of an optax mask (a prefix tree of bools or a
    callable on params), aligned with the flattened params."""
    if mask is None:
        return [True] * n_leaves
    mask_tree = mask(params) if callable(mask) else mask
    m_leaves, m_td = _tree.flatten(mask_tree, is_leaf=lambda x: isinstance(x, bool))
    subtrees = _tree.flatten_up_to(m_td, params)
    out: list = []
    for mval, sub in zip(m_leaves, subtrees):
        count = len(_tree.leaves(sub, is_leaf=_is_passthrough_leaf))
        out.extend([bool(mval)] * count)
    if len(out) != n_leaves:
        raise ValueError("weight_decay_mask does not match the params tree")
    return out


def decay_link_state(weight_decay, weight_decay_mask):
    """Initial state of the chain's add_decayed_weights link: empty for a
    scalar decay, the schedule's step count (0) for a schedule; wrapped by
    optax.masked's state when a mask is given."""
    inner = ScaleByScheduleState(count=np.zeros((), dtype=np.int32)) if callable(weight_decay) else EmptyState()
    return MaskedState(inner) if weight_decay_mask is not None else inner


class _Adamw8Update:
    """``adamw8(...).update``: the optax chain scale_by_adam8 ->
    add_decayed_weights -> scale_by_learning_rate in one launch."""

    def __init__(self, engine: _Engine, learning_rate, weight_decay, weight_decay_mask, wd_nonzero: bool):
        self.engine = engine
        self.learning_rate = learning_rate
        self.weight_decay = weight_decay
        self.weight_decay_mask = weight_decay_mask
        self.wd_nonzero = wd_nonzero

    def _lr(self, lr_state):
        """(-lr as f32, new lr state) per optax scale_by_learning_rate."""
        lr = self.learning_rate
        if callable(lr):
            count = int(np.asarray(lr_state.count))
            value = _as_f32(lr(np.asarray(count, dtype=np.int32)))
            return np.float32(-value), ScaleByScheduleState(
                count=np.asarray(safe_int32_increment(count), dtype=np.int32))
        return np.float32(-_as_f32(lr)) if not isinstance(lr, (int, float)) else np.float32(-lr), lr_state

    def _wd(self, state):
        """(decay for the launch, new add_decayed_weights state) of the
        chain's decay link (adam8.py:433-443).  A Python scalar stays a
        Python scalar: wd * p is then weak-typed (kept in the dtype of bf16
        and f16 params).  A schedule (weight_decay is ScalarOrSchedule,
        adam8.py:400) is evaluated at the link's own step count, which starts
        at 0 and advances with a saturating increment, as optax's schedules
        are (scale_by_learning_rate; the reference's own decay,
        optim/adam.py:186, likewise reads the count before the step).  Its
        value is an f32 array scalar, so wd * p is an f32 product for every
        param dtype.  ``state``: the whole chain state."""
        wd = self.weight_decay
        if not self.wd_nonzero:
            return None, None
        link = state[1]
        if not callable(wd):
            return wd, link
        inner = link.inner_state if isinstance(link, MaskedState) else link
        count = int(np.asarray(inner.count))
        value = np.float32(_as_f32(wd(np.asarray(count, dtype=np.int32))))
        new_inner = ScaleByScheduleState(count=np.asarray(safe_int32_increment(count), dtype=np.int32))
        return value, (MaskedState(new_inner) if isinstance(link, MaskedState) else new_inner)

    def new_chain_state(self, state, new_adam, new_decay, new_lr_state):
        """The chain's state tuple after a step."""
        mid = tuple(state[1:-1])
        if self.wd_nonzero:
            mid = (new_decay,) + mid[1:]
        return (new_adam,) + mid + (new_lr_state,)

    def _step(self, updates, state, params, *, apply: bool, param_key=None, param_sr=False, random_bits=None,
              clip_global_norm=None, clip_stats=None, skip_nonfinite=False, finite_out=None, finite_host=None):
        adam_state = state[0]
        lr_state = state[-1]
        neg_lr, new_lr_state = self._lr(lr_state)
        wd, new_decay = self._wd(state)
        decay_mask = None
        if self.wd_nonzero:
            if params is None:
                raise ValueError(NO_PARAMS_MSG)
            if self.weight_decay_mask is None:
                decay_mask = ALL_LEAVES
            else:
                n = len(_tree.leaves(updates, is_leaf=_is_passthrough_leaf))
                decay_mask = _decay_mask_leaves(self.weight_decay_mask, params, n)
        out, new_adam = self.engine.run(
            updates, adam_state, params, apply=apply, decay_mask=decay_mask, weight_decay=wd, neg_lr=neg_lr,
            param_key=param_key, param_sr=param_sr, random_bits=random_bits,
            clip_global_norm=clip_global_norm, clip_stats=clip_stats, skip_nonfinite=skip_nonfinite,
            finite_out=finite_out, finite_host=finite_host,
            zero_decay=self.engine.own_zero_decay and params is not None,
        )
        return out, self.new_chain_state(state, new_adam, new_decay, new_lr_state)

    def __call__(self, updates, state, params=None, **extra_args):
        del extra_args
        return self._step(updates, state, params, apply=False)


def adamw8(
    learning_rate,
    b1=0.9,
    b2=0.999,
    eps=1e-8,
    eps_root=0.0,
    weight_decay=1e-4,
    weight_decay_mask: Optional[Union[Any, Callable[[Any], Any]]] = None,
    *,
    block_size: int = 2048,
    min_size: int = 4096,
    scale_dtype=None,
    fallback_dtype=None,
    stochastic_rounding: bool = False,
    block_layout: BlockLayout = "shard_local",
    quantize: bool = True,
    nesterov: bool = False,
    use_magma: bool = False,
    key=None,
    exact: bool = False,
    sr_bits: str = "jax",
) -> GradientTransformationExtraArgs:
    """AdamW whose eligible moment leaves use blockwise 8-bit codebook state
    (adam8.py:394-443).  ``exact`` and ``sr_bits``: as for scale_by_adam8.  The state is the chain's tuple
    ``(ScaleByAdam8State, add_decayed_weights state?, lr state)``."""
    if use_magma:
        raise NotImplementedError("Magma is not supported by adamw8 yet.")
    inner = scale_by_adam8(
        b1=b1, b2=b2, eps=eps, eps_root=eps_root, block_size=block_size, min_size=min_size,
        scale_dtype=scale_dtype, fallback_dtype=fallback_dtype, stochastic_rounding=stochastic_rounding,
        block_layout=block_layout, quantize=quantize, nesterov=nesterov, key=key, exact=exact, sr_bits=sr_bits,
    )
    weight_decay_is_nonzero = weight_decay > 0.0 if isinstance(weight_decay, (int, float)) else True
    engine = inner.update.engine

    def init_fn(params):
        states = [inner.init(params)]
        if weight_decay_is_nonzero:
            states.append(decay_link_state(weight_decay, weight_decay_mask))
        if callable(learning_rate):
            states.append(ScaleByScheduleState(count=np.zeros((), dtype=np.int32)))
        else:
            states.append(EmptyState())
        return tuple(states)

    update = _Adamw8Update(engine, learning_rate, weight_decay, weight_decay_mask, weight_decay_is_nonzero)
    return GradientTransformationExtraArgs(init_fn, update)


def adamw8_step(tx, params, grads, state, key=None, stochastic: bool = True, *, random_bits=None,
                clip_global_norm: Optional[float] = None, clip_stats=None):
    """Fused ``tx.update`` + ``rollfast.apply_updates`` in one HBM pass (no
    reference counterpart: the reference runs them as two XLA programs).

    Equivalent to::

        updates, state = tx.update(grads, state, params)
        params = rollfast.apply_updates(params, updates, key, stochastic)

    for ``tx = adamw8(...)``: the same state bit for bit, and with
    ``exact=True`` the same params; in the default mode the fused form folds
    the learning rate into the direction, and both forms stay within one
    bf16 ulp of the reference's params.  Params are updated in place and
    returned with the new state.  ``random_bits`` (testing): ``{leaf_index: (mu_bits,
    nu_bits, param_bits)}`` device uint32 arrays replacing in-kernel bits.

    ``clip_global_norm``: the grads are first clipped by their global L2 norm
    as rollfast's ``finetune.transforms.clip_by_global_norm(max_norm)`` does
    (transforms.py:20-82), fused: a norm pre-pass reads the grads once and
    the step scales them as it loads them (the grads are not modified).
    ``clip_stats``: optional float32 device tensor of 2 elements that receives
    (scale, norm).

    ``tx`` may also be a composition the fine-tune builders use, still one
    launch: ``apply_if_finite(...)`` (a step whose grads hold an Inf or NaN
    is rejected on the device: moments untouched, params given the zero
    update, the guard's counters updated), ``chain(clip_by_global_norm(m),
    ...)`` and ``multi_transform({label: adamw8(...) or adamw(...)}, labels)``
    (one grouped launch).
    """
    upd = tx.update
    if not hasattr(upd, "_step") or isinstance(upd, _ScaleByAdam8Update):
        raise TypeError("adamw8_step needs a transformation built by adamw8(...), adamw(...) or a composition "
                        "of them (apply_if_finite, chain with clip_by_global_norm, multi_transform)")
    if stochastic and key is None:
        raise ValueError(
            "apply_updates requires a PRNG `key` when stochastic=True. "
            "Pass stochastic=False for deterministic rounding."
        )
    _, new_state = upd._step(grads, state, params, apply=True, param_key=key, param_sr=bool(stochastic),
                             random_bits=random_bits, clip_global_norm=clip_global_norm, clip_stats=clip_stats)
    return params, new_state


__all__ = (
    "QuantizedBlocks",
    "BlockLayout",
    "CodebookQuantizer",
    "ScaleByAdam8State",
    "DYNAMIC_SIGNED_CODEBOOK_ID",
    "DYNAMIC_UNSIGNED_CODEBOOK_ID",
    "SYMMETRIC_INT8_CODEBOOK_ID",
    "adamw8",
    "adamw8_step",
    "dequantize_blocks",
    "estimate_quantized_moment_bytes",
    "quantize_blocks",
    "quantized_nbytes",
    "scale_by_adam8",
    "tree_state_nbytes",
)


# --------------------------------------------------- grouped launches -----
def _group_key(upd) -> tuple:
    """What a group must share with the others to join one grouped launch:
    everything but the learning rate, weight decay, EMA-weight convention
    and keys (those travel per group).  Moment stochastic rounding is
    compared separately: only groups with quantized moments have it."""
    cfg = upd.engine.cfg
    wd = upd.weight_decay if upd.wd_nonzero else 0.0
    return (_as_f32(cfg.b1).item(), _as_f32(cfg.b2).item(), _as_f32(cfg.eps).item(), _as_f32(cfg.eps_root).item(),
            bool(cfg.nesterov), bool(cfg.exact), cfg.sr_bits, isinstance(wd, (int, float)))


def _moment_sr(upd) -> Optional[bool]:
    """adamw8(stochastic_rounding=...) of a group; None for optim/adam.py's
    adamw, whose moments are never requantized."""
    return bool(upd.engine.cfg.stochastic_rounding) if type(upd.engine) is _Engine else None


class _GroupedRunner:
    """One launch over several adamw8 / adamw transforms that each own a
    disjoint subset of the leaves (optax.multi_transform with masked inner
    transforms, finetune/builders.py:1529-1621).  Each leaf row carries its
    group index; the per-group learning rate, weight decay, EMA weight and
    moment keys travel in the launch's group table, the rest is shared."""

    def __init__(self):
        self._plans: dict = {}
        self._last = None  # the previous fused call's table, for run_cached

    @staticmethod
    def compatible(updates_objs, adam_states) -> bool:
        if not updates_objs or not all(isinstance(u, _Adamw8Update) for u in updates_objs):
            return False
        keys = {_group_key(u) for u in updates_objs}
        srs = {_moment_sr(u) for u in updates_objs} - {None}
        counts = {int(np.asarray(s.count)) for s in adam_states}
        return len(keys) == 1 and len(srs) <= 1 and len(counts) == 1

    @staticmethod
    def _scalars(groups_in):
        """Per group (update object, chain state): its group record (-lr,
        decay, EMA weight, moment keys) and its new chain state."""
        records, new_states = [], []
        for upd, state in groups_in:
            eng = upd.engine
            adam_state, lr_state = state[0], state[-1]
            neg_lr, new_lr_state = upd._lr(lr_state)
            wd, new_decay = upd._wd(state)
            key_mu, key_nu, next_key = eng.split_keys(adam_state.key)
            grp = _lib.Adam8Group()
            grp.neg_lr = neg_lr
            grp.weight_decay = _as_f32(wd) if upd.wd_nonzero else np.float32(0.0)
            grp.one_minus_b1 = eng.ema_weight(eng.cfg.b1)
            grp.key_mu[0], grp.key_mu[1] = int(key_mu[0]), int(key_mu[1])
            grp.key_nu[0], grp.key_nu[1] = int(key_nu[0]), int(key_nu[1])
            records.append(grp)
            count_inc = safe_int32_increment(int(np.asarray(adam_state.count)))
            new_states.append(upd.new_chain_state(state, eng.new_state(adam_state, count_inc, next_key), new_decay,
                                                  new_lr_state))
        return records, new_states

    @staticmethod
    def _launch(groups_in, records, table, n_rows, n_groups, device, plan, *, apply, param_key=None, param_sr=False,
                random_bits=None, clip_global_norm=None, clip_stats=None, skip_nonfinite=False, finite_out=None,
                finite_host=None):
        torch = _torch()
        upd0, state0 = groups_in[0]
        cfg = upd0.engine.cfg
        flags = _lib.RF_LR
        if cfg.nesterov:
            flags |= _lib.RF_NESTEROV
        if _group_key(upd0)[-1]:
            flags |= _lib.RF_DECAY_WEAK
        if any(_moment_sr(u) for u, _ in groups_in):
            flags |= _lib.RF_MOMENT_SR
        if apply and param_sr:
            flags |= _lib.RF_PARAM_SR
        if cfg.exact:
            flags |= _lib.RF_EXACT
        if random_bits is not None:
            flags |= _lib.RF_FED_BITS
        elif cfg.sr_bits == "packed":
            flags |= _lib.RF_PACKED_BITS
        if skip_nonfinite:
            flags |= _lib.RF_SKIP_NONFINITE
        count_inc = safe_int32_increment(int(np.asarray(state0[0].count)))
        hp = _common_hparams(cfg, count_inc, flags, param_key, clip_global_norm, clip_stats, finite_out,
                             finite_host)
        if n_rows:
            gtab = (_lib.Adam8Group * len(records))(*records)
            hp.groups = ctypes.cast(gtab, ctypes.c_void_p)
            hp.n_groups = n_groups
            with torch.cuda.device(device):
                plan.run(table, hp, _lib.stream_ptr())
                if finite_host is not None:
                    plan.wait_prepass()

    def run_cached(self, groups_in, labels_obj, updates, params, **kw):
        """Steady state of the fused grouped step: the same labels object and,
        per group, the same moment and param objects as the previous call.
        The native fast path rewrites each group's grad pointers in the cached
        table.  Returns the new chain states, or None (run() then rebuilds)."""
        last = self._last
        if (last is None or labels_obj is not last["labels"] or kw.get("random_bits") is not None
                or len(groups_in) != len(last["groups"])):
            return None
        if not self.compatible([u for u, _ in groups_in], [st[0] for _, st in groups_in]):
            return None
        host = _lib.pyhost()
        base = ctypes.addressof(last["table"])
        size = ctypes.sizeof(_lib.Adam8Leaf)
        for (upd, state), (first, refs) in zip(groups_in, last["groups"]):
            if upd.wd_nonzero and upd.weight_decay_mask is not None:
                return None
            adam = state[0]
            lists = host.gather(updates, adam.mu, adam.nu, params)
            if lists is None or not host.refresh(*lists, refs, base + first * size, last["device"].index):
                return None
        records, new_states = self._scalars(groups_in)
        self._launch(groups_in, records, last["table"], last["n"], last["n_groups"], last["device"], last["plan"],
                     apply=True, **kw)
        return new_states

    def run(self, members, updates, params, *, apply: bool, labels_obj=None, param_key=None, param_sr=False,
            random_bits=None, clip_global_norm=None, clip_stats=None, skip_nonfinite=False, finite_out=None,
            finite_host=None):
        """``members``: list of (update object, chain state, per-leaf membership
        list).  Returns (out leaves or None, the grads treedef, list of new
        chain states)."""
        torch = _torch()
        self._last = None
        g_leaves, g_td = _tree.flatten(updates, is_leaf=_is_passthrough_leaf)
        n = len(g_leaves)
        p_leaves = _tree.flatten_up_to(g_td, params) if params is not None else None
        masked = MaskedNode()
        rows, structure, group_rows = [], [], []
        out_leaves = [None] * n
        device = None
        for gi, (upd, state, member) in enumerate(members):
            eng = upd.engine
            adam_state = state[0]
            gm = [g_leaves[i] if member[i] else masked for i in range(n)]
            pm = None if p_leaves is None else [p_leaves[i] if member[i] else masked for i in range(n)]
            decay_mask = None
            if upd.wd_nonzero:
                if params is None:
                    raise ValueError(NO_PARAMS_MSG)
                decay_mask = _decay_mask_leaves(upd.weight_decay_mask, _tree.unflatten(g_td, pm), n)
            mu_leaves = _tree.flatten_up_to(g_td, adam_state.mu) if n else []
            nu_leaves = _tree.flatten_up_to(g_td, adam_state.nu) if n else []
            grows, gstruct, grefs, gouts, gdev = eng._build_rows(
                gm, mu_leaves, nu_leaves, pm, apply=apply, decay_mask=decay_mask, random_bits=random_bits,
                zero_decay=eng.own_zero_decay and params is not None)
            if gdev is not None:
                if device is not None and gdev != device:
                    raise ValueError("all leaves must live on the same device")
                device = gdev
            for row in grows:
                row.group = gi
            group_rows.append((len(rows), grefs))
            rows.extend(grows)
            structure.extend(s + (gi,) for s in gstruct)
            for i in range(n):
                if member[i]:
                    out_leaves[i] = gouts[i]
        for i in range(n):
            if out_leaves[i] is None:  # passthrough leaves and leaves of no group keep their update
                out_leaves[i] = g_leaves[i]
        groups_in = [(upd, state) for upd, state, _ in members]
        records, new_states = self._scalars(groups_in)
        table = plan = None
        n_groups = 0
        if rows:
            table = (_lib.Adam8Leaf * len(rows))(*rows)
            n_groups = 1 + max(r.group for r in rows)
            skey = (bool(apply), device.index, tuple(structure))
            plan = self._plans.get(skey)
            if plan is None:
                with torch.cuda.device(device):
                    plan = _LeafPlan(table, len(rows), apply)
                if len(self._plans) > 16:
                    self._plans.clear()
                self._plans[skey] = plan
        self._launch(groups_in, records, table, len(rows), n_groups, device, plan, apply=apply, param_key=param_key,
                     param_sr=param_sr, random_bits=random_bits, clip_global_norm=clip_global_norm,
                     clip_stats=clip_stats, skip_nonfinite=skip_nonfinite, finite_out=finite_out,
                     finite_host=finite_host)
        if apply and rows and random_bits is None and labels_obj is not None:
            self._last = {"labels": labels_obj, "groups": group_rows, "table": table, "n": len(rows),
                          "n_groups": n_groups, "device": device, "plan": plan}
        return (out_leaves if not apply else None), g_td, new_states
