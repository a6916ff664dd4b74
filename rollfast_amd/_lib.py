"""ctypes binding of ``librfadam8.so`` (C ABI declared in ``include/rfadam8.h``).

The library is required: there is no fallback implementation.  Importing
works without a GPU (the symbols load), but every compute entry point needs
its tensors on a ROCm device and raises if the library was not built.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "librfadam8.so")

RF_OK, RF_ERR_INVALID, RF_ERR_HIP, RF_ERR_UNSUPPORTED = 0, 1, 2, 3
RF_F32, RF_BF16, RF_F16 = 0, 1, 2
RF_MOMENT_QUANTIZED, RF_MOMENT_F32, RF_MOMENT_BF16, RF_MOMENT_F16 = 0, 1, 2, 3
RF_Q_DYNAMIC_SIGNED, RF_Q_DYNAMIC_UNSIGNED, RF_Q_SYMMETRIC_INT8 = 0, 1, 2
RF_NESTEROV = 1
RF_DECAY_WEAK = 4
RF_LR = 8
RF_MOMENT_SR = 16
RF_PARAM_SR = 32
RF_EXACT = 128
RF_FED_BITS = 256
RF_SKIP_NONFINITE = 512
RF_PACKED_BITS = 1024
RF_ABI_VERSION = 2
RF_LEAF_DECAY = 1
RF_LEAF_STORE_SR = 2
RF_LEAF_ZERO_DECAY = 4
RF_LEAF_SCALE_BF16 = 8
RF_LEAF_SCALE_F16 = 16
RF_ACC_SUM, RF_ACC_MEAN, RF_ACC_ZERO = 0, 1, 2
RF_NOALLOC_SCRATCH_BYTES = 8 << 20

_p = ctypes.c_void_p


class Adam8Leaf(ctypes.Structure):
    _fields_ = [
        ("param", _p),
        ("grad", _p),
        ("updates", _p),
        ("mu", _p),
        ("mu_scales", _p),
        ("nu", _p),
        ("nu_scales", _p),
        ("mu_bits", _p),
        ("nu_bits", _p),
        ("param_bits", _p),
        ("size", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("param_dtype", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("moment_kind", ctypes.c_int32),
        ("state_index", ctypes.c_int32),
        ("param_index", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("group", ctypes.c_int32),
    ]


class Adam8Group(ctypes.Structure):
    _fields_ = [
        ("neg_lr", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("one_minus_b1", ctypes.c_float),
        ("reserved", ctypes.c_uint32),
        ("key_mu", ctypes.c_uint32 * 2),
        ("key_nu", ctypes.c_uint32 * 2),
    ]


class Adam8Hparams(ctypes.Structure):
    _fields_ = [
        ("b1", ctypes.c_float),
        ("one_minus_b1", ctypes.c_float),
        ("b2", ctypes.c_float),
        ("one_minus_b2", ctypes.c_float),
        ("bc1", ctypes.c_float),
        ("bc2", ctypes.c_float),
        ("bc1_next", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("eps_root", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("neg_lr", ctypes.c_float),
        ("flags", ctypes.c_uint32),
        ("key_mu", ctypes.c_uint32 * 2),
        ("key_nu", ctypes.c_uint32 * 2),
        ("key_param", ctypes.c_uint32 * 2),
        ("nesterov_one_minus_b1", ctypes.c_float),
        ("clip_max_norm", ctypes.c_float),
        ("clip_out", _p),
        ("finite_out", _p),
        ("finite_host", _p),
        ("groups", _p),
        ("n_groups", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("magma_sums", _p),
    ]


class ClipLeaf(ctypes.Structure):
    _fields_ = [
        ("grad", _p),
        ("out", _p),
        ("size", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class MagmaLeaf(ctypes.Structure):
    _fields_ = [
        ("grad", _p),
        ("mu", _p),
        ("updates", _p),
        ("size", ctypes.c_int64),
        ("grad_dtype", ctypes.c_int32),
        ("mu_dtype", ctypes.c_int32),
        ("key_index", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class AccumLeaf(ctypes.Structure):
    _fields_ = [
        ("grad", _p),
        ("acc", _p),
        ("size", ctypes.c_int64),
        ("grad_dtype", ctypes.c_int32),
        ("acc_dtype", ctypes.c_int32),
    ]


class ApplyLeaf(ctypes.Structure):
    _fields_ = [
        ("param", _p),
        ("updates", _p),
        ("bits", _p),
        ("size", ctypes.c_int64),
        ("param_dtype", ctypes.c_int32),
        ("param_index", ctypes.c_int32),
    ]


assert ctypes.sizeof(Adam8Leaf) == 120
assert ctypes.sizeof(Adam8Hparams) == 128
assert ctypes.sizeof(Adam8Group) == 32
assert ctypes.sizeof(ApplyLeaf) == 40
assert ctypes.sizeof(ClipLeaf) == 32
assert ctypes.sizeof(AccumLeaf) == 32

# Every symbol the header declares (checked by the CPU test suite).
EXPORTS = (
    "rf_adam8_plan_create",
    "rf_adam8_plan_run",
    "rf_adam8_plan_run_leaves",
    "rf_adam8_plan_wait_prepass",
    "rf_adam8_plan_info",
    "rf_adam8_plan_stream_probe",
    "rf_adam8_plan_destroy",
    "rf_adam8_step",
    "rf_adam8_step_noalloc",
    "rf_blockwise_quantize",
    "rf_blockwise_dequantize",
    "rf_sr_bf16",
    "rf_sr_bf16_packed",
    "rf_apply_updates",
    "rf_apply_updates_packed",
    "rf_clip_by_global_norm",
    "rf_magma_reduce",
    "rf_magma_scale",
    "rf_magma_apply_updates",
    "rf_accumulate",
    "rf_codebook",
    "rf_host_table_codes",
    "rf_host_search_index",
    "rf_host_sr_records",
    "rf_version",
    "rf_abi_version",
    "rf_last_error",
)

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m rollfast_amd.build` "
            "(hipcc --offload-arch=gfx950) first"
        )
    L = ctypes.CDLL(LIB_PATH)
    i32, i64, u32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
    L.rf_version.restype = ctypes.c_char_p
    L.rf_last_error.restype = ctypes.c_char_p
    L.rf_adam8_plan_create.argtypes = [ctypes.POINTER(Adam8Leaf), i32, i32, ctypes.POINTER(_p)]
    L.rf_adam8_plan_run.argtypes = [_p, ctypes.POINTER(Adam8Hparams), _p]
    L.rf_adam8_plan_run_leaves.argtypes = [_p, ctypes.POINTER(Adam8Leaf), i32, ctypes.POINTER(Adam8Hparams), _p]
    L.rf_adam8_plan_info.argtypes = [_p, ctypes.POINTER(i64), ctypes.POINTER(i64), ctypes.POINTER(i64)]
    L.rf_adam8_plan_stream_probe.argtypes = [_p, _p, ctypes.POINTER(i64)]
    L.rf_adam8_plan_destroy.argtypes = [_p]
    L.rf_adam8_step.argtypes = [ctypes.POINTER(Adam8Leaf), i32, i32, ctypes.POINTER(Adam8Hparams), _p]
    L.rf_adam8_step_noalloc.argtypes = [ctypes.POINTER(Adam8Leaf), i32, i32, ctypes.POINTER(Adam8Hparams), _p]
    L.rf_blockwise_quantize.argtypes = [i32, _p, i32, i64, i32, i32, u32, u32, _p, _p, _p, i32, _p]
    L.rf_blockwise_dequantize.argtypes = [i32, _p, _p, i32, i64, i32, i32, _p, _p]
    L.rf_sr_bf16.argtypes = [_p, i64, u32, u32, _p, _p, _p]
    L.rf_apply_updates.argtypes = [ctypes.POINTER(ApplyLeaf), i32, i32, u32, u32, _p]
    L.rf_sr_bf16_packed.argtypes = [_p, i64, u32, u32, _p, _p]
    L.rf_apply_updates_packed.argtypes = [ctypes.POINTER(ApplyLeaf), i32, u32, u32, _p]
    f32 = ctypes.c_float
    L.rf_magma_reduce.argtypes = [ctypes.POINTER(MagmaLeaf), i32, f32, f32, _p, _p]
    L.rf_magma_scale.argtypes = [ctypes.POINTER(MagmaLeaf), i32, _p, _p, f32, f32, u32, u32, i32, f32, _p, _p]
    L.rf_magma_apply_updates.argtypes = [ctypes.POINTER(ApplyLeaf), i32, _p, f32, i32, u32, u32, _p]
    L.rf_accumulate.argtypes = [ctypes.POINTER(AccumLeaf), i32, i32, i32, _p]
    L.rf_codebook.argtypes = [i32, _p]
    L.rf_host_table_codes.argtypes = [i32, u32, i64, _p]
    L.rf_host_search_index.argtypes = [i32, u32, i64, _p]
    L.rf_host_sr_records.argtypes = [i32, _p]
    for name in EXPORTS:
        if name not in ("rf_version", "rf_last_error"):
            getattr(L, name).restype = i32
    if L.rf_abi_version() != RF_ABI_VERSION:
        raise LibraryMissing(f"{LIB_PATH} has ABI revision {L.rf_abi_version()}, this binding is written for "
                             f"{RF_ABI_VERSION}; rebuild with `python -m rollfast_amd.build`")
    _lib = L
    return L


_pyhost = None


def pyhost():
    """The native host fast-path module ``_rfhost`` (built with the library
    by ``rollfast_amd.build``); raises if it is not built."""
    global _pyhost
    if _pyhost is not None:
        return _pyhost
    import importlib.util
    import sysconfig

    from ._base import MaskedNode

    path = os.path.join(os.path.dirname(LIB_PATH), "_rfhost" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.exists(path):
        raise LibraryMissing(f"{path} is not built; run `python -m rollfast_amd.build` first")
    spec = importlib.util.spec_from_file_location("rollfast_amd._lib._rfhost", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.set_masked_node_type(MaskedNode)
    _pyhost = mod
    return mod


def check(status: int, what: str) -> None:
    """Map an rf_status to the reference's exception types."""
    if status == RF_OK:
        return
    msg = lib().rf_last_error().decode(errors="replace")
    text = f"{what}: {msg}"
    if status == RF_ERR_INVALID:
        raise ValueError(text)
    if status == RF_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)


def version() -> str:
    return lib().rf_version().decode()


def codebook(signed: bool) -> np.ndarray:
    out = np.empty(256, dtype=np.float32)
    q = RF_Q_DYNAMIC_SIGNED if signed else RF_Q_DYNAMIC_UNSIGNED
    check(lib().rf_codebook(q, out.ctypes.data_as(_p)), "rf_codebook")
    return out


def host_table_codes(quantizer: int, first_bits: int, count: int) -> np.ndarray:
    out = np.empty(int(count), dtype=np.uint8)
    check(lib().rf_host_table_codes(quantizer, int(first_bits), int(count), out.ctypes.data_as(_p)),
          "rf_host_table_codes")
    return out


def host_search_index(quantizer: int, first_bits: int, count: int) -> np.ndarray:
    out = np.empty(int(count), dtype=np.uint16)
    check(lib().rf_host_search_index(quantizer, int(first_bits), int(count), out.ctypes.data_as(_p)),
          "rf_host_search_index")
    return out


def host_sr_records(quantizer: int) -> np.ndarray:
    """The moment-SR neighbour records [256, 4] (cb[li], gap, RN(1/gap) or
    0, 0) of a dynamic codebook."""
    out = np.empty((256, 4), dtype=np.float32)
    check(lib().rf_host_sr_records(quantizer, out.ctypes.data_as(_p)), "rf_host_sr_records")
    return out


def stream_ptr(device=None) -> ctypes.c_void_p:
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
