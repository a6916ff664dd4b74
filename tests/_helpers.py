"""Shared helpers for the parity tests: synthetic inputs, host/device copies,
and the oracle run of one adamw8 step over a whole tree."""

from __future__ import annotations

import numpy as np

from oracle import oracle as orc


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even."""
    return orc.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return orc.bf16_bits_to_f32(h)


def to_device(arr: np.ndarray, dtype: str, device="cuda"):
    """NumPy -> torch on device.  dtype 'f32' takes f32 values; 'bf16' and
    'f16' take bit patterns (uint16)."""
    import torch

    if dtype == "bf16":
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    elif dtype == "f16":
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.uint16).view(np.int16)).view(torch.float16)
    elif dtype == "f32":
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32))
    elif dtype == "u8":
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.uint8))
    elif dtype == "u32":
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.uint32).view(np.int32)).view(torch.uint32)
    else:
        raise ValueError(dtype)
    return t.to(device)


def to_host(t) -> np.ndarray:
    """torch -> NumPy: bf16 as uint16 bit patterns, uint32 as uint32."""
    import torch

    t = t.detach().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    if t.dtype == torch.uint32:
        return t.view(torch.int32).cpu().numpy().view(np.uint32).reshape(-1)
    return t.cpu().numpy().reshape(-1)


def bf16_ulp_distance(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in ulps between two arrays of bf16 (or f16) bit patterns
    (sign-magnitude order)."""

    def key(h):
        h = h.astype(np.int64)
        return np.where(h & 0x8000, -(h & 0x7FFF), h & 0x7FFF)

    return np.abs(key(a_bits) - key(b_bits))


def f32_within_bf16_ulp(a: np.ndarray, b: np.ndarray, before: np.ndarray | None = None) -> np.ndarray:
    """|a - b| <= one bf16 ulp of the largest magnitude among the two results
    and the param before the step (f32 params): when an update cancels the
    param, the new value is tiny but the step's rounding error scales with
    the operands."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    m = np.maximum(np.abs(a), np.abs(b))
    if before is not None:
        m = np.maximum(m, np.abs(before.astype(np.float64)))
    e = np.floor(np.log2(np.where(m > 0, m, 1.0)))
    ulp = np.exp2(e - 7)
    return np.abs(a - b) <= ulp


def f32_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of f32 values at |x| (2^-149 in the subnormal range)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.where(x > 0, x, 1.0)))
    return np.exp2(np.maximum(e, -126.0) - 23.0)


def f32_params_close(got: np.ndarray, want: np.ndarray, before: np.ndarray, steps: int = 1) -> np.ndarray:
    """f32 params of the default (hardware rcp/sqrt) direction: the update
    u = want - before carries a few f32 ulps of error and the fused add
    rounds once more, so |got - want| <= 8 ulp(|want - before|) + ulp(want)
    per step (where p + u nearly cancels the kernel recomputes in IEEE
    arithmetic, which is exact).  ``steps``: device params that followed
    their own trajectory for that many steps of similar updates."""
    g = got.astype(np.float64)
    w = want.astype(np.float64)
    b = before.astype(np.float64)
    bound = 8.0 * f32_ulp(w - b) + f32_ulp(np.maximum(np.abs(w), np.abs(g)))
    return np.abs(g - w) <= steps * bound


def gaussian(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


class OracleTree:
    """Host copy of one adamw8 state (leaf list) advanced by the oracle."""

    def __init__(self, leaves):
        # leaves: list of dicts with keys pdtype ('f32'|'bf16'), gdtype, kind
        # ('quant'|'f32'|'bf16'), size, block_size, param (np), mu, mu_scales,
        # nu, nu_scales (np, host copies).
        self.leaves = leaves

    def step(self, grads, *, b1=0.9, b2=0.999, eps=1e-8, eps_root=0.0, weight_decay=0.0, lr=1e-3,
             count=1, decay_mask=None, nesterov=False, moment_sr=False, param_sr=False, apply=True,
             mu_bits=None, nu_bits=None, p_bits=None, lr_scale=True, decay_weak=True, ema_weight_f32=False,
             store_sr=False, zero_decay=False, scale_dtype=None):
        outs = []
        for i, L in enumerate(self.leaves):
            decays = weight_decay != 0.0 and (decay_mask is None or decay_mask[i])
            hp = orc.make_hparams(b1=b1, b2=b2, eps=eps, eps_root=eps_root, weight_decay=weight_decay,
                                  lr=lr if lr_scale else None, count=count, nesterov=nesterov, decay=decays,
                                  decay_weak=decay_weak, moment_sr=moment_sr, param_sr=param_sr, apply=apply,
                                  ema_weight_f32=ema_weight_f32, store_sr=store_sr and L["kind"] == "bf16",
                                  zero_decay=zero_decay,
                                  scale_dtype=orc.F32 if scale_dtype is None else scale_dtype)
            dt = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}
            pd, gd = dt[L["pdtype"]], dt[L["gdtype"]]
            mk = {"quant": orc.MOM_QUANT, "f32": orc.MOM_F32, "bf16": orc.MOM_BF16, "f16": orc.MOM_F16}[L["kind"]]
            upd = None if apply else np.empty(L["size"], dtype=np.float32)
            orc.adam8_leaf(hp, L["param"], pd, grads[i], gd, mk, L["mu"], L.get("mu_scales"), L["nu"],
                           L.get("nu_scales"), L.get("block_size", 2048),
                           mu_bits=None if mu_bits is None else mu_bits[i],
                           nu_bits=None if nu_bits is None else nu_bits[i],
                           p_bits=None if p_bits is None else p_bits[i], updates_out=upd)
            outs.append(upd)
        return outs
