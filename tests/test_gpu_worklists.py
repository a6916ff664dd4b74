"""GPU parity of the work-list kernels at sizes where every wave walks
several units: k_quantize's register ring across a wave's blocks (a
full block followed by the partial last one), k_accumulate and k_apply
over ~10^8 elements (a grid of whole chip-fulls, 1.5-4 units per wave).

Bars: codes, scales and bf16 / f32 bit patterns bit-exact, against the
oracle where it runs in seconds and otherwise against exact properties
(a running mean started from zeros is the grad, the sum of a grad with
itself is twice it, the reset is a zero of the accumulator's sign) or a
torch reference whose operations are single IEEE roundings
(f32 add and multiply, the round-to-nearest-even float -> bf16 cast).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import to_device, to_host

pytestmark = pytest.mark.gpu


def _rf():
    import rollfast_amd as rf

    return rf


@pytest.mark.parametrize("quantizer,x_dtype", [("dynamic_signed", "f32"), ("symmetric_int8", "f32"),
                                               ("dynamic_unsigned", "bf16")])
def test_quantize_many_blocks_per_wave_with_partial_tail(quantizer, x_dtype):
    """16,385 blocks of 2048 (the last one 333 elements) over a grid of one
    chip-full: about 2.7 blocks per wave, each wave's next full block
    loaded into the registers its current block frees, then the partial
    block by the element path."""
    import torch

    rf = _rf()
    qid = {"dynamic_signed": orc.Q_SIGNED, "dynamic_unsigned": orc.Q_UNSIGNED,
           "symmetric_int8": orc.Q_SYMMETRIC}[quantizer]
    n = 2048 * 16384 + 333
    rng = np.random.default_rng(31)
    mag = np.exp(rng.uniform(np.log(1e-8), np.log(1e2), size=n)).astype(np.float32)
    x = np.where(rng.random(n) < 0.5, -mag, mag).astype(np.float32)
    x[::97] = 0.0
    if quantizer == "dynamic_unsigned":
        x = np.abs(x)
    if x_dtype == "bf16":
        xh = orc.f32_to_bf16_bits(x)
        xd = to_device(xh, "bf16")
        x = orc.bf16_bits_to_f32(xh)
    else:
        xd = to_device(x, "f32")
    print(f"quantize {quantizer} {x_dtype} n={n}", flush=True)
    qb = rf.quantize_blocks(xd, block_size=2048, quantizer=quantizer)
    torch.cuda.synchronize()
    codes, scales = orc.quantize(x, 2048, qid)
    np.testing.assert_array_equal(to_host(qb.values).view(np.uint8), codes.reshape(-1).view(np.uint8))
    np.testing.assert_array_equal(to_host(qb.scales).view(np.uint32), scales.view(np.uint32))


def _accum_rows(pairs, mode_zero=False):
    from rollfast_amd import _lib

    rows = []
    for g, a in pairs:
        row = _lib.AccumLeaf()
        row.grad = None if mode_zero else g.data_ptr()
        row.acc = a.data_ptr()
        row.size = a.numel()
        row.grad_dtype = _lib.RF_BF16
        row.acc_dtype = _lib.RF_F32
        rows.append(row)
    return (_lib.AccumLeaf * len(rows))(*rows), len(rows)


def test_accumulate_at_scale_exact_properties():
    """~2 x 10^8 elements in three leaves (bf16 grads, f32 accumulator):
    the running mean started from zeros is the widened grad, summing the
    same grad is twice it, and the reset is a zero of the accumulator's
    sign."""
    import torch

    from rollfast_amd import _lib

    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    sizes = [80_000_000, 67_108_864 + 7, 53_000_013]
    grads = [torch.randn(n, generator=gen, device="cuda").to(torch.bfloat16) for n in sizes]
    accs = [torch.zeros(n, device="cuda") for n in sizes]
    table, n = _accum_rows(zip(grads, accs))
    print("accumulate mean n_acc=0", flush=True)
    _lib.check(_lib.lib().rf_accumulate(table, n, _lib.RF_ACC_MEAN, 0, _lib.stream_ptr()), "rf_accumulate")
    torch.cuda.synchronize()
    for g, a in zip(grads, accs):
        assert torch.equal(a.view(torch.int32), g.float().view(torch.int32))
    print("accumulate sum", flush=True)
    _lib.check(_lib.lib().rf_accumulate(table, n, _lib.RF_ACC_SUM, 1, _lib.stream_ptr()), "rf_accumulate")
    torch.cuda.synchronize()
    for g, a in zip(grads, accs):
        assert torch.equal(a.view(torch.int32), (2.0 * g.float()).view(torch.int32))
    ztable, zn = _accum_rows(zip(grads, accs), mode_zero=True)
    print("accumulate reset", flush=True)
    _lib.check(_lib.lib().rf_accumulate(ztable, zn, _lib.RF_ACC_ZERO, 0, _lib.stream_ptr()), "rf_accumulate")
    torch.cuda.synchronize()
    for g, a in zip(grads, accs):
        assert not torch.any(a != 0).item()
        assert torch.equal(torch.signbit(a), torch.signbit(g.float()))


@pytest.mark.parametrize("pdtype", ["bf16", "f32"])
def test_apply_nearest_even_at_scale(pdtype):
    """apply_updates(stochastic=False) over ~1.2 x 10^8 params against
    torch: bf16 params take the nearest-even cast of f32(p) + u, f32 params
    the f32 sum."""
    import torch

    rf = _rf()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(6)
    dt = torch.bfloat16 if pdtype == "bf16" else torch.float32
    sizes = [(8192, 8192), (11008, 4096 + 3), (5,)]
    params = {f"l{i}": (torch.randn(s, generator=gen, device="cuda") * 0.02).to(dt) for i, s in enumerate(sizes)}
    ups = {k: torch.randn(v.shape, generator=gen, device="cuda") * 1e-3 for k, v in params.items()}
    want = {k: (v.float() + ups[k]).to(dt) for k, v in params.items()}
    print(f"apply nearest-even {pdtype}", flush=True)
    out = rf.apply_updates(params, ups, stochastic=False)
    torch.cuda.synchronize()
    for k in params:
        a, b = out[k], want[k]
        ia = a.view(torch.int16) if dt == torch.bfloat16 else a.view(torch.int32)
        ib = b.view(torch.int16) if dt == torch.bfloat16 else b.view(torch.int32)
        assert torch.equal(ia, ib), k


def test_apply_stochastic_at_scale_matches_oracle():
    """apply_updates(stochastic=True) with in-kernel Threefry bits over two
    bf16 leaves of 2.6 x 10^7 and 2.3 x 10^7 params, against the oracle
    (per-leaf key split(key, 2)[i], bits of the flat index)."""
    import torch

    rf = _rf()
    rng = np.random.default_rng(8)
    sizes = [26_000_011, 23_068_672]
    host_p, host_u, params, ups = [], [], {}, {}
    for i, n in enumerate(sizes):
        p = orc.f32_to_bf16_bits((rng.standard_normal(n) * 0.02).astype(np.float32))
        u = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        host_p.append(p.copy())
        host_u.append(u)
        params[f"l{i}"] = to_device(p, "bf16")
        ups[f"l{i}"] = to_device(u, "f32")
    key = rf.prng.PRNGKey(17)
    print("apply stochastic", flush=True)
    out = rf.apply_updates(params, ups, key=key, stochastic=True)
    torch.cuda.synchronize()
    keys = orc.split(key, len(sizes))
    for i, n in enumerate(sizes):
        orc.apply_updates(host_p[i], orc.BF16, host_u[i], bits=orc.random_bits(keys[i], n))
        np.testing.assert_array_equal(to_host(out[f"l{i}"]), host_p[i])
