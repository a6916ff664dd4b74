"""One bf16 leaf of 2^32 + 10,240 + 777 elements (2,097,158 blocks, the last
one partial) through ``adamw8_step`` with param and moment stochastic
rounding drawn in the kernel, for 2 steps.

The leaf's element index passes 2^31 and 2^32: the Threefry counter of
jax.random.bits (``jax_threefry_partitionable``: the element index as the
(high, low) 32-bit counter words) takes a non-zero high word there, and
every offset into the params, grads, codes and scales needs 64 bits.  Blocks
are independent (adam8.py:137-187), so the blocks on both sides of 2^31 and
2^32 elements, the first, the last full and the partial last block and 6
random ones are checked against the oracle run on that block alone, its
bits drawn with ``orc.random_bits(key, n, offset=block * 2048)`` from the
leaf's keys (adam8.py:306 for the moment keys, utils.py:648-708 for the
param key).  Bar: codes and scales bit-exact; params within one bf16 ulp
(default hardware rcp/sqrt direction).

The second test takes the standalone kernels (stochastic rounding to bf16,
apply_updates, quantize and dequantize) past 2^32 elements the same way.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as orc
from tests._helpers import bf16_ulp_distance

pytestmark = pytest.mark.gpu

BS = 2048
N = (1 << 32) + 5 * BS + 777
NB = (N + BS - 1) // BS


def _block(t, b, n):
    """Elements [b*BS, min((b+1)*BS, n)) of a flat device tensor, on the host
    (bf16 as uint16 patterns)."""
    import torch

    lo, hi = b * BS, min((b + 1) * BS, n)
    v = t.reshape(-1)[lo:hi]
    if v.dtype == torch.bfloat16:
        v = v.view(torch.int16)
        return v.cpu().numpy().view(np.uint16)
    return v.cpu().numpy()


def _fill_normal(t, std, gen):
    """t (flat bf16 or f32, device) <- N(0, std^2), 2^28 elements at a time."""
    import torch

    flat = t.reshape(-1)
    step = 1 << 28
    for lo in range(0, flat.numel(), step):
        hi = min(lo + step, flat.numel())
        flat[lo:hi] = (torch.randn(hi - lo, generator=gen, device="cuda") * std).to(t.dtype)


def _windows(n):
    """2048-element windows on both sides of 2^31 and 2^32 elements and at
    the end of an n-element array: (start, length)."""
    return [(0, BS), ((1 << 31) - BS // 2, BS), ((1 << 32) - BS // 2, BS), (n - 1500, 1500)]


def test_leaf_beyond_2p32_elements_sr_in_kernel_bits():
    import torch

    import rollfast_amd as rf

    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    print(f"[bigleaf] allocating a {N}-element bf16 leaf ({NB} blocks)", flush=True)
    params = {"w": torch.empty(N, dtype=torch.bfloat16, device="cuda")}
    _fill_normal(params["w"], 0.02, gen)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, stochastic_rounding=True, key=rf.prng.PRNGKey(5))
    state = tx.init(params)
    m, v = state[0].mu["w"], state[0].nu["w"]
    assert tuple(m.values.shape) == (NB, BS)
    rng = np.random.default_rng(4)
    edges = [0, (1 << 31) // BS - 1, (1 << 31) // BS, (1 << 32) // BS - 1, (1 << 32) // BS, NB - 2, NB - 1]
    idx = np.unique(np.concatenate([edges, rng.choice(NB, size=6, replace=False)]))
    orc_m = {int(b): {"mc": m.values[b].cpu().numpy().copy(), "vc": v.values[b].cpu().numpy().copy(),
                      "ms": m.scales[b:b + 1].cpu().numpy().copy(), "vs": v.scales[b:b + 1].cpu().numpy().copy()}
             for b in idx}
    grads = {"w": torch.empty(N, dtype=torch.bfloat16, device="cuda")}
    for step in range(2):
        print(f"[bigleaf] step {step + 1}", flush=True)
        _fill_normal(grads["w"], 1e-3, gen)
        before = {int(b): (_block(params["w"], b, N), _block(grads["w"], b, N)) for b in idx}
        key_mu, key_nu, _ = orc.split(state[0].key, 3)
        kmu, knu = orc.split(key_mu, 1)[0], orc.split(key_nu, 1)[0]
        pkey = rf.prng.PRNGKey(200 + step)
        kp = orc.split(pkey, 1)[0]
        params, state = rf.adamw8_step(tx, params, grads, state, key=pkey, stochastic=True)
        torch.cuda.synchronize()
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=step + 1, decay=True, apply=True,
                              moment_sr=True, param_sr=True)
        m, v = state[0].mu["w"], state[0].nu["w"]
        worst = 0
        for b in idx:
            b = int(b)
            p, g = before[b]
            p = p.copy()
            o = orc_m[b]
            orc.adam8_leaf(hp, p, orc.BF16, g, orc.BF16, orc.MOM_QUANT, o["mc"], o["ms"], o["vc"], o["vs"], BS,
                           mu_bits=orc.random_bits(kmu, BS, offset=b * BS),
                           nu_bits=orc.random_bits(knu, BS, offset=b * BS),
                           p_bits=orc.random_bits(kp, g.size, offset=b * BS))
            where = f"step {step + 1} block {b} (elements from {b * BS})"
            np.testing.assert_array_equal(m.values[b].cpu().numpy(), o["mc"], err_msg=f"{where}: mu codes")
            np.testing.assert_array_equal(v.values[b].cpu().numpy(), o["vc"], err_msg=f"{where}: nu codes")
            assert m.scales[b:b + 1].cpu().numpy().view(np.uint32)[0] == o["ms"].view(np.uint32)[0], where
            assert v.scales[b:b + 1].cpu().numpy().view(np.uint32)[0] == o["vs"].view(np.uint32)[0], where
            worst = max(worst, int(bf16_ulp_distance(_block(params["w"], b, N), p).max()))
        assert worst <= 1, f"step {step + 1}: params differ by {worst} bf16 ulp"
    del params, grads, state
    torch.cuda.empty_cache()


def test_standalone_kernels_beyond_2p32_elements():
    """_stochastic_round_bf16 (utils.py:342-371) and apply_updates with
    stochastic rounding (utils.py:648-708) of 2^32 + 777 elements with bits
    drawn in the kernel, and quantize_blocks with stochastic rounding plus
    dequantize_blocks (adam8.py:113-204) of the same count: windows across
    2^31 and 2^32 elements and at the end against the oracle (bit-exact)."""
    import torch

    import rollfast_amd as rf
    from rollfast_amd import prng
    from rollfast_amd.utils import _stochastic_round_bf16

    n = (1 << 32) + 777
    gen = torch.Generator(device="cuda")
    gen.manual_seed(33)
    key = rf.prng.PRNGKey(9)
    k = prng.as_key(key)

    print(f"[bigleaf] sr_bf16 of {n} f32 elements", flush=True)
    x = torch.empty(n, dtype=torch.float32, device="cuda")
    _fill_normal(x, 1.0, gen)
    out = _stochastic_round_bf16(x, key)
    torch.cuda.synchronize()
    for lo, ln in _windows(n):
        want = orc.sr_bf16(x[lo:lo + ln].cpu().numpy(), orc.random_bits(k, ln, offset=lo))
        got = out[lo:lo + ln].view(torch.int16).cpu().numpy().view(np.uint16)
        np.testing.assert_array_equal(got, want, err_msg=f"sr_bf16 elements {lo}..{lo + ln}")
    del out

    print("[bigleaf] apply_updates with stochastic rounding", flush=True)
    p = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    _fill_normal(p, 0.02, gen)
    x.mul_(1e-4)  # the updates
    before = {lo: p[lo:lo + ln].view(torch.int16).cpu().numpy().view(np.uint16).copy() for lo, ln in _windows(n)}
    new = rf.apply_updates({"w": p}, {"w": x}, key=key, stochastic=True)
    torch.cuda.synchronize()
    kp = orc.split(k, 1)[0]  # the leaf's key: split(key, n_leaves)[leaf index]
    for lo, ln in _windows(n):
        want = before[lo].copy()
        orc.apply_updates(want, orc.BF16, x[lo:lo + ln].cpu().numpy(), bits=orc.random_bits(kp, ln, offset=lo))
        got = new["w"][lo:lo + ln].view(torch.int16).cpu().numpy().view(np.uint16)
        np.testing.assert_array_equal(got, want, err_msg=f"apply_updates elements {lo}..{lo + ln}")
    del p, new

    print("[bigleaf] quantize_blocks (stochastic rounding) and dequantize_blocks", flush=True)
    _fill_normal(x, 1.0, gen)
    q = rf.quantize_blocks(x, stochastic_rounding=True, key=key)
    nb = (n + BS - 1) // BS
    assert tuple(q.values.shape) == (nb, BS)
    blocks = sorted({0, (1 << 31) // BS - 1, (1 << 31) // BS, (1 << 32) // BS - 1, (1 << 32) // BS, nb - 1})
    for b in blocks:
        lo, hi = b * BS, min((b + 1) * BS, n)
        codes, scales = orc.quantize(x[lo:hi].cpu().numpy(), BS, orc.Q_SIGNED,
                                     bits=orc.random_bits(k, BS, offset=lo))
        np.testing.assert_array_equal(q.values[b].cpu().numpy(), codes[0], err_msg=f"quantize block {b}")
        assert q.scales[b:b + 1].cpu().numpy().view(np.uint32)[0] == scales.view(np.uint32)[0], f"scale {b}"
    del x
    y = rf.dequantize_blocks(q)
    torch.cuda.synchronize()
    for b in blocks:
        lo, hi = b * BS, min((b + 1) * BS, n)
        want = orc.dequantize(q.values[b].cpu().numpy(), q.scales[b:b + 1].cpu().numpy(), hi - lo, BS)
        np.testing.assert_array_equal(y[lo:hi].cpu().numpy().view(np.uint32), want.view(np.uint32),
                                      err_msg=f"dequantize block {b}")
    del q, y
    torch.cuda.empty_cache()
