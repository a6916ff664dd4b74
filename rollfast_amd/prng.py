"""Host-side PRNG keys with ``jax.random``'s default (Threefry-2x32) layout.

The reference keeps a ``uint32[2]`` key in the optimizer state and derives
per-leaf keys with ``jax.random.split`` (``src/rollfast/optim/adam8.py:274``,
``:306``, ``:585``, ``:645``; ``src/rollfast/utils.py:682``).  Keys here are
NumPy ``uint32[2]`` arrays kept on the host: key arithmetic is a handful of
block-cipher evaluations, and keeping it off the device means a step never
waits for a device-to-host copy.  The kernels derive the same per-leaf keys
and the per-element random bits on the GPU.

Layout (``jax_threefry_partitionable``, the JAX default since 0.5):
``split(key, n)[i] = threefry2x32(key, (0, i))`` and
``bits(key, shape)[i] = y0 ^ y1`` of ``threefry2x32(key, (hi32(i), lo32(i)))``.
Threefry-2x32 with 20 rounds follows Salmon et al., "Parallel random
numbers: as easy as 1, 2, 3" (SC'11).
"""

from __future__ import annotations

import numpy as np

_ROT = ((13, 15, 26, 6), (17, 29, 16, 24))
_PARITY = np.uint32(0x1BD11BDA)


def _rotl(x, r):
    return (x << np.uint32(r)) | (x >> np.uint32(32 - r))


def threefry2x32(key, c0, c1):
    """Vectorised Threefry-2x32-20 of counters (c0, c1) under ``key``."""
    k0 = np.uint32(key[0])
    k1 = np.uint32(key[1])
    ks = (k0, k1, k0 ^ k1 ^ _PARITY)
    with np.errstate(over="ignore"):
        x0 = np.asarray(c0, dtype=np.uint32) + ks[0]
        x1 = np.asarray(c1, dtype=np.uint32) + ks[1]
        for blk in range(5):
            for r in _ROT[blk & 1]:
                x0 = x0 + x1
                x1 = _rotl(x1, r)
                x1 = x1 ^ x0
            x0 = x0 + ks[(blk + 1) % 3]
            x1 = x1 + ks[(blk + 2) % 3] + np.uint32(blk + 1)
    return x0, x1


_M32 = 0xFFFFFFFF


def _threefry_int(k0: int, k1: int, c0: int, c1: int):
    """threefry2x32 of one counter pair on Python ints (the same rounds and
    key schedule as threefry2x32): a few times faster than NumPy for the
    handful of blocks a step's key derivation needs."""
    ks = (k0, k1, k0 ^ k1 ^ 0x1BD11BDA)
    x0 = (c0 + k0) & _M32
    x1 = (c1 + k1) & _M32
    for blk in range(5):
        for r in _ROT[blk & 1]:
            x0 = (x0 + x1) & _M32
            x1 = ((x1 << r) | (x1 >> (32 - r))) & _M32
            x1 ^= x0
        x0 = (x0 + ks[(blk + 1) % 3]) & _M32
        x1 = (x1 + ks[(blk + 2) % 3] + blk + 1) & _M32
    return x0, x1


def as_key(key) -> np.ndarray:
    """Normalise a key (NumPy array, sequence, or host/device tensor) to
    ``uint32[2]``."""
    if hasattr(key, "detach"):
        key = key.detach().cpu().numpy()
    k = np.asarray(key)
    if k.shape != (2,):
        raise ValueError(f"a PRNG key is uint32[2], got shape {k.shape}")
    return k.astype(np.uint32, copy=True)


def PRNGKey(seed: int) -> np.ndarray:
    """``jax.random.PRNGKey(seed)`` (32-bit seeds give ``[0, seed]``)."""
    seed = int(seed)
    if -(1 << 31) <= seed < (1 << 31):
        return np.array([0, seed & 0xFFFFFFFF], dtype=np.uint32)
    return np.array([(seed >> 32) & 0xFFFFFFFF, seed & 0xFFFFFFFF], dtype=np.uint32)


def split(key, num: int = 2) -> np.ndarray:
    """``jax.random.split(key, num)`` -> ``uint32[num, 2]``."""
    k = as_key(key)
    num = int(num)
    if num <= 16:
        k0, k1 = int(k[0]), int(k[1])
        return np.array([_threefry_int(k0, k1, 0, i) for i in range(num)], dtype=np.uint32).reshape(num, 2)
    i = np.arange(num, dtype=np.uint32)
    y0, y1 = threefry2x32(k, np.zeros_like(i), i)
    return np.stack([y0, y1], axis=1).astype(np.uint32)


def fold_in(key, data: int) -> np.ndarray:
    """``jax.random.fold_in(key, data)`` -> ``uint32[2]``.

    JAX converts ``data`` to uint32 (out-of-range Python ints raise
    OverflowError), makes it a seed pair ``[data >> 32, data & 0xFFFFFFFF]``
    = ``[0, data]`` and hashes that pair as one Threefry counter:
    ``threefry2x32(key, (0, data))``.  The fine-tune builders key each
    adamw8 group with ``fold_in(root_key, group_index)``
    (``src/rollfast/finetune/builders.py:1582``, ``:1123``, ``:1280``).  In
    the partitionable layout this is row ``data`` of ``split(key, n)`` for
    any ``n > data``."""
    k = as_key(key)
    d = int(data)
    if not 0 <= d < (1 << 32):
        raise OverflowError(f"Python int {d} too large to convert to uint32")
    return np.array(_threefry_int(int(k[0]), int(k[1]), 0, d), dtype=np.uint32)


def bits(key, n: int, offset: int = 0) -> np.ndarray:
    """``jax.random.bits(key, (n,), uint32)`` over flat indices
    ``offset .. offset+n-1``."""
    k = as_key(key)
    idx = np.arange(int(offset), int(offset) + int(n), dtype=np.uint64)
    y0, y1 = threefry2x32(k, (idx >> np.uint64(32)).astype(np.uint32), idx.astype(np.uint32))
    return (y0 ^ y1).astype(np.uint32)


def fresh_key(key, seed: int = 42) -> np.ndarray:
    """``rollfast.utils._fresh_prng_key`` (utils.py:73-76): a copy of ``key``,
    or ``PRNGKey(42)`` when ``key`` is None."""
    return PRNGKey(seed) if key is None else as_key(key)
