"""rf_adam8_step_noalloc (the step with its tables in a device-scope array,
no allocation) through the C ABI: two calls in a row, the second over a
smaller tree, each equal bit for bit to rf_adam8_step on copies of the same
buffers; and a tree too large for the array is refused before any work."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BS = 2048


def _leaf_set(specs, seed):
    """Device buffers of a tree: specs are (size, param dtype, grad dtype,
    moment kind) with kind 'q' (quantized) or 'f32' (fallback moments)."""
    import torch

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    leaves = []
    for n, pdt, gdt, kind in specs:
        p = torch.randn(n, generator=gen, device="cuda") * 0.02
        g = torch.randn(n, generator=gen, device="cuda") * 0.5
        d = {"p": p.to(torch.bfloat16 if pdt == "bf16" else torch.float32),
             "g": g.to(torch.bfloat16 if gdt == "bf16" else torch.float32), "kind": kind}
        if kind == "q":
            nb = -(-n // BS)
            d["mc"] = torch.randint(0, 256, (nb * BS,), generator=gen, device="cuda", dtype=torch.int64).to(torch.uint8)
            d["vc"] = torch.randint(0, 256, (nb * BS,), generator=gen, device="cuda", dtype=torch.int64).to(torch.uint8)
            d["ms"] = torch.rand(nb, generator=gen, device="cuda") * 1e-3
            d["vs"] = torch.rand(nb, generator=gen, device="cuda") * 1e-6
        else:
            d["mc"] = torch.randn(n, generator=gen, device="cuda") * 1e-3
            d["vc"] = torch.rand(n, generator=gen, device="cuda") * 1e-6
        leaves.append(d)
    return leaves


def _clone(leaves):
    return [{k: (v.clone() if hasattr(v, "clone") else v) for k, v in d.items()} for d in leaves]


def _table(leaves):
    from rollfast_amd import _lib

    table = (_lib.Adam8Leaf * len(leaves))()
    for i, d in enumerate(leaves):
        L = table[i]
        L.param = d["p"].data_ptr()
        L.grad = d["g"].data_ptr()
        L.mu = d["mc"].data_ptr()
        L.nu = d["vc"].data_ptr()
        L.size = d["p"].numel()
        L.param_dtype = _lib.RF_BF16 if d["p"].element_size() == 2 else _lib.RF_F32
        L.grad_dtype = _lib.RF_BF16 if d["g"].element_size() == 2 else _lib.RF_F32
        if d["kind"] == "q":
            L.moment_kind = _lib.RF_MOMENT_QUANTIZED
            L.block_size = BS
            L.mu_scales = d["ms"].data_ptr()
            L.nu_scales = d["vs"].data_ptr()
        else:
            L.moment_kind = _lib.RF_MOMENT_F32
        L.state_index = L.param_index = i
        L.flags = _lib.RF_LEAF_DECAY if i % 3 != 2 else 0
    return table


def _hparams(count, flags, clip):
    from rollfast_amd import _lib
    from rollfast_amd.prng import PRNGKey

    hp = _lib.Adam8Hparams()
    b1, b2 = np.float32(0.9), np.float32(0.999)
    hp.b1, hp.one_minus_b1 = b1, np.float32(1.0 - 0.9)
    hp.b2, hp.one_minus_b2 = b2, np.float32(1.0 - 0.999)
    hp.bc1 = np.float32(1) - np.power(b1, np.float32(count))
    hp.bc2 = np.float32(1) - np.power(b2, np.float32(count))
    hp.bc1_next = np.float32(1) - np.power(b1, np.float32(count + 1))
    hp.eps, hp.eps_root = 1e-8, 0.0
    hp.weight_decay = 0.01
    hp.neg_lr = -1e-3
    hp.nesterov_one_minus_b1 = hp.one_minus_b1
    hp.flags = flags
    k = np.asarray(PRNGKey(count), dtype=np.uint32).reshape(-1)
    for f, off in (("key_mu", 0), ("key_nu", 1), ("key_param", 2)):
        arr = getattr(hp, f)
        arr[0], arr[1] = int(k[0]) ^ off, int(k[1]) + off
    hp.clip_max_norm = clip
    return hp


def _same(a, b, what):
    """Every output buffer equal byte for byte."""
    import torch

    for i, (x, y) in enumerate(zip(a, b)):
        for key in ("p", "mc", "vc", "ms", "vs"):
            if key in x:
                assert torch.equal(x[key].view(torch.uint8), y[key].view(torch.uint8)), \
                    f"{what}: leaf {i} {key} differs between rf_adam8_step_noalloc and rf_adam8_step"


def _run_both(specs, seed, count, flags, clip):
    import torch

    from rollfast_amd import _lib

    lib = _lib.lib()
    a = _leaf_set(specs, seed)
    b = _clone(a)
    ta, tb = _table(a), _table(b)
    fa = torch.full((2,), -1, dtype=torch.int32, device="cuda")
    ca = torch.zeros(2, device="cuda")
    cb = torch.zeros(2, device="cuda")
    hpa = _hparams(count, flags, clip)
    hpb = _hparams(count, flags, clip)
    hpa.finite_out, hpb.finite_out = fa[0:1].data_ptr(), fa[1:2].data_ptr()
    if clip > 0:
        hpa.clip_out, hpb.clip_out = ca.data_ptr(), cb.data_ptr()
    print(f"[no_alloc] {len(specs)} leaves, flags {flags}, clip {clip}: rf_adam8_step", flush=True)
    st = lib.rf_adam8_step(ta, len(specs), 1, ctypes.byref(hpa), _lib.stream_ptr())
    assert st == _lib.RF_OK, lib.rf_last_error()
    print("[no_alloc] rf_adam8_step_noalloc", flush=True)
    st = lib.rf_adam8_step_noalloc(tb, len(specs), 1, ctypes.byref(hpb), _lib.stream_ptr())
    assert st == _lib.RF_OK, lib.rf_last_error()
    torch.cuda.synchronize()
    _same(a, b, f"count {count}")
    assert fa.tolist() == [1, 1]
    if clip > 0:
        assert torch.equal(ca.view(torch.int32), cb.view(torch.int32))
        assert 0.0 < float(cb[0]) < 1.0, "the clipping scale should be active"


def test_noalloc_equals_step_two_calls_second_smaller():
    from rollfast_amd import _lib

    big = [(37 * BS, "bf16", "bf16", "q"), (5 * BS + 77, "bf16", "bf16", "q"), (9 * BS, "f32", "f32", "q"),
           (3 * BS, "bf16", "f32", "q"), (1000, "bf16", "bf16", "f32"), (4 * BS + 5, "f32", "bf16", "f32"),
           (65536 + 3, "bf16", "bf16", "q")]
    small = [(2 * BS, "bf16", "bf16", "q"), (777, "f32", "f32", "f32")]
    # first call: the larger tree, clipping and the finite flag (norm sums in the scratch)
    _run_both(big, 1, 1, _lib.RF_LR | _lib.RF_DECAY_WEAK, 1.0)
    # second call: a smaller tree over what the first left in the scratch;
    # param and moment stochastic rounding with in-kernel bits, no clipping
    _run_both(small, 2, 2, _lib.RF_LR | _lib.RF_DECAY_WEAK | _lib.RF_PARAM_SR | _lib.RF_MOMENT_SR, 0.0)


def test_noalloc_refuses_a_tree_beyond_its_scratch():
    import torch

    from rollfast_amd import _lib

    lib = _lib.lib()
    p = torch.zeros(1, device="cuda")
    g = torch.zeros(1, device="cuda")
    m = torch.zeros(1, device="cuda")
    v = torch.zeros(1, device="cuda")
    n = _lib.RF_NOALLOC_SCRATCH_BYTES // 120 + 1   # the leaf table alone exceeds it
    table = (_lib.Adam8Leaf * n)()
    for i in range(n):
        L = table[i]
        L.param, L.grad, L.mu, L.nu = p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr()
        L.size = 1
        L.moment_kind = _lib.RF_MOMENT_F32
        L.state_index = L.param_index = i
    hp = _hparams(1, _lib.RF_LR, 0.0)
    before = p.clone()
    st = lib.rf_adam8_step_noalloc(table, n, 1, ctypes.byref(hp), _lib.stream_ptr())
    assert st == _lib.RF_ERR_INVALID
    assert b"maximum" in lib.rf_last_error()
    torch.cuda.synchronize()
    assert torch.equal(p, before)


def _hip():
    """The HIP runtime (stream capture calls the tests make directly)."""
    lib = ctypes.CDLL("libamdhip64.so")
    lib.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    lib.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    lib.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    return lib


def test_noalloc_refuses_stream_capture():
    """On a capturing stream the call returns RF_ERR_UNSUPPORTED and
    enqueues nothing: the capture ends with an empty graph and the tree's
    params are unchanged."""
    import torch

    from rollfast_amd import _lib

    lib = _lib.lib()
    hip = _hip()
    leaves = _leaf_set([(2 * BS, "bf16", "bf16", "q")], 5)
    before = leaves[0]["p"].clone()
    table = _table(leaves)
    hp = _hparams(1, _lib.RF_LR, 0.0)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    print("[no_alloc] capture refusal", flush=True)
    assert hip.hipStreamBeginCapture(ctypes.c_void_p(s.cuda_stream), 2) == 0  # hipStreamCaptureModeRelaxed
    st = lib.rf_adam8_step_noalloc(table, 1, 1, ctypes.byref(hp), ctypes.c_void_p(s.cuda_stream))
    msg = lib.rf_last_error()
    graph = ctypes.c_void_p()
    assert hip.hipStreamEndCapture(ctypes.c_void_p(s.cuda_stream), ctypes.byref(graph)) == 0
    if graph.value:
        hip.hipGraphDestroy(graph)
    assert st == _lib.RF_ERR_UNSUPPORTED and b"graph" in msg
    torch.cuda.synchronize()
    assert torch.equal(leaves[0]["p"], before)


def test_noalloc_calls_on_two_streams_are_ordered():
    """A call on stream A behind pending work, then at once a call on stream
    B over another tree: B's table copy waits for A's launches (the
    library's per-device event), so both trees equal rf_adam8_step's."""
    import torch

    from rollfast_amd import _lib

    lib = _lib.lib()
    specs_a = [(64 * BS, "bf16", "bf16", "q"), (3 * BS + 11, "f32", "bf16", "q"), (900, "bf16", "bf16", "f32")]
    specs_b = [(5 * BS, "bf16", "f32", "q"), (2 * BS, "f32", "f32", "q")]
    a, b = _leaf_set(specs_a, 7), _leaf_set(specs_b, 8)
    ra, rb = _clone(a), _clone(b)
    flags = _lib.RF_LR | _lib.RF_DECAY_WEAK
    for ref, specs in ((ra, specs_a), (rb, specs_b)):
        hp = _hparams(1, flags, 0.0)
        assert lib.rf_adam8_step(_table(ref), len(specs), 1, ctypes.byref(hp), _lib.stream_ptr()) == _lib.RF_OK
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    x = torch.ones(1 << 28, device="cuda")
    ta, tb = _table(a), _table(b)
    hpa, hpb = _hparams(1, flags, 0.0), _hparams(1, flags, 0.0)
    print("[no_alloc] two streams", flush=True)
    with torch.cuda.stream(sa):
        for _ in range(8):
            x.mul_(1.0)   # pending work ahead of A's call
        st = lib.rf_adam8_step_noalloc(ta, len(specs_a), 1, ctypes.byref(hpa), ctypes.c_void_p(sa.cuda_stream))
        assert st == _lib.RF_OK, lib.rf_last_error()
    st = lib.rf_adam8_step_noalloc(tb, len(specs_b), 1, ctypes.byref(hpb), ctypes.c_void_p(sb.cuda_stream))
    assert st == _lib.RF_OK, lib.rf_last_error()
    torch.cuda.synchronize()
    _same(ra, a, "stream A")
    _same(rb, b, "stream B")


def test_noalloc_return_time_behind_pending_work():
    """How long the call holds the host when the stream still has work ahead
    of it (the table copy is from pageable memory).  Measured and printed;
    the call's results are checked as in the other tests."""
    import time

    import torch

    from rollfast_amd import _lib

    lib = _lib.lib()
    specs = [(4 * BS, "bf16", "bf16", "q")]
    a = _leaf_set(specs, 9)
    r = _clone(a)
    hp = _hparams(1, _lib.RF_LR, 0.0)
    assert lib.rf_adam8_step(_table(r), 1, 1, ctypes.byref(hp), _lib.stream_ptr()) == _lib.RF_OK
    x = torch.ones(1 << 30, device="cuda")
    t = _table(a)
    # warm: the first call on a stream may set up runtime state
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(8):
        x.mul_(1.0)
    e1.record()
    t0 = time.perf_counter()
    st = lib.rf_adam8_step_noalloc(t, 1, 1, ctypes.byref(_hparams(1, _lib.RF_LR, 0.0)), _lib.stream_ptr())
    held = (time.perf_counter() - t0) * 1e3
    t_enq = time.perf_counter()
    torch.cuda.synchronize()
    rest = (time.perf_counter() - t_enq) * 1e3
    assert st == _lib.RF_OK, lib.rf_last_error()
    pending = e0.elapsed_time(e1)
    print(f"[no_alloc] call returned after {held:.3f} ms with {pending:.3f} ms of work ahead on the stream; "
          f"the stream finished {rest:.3f} ms after the return", flush=True)
    _same(r, a, "behind pending work")
