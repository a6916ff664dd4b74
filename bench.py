#!/usr/bin/env python
"""Throughput of the 8-bit AdamW step (and its standalone kernels) on one
MI355X.

Default workload (``--workload llama7b``): the Llama-7B-shaped bf16 pytree
(32 layers, hidden 4096, SwiGLU MLP 11008, vocab 32000, RMSNorm vectors;
6,738,415,616 params in 291 leaves, all quantized: uint8 codes + f32 scales
per 2048-element block), params ~N(0, 0.02^2), grads ~N(0, 1e-3^2).  A step
is one fused adamw8_step over the whole tree (one launch): dequantize both
moments, AdamW update (lr 1e-3, wd 0.01, betas 0.9/0.999), bf16 params
written with round-to-nearest-even, moments requantized.  Gradients are
drawn before the timed region into a pool of distinct buffers that the steps
cycle through.

Other workloads (one JSON line each, same fields):
  llama7b_msr      the default step with moment stochastic rounding
                   (adamw8(stochastic_rounding=True)): two in-kernel Threefry
                   draws per element for the requantization of both moments.
  llama7b_f32      the default step over the same tree with f32 params and
                   grads (16.0078 B/param).
  gpt2             GPT-2-small bf16 tree (74 leaves, LayerNorms on f32
                   fallback moments), param stochastic rounding on.
  ragged           2256 leaves, most below min_size (fallback moments),
                   Student-t(3) grads with per-leaf scales, 10 % zero blocks.
  llama7b_clip     the default step with fused global-norm clipping (max norm
                   1.0): a norm pre-pass reads the grads once more (+2 B/param).
  llama7b_finetune the fine-tune builders' gradient policy around the step:
                   clipping at 1.0 and apply_if_finite (skip non-finite
                   steps); the finite flag is read back once per step.
  llama7b_finetune_groups  the same around a three-group multi_transform
                   (base / embeddings / norms with their own learning rates,
                   decays and keys), as the fine-tune builders compose it.
  llama7b_finetune_accum4  that composition inside MultiSteps(every_k=4,
                   f32 accumulator): a step is one window of four micro-steps
                   (one accumulate launch each; the fourth then runs the
                   guarded grouped step on the accumulator and resets it).
  llama7b_optax    update-only (Optax) mode over the Llama tree: f32 updates
                   written, params read for weight decay.
  llama7b_adamw_f32   full-precision AdamW (adamw, f32 moments) over the Llama
                   tree: 22 B/param.
  llama7b_adamw_bf16  the same with stochastically rounded bf16 moments.
  llama7b_adamw_magma full-precision AdamW with Magma (use_magma=True) by
                   adamw_step: the Magma factor folded into apply_updates.
  llama7b_apply    apply_updates of f32 updates to the bf16 Llama params with
                   stochastic rounding (in-kernel Threefry bits).
  quantize_2p30    quantize_blocks, dynamic signed, 2^30 f32 elements
                   (log-uniform magnitudes 1e-8..1e2, random sign).
  dequantize_2p30  dequantize_blocks of the same codes to f32.
  sr_bf16_2p30     f32 -> bf16 stochastic rounding of 2^30 elements.

Prints one JSON line: throughput (whole job), ms per step, the HBM roofline of
the measured kernel (algorithmic bytes / kernel time from HIP events on the
launch stream) and the CPU oracle's throughput on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
METRIC = "adam8 step params/sec + achieved HBM GB/s (% peak), 7B Llama pytree, 1 GPU"
BS = 2048
MIN_SIZE = 4096


# ------------------------------------------------------------- shapes -----
def llama7b_shapes():
    h, f, v, layers = 4096, 11008, 32000, 32
    shapes = [("embed", (v, h)), ("lm_head", (v, h)), ("norm", (h,))]
    for i in range(layers):
        for n, s in (("q", (h, h)), ("k", (h, h)), ("v", (h, h)), ("o", (h, h)), ("gate", (f, h)),
                     ("up", (f, h)), ("down", (h, f)), ("attn_norm", (h,)), ("mlp_norm", (h,))):
            shapes.append((f"layer{i:02d}.{n}", s))
    return shapes


def gpt2_small_shapes():
    d, v, layers = 768, 50304, 12
    shapes = [("wte", (v, d)), ("ln_f", (d,))]
    for i in range(layers):
        for n, s in (("qkv", (d, 3 * d)), ("proj", (d, d)), ("fc", (d, 4 * d)), ("fc_proj", (4 * d, d)),
                     ("ln1", (d,)), ("ln2", (d,))):
            shapes.append((f"h{i:02d}.{n}", s))
    return shapes


def ragged_shapes(seed=0):
    import numpy as np

    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(2000):
        n = int(np.exp(rng.uniform(np.log(16), np.log(4096))))
        shapes.append((f"v{i:04d}", (n,)))
    for i in range(256):
        r = int(np.exp(rng.uniform(np.log(64), np.log(4096))))
        c = int(np.exp(rng.uniform(np.log(64), np.log(4096))))
        shapes.append((f"m{i:03d}", (r, c)))
    return shapes


def _numel(s):
    return int(math.prod(s))


def step_bytes(shapes, pbytes=2, gbytes=2, apply=True):
    """Bytes one step must read and write once.  Quantized leaves: param r
    (+ w when fused), grad r, codes r+w and f32 block scales r+w for both
    moments; update-only mode writes f32 updates instead of params.
    Fallback leaves (below min_size) move f32 moments instead of codes."""
    total = 0
    for _, s in shapes:
        n = _numel(s)
        pio = n * pbytes * (2 if apply else 1) + (0 if apply else 4 * n)
        if n >= MIN_SIZE:
            nb = -(-n // BS)
            total += pio + n * gbytes + 2 * (nb * BS) * 2 + nb * 16
        else:
            total += pio + n * gbytes + n * 16
    return total


def algorithmic_bytes(shapes):
    """Fused-step bytes (bf16 params and grads)."""
    return step_bytes(shapes)


def profiled_traffic(workload, exact, param_sr):
    """HBM bytes per launch of the step kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of the same workload (default flags only),
    or None when no such summary exists."""
    if exact or param_sr:
        return None
    name = {"llama7b_bf16_adamw8": "k_adam8_llama7b_traffic.md"}.get(workload)
    path = os.path.join(ROOT, "profiles", name) if name else None
    if not path or not os.path.exists(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch = (\d+)$", open(path).read(), re.M)
    return int(m.group(1)) if m else None


# ------------------------------------------------------- CPU baselines ----
def _threads(threads=None):
    from oracle import oracle as orc

    n = threads or int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    orc.set_threads(n)
    return n


def _timed_loop(body, seconds_target):
    done = 0
    reps = 0
    t0 = time.perf_counter()
    while True:
        done += body()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds_target:
            return done, reps, el


def cpu_baseline(seconds_target=12.0, threads=None, shapes=None, sample_name="the 9 leaves of one Llama-7B layer",
                 param_sr=False, moment_sr=False, pdtype="bf16", packed=False):
    """The CPU oracle (C, OpenMP over blocks) on a bounded sample of the same
    workload (default: the 9 leaves of one Llama layer), one step per leaf,
    repeated until about `seconds_target` seconds of CPU work have run.  With
    stochastic rounding each step also draws its Threefry bits on the CPU
    (the kernel draws them in-kernel), from the packed stream with
    ``packed``.  ``pdtype`` "f32": f32 params and grads."""
    import numpy as np

    from oracle import oracle as orc

    nthreads = _threads(threads)
    rng = np.random.default_rng(0)
    if shapes is None:
        shapes = [s for name, s in llama7b_shapes() if name.startswith("layer00.")]
    leaves = []
    for s in shapes:
        n = _numel(s)
        nb = -(-n // BS)
        quant = n >= MIN_SIZE
        p = rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)
        g = rng.standard_normal(n, dtype=np.float32) * np.float32(1e-3)
        if pdtype != "f32":
            p, g = orc.f32_to_bf16_bits(p), orc.f32_to_bf16_bits(g)
        leaves.append(dict(
            n=n, quant=quant, p=p, g=g,
            mc=np.full(nb * BS, 127, np.uint8) if quant else np.zeros(n, np.float32),
            ms=np.ones(nb, np.float32) if quant else None,
            vc=np.zeros(nb * BS, np.uint8) if quant else np.zeros(n, np.float32),
            vs=np.ones(nb, np.float32) if quant else None))
    state = {"step": 0}

    def body():
        state["step"] += 1
        t = state["step"]
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=t, decay=True, apply=True,
                              param_sr=param_sr, moment_sr=moment_sr)
        done = 0
        for i, L in enumerate(leaves):
            pb = None
            if param_sr:
                pb = orc.packed_param_bits((t, i), L["n"]) if packed else orc.random_bits((t, i), L["n"])
            mb = vb = None
            if moment_sr and L["quant"]:
                if packed:
                    mb, vb = orc.packed_moment_bits((t, 1000 + i), L["mc"].size)
                else:
                    mb = orc.random_bits((t, 1000 + i), L["mc"].size)
                    vb = orc.random_bits((t, 2000 + i), L["vc"].size)
            dt = orc.F32 if pdtype == "f32" else orc.BF16
            orc.adam8_leaf(hp, L["p"], dt, L["g"], dt, orc.MOM_QUANT if L["quant"] else orc.MOM_F32,
                           L["mc"], L["ms"], L["vc"], L["vs"], BS, mu_bits=mb, nu_bits=vb, p_bits=pb)
            done += L["n"]
        return done

    done, reps, el = _timed_loop(body, seconds_target)
    return {
        "value": done / el,
        "unit": "params/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"CPU oracle (C restatement, OpenMP, {nthreads} threads) over {sample_name} "
                  f"({sum(L['n'] for L in leaves)} params), {reps} steps in {el:.1f} s",
    }


def cpu_baseline_kernel(kind, seconds_target=12.0, threads=None, n=1 << 22, packed=False):
    """The CPU oracle's standalone quantize / dequantize / SR / apply over a
    2^22-element sample of the same input distribution (SR bits from the
    packed stream with ``packed``)."""
    import numpy as np

    from oracle import oracle as orc

    nthreads = _threads(threads)
    rng = np.random.default_rng(0)
    x = (np.exp(rng.uniform(np.log(1e-8), np.log(1e2), n)) * rng.choice([-1.0, 1.0], n)).astype(np.float32)
    if kind == "quantize":
        def body():
            orc.quantize(x, BS, orc.Q_SIGNED)
            return n
    elif kind == "dequantize":
        codes, scales = orc.quantize(x, BS, orc.Q_SIGNED)

        def body():
            orc.dequantize(codes, scales, n, BS, orc.Q_SIGNED)
            return n
    elif kind == "sr_bf16":
        def body():
            orc.sr_bf16(x, orc.packed_param_bits((0, 1), n) if packed else orc.random_bits((0, 1), n))
            return n
    elif kind in ("apply", "apply_rne"):
        p = orc.f32_to_bf16_bits(x * np.float32(1e-3))
        u = (x * np.float32(1e-6)).astype(np.float32)

        def body():
            bits = None
            if kind == "apply":
                bits = orc.packed_param_bits((0, 1), n) if packed else orc.random_bits((0, 1), n)
            orc.apply_updates(p, orc.BF16, u, bits=bits)
            return n
    else:
        raise ValueError(kind)
    done, reps, el = _timed_loop(body, seconds_target)
    return {
        "value": done / el,
        "unit": "params/s" if kind in ("apply", "apply_rne") else "elements/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"CPU oracle ({kind}, C, OpenMP, {nthreads} threads; Threefry bits generated on the CPU where "
                  f"the kernel draws them) over {n} elements, {reps} reps in {el:.1f} s",
    }


# ------------------------------------------------------------ workloads ---
class Workload:
    """What one bench line measures: units per step, algorithmic HBM bytes
    per step, the step closure, its config and its CPU baseline."""

    def __init__(self, name, units, unit, nbytes, step, config, cpu, metric):
        self.name, self.units, self.unit, self.nbytes = name, units, unit, nbytes
        self.step, self.config, self.cpu, self.metric = step, config, cpu, metric
        self.probe = None  # the memory ceiling of the step's byte mix, where the library can measure it


def _tree_workload(args, shapes_fn, workload, *, param_sr, grads="normal", optax=False, adam_mu=None, clip=None,
                   guard=False, groups=False, magma=False, moment_sr=False, accum=1, pdtype="bf16"):
    import numpy as np
    import torch

    import rollfast_amd as rf

    shapes = shapes_fn()
    n_params = sum(_numel(s) for _, s in shapes)
    print(f"[bench] {workload}: {n_params} params in {len(shapes)} leaves; allocating", file=sys.stderr, flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    tdt = torch.float32 if pdtype == "f32" else torch.bfloat16  # params and grads
    params = {name: (torch.randn(s, generator=gen, device="cuda", dtype=torch.float32) * 0.02).to(tdt)
              for name, s in shapes}
    packed = args.sr_bits == "packed"
    if adam_mu is None:
        tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=args.exact, stochastic_rounding=moment_sr,
                       sr_bits=args.sr_bits)
    else:
        tx = rf.adamw(learning_rate=1e-3, weight_decay=0.01, exact=args.exact,
                      mu_dtype=torch.bfloat16 if adam_mu == "bf16" else None, use_magma=magma,
                      sr_bits="jax" if magma else args.sr_bits)
    chain_clip = None
    if groups:
        # the fine-tune builders' shape: groups with their own lr / decay / key
        # (embeddings and norms undecayed), clipping and the non-finite guard
        # around the multi_transform, all one launch
        def group_of(name):
            return "embed" if "embed" in name or "lm_head" in name else ("norm" if "norm" in name else "base")

        labels = {name: group_of(name) for name, _ in shapes}
        tx = rf.multi_transform({
            "base": rf.adamw8(learning_rate=1e-3, weight_decay=0.05, exact=args.exact, key=rf.prng.PRNGKey(1)),
            "embed": rf.adamw8(learning_rate=2e-4, weight_decay=0.0, exact=args.exact, key=rf.prng.PRNGKey(2)),
            "norm": rf.adamw8(learning_rate=1e-3, weight_decay=0.0, exact=args.exact, key=rf.prng.PRNGKey(3)),
        }, labels)
        if clip is not None:
            tx = rf.chain(rf.clip_by_global_norm(clip), tx)
            chain_clip, clip = clip, None
    if guard:
        tx = rf.apply_if_finite(tx, 1)
    if accum > 1:
        # the builders' accumulation wrapper (AccumulationConfig defaults:
        # mean of the micro-steps' grads in an f32 accumulator)
        tx = rf.MultiSteps(tx, every_k_schedule=accum, use_grad_mean=True, accumulator_dtype=torch.float32)
    state = tx.init(params)
    pool = []
    rng = np.random.default_rng(0)
    for k in range(args.grad_pool):
        gen.manual_seed(1000 + k)
        g = {}
        for name, s in shapes:
            if grads == "student_t":
                # Student-t(3) = N / sqrt(chi2_3 / 3), times a log-uniform per-leaf scale
                z = torch.randn(s, generator=gen, device="cuda")
                c = sum(torch.randn(s, generator=gen, device="cuda") ** 2 for _ in range(3)) / 3
                t = z / torch.sqrt(c) * float(np.exp(rng.uniform(np.log(1e-6), 0.0)))
                flat = t.view(-1)
                nb = flat.numel() // BS
                if nb:
                    zero = torch.from_numpy(rng.random(nb) < 0.1).cuda()
                    flat[: nb * BS].view(nb, BS)[zero] = 0.0
                g[name] = t.to(torch.bfloat16)
            else:
                g[name] = (torch.randn(s, generator=gen, device="cuda", dtype=torch.float32) * 1e-3).to(tdt)
        pool.append(g)
    key = rf.prng.PRNGKey(0)
    holder = {"params": params, "state": state, "k": 0}

    def micro_step():
        g = pool[holder["k"] % len(pool)]
        holder["k"] += 1
        if optax:
            _, holder["state"] = tx.update(g, holder["state"], holder["params"])
        elif magma:  # the step (with the Magma sums), the Magma factors, then apply_updates with them
            holder["params"], holder["state"] = rf.adamw_step(tx, holder["params"], g, holder["state"], key=key,
                                                              stochastic=param_sr)
        else:
            holder["params"], holder["state"] = rf.adamw8_step(tx, holder["params"], g, holder["state"], key=key,
                                                               stochastic=param_sr, clip_global_norm=clip)

    def step():
        # one optimizer step: with accumulation, a whole window of micro-steps
        for _ in range(accum):
            micro_step()

    n_quant = sum(1 for _, s in shapes if _numel(s) >= MIN_SIZE) if adam_mu is None else 0
    config = {
        "workload": workload,
        "params": n_params,
        "leaves": len(shapes),
        "quantized_leaves": n_quant,
        "block_size": BS,
        "param_dtype": pdtype,
        "grad_dtype": pdtype,
        "moments": ("uint8 codebook codes + f32 block scales (f32 fallback below 4096 elements)"
                    if adam_mu is None else f"{adam_mu} (full-precision AdamW"
                    + (", stochastically rounded storage)" if adam_mu == "bf16" else ")")),
        "param_rounding": (("stochastic" + (" (packed bits: a Threefry block per 4 elements)" if packed else ""))
                           if param_sr else "nearest-even") if pdtype == "bf16" else "f32 add",
        "moment_rounding": (("stochastic (packed bits: a Threefry block per pair of elements for both moments)" if packed
                             else "stochastic (in-kernel Threefry bits)") if moment_sr else "nearest"),
        "direction": "ieee" if args.exact else "hw rcp/sqrt",
        "mode": "optax update-only (f32 updates)" if optax else "fused step (params written)",
        "launches_per_step": 1 if clip is None else 4,
        "grad_pool": len(pool),
    }
    if clip is not None:
        config["clip_global_norm"] = clip
    if groups:
        config["groups"] = "multi_transform: base (lr 1e-3, wd 0.05), embed (lr 2e-4), norm (lr 1e-3), one launch"
        config["clip_global_norm"] = chain_clip
        config["launches_per_step"] = 4
    if guard:
        config["nonfinite"] = "skip (apply_if_finite, max_consecutive_errors=1; one int32 read back per step)"
        config["launches_per_step"] = 4
    if accum > 1:
        config["accumulation"] = (f"MultiSteps(every_k_schedule={accum}, use_grad_mean=True, f32 accumulator) "
                                  "around the whole transformation; a step is one window: "
                                  f"{accum} micro-steps, the last running the inner step on the accumulator")
        config["launches_per_step"] += accum + 1
    if magma:
        config["magma"] = ("use_magma=True (p 0.5, tau 2): sums written by the step, per-leaf factors after "
                           "it, folded into apply_updates")
        config["mode"] = "adamw_step (update-only step, then apply_updates with the Magma factor)"
        config["launches_per_step"] = 4
    if shapes_fn is llama7b_shapes and pdtype == "f32":
        cpu = lambda: cpu_baseline(args.cpu_seconds, pdtype="f32")  # noqa: E731
    elif shapes_fn is llama7b_shapes:
        cpu = lambda: cpu_baseline(args.cpu_seconds, param_sr=param_sr, moment_sr=moment_sr,  # noqa: E731
                                   packed=packed)
    else:
        sub = [s for _, s in shapes][:400]
        cpu = lambda: cpu_baseline(args.cpu_seconds, shapes=sub,  # noqa: E731
                                   sample_name=f"the first {len(sub)} leaves", param_sr=param_sr,
                                   moment_sr=moment_sr, packed=packed)
    if accum > 1:
        cpu = None  # the oracle baseline times the plain step, not a window
    metric = METRIC if workload == "llama7b_bf16_adamw8" else f"adam8 params/sec + achieved HBM GB/s, {workload}, 1 GPU"
    if adam_mu is None:
        g_extra = 2 if (clip is not None or guard or groups) else 0  # the norm pre-pass's grad read
        if accum > 1:
            # micro-steps: bf16 grad read, f32 accumulator read and written
            # (10 B); the inner step reads f32 grads (+2 B over bf16, and its
            # pre-pass reads 4 B instead of 2); the reset reads and writes
            # the accumulator (8 B)
            g_extra = 2 * g_extra + 2 + accum * 10 + 8
        pb = 4 if pdtype == "f32" else 2
        nbytes = step_bytes(shapes, pbytes=pb, gbytes=pb, apply=not optax) + n_params * g_extra
    else:
        mb = 4 if adam_mu == "f32" else 2
        nbytes = n_params * (2 + 2 + 2 + 2 * 2 * mb)  # p r+w, g r, two moments r+w
        if magma:
            # update-only step writes f32 updates (4) instead of params (2)
            # and the Magma sums (24 B per 2048 elements, left out);
            # apply_updates with the per-leaf Magma factor folded in reads
            # the updates (4) and the params and writes the params (2 + 2)
            nbytes = n_params * ((2 + 2 + 2 * 2 * mb + 4) + (4 + 2 + 2))
        cpu = None
    wl = Workload(workload, n_params, "params/s", nbytes, step, config, cpu, metric)
    wl.holder = holder  # params and optimizer state, for the placement study's cross pairs
    if (shapes_fn is llama7b_shapes and adam_mu is None and not (optax or groups or guard or accum > 1)
            and clip is None):
        # every leaf is whole 2048-blocks: the stream probe moves the step's bytes
        pb = 4 if pdtype == "f32" else 2
        block_bytes = BS * (2 * pb + pb + 4) + 16

        def probe():
            from rollfast_amd import _lib

            plan = tx.update.engine._last["plan"]
            return plan.stream_probe(_lib.stream_ptr()) * block_bytes

        wl.probe = probe
    return wl


def _c5_input(n, seed=5):
    """|x| log-uniform in [1e-8, 1e2] with a random sign, plus zeros (half of
    them -0) at every 97th element and f32 denormals with random mantissa and
    sign at every 89th from element 1."""
    import torch

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    x = torch.empty(n, device="cuda").uniform_(math.log(1e-8), math.log(1e2), generator=gen).exp_()
    sign = torch.rand(n, device="cuda", generator=gen) < 0.5
    x[sign] *= -1.0
    d = x[1::89]
    mant = torch.randint(1, 1 << 23, (d.numel(),), device="cuda", generator=gen, dtype=torch.int32)
    den = mant.view(torch.float32)
    d.copy_(torch.where(torch.rand(d.numel(), device="cuda", generator=gen) < 0.5, -den, den))
    z = x[::97]  # after the denormals: where the two strides meet, a zero
    z.copy_(torch.where(torch.arange(z.numel(), device="cuda") % 2 == 1, -0.0, 0.0))
    return x


def _kernel_workload(args, kind):
    import torch

    from rollfast_amd import _lib

    L = _lib.lib()
    sp = _lib.stream_ptr
    packed = args.sr_bits == "packed"
    if kind in ("apply", "apply_rne"):
        sr = kind == "apply"
        shapes = llama7b_shapes()
        n = sum(_numel(s) for _, s in shapes)
        print(f"[bench] llama7b_{kind}: {n} params; allocating", file=sys.stderr, flush=True)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(0)
        params = [(torch.randn(s, generator=gen, device="cuda") * 0.02).to(torch.bfloat16) for _, s in shapes]
        upd = [torch.randn(s, generator=gen, device="cuda") * 1e-5 for _, s in shapes]
        rows = (_lib.ApplyLeaf * len(shapes))()
        for i, (p, u) in enumerate(zip(params, upd)):
            rows[i].param = p.data_ptr()
            rows[i].updates = u.data_ptr()
            rows[i].bits = None
            rows[i].size = p.numel()
            rows[i].param_dtype = _lib.RF_BF16
            rows[i].param_index = i

        def step():
            if sr and packed:
                _lib.check(L.rf_apply_updates_packed(rows, len(shapes), 0, 42, sp()), "apply")
            else:
                _lib.check(L.rf_apply_updates(rows, len(shapes), 1 if sr else 0, 0, 42, sp()), "apply")

        name = "llama7b_bf16_apply_updates_" + ("sr" if sr else "rne") + ("_packed_bits" if sr and packed else "")
        return Workload(name, n, "params/s", n * (2 + 4 + 2), step,
                        {"workload": name, "params": n, "leaves": len(shapes), "param_dtype": "bf16",
                         "update_dtype": "f32",
                         "rounding": ("stochastic (packed bits: a Threefry block per 4 elements)" if packed
                                      else "stochastic (in-kernel Threefry)") if sr else "nearest-even",
                         "launches_per_step": 1},
                        lambda: cpu_baseline_kernel(kind, args.cpu_seconds, packed=packed),
                        "apply_updates params/sec + achieved HBM GB/s, 7B Llama pytree bf16 "
                        + ("SR" if sr else "nearest-even") + ", 1 GPU")
    n = 1 << 30
    nb = n // BS
    print(f"[bench] {kind}: 2^30 elements; allocating", file=sys.stderr, flush=True)
    x = _c5_input(n)
    codes = torch.empty(n, dtype=torch.uint8, device="cuda")
    scales = torch.empty(nb, dtype=torch.float32, device="cuda")

    def quantize():
        _lib.check(L.rf_blockwise_quantize(0, x.data_ptr(), _lib.RF_F32, n, BS, 0, 0, 0, None, codes.data_ptr(),
                                           scales.data_ptr(), _lib.RF_F32, sp()), "quantize")

    if kind == "quantize":
        step = quantize
        nbytes = n * 4 + n + nb * 4
    elif kind == "dequantize":
        quantize()
        out = torch.empty(n, dtype=torch.float32, device="cuda")

        def step():
            _lib.check(L.rf_blockwise_dequantize(0, codes.data_ptr(), scales.data_ptr(), _lib.RF_F32, n, BS,
                                                 _lib.RF_F32, out.data_ptr(), sp()), "dequantize")
        nbytes = n + nb * 4 + n * 4
    elif kind == "sr_bf16":
        out = torch.empty(n, dtype=torch.bfloat16, device="cuda")

        def step():
            if packed:
                _lib.check(L.rf_sr_bf16_packed(x.data_ptr(), n, 0, 42, out.data_ptr(), sp()), "sr_bf16")
            else:
                _lib.check(L.rf_sr_bf16(x.data_ptr(), n, 0, 42, None, out.data_ptr(), sp()), "sr_bf16")
        nbytes = n * 4 + n * 2
    else:
        raise ValueError(kind)
    name = f"{kind}_2p30_f32" + ("_packed_bits" if kind == "sr_bf16" and packed else "")
    return Workload(name, n, "elements/s", nbytes, step,
                    {"workload": name, "elements": n, "block_size": BS, "quantizer": "dynamic_signed",
                     "input": "log-uniform |x| in [1e-8, 1e2], random sign, +-0 every 97th and denormals "
                              "every 89th element", "launches_per_step": 1},
                    lambda: cpu_baseline_kernel(kind, args.cpu_seconds, packed=packed),
                    f"{kind} elements/sec + achieved HBM GB/s, 2^30 f32, 1 GPU")


WORKLOADS = {
    "llama7b": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw8", param_sr=a.param_sr),
    "llama7b_f32": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_f32_adamw8", param_sr=False, pdtype="f32"),
    "gpt2": lambda a: _tree_workload(a, gpt2_small_shapes, "gpt2_small_bf16_adamw8", param_sr=True),
    "ragged": lambda a: _tree_workload(a, ragged_shapes, "ragged_2256_leaves_bf16_adamw8", param_sr=a.param_sr,
                                       grads="student_t"),
    "llama7b_msr": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw8_moment_sr", param_sr=a.param_sr,
                                            moment_sr=True),
    "llama7b_clip": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw8_clip_global_norm",
                                             param_sr=False, clip=1.0),
    "llama7b_finetune": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw8_clip_skip_nonfinite",
                                                 param_sr=False, clip=1.0, guard=True),
    "llama7b_finetune_groups": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw8_grouped_finetune",
                                                        param_sr=False, clip=1.0, guard=True, groups=True),
    "llama7b_finetune_accum4": lambda a: _tree_workload(a, llama7b_shapes,
                                                        "llama7b_bf16_adamw8_grouped_finetune_multisteps4",
                                                        param_sr=a.param_sr, clip=1.0, guard=True, groups=True,
                                                        accum=4),
    "llama7b_optax": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw8_optax_update",
                                              param_sr=False, optax=True),
    "llama7b_adamw_f32": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw_f32_moments",
                                                  param_sr=False, adam_mu="f32"),
    "llama7b_adamw_bf16": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw_bf16_moments",
                                                   param_sr=False, adam_mu="bf16"),
    "llama7b_adamw_magma": lambda a: _tree_workload(a, llama7b_shapes, "llama7b_bf16_adamw_f32_moments_magma",
                                                    param_sr=False, adam_mu="f32", magma=True),
    "llama7b_apply": lambda a: _kernel_workload(a, "apply"),
    "llama7b_apply_rne": lambda a: _kernel_workload(a, "apply_rne"),
    "quantize_2p30": lambda a: _kernel_workload(a, "quantize"),
    "dequantize_2p30": lambda a: _kernel_workload(a, "dequantize"),
    "sr_bf16_2p30": lambda a: _kernel_workload(a, "sr_bf16"),
}


def placement_study(args):
    """Times args.copies independent copies of one workload in one process.

    The copies run the same kernels on the same shapes and differ only in
    where their buffers landed in device memory.  Each round steps every
    copy once, in ascending order on even rounds and descending on odd ones,
    each step bracketed by HIP events and a synchronize.  The JSON line lists
    the copies in step order (warmup steps included) so that a profiler's
    dispatches can be matched to their copy."""
    import statistics

    import torch

    wls = []
    for c in range(args.copies):
        wls.append(WORKLOADS[args.workload](args))
        torch.cuda.synchronize()
        print(f"[bench] copy {c} built; {torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated",
              file=sys.stderr, flush=True)
    order = []
    for c, wl in enumerate(wls):
        for _ in range(args.warmup):
            wl.step()
            order.append(c)
    torch.cuda.synchronize()
    times = [[] for _ in wls]
    for r in range(args.steps):
        for c in (range(len(wls)) if r % 2 == 0 else reversed(range(len(wls)))):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            wls[c].step()
            e1.record()
            torch.cuda.synchronize()
            times[c].append(e0.elapsed_time(e1))
            order.append(c)
    for c, t in enumerate(times):
        print(f"[bench] copy {c}: median {statistics.median(t):.3f} ms, min {min(t):.3f}, max {max(t):.3f}",
              file=sys.stderr, flush=True)
    cross = None
    if args.cross:
        # copy a's params and grads stepped with copy b's optimizer state:
        # three steps per pair, the best of the last two, two rounds in
        # opposite pair order
        holders = [getattr(wl, "holder", None) for wl in wls]
        if any(h is None for h in holders):
            raise SystemExit(f"--cross needs an optimizer-step workload, not {args.workload}")
        n = len(wls)
        best = [[float("inf")] * n for _ in range(n)]
        pairs = [(a, b) for a in range(n) for b in range(n)]
        for r in range(2):
            for a, b in (pairs if r == 0 else pairs[::-1]):
                own = holders[a]["state"]
                holders[a]["state"] = holders[b]["state"]
                t = []
                for _ in range(3):
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    wls[a].step()
                    e1.record()
                    torch.cuda.synchronize()
                    t.append(e0.elapsed_time(e1))
                holders[b]["state"] = holders[a]["state"]  # the stepped state stays copy b's
                if a != b:
                    holders[a]["state"] = own
                best[a][b] = min(best[a][b], min(t[1:]))
        cross = best
        for a in range(n):
            print("[bench] params/grads of copy %d with the state of copies 0..%d: %s"
                  % (a, n - 1, " ".join(f"{x:.3f}" for x in best[a])), file=sys.stderr, flush=True)
    print(json.dumps({
        "study": "placement",
        "config": wls[0].config,
        "copies": args.copies,
        "steps_per_copy": args.steps,
        "warmup_per_copy": args.warmup,
        "ms_median": [statistics.median(t) for t in times],
        "ms_min": [min(t) for t in times],
        "ms_max": [max(t) for t in times],
        "step_order": order,
        "cross_ms": cross,
    }), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="llama7b")
    ap.add_argument("--grad-pool", type=int, default=2, help="distinct gradient buffers cycled by the steps")
    ap.add_argument("--exact", action="store_true", help="IEEE div/sqrt in the update direction")
    ap.add_argument("--param-sr", action="store_true", help="stochastic rounding of bf16 params")
    ap.add_argument("--sr-bits", choices=("jax", "packed"), default="jax",
                    help="bit source of the stochastic roundings: jax.random.bits' stream (one Threefry block per "
                         "32-bit word) or the packed one (a block per four param roundings, or per pair of "
                         "elements for both moments)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copies", type=int, default=1,
                    help="placement study: build this many independent copies of the workload, time their "
                         "steps in alternating order and print each copy's times instead of the benchmark line")
    ap.add_argument("--cross", action="store_true",
                    help="with --copies: also time every pair (params and grads of copy a, optimizer state of copy b)")
    ap.add_argument("--calibrate-copy-gib", type=float, default=0.0,
                    help="after the timed steps, run three device copies of this many GiB "
                         "(reference kernel of known traffic for profiler byte counters)")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the step has no cross-GPU "
              "communication and rollfast_amd runs on one GPU.", file=sys.stderr)
        return 2

    import torch

    torch.cuda.set_device(0)
    if args.copies > 1:
        return placement_study(args)
    wl = WORKLOADS[args.workload](args)
    torch.cuda.synchronize()
    print(f"[bench] warmup {args.warmup} steps", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()

    # One event pair around the timed steps (on the launch stream): markers
    # between steps would add idle gaps of their own to short steps.
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for k in range(args.steps):
        wl.step()
    end.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    kernel_ms_avg = start.elapsed_time(end) / args.steps
    achieved = wl.nbytes / (kernel_ms_avg * 1e-3)
    value = wl.units / (ms_per_step * 1e-3)
    print(f"[bench] {ms_per_step:.3f} ms/step wall, {kernel_ms_avg:.3f} ms/step events, "
          f"{achieved / 1e9:.1f} GB/s", file=sys.stderr, flush=True)

    ceiling = None
    if wl.probe is not None:
        # The same bytes in the same buffers, layout and grid, without the
        # step's arithmetic: what this memory placement gives the byte mix.
        for _ in range(2):
            wl.probe()
        pstart, pend = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        pbytes = 0
        pstart.record()
        for k in range(args.steps):
            pbytes = wl.probe()
        pend.record()
        torch.cuda.synchronize()
        probe_ms = pstart.elapsed_time(pend) / args.steps
        ceiling = pbytes / (probe_ms * 1e-3)
        print(f"[bench] stream probe: {probe_ms:.3f} ms, {ceiling / 1e9:.1f} GB/s", file=sys.stderr, flush=True)

    if args.calibrate_copy_gib > 0:
        nbytes = int(args.calibrate_copy_gib * (1 << 30))
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"[bench] calibration copy: 3 x {nbytes} bytes read + written", file=sys.stderr, flush=True)
        del src, dst

    cpu = None
    if not args.no_cpu_baseline and wl.cpu is not None:
        print("[bench] CPU oracle baseline", file=sys.stderr, flush=True)
        cpu = wl.cpu()

    traffic = profiled_traffic(wl.name, args.exact, args.param_sr)
    line = {
        "metric": wl.metric,
        "value": value,
        "unit": wl.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": wl.config,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved / 1e9,
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK,
            "traffic": traffic,
            "traffic_source": "profiles/ rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated" if traffic else None,
            "algorithmic_bytes_per_step": wl.nbytes,
            "kernel_ms": kernel_ms_avg,
        },
        "cpu_baseline": cpu,
    }
    if ceiling is not None:
        line["roofline"]["ceiling"] = ceiling / 1e9
        line["roofline"]["ceiling_frac"] = achieved / ceiling
        line["roofline"]["ceiling_source"] = (
            "rf_adam8_plan_stream_probe timed after the steps: the step's bytes, lane layout and grid over the "
            "same buffers, no arithmetic")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
