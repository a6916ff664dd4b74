#!/usr/bin/env python
"""Throughput of the fused 8-bit AdamW step on one MI355X.

Default workload: the Llama-7B-shaped bf16 pytree (32 layers, hidden 4096,
SwiGLU MLP 11008, vocab 32000, RMSNorm vectors; 6,738,415,616 params in 291
leaves, all quantized: uint8 codes + f32 scales per 2048-element block),
params ~N(0, 0.02^2), grads ~N(0, 1e-3^2).  A step is one fused
adamw8_step over the whole tree (one launch): dequantize both moments, AdamW
update (lr 1e-3, wd 0.01, betas 0.9/0.999), bf16 params written with
round-to-nearest-even, moments requantized.  Gradients are drawn before the
timed region into a pool of distinct buffers that the steps cycle through.

Prints one JSON line: params/s (whole job), ms per step, the HBM roofline of
the step kernel (algorithmic bytes / kernel time, measured with HIP events on
the launch stream) and the CPU oracle's throughput on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
METRIC = "adam8 step params/sec + achieved HBM GB/s (% peak), 7B Llama pytree, 1 GPU"


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


WORKLOADS = {
    "llama7b": (llama7b_shapes, "llama7b_bf16_adamw8"),
    "gpt2": (gpt2_small_shapes, "gpt2_small_bf16_adamw8"),
    "ragged": (ragged_shapes, "ragged_2256_leaves_bf16_adamw8"),
}


def algorithmic_bytes(shapes, block_size=2048, min_size=4096):
    """Bytes one step must read and write once: bf16 param r+w, bf16 grad r,
    codes r+w (2 moments), f32 block scales r+w (2 moments); fallback leaves
    move f32 moments instead of codes."""
    total = 0
    for _, s in shapes:
        n = 1
        for d in s:
            n *= d
        if n >= min_size:
            nb = -(-n // block_size)
            total += n * (2 + 2 + 2) + 2 * (nb * block_size) * 2 + nb * 16
        else:
            total += n * (2 + 2 + 2) + n * 16
    return total


def profiled_traffic(workload, exact, param_sr):
    """HBM bytes per launch of the step kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of the same workload (default flags only),
    or None when no such summary exists."""
    if exact or param_sr:
        return None
    import re

    name = {"llama7b_bf16_adamw8": "k_adam8_llama7b_traffic.md"}.get(workload)
    path = os.path.join(ROOT, "profiles", name) if name else None
    if not path or not os.path.exists(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch = (\d+)$", open(path).read(), re.M)
    return int(m.group(1)) if m else None


def cpu_baseline(seconds_target=12.0, threads=None):
    """The CPU oracle (C, OpenMP over blocks) on a bounded sample of the same
    workload: the leaves of one Llama layer, one step each, repeated until
    about `seconds_target` seconds of CPU work have run."""
    import numpy as np

    from oracle import oracle as orc

    nthreads = threads or int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    orc.set_threads(nthreads)
    rng = np.random.default_rng(0)
    shapes = [s for name, s in llama7b_shapes() if name.startswith("layer00.")]
    leaves = []
    for s in shapes:
        n = int(np.prod(s))
        nb = -(-n // 2048)
        leaves.append(dict(
            n=n,
            p=orc.f32_to_bf16_bits(rng.standard_normal(n, dtype=np.float32) * np.float32(0.02)),
            g=orc.f32_to_bf16_bits(rng.standard_normal(n, dtype=np.float32) * np.float32(1e-3)),
            mc=np.full(nb * 2048, 127, np.uint8), ms=np.ones(nb, np.float32),
            vc=np.zeros(nb * 2048, np.uint8), vs=np.ones(nb, np.float32)))
    done = 0
    step = 0
    t0 = time.perf_counter()
    while True:
        step += 1
        hp = orc.make_hparams(weight_decay=0.01, lr=1e-3, count=step, decay=True, apply=True)
        for L in leaves:
            orc.adam8_leaf(hp, L["p"], orc.BF16, L["g"], orc.BF16, orc.MOM_QUANT, L["mc"], L["ms"], L["vc"],
                           L["vs"], 2048)
            done += L["n"]
        el = time.perf_counter() - t0
        if el >= seconds_target:
            break
    return {
        "value": done / el,
        "unit": "params/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"CPU oracle (C restatement, OpenMP, {nthreads} threads) over the 9 leaves of one Llama-7B "
                  f"layer ({sum(L['n'] for L in leaves)} params), {step} steps in {el:.1f} s",
    }


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="llama7b")
    ap.add_argument("--grad-pool", type=int, default=2, help="distinct gradient buffers cycled by the steps")
    ap.add_argument("--exact", action="store_true", help="IEEE div/sqrt in the update direction")
    ap.add_argument("--param-sr", action="store_true", help="stochastic rounding of bf16 params")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--calibrate-copy-gib", type=float, default=0.0,
                    help="after the timed steps, run three device copies of this many GiB "
                         "(reference kernel of known traffic for profiler byte counters)")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the step has no cross-GPU "
              "communication and multi-GPU runs are not part of this build.", file=sys.stderr)
        return 2

    import torch

    import rollfast_amd as rf

    torch.cuda.set_device(0)
    shapes_fn, workload = WORKLOADS[args.workload]
    shapes = shapes_fn()
    n_params = sum(int(torch.Size(s).numel()) for _, s in shapes)
    print(f"[bench] {workload}: {n_params} params in {len(shapes)} leaves; allocating", file=sys.stderr, flush=True)

    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    params = {}
    for name, s in shapes:
        params[name] = (torch.randn(s, generator=gen, device="cuda", dtype=torch.float32) * 0.02).to(torch.bfloat16)
    tx = rf.adamw8(learning_rate=1e-3, weight_decay=0.01, exact=args.exact)
    state = tx.init(params)
    pool = []
    for k in range(args.grad_pool):
        gen.manual_seed(1000 + k)
        pool.append({name: (torch.randn(s, generator=gen, device="cuda", dtype=torch.float32) * 1e-3)
                     .to(torch.bfloat16) for name, s in shapes})
    torch.cuda.synchronize()
    key = rf.prng.PRNGKey(0)
    print(f"[bench] warmup {args.warmup} steps", file=sys.stderr, flush=True)
    for w in range(args.warmup):
        params, state = rf.adamw8_step(tx, params, pool[w % len(pool)], state, key=key, stochastic=args.param_sr)
    torch.cuda.synchronize()

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    print(f"[bench] timing {args.steps} steps", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        starts[k].record()
        params, state = rf.adamw8_step(tx, params, pool[k % len(pool)], state, key=key, stochastic=args.param_sr)
        ends[k].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    kernel_ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    kernel_ms_avg = sum(kernel_ms) / len(kernel_ms)
    bytes_step = algorithmic_bytes(shapes)
    achieved = bytes_step / (kernel_ms_avg * 1e-3)
    value = n_params / (ms_per_step * 1e-3)
    print(f"[bench] {ms_per_step:.3f} ms/step wall, {kernel_ms_avg:.3f} ms/step events, "
          f"{achieved / 1e9:.1f} GB/s", file=sys.stderr, flush=True)

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
    if not args.no_cpu_baseline:
        print("[bench] CPU oracle baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(args.cpu_seconds)

    traffic = profiled_traffic(workload, args.exact, args.param_sr)
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "params": n_params,
            "leaves": len(shapes),
            "block_size": 2048,
            "param_dtype": "bf16",
            "grad_dtype": "bf16",
            "moments": "uint8 codebook codes + f32 block scales",
            "param_rounding": "stochastic" if args.param_sr else "nearest-even",
            "direction": "ieee" if args.exact else "hw rcp/sqrt",
            "launches_per_step": 1,
            "grad_pool": len(pool),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved / 1e9,
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK,
            "traffic": traffic,
            "traffic_source": "profiles/ rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated" if traffic else None,
            "algorithmic_bytes_per_step": bytes_step,
            "kernel_ms": kernel_ms_avg,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
