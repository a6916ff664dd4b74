"""Build recipe for the gfx950 shared library ``rollfast_amd/_lib/librfadam8.so``.

The library is built in-tree with ``hipcc`` (cross-compiles without a GPU)
so the ``.so`` travels with the source tree to the machine that runs it.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
LIB_NAME = "librfadam8.so"
LIB_PATH = os.path.join(OUT_DIR, LIB_NAME)
OBJ_DIR = os.path.join(HERE, "_lib", "obj")
HOST_SRC = os.path.join(CSRC, "rf_host.hip")
INST_SRC = os.path.join(CSRC, "rf_adam8_inst.hip")
# One object per (apply, moment SR, exact) instance of the step kernel.
VARIANTS = [(a, m, e) for a in (0, 1) for m in (0, 1) for e in (0, 1)]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -ffp-contract=off: every multiply and add rounds separately, as in the
#   reference's elementwise f32 program; FMAs appear only where written.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 generation.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _compile_jobs():
    inc = ["-I", os.path.join(REPO, "include")]
    jobs = [([HIPCC, *FLAGS, *inc, "-c", HOST_SRC, "-o", os.path.join(OBJ_DIR, "rf_host.o")],
             os.path.join(OBJ_DIR, "rf_host.o"))]
    for a, m, e in VARIANTS:
        obj = os.path.join(OBJ_DIR, f"rf_adam8_a{a}_m{m}_e{e}.o")
        defs = [f"-DRFI_APPLY={a}", f"-DRFI_MSR={m}", f"-DRFI_EXACT={e}"]
        jobs.append(([HIPCC, *FLAGS, *inc, *defs, "-c", INST_SRC, "-o", obj], obj))
    return jobs


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile the HIP library (objects in parallel, then link); returns
    the path of the built ``.so``."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    max_par = jobs or min(len(VARIANTS) + 1, max(1, os.cpu_count() or 1))
    pending = _compile_jobs()
    running = []
    failures = []
    while pending or running:
        while pending and len(running) < max_par:
            cmd, obj = pending.pop(0)
            if verbose:
                print(" ".join(cmd), flush=True)
            running.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), obj))
        proc, obj = running.pop(0)
        out, _ = proc.communicate()
        if proc.returncode != 0:
            failures.append((obj, out))
    if failures:
        for obj, out in failures:
            sys.stderr.write(f"--- {obj}\n{out}\n")
        raise RuntimeError(f"hipcc failed for {len(failures)} object(s)")
    tmp = LIB_PATH + ".tmp"
    objs = [obj for _, obj in _compile_jobs()]
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(link), flush=True)
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"link failed with exit code {proc.returncode}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
