"""Build recipe for the gfx950 shared library ``rollfast_amd/_lib/librfadam8.so``
and the host fast-path module ``rollfast_amd/_lib/_rfhost*.so``.

Both are built in-tree (``hipcc`` cross-compiles without a GPU; the module
with ``g++`` against torch's headers) so they travel with the source tree to
the machine that runs them.
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
# The soname carries the ABI revision of include/rfadam8.h (RF_ABI_VERSION):
# a program linked against another revision does not load this library.
ABI_VERSION = 2
SONAME = f"{LIB_NAME}.{ABI_VERSION}"
OBJ_DIR = os.path.join(HERE, "_lib", "obj")
HOST_SRC = os.path.join(CSRC, "rf_host.hip")
# The native host fast path of the fused step: a CPython module built against
# torch's C++ headers (tensor data pointers without a Python call).
PYHOST_SRC = os.path.join(CSRC, "rf_pyhost.cpp")
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


def pyhost_path() -> str:
    import sysconfig

    return os.path.join(OUT_DIR, "_rfhost" + sysconfig.get_config_var("EXT_SUFFIX"))


def _pyhost_job():
    """g++ command for the host fast-path module (compiled and linked at once)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{d}" for d in cpp_extension.include_paths()] + [f"-I{sysconfig.get_paths()['include']}",
                                                               f"-I{os.path.join(REPO, 'include')}"]
    libdirs = cpp_extension.library_paths()
    libs = [f"-L{d}" for d in libdirs] + [f"-Wl,-rpath,{d}" for d in libdirs]
    out = pyhost_path() + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *inc, PYHOST_SRC, "-o", out, *libs,
           "-ltorch_python", "-ltorch", "-lc10"]
    return cmd, out


def _sources_of(obj: str) -> list:
    """The source files an output is built from (headers included)."""
    inc = [os.path.join(REPO, "include", "rfadam8.h")]
    dev = [os.path.join(CSRC, "rf_device.h"), os.path.join(CSRC, "rf_tables.h")]
    if obj.endswith("rf_host.o"):
        return [HOST_SRC, *dev, *inc]
    if obj.endswith(".o"):
        return [INST_SRC, *dev, *inc]
    return [PYHOST_SRC, *inc, __file__]


def _stale(obj: str) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(src) > t for src in _sources_of(obj))


def build(verbose: bool = False, jobs: int | None = None, incremental: bool = False) -> str:
    """Compile the HIP library (objects in parallel, then link); returns
    the path of the built ``.so``.  ``incremental``: recompile only the
    objects older than their sources."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    max_par = jobs or min(len(VARIANTS) + 1, max(1, os.cpu_count() or 1))
    pending = [_pyhost_job()] + _compile_jobs()
    if incremental:
        pending = [(cmd, obj) for cmd, obj in pending
                   if _stale(pyhost_path() if obj.endswith(".tmp") else obj)]
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
        raise RuntimeError(f"compilation failed for {len(failures)} object(s)")
    if os.path.exists(pyhost_path() + ".tmp"):
        os.replace(pyhost_path() + ".tmp", pyhost_path())
    tmp = LIB_PATH + ".tmp"
    objs = [obj for _, obj in _compile_jobs()]
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{SONAME}", "-o", tmp, *objs]
    if verbose:
        print(" ".join(link), flush=True)
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"link failed with exit code {proc.returncode}")
    os.replace(tmp, LIB_PATH)
    # programs linked with -lrfadam8 ask the loader for the soname
    link_name = os.path.join(OUT_DIR, SONAME)
    if os.path.lexists(link_name):
        os.remove(link_name)
    os.symlink(LIB_NAME, link_name)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True, incremental="--incremental" in sys.argv))
