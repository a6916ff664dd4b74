"""The C-ABI library (no GPU): it loads, exports every entry point that
include/rfadam8.h declares, its structs have the sizes the header fixes,
and host-only entry points validate arguments and report errors the way the
header documents."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest

from oracle import oracle as orc
from rollfast_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rfadam8.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:RF_API\s+)?(?:const\s+)?[a-z_0-9]+\s*\*?\s*(rf_[a-z_0-9]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    assert len(names) >= 14
    assert set(names) == set(_lib.EXPORTS), set(names) ^ set(_lib.EXPORTS)


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.lib()
    for name in _declared_functions():
        assert hasattr(L, name), name
    # nothing else with the rf_ prefix is part of the ABI contract
    assert os.path.basename(L._name) == "librfadam8.so"


def test_dynamic_symbols_are_exactly_the_declared_entry_points():
    """The library exports the C ABI and nothing else (hidden visibility)."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    path = _lib.lib()._name
    out = subprocess.run([nm, "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.split()[1:2] == ["T"]}
    assert exported == set(_declared_functions()), exported ^ set(_declared_functions())


def test_struct_sizes_match_header():
    assert ctypes.sizeof(_lib.Adam8Leaf) == 120
    assert ctypes.sizeof(_lib.Adam8Hparams) == 128
    assert ctypes.sizeof(_lib.Adam8Group) == 32
    assert ctypes.sizeof(_lib.ApplyLeaf) == 40
    assert ctypes.sizeof(_lib.MagmaLeaf) == 48


def test_header_compiles_as_c_with_the_same_struct_sizes(tmp_path):
    """A C host (cgo, JNI or N-API glue) includes the header as C99; the
    struct sizes it sees are the ones the library and the binding use."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "h.c"
    src.write_text(
        '#include "rfadam8.h"\n'
        "typedef char leaf_120[sizeof(rf_adam8_leaf) == 120 ? 1 : -1];\n"
        "typedef char hparams_128[sizeof(rf_adam8_hparams) == 128 ? 1 : -1];\n"
        "typedef char group_32[sizeof(rf_adam8_group) == 32 ? 1 : -1];\n"
        "typedef char apply_40[sizeof(rf_apply_leaf) == 40 ? 1 : -1];\n"
        "typedef char magma_48[sizeof(rf_magma_leaf) == 48 ? 1 : -1];\n"
        "typedef char accum_32[sizeof(rf_accum_leaf) == 32 ? 1 : -1];\n"
        "typedef char clip_%d[sizeof(rf_clip_leaf) == %d ? 1 : -1];\n"
        % (ctypes.sizeof(_lib.ClipLeaf), ctypes.sizeof(_lib.ClipLeaf))
        + "int main(void) { return 0; }\n"
    )
    r = subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", os.path.dirname(HEADER),
                        "-fsyntax-only", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_version_string():
    v = _lib.version()
    assert v.startswith("rfadam8 ")


def test_codebook_entry_point_matches_oracle():
    for signed in (True, False):
        np.testing.assert_array_equal(_lib.codebook(signed).view(np.uint32), orc.codebook(signed).view(np.uint32))


def test_invalid_arguments_are_reported_not_thrown():
    L = _lib.lib()
    out = np.empty(256, np.float32)
    st = L.rf_codebook(7, out.ctypes.data_as(ctypes.c_void_p))
    assert st == 1  # RF_ERR_INVALID
    assert L.rf_last_error().decode()
    with pytest.raises(ValueError):
        _lib.check(st, "rf_codebook")
    st = L.rf_codebook(0, None)
    assert st == 1
    st = L.rf_host_table_codes(0, 0, -1, out.ctypes.data_as(ctypes.c_void_p))
    assert st == 1
    # a null leaf table is rejected before any device work
    st = L.rf_adam8_step(None, 1, 1, None, None)
    assert st == 1


def test_status_mapping():
    with pytest.raises(NotImplementedError):
        _lib.check(3, "x")
    with pytest.raises(RuntimeError):
        _lib.check(2, "x")
    _lib.check(0, "x")
