"""The C-ABI library loads and exports every symbol include/*.h declares (no
compute calls: this runs without a GPU)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(zs_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


@pytest.fixture(scope="module")
def libzs():
    path = os.path.join(ROOT, "zllm_amd", "libzs.so")
    if not os.path.exists(path):
        from zllm_amd import build
        build.build()
    return ctypes.CDLL(path)


def test_header_declares_entry_points():
    names = _declared()
    for n in ("zs_abi_version", "zs_ctx_create", "zs_sample", "zs_dfa_mask", "zs_vocab_create"):
        assert n in names


def test_library_exports_every_declared_symbol(libzs):
    missing = [n for n in _declared() if not hasattr(libzs, n)]
    assert not missing, missing


def test_abi_version(libzs):
    libzs.zs_abi_version.restype = ctypes.c_int
    assert libzs.zs_abi_version() == 2


def test_struct_layouts_match_binding(libzs):
    """sizeof and every field offset of the ABI structs, as compiled into the
    library, equal the ctypes binding's (the Rust binding in INTEGRATION.md
    mirrors the same field lists)."""
    from zllm_amd import _lib
    fn = libzs.zs_struct_layout
    fn.restype = ctypes.c_int
    fn.argtypes = _lib.SIGNATURES["zs_struct_layout"][1]
    assert _lib.layout_mismatches(libzs) == []
    # the batch ends with the pass_event pointer that ABI 2 added
    size = ctypes.c_size_t()
    offs = (ctypes.c_size_t * 64)()
    n = fn(0, ctypes.byref(size), offs, 64)
    assert n == len(_lib.Batch._fields_) and _lib.Batch._fields_[-1][0] == "pass_event"
    assert offs[n - 1] + 8 == size.value
    assert fn(99, ctypes.byref(size), offs, 64) == -1


def test_python_binding_covers_header():
    from zllm_amd._lib import SIGNATURES
    assert set(_declared()) <= set(SIGNATURES), set(_declared()) - set(SIGNATURES)
