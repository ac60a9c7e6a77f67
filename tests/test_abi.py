"""The C-ABI library loads and exports every symbol ``include/*.h`` declares; host-side argument
checks fail before any GPU call. No compute is launched here."""

from __future__ import annotations

import ctypes
import glob
import os
import re
import subprocess

import pytest

from tests.conftest import ROOT

HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))
DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(rt_\w+)\s*\(", re.M)


def declared() -> set[str]:
    names: set[str] = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(DECL.findall(text))
    return names


def test_headers_declare_entry_points():
    assert HEADERS and "rt_int8_scan_topk" in declared()


def test_library_exports_every_declared_symbol():
    from retrieve_amd import _native

    assert os.path.exists(_native.LIB_PATH), "build first: make -C retrieve_amd/csrc"
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = declared() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_ctypes_table_covers_the_header():
    import torch  # noqa: F401  (the library binds to torch's HIP runtime)

    from retrieve_amd import _native

    assert set(_native.SIGNATURES) == declared()
    lib = _native.lib()
    for name in declared():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_argument_errors_need_no_gpu():
    import torch  # noqa: F401

    from retrieve_amd import _native

    lib = _native.lib()
    # k = 0 is rejected before any HIP call
    st = lib.rt_int8_scan_topk(None, 1, None, 10, 64, 0, None, 0, None, None, None, 0, None)
    assert st == 1
    assert b"k must be" in lib.rt_last_error()
    with pytest.raises(ValueError, match="k must be"):
        _native.check(st)


def test_workspace_grows_with_batch():
    import torch  # noqa: F401

    from retrieve_amd import _native

    lib = _native.lib()
    small = lib.rt_int8_scan_topk_workspace(1, 30_000_000, 512, 100)
    big = lib.rt_int8_scan_topk_workspace(1024, 30_000_000, 512, 100)
    assert 0 < small <= big


def test_no_alloc_rejections_need_no_gpu():
    """The allocation-free int8 scan rejects null pointers before any device call. (Its
    rejection of a plan above the fixed scratch is tested with real device buffers, on the GPU,
    in ``tests/test_zz_no_alloc.py``: no call here passes an address that is not a buffer.)"""
    import torch  # noqa: F401

    from retrieve_amd import _native

    lib = _native.lib()
    st = lib.rt_int8_scan_topk_noalloc(None, 2, None, 10, 64, 5, None, 0, None, None, None)
    assert st == 1 and b"must not be null" in lib.rt_last_error()
    st = lib.rt_int8_scan_topk(None, 2, None, 10, 64, 5, None, 0, None, None, None, 0, None)
    assert st == 1 and b"null" in lib.rt_last_error()
