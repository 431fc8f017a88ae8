"""C-ABI checks that need no GPU: the library loads, exports what include/*.h declares, and rejects
bad arguments before launching anything."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

from conftest import REPO


def _declared_functions():
    names = []
    for hdr in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(hdr).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*;", text, re.M):
            names.append(m.group(1))
    return names


def test_header_declares_reference_symbol():
    names = _declared_functions()
    assert "h4mv_launch" in names and "h4mv_launch_status" in names


def test_library_exports_every_declared_symbol(lib):
    from fp8kv_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.lib_path()], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in _declared_functions():
        assert name in exported, name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        getattr(lib, name)


def test_status_strings(lib):
    assert lib.fp8kv_status_string(0) == b"ok"
    assert lib.fp8kv_status_string(5).startswith(b"scratch")
    assert lib.fp8kv_status_string(99) == b"unknown status"


# Pointer values below are never dereferenced: every call is rejected before any launch.
A = 0x10000


@pytest.mark.parametrize("args,code", [
    ((0, A, A, A, 64, 64, 1), 1),          # null W
    ((A, A, A, A, 0, 64, 1), 1),           # N = 0
    ((A, A, A, A, 64, 64, 0), 1),          # M = 0
    ((A, A, A, A, 64, 64, 17), 2),         # M > 16
    ((A, A, A, A, 64, 48, 1), 2),          # K % 32 != 0
    ((A + 1, A, A, A, 64, 64, 1), 3),      # W not 16-byte aligned
    ((A, A, A + 8, A, 64, 64, 1), 3),      # X not 16-byte aligned
])
def test_h4mv_rejects_before_launch(lib, args, code):
    assert lib.h4mv_launch_status(*args, None) == code
    lib.h4mv_launch(*args, None)
    assert lib.fp8kv_last_status() == code


def test_loader_fails_loudly_without_library(monkeypatch, tmp_path):
    from fp8kv_amd import _lib
    monkeypatch.setenv("FP8KV_AMD_LIB", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(FileNotFoundError):
        _lib.load()
