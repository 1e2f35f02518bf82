"""CPU checks of the C-ABI boundary: libhipbackend.so loads, exports every
entry point include/laya_hip.h declares, and the ctypes table binds exactly
that set.  No GPU call is made."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "laya_hip.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"^\s*(?:const\s+char\s*\*|int)\s+(hb_\w+)\s*\(", src, flags=re.M))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ("hb_init", "hb_linear", "hb_qlinear", "hb_layernorm", "hb_rope", "hb_sdpa", "hb_geglu", "hb_upload",
              "hb_download", "hb_last_error"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from laya_hip.lib import resolve_lib
    lib = ctypes.CDLL(resolve_lib())
    missing = [s for s in sorted(declared_symbols()) if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"


def test_ffi_table_matches_header():
    from laya_hip import ffi
    assert set(ffi.SYMBOLS) == declared_symbols()


def test_abi_version_and_error_path_without_gpu():
    """A failed call returns -1 with a message and never aborts (the
    reference's FFI rule, packages/backend-mlx/src/ffi.ts:15-16)."""
    from laya_hip import ffi
    n = ffi.native()
    assert n.lib.hb_abi_version() == 1
    assert n.lib.hb_sync(0) == -1
    assert "null context" in n.last_error()
    with pytest.raises(ffi.HipError, match="flush: null context"):
        n.call("flush", "hb_sync", 0)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from laya_hip import lib
    monkeypatch.setenv(lib.ENV_VAR, str(tmp_path / "nowhere.so"))
    monkeypatch.setattr(lib.os.path, "dirname", lambda p: str(tmp_path))
    with pytest.raises(lib.HipLibraryNotFound):
        lib.resolve_lib()
