"""CPU checks of the C-ABI boundary: libhipbackend.so loads, exports every
entry point include/laya_hip.h declares, and the ctypes table binds exactly
that set, with the header's parameter and return types.  No GPU call is made."""
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


# C parameter / return types of the header -> the ctypes type that passes them
# (LP64: uintptr_t, uint64_t and size_t are unsigned long, int64_t is long)
_CTYPE = {
    "int": ctypes.c_int, "unsigned": ctypes.c_uint, "int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t,
    "uintptr_t": ctypes.c_uint64, "float": ctypes.c_float, "double": ctypes.c_double,
    "void *": ctypes.c_void_p, "const void *": ctypes.c_void_p, "char *": ctypes.c_char_p,
    "const char *": ctypes.c_char_p, "const int64_t *": ctypes.POINTER(ctypes.c_int64),
    "float *": ctypes.POINTER(ctypes.c_float), "size_t *": ctypes.POINTER(ctypes.c_size_t),
    "uint64_t *": ctypes.POINTER(ctypes.c_uint64), "uintptr_t *": ctypes.POINTER(ctypes.c_uint64),
}


def _norm(t):
    return re.sub(r"\s+", " ", t.replace("*", " * ")).strip()


def declared_signatures():
    """name -> (return type, [parameter types]) as written in the header."""
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    out = {}
    for rt, name, params in re.findall(r"^\s*(const\s+char\s*\*|int)\s+(hb_\w+)\s*\(([^)]*)\)\s*;", src,
                                       flags=re.M | re.S):
        ps = [p.strip() for p in params.split(",") if p.strip() and p.strip() != "void"]
        out[name] = (_norm(rt), [_norm(re.sub(r"\b\w+\s*$", "", p)) for p in ps])
    return out


def signature_mismatches(table):
    bad = []
    for name, (rt, ps) in declared_signatures().items():
        res, args = table[name]
        if _CTYPE[rt] is not res:
            bad.append(f"{name}: returns {rt}, bound as {res.__name__}")
        if len(ps) != len(args):
            bad.append(f"{name}: {len(ps)} parameters, bound with {len(args)}")
            continue
        for i, (p, a) in enumerate(zip(ps, args)):
            if _CTYPE[p] is not a:
                bad.append(f"{name}: parameter {i} is {p}, bound as {a.__name__}")
    return bad


def test_ffi_argument_types_match_header():
    """Each entry point's ctypes binding passes exactly the header's
    parameter types (count, width, signedness, pointee), so no argument is
    truncated or misplaced at the boundary.  A table with one parameter
    narrowed from int64_t to int is caught."""
    from laya_hip import ffi
    sigs = declared_signatures()
    assert len(sigs) == len(declared_symbols())
    assert signature_mismatches(ffi.SYMBOLS) == []
    planted = dict(ffi.SYMBOLS)
    res, args = planted["hb_linear"]
    planted["hb_linear"] = (res, args[:3] + [ctypes.c_int] + args[4:])  # ldx narrowed
    assert signature_mismatches(planted) == ["hb_linear: parameter 3 is int64_t, bound as c_int"]


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
