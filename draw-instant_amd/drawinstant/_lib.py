"""ctypes binding of libdrawinstant_hip.so.

Signatures are read from the C header (``include/drawinstant.h``), the single
source of truth for the ABI, so every declared entry point is bound and a
missing export fails at load time.  There is no fallback: if the HIP library
is not built, importing the binding raises.
"""
from __future__ import annotations

import ctypes
import os
import re

_PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.abspath(os.path.join(_PKG, "..", ".."))
HEADER = os.path.join(REPO, "include", "drawinstant.h")
LIBRARY = os.path.join(_PKG, "libdrawinstant_hip.so")

_SCALARS = {
    "int32_t": ctypes.c_int32,
    "uint32_t": ctypes.c_uint32,
    "int64_t": ctypes.c_int64,
    "uint64_t": ctypes.c_uint64,
    "float": ctypes.c_float,
    "double": ctypes.c_double,
    "di_handle": ctypes.c_uint64,
}


class LibraryMissing(ImportError):
    pass


def _ctype(decl: str):
    """Map one C parameter / return type (without the name) to ctypes."""
    t = " ".join(decl.replace("*", " * ").split())
    stars = t.count("*")
    base = t.replace("*", "").replace("const", "").strip()
    if base == "void" and stars == 0:
        return None
    if base == "char" and stars == 1:
        return ctypes.c_char_p
    if base == "di_ctx":
        return ctypes.c_void_p if stars == 1 else ctypes.POINTER(ctypes.c_void_p)
    if base in _SCALARS:
        ct = _SCALARS[base]
        for _ in range(stars):
            ct = ctypes.POINTER(ct)
        return ct
    # void* and struct pointers travel as raw addresses
    if stars >= 1:
        return ctypes.c_void_p
    raise TypeError(f"unmapped C type {decl!r}")


def parse_header(path: str = HEADER):
    """Return {name: (restype, [argtypes], [param decls])} for every di_* prototype."""
    with open(path) as f:
        src = f.read()
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    src = re.sub(r"//[^\n]*", " ", src)
    src = re.sub(r"#[^\n]*", " ", src)
    protos = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(di_\w+)\s*\(([^)]*)\)\s*;", src):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        decls = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        argtypes = []
        for d in decls:
            pm = re.match(r"(.*?)(\w+)$", d.strip())
            argtypes.append(_ctype(pm.group(1)))
        protos[name] = (_ctype(ret.strip()), argtypes, decls)
    return protos


_lib = None


def load():
    """Load and bind the library (once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise LibraryMissing(
            f"{LIBRARY} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    lib = ctypes.CDLL(LIBRARY, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args, _) in parse_header().items():
        fn = getattr(lib, name)  # AttributeError = declared but not exported
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
