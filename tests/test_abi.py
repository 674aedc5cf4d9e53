"""C-ABI checks that need no GPU: the library loads, every prototype in
include/drawinstant.h is exported, and argument validation that precedes any
device use fails loudly with a message (reference fail-loud convention,
wgsl-executor.js:1344-1348)."""
import ctypes
import glob
import os
import re

import pytest

from conftest import REPO


def _declared():
    names = set()
    for h in glob.glob(os.path.join(REPO, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
        names |= set(re.findall(r"\b(di_\w+)\s*\(", src))
    return names


def test_header_declares_entry_points():
    names = _declared()
    for must in ("di_create", "di_destroy", "di_alloc", "di_upload", "di_download", "di_sync",
                 "di_group_norm", "di_gn_silu", "di_layer_norm"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from drawinstant import _lib
    lib = ctypes.CDLL(_lib.LIBRARY)
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    from drawinstant import _lib
    protos = _lib.parse_header()
    assert set(protos) == _declared()
    lib = _lib.load()
    for name in protos:
        assert getattr(lib, name).restype is not None or name == "di_last_error"


def test_null_context_is_rejected():
    import drawinstant
    from drawinstant import DiError, call
    with pytest.raises(DiError) as e:
        call("di_sync", None)
    assert e.value.code == 1 and "null context" in str(e.value)
    with pytest.raises(DiError):
        call("di_alloc", None, 16, None)


def test_create_rejects_null_out_pointer():
    from drawinstant import DiError, call
    with pytest.raises(DiError) as e:
        call("di_create", 0, None)
    assert "null out pointer" in str(e.value)


def test_create_without_gpu_fails_loudly():
    from drawinstant import DiError, Device
    try:
        import torch
        has_gpu = torch.cuda.device_count() > 0
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    with pytest.raises(DiError) as e:
        Device(0)
    assert e.value.code == 3 and "no HIP device" in str(e.value)


def _deno_table():
    """{name: parameter count} of the Deno.dlopen table in INTEGRATION.md."""
    src = open(os.path.join(REPO, "INTEGRATION.md")).read()
    block = src[src.index("Deno.dlopen("):]
    block = block[:block.index("\n})")]
    return {m.group(1): len([p for p in m.group(2).split(",") if p.strip()])
            for m in re.finditer(r"^\s*(di_\w+):\s*\{\s*parameters:\s*\[([^\]]*)\]", block, re.M)}


def test_deno_table_matches_exports():
    """The maintainer's FFI table names every exported entry point, and each
    with the header prototype's parameter count."""
    import subprocess
    from drawinstant import _lib
    table = _deno_table()
    protos = _lib.parse_header()
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIBRARY], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if ln.split()[-1].startswith("di_")}
    assert set(table) == exported == set(protos)
    wrong = {n: (table[n], len(protos[n][1])) for n in table if table[n] != len(protos[n][1])}
    assert not wrong, f"parameter counts differ (table, header): {wrong}"
