"""The C-ABI library loads (no GPU needed) and exports every declared symbol."""
import ctypes
import os
import re

from wnw_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = []
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(wnw_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_functions():
    names = _declared_functions()
    assert "wnw_decode_attn" in names and "wnw_interleave_append" in names and "wnw_rebuild_append_kv" in names


def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared_functions() if not hasattr(handle, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_every_symbol():
    declared = set(_declared_functions())
    bound = set(_lib.exported_symbols())
    assert declared <= bound, f"unbound: {sorted(declared - bound)}"
    _lib.lib()  # argtypes install without error


def test_host_only_queries_work_without_gpu():
    l = _lib.lib()
    assert l.wnw_abi_version() >= 1
    ws = l.wnw_decode_attn_workspace_bytes(64, 4, 128)
    assert ws > 0 and ws % 256 == 0
    assert l.wnw_decode_attn_workspace_bytes(64, 0, 128) == -1
