"""CPU checks of the C ABI: the library loads and exports every function that
include/hn_int4.h declares, and the ctypes table covers exactly that set.
No kernel is launched."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = []
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            names += re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(hn_\w+)\s*\(", src, re.M)
    return sorted(set(names))


def test_header_declares_entry_points():
    names = _declared()
    assert "hn_int4_linear" in names and "hn_expert_mlp_int4" in names
    assert len(names) >= 14


def test_library_exports_every_declared_symbol():
    from hydranet_amd import _lib
    h = _lib.lib()
    for name in _declared():
        assert hasattr(h, name), name
    assert h.hn_abi_version() == 1


def test_ctypes_table_matches_header():
    from hydranet_amd import _lib
    declared = set(_declared()) - {"hn_last_error_string", "hn_abi_version"}
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def _declared_params():
    """name -> parameter kinds ('P' pointer, 'L' long, 'I' int, 'F' float) of
    every function include/*.h declares."""
    out = {}
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if not fn.endswith(".h"):
            continue
        src = re.sub(r"/\*.*?\*/", " ", open(os.path.join(ROOT, "include", fn)).read(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?\w+\*?\s+\*?(hn_\w+)\s*\(([^)]*)\)\s*;", src,
                             re.M):
            params = " ".join(m.group(2).split())
            kinds = []
            if params and params != "void":
                for prm in params.split(","):
                    t = prm.strip()
                    if "*" in t:
                        kinds.append("P")
                    elif re.match(r"(const\s+)?long\b", t):
                        kinds.append("L")
                    elif re.match(r"(const\s+)?int\b", t):
                        kinds.append("I")
                    elif re.match(r"(const\s+)?float\b", t):
                        kinds.append("F")
                    else:
                        kinds.append("?" + t)
            out[m.group(1)] = kinds
    return out


def test_ctypes_argument_kinds_match_header():
    """Every ctypes signature has the header's parameter count and kinds, so a
    changed declaration cannot silently shift the arguments of a call."""
    from hydranet_amd import _lib
    code = {_lib.P: "P", _lib.L: "L", _lib.I: "I", _lib.F: "F"}
    decl = _declared_params()
    assert set(_lib.SIGNATURES) <= set(decl)
    for name, sig in _lib.SIGNATURES.items():
        assert [code[t] for t in sig] == decl[name], name


def test_workspace_query():
    from hydranet_amd import _lib
    h = _lib.lib()
    ctr = 2 << 20  # fixed counter region at the start of every workspace
    # one token: every tile reduces K inside a workgroup -> counters only
    assert h.hn_skinny_workspace_bytes(2, 1, 4096, 14336, 0) == ctr
    assert h.hn_skinny_workspace_bytes(0, 1, 64, 256, 0) == ctr
    # 64 tokens x K=14336 do not fit one workgroup's LDS -> fp32 partials
    b = h.hn_skinny_workspace_bytes(0, 64, 4096, 14336, 0)
    assert b >= ctr + 2 * 64 * 4096 * 4
    # the grouped query at decode sizes covers E x tiles counters + partials
    assert h.hn_skinny_workspace_bytes(3, 32, 4096, 14336, 8) >= ctr


def test_argument_errors_raise_without_gpu():
    # rejected arguments return before any HIP call
    from hydranet_amd import _lib
    import pytest
    with pytest.raises(RuntimeError, match="multiple of 32"):
        _lib.call("hn_int4_linear", None, 8, None, 16, None, 1, None, 8, 1, 1, 48, 16, None, 0,
                  None)
    with pytest.raises(RuntimeError, match="mode must be"):
        _lib.call("hn_router_topk", None, None, 1, 8, 2, 5, ctypes.c_float(0), ctypes.c_float(1),
                  None, None, None)
    with pytest.raises(RuntimeError, match="E <= 256"):
        _lib.call("hn_router_topk", None, None, 1, 257, 2, 1, ctypes.c_float(0),
                  ctypes.c_float(1), None, None, None)
    with pytest.raises(RuntimeError, match="negative dims"):
        _lib.call("hn_silu_then_mul", None, 8, None, 8, None, 8, -1, 8, None)
    # empty products return before any HIP call
    _lib.call("hn_silu_then_mul", None, 8, None, 8, None, 8, 0, 8, None)
    _lib.call("hn_silu_mul", None, 8, None, 8, None, 8, 4, 0, None)
    with pytest.raises(RuntimeError, match="decode sizes"):
        _lib.call("hn_moe_route", None, 4096, None, 4096, 0, None, None, 2048, 8, 4096, 2, 0,
                  ctypes.c_float(0), ctypes.c_float(1), None, None, None, None, None, None, None,
                  None, None, None, 4096, None)


def test_growing_a_workspace_keeps_the_old_buffer_allocated():
    # a captured graph holds the raw pointer of the workspace it was captured
    # with: growing must not hand the old buffer back to the allocator
    from hydranet_amd import _lib
    a = _lib.workspace(1000, "cpu")
    pa = a.data_ptr()
    b = _lib.workspace(1 << 20, "cpu")
    assert b.data_ptr() != pa and b.numel() >= 1 << 20
    assert any(t.data_ptr() == pa for t in _lib._RETIRED[("cpu", 0)])
    assert _lib.workspace(10, "cpu") is b  # smaller requests reuse the current one
