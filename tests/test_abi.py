"""CPU checks of the C ABI: the library loads (no GPU needed to dlopen) and
exports every function include/klearu_hip.h declares; the Python binding
covers each of them."""
import ctypes
import os
import re

import pytest

from klearu_amd import _lib


def test_header_symbols_exported():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libklearu_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _lib.header_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    names = set(_lib.header_functions())
    assert names == set(_lib.SIGS), (names ^ set(_lib.SIGS))


def _header_declarations():
    """{name: [parameter type, ...]} of every function include/klearu_hip.h declares."""
    txt = open(os.path.join(os.path.dirname(_lib.LIB_PATH), "..", "include", "klearu_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    txt = re.sub(r"//[^\n]*", "", txt)
    out = {}
    for m in re.finditer(r"\b(kh_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", txt):
        params = m.group(2).strip()
        ps = [] if params in ("", "void") else [p.strip() for p in params.split(",")]
        # drop the parameter name, keep its type
        out[m.group(1)] = [re.sub(r"\b[A-Za-z_][A-Za-z0-9_]*$", "", p).strip() for p in ps]
    return out


def _c_kind(t):
    t = " ".join(t.replace("*", " * ").split())
    if t.count("*") >= 2:
        return "pp"
    if t.count("*") == 1:
        return "char*" if re.search(r"\bchar\b", t) else "p"
    if re.search(r"\b(int64_t|uint64_t|size_t)\b", t):
        return "i64"
    if re.search(r"\b(int|int32_t|uint32_t|unsigned)\b", t):
        return "i32"
    return {"float": "f32", "double": "f64"}.get(t.replace("const ", ""), "other " + t)


def _ctypes_kind(c):
    if c is ctypes.c_char_p:
        return "char*"
    if c is ctypes.c_void_p:
        return "p"
    if isinstance(c, type) and issubclass(c, ctypes._Pointer):
        return "pp" if c._type_ is ctypes.c_void_p else "p"
    for kind, group in (("i32", (ctypes.c_int, ctypes.c_uint, ctypes.c_int32, ctypes.c_uint32)),
                        ("i64", (ctypes.c_int64, ctypes.c_uint64)),
                        ("f32", (ctypes.c_float,)), ("f64", (ctypes.c_double,))):
        if c in group:
            return kind
    return f"other {c!r}"


def test_binding_signatures_match_header():
    """Every binding passes as many arguments as its C declaration takes, each of
    the declared kind (pointer, pointer to pointer, 32- or 64-bit integer, float,
    double, string): a stale ctypes signature would otherwise truncate or
    misplace arguments only at call time on the GPU box."""
    decls = _header_declarations()
    assert set(decls) == set(_lib.SIGS)
    bad = []
    for name, params in sorted(decls.items()):
        want = [_c_kind(p) for p in params]
        got = [_ctypes_kind(a) for a in _lib.SIGS[name][1]]
        ok = len(want) == len(got) and all(w == g or (w == "char*" and g == "p") for w, g in zip(want, got))
        if not ok:
            bad.append((name, want, got))
    assert not bad, bad


def test_error_reporting_without_gpu():
    lib = _lib.load()
    # argument validation happens before any device call
    rc = lib.kh_sparse_ffn_forward(None, None, 1, None, 0, None, None, 0, None)
    assert rc == _lib.KH_ERR_ARG
    assert b"null" in lib.kh_last_error()
    assert lib.kh_version() >= 1


@pytest.mark.parametrize("base,decay,steps", [(10, 0.0, 40), (5, 0.0, 31), (10, 0.5, 400), (1, 0.0, 5),
                                              (5, 2.0, 3000), (3, -1.0, 40), (7, 0.25, 1000)])
def test_rebuild_scheduler_host_matches_oracle(base, decay, steps):
    """RebuildScheduler is host logic (no GPU): the C entry points against the
    oracle's scheduler, which the reference's own tests pin."""
    import oracle
    from klearu_amd.slide import RebuildScheduler
    s, o = RebuildScheduler(base, decay), oracle.RebuildScheduler(base, decay)
    for i in range(steps):
        assert s.step() == o.step(), i
        assert (s.rebuild_count, s.next_rebuild_step, s.current_step) == (
            o.rebuild_count, o.next_rebuild_step, o.current_step)
    for jump in (steps + 3, steps + 1000, 2 ** 40):
        assert s.should_rebuild(jump) == o.should_rebuild(jump)
        assert (s.rebuild_count, s.next_rebuild_step) == (o.rebuild_count, o.next_rebuild_step)
