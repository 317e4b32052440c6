"""CPU checks of the C ABI: the library loads (no GPU needed to dlopen) and
exports every function include/klearu_hip.h declares; the Python binding
covers each of them."""
import ctypes
import os

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
