"""klearu_amd -- MI355X (gfx950) implementation of klearu's activation-sparse
inference path (SLIDE LSH layers, Deja Vu predictors / sparse FFN / head-sparse
attention, klearu-accel kernels) behind a C ABI (include/klearu_hip.h).

The compute lives in libklearu_hip.so (hand-written HIP kernels); this package
is a thin host mirror of the reference's Rust interfaces for tests and
benchmarks.  There is no CPU fallback: without the built library or a GPU,
calls raise.
"""
from ._lib import KlearuError, header_functions, load  # noqa: F401
from ._dev import require_gpu  # noqa: F401

__all__ = ["KlearuError", "header_functions", "load", "require_gpu"]
