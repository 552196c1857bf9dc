"""MI355X-native (gfx950) affine group-quantized matmul: qmv (decode), qmm
(prefill) and gather_qmm (routed experts) over MLX-packed 4/8-bit weights.

The compute path is libcpq.so (hand-written HIP kernels behind the C ABI in
include/cpq.h).  This package is a thin Python mirror of the reference's
kernels-crate op API (`cider_press_amd.kernels`) and runtime node
(`cider_press_amd.runtime`) used by the tests and the benchmark.
"""
from . import _lib  # noqa: F401

__all__ = ["kernels", "runtime", "synthetic"]


def __getattr__(name):
    if name in ("kernels", "runtime", "synthetic"):
        import importlib

        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
