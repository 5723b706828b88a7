"""flydsl_amd -- MI355X (gfx950) quantized preshuffle GEMM.

Drop-in launchers (``flydsl_amd.kernels.preshuffle_gemm``,
``flydsl_amd.kernels.blockscale_preshuffle_gemm``) over hand-written HIP kernels
reached through a C ABI (``include/flygemm.h``, loaded with ctypes).
"""
from .quant import pack_int4, pertoken_quant, shuffle_weight, blockscale_quant  # noqa: F401


class CompiledFunction:
    """Fast callable returned by :func:`compile`: positional arguments only, in the launcher's
    order; each call reads the tensors' data pointers, M, N and the stream and calls the C
    entry point directly (reference ``python/flydsl/compiler/jit_function.py:895-915``)."""

    __slots__ = ("_call", "_launcher")

    def __init__(self, call, launcher):
        self._call = call
        self._launcher = launcher

    def __call__(self, *args):
        return self._call(*args)


def compile(launch_fn, *args):
    """The reference's ``flyc.compile(fn, *args)`` (``python/flydsl/compiler/jit_function.py:
    917-954``): run ``launch_fn(*args)`` once -- with every argument check -- and return a
    :class:`CompiledFunction` that repeats the launch for new tensors, M, N and stream with only
    a capacity check of each tensor (no dtype, device or layout checks).  The kernels are built
    ahead of time, so nothing is compiled here; launchers of this package are pre-bound to their
    C entry point, any other callable is returned as it is after the first call."""
    launch_fn(*args)
    bind = getattr(launch_fn, "_bind", None)
    if bind is None:
        return launch_fn
    return CompiledFunction(bind(), launch_fn)


__version__ = "0.1.0"
