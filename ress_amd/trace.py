"""Stage ranges for the profiler: each stage of a layer's sparse attention (operand prep, pooled
map, budget, block selection, attention) runs inside a named roctx range, which
`rocprofv3 --marker-trace` records beside the kernels the stage launched. The reference has no
profiler hooks (its diagnostics are the drift recorders, src/ress/scoring/projected.py:41-128);
the ranges are this build's equivalent for a GPU timeline.

Off by default, so a layer step pays one flag test per stage. Set RESS_ROCTX=1 in the
environment, or call enable(), to turn them on; the ranges then need ROCm's roctx library
(librocprofiler-sdk-roctx, or the older libroctx64), and enable() raises if neither loads.
Ranges are host-side markers: they bracket the launches, not the kernels' execution."""

import ctypes
import os

_LIBS = ("librocprofiler-sdk-roctx.so.1", "libroctx64.so.4")
_roctx = None
_on = False


def _load():
    root = os.environ.get("ROCM_PATH", "/opt/rocm")
    errors = []
    for name in _LIBS:
        for path in (os.path.join(root, "lib", name), name):
            try:
                lib = ctypes.CDLL(path)
            except OSError as e:
                errors.append(str(e))
                continue
            lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
            lib.roctxRangePushA.restype = ctypes.c_int
            lib.roctxRangePop.argtypes = []
            lib.roctxRangePop.restype = ctypes.c_int
            return lib
    raise RuntimeError("ress_amd.trace: no roctx library could be loaded (%s)" % "; ".join(errors))


def enable(on=True, lib=None):
    """Turn the stage ranges on or off. `lib` replaces the roctx library (an object with
    roctxRangePushA(bytes) and roctxRangePop()), for tests."""
    global _roctx, _on
    if on and lib is not None:
        _roctx = lib
    elif on and _roctx is None:
        _roctx = _load()
    _on = bool(on)


def enabled():
    return _on


class stage:
    """`with stage("ress.select"): ...` -- one named range around the block, when enabled."""

    __slots__ = ("name", "pushed")

    def __init__(self, name):
        self.name = name
        self.pushed = False

    def __enter__(self):
        if _on:
            _roctx.roctxRangePushA(self.name.encode())
            self.pushed = True
        return self

    def __exit__(self, *exc):
        if self.pushed:
            _roctx.roctxRangePop()
        return False


if os.environ.get("RESS_ROCTX", "") not in ("", "0"):
    enable()
