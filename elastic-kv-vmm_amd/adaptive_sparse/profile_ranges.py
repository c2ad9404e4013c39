"""Opt-in profiler ranges around the host entry points of the sparse-KV path.

The reference's diagnostic switch (adaptive_sparse/profile_ranges.py:7-45):
with EKV_PROFILE_RANGES=1 in the environment when a module is imported, each
call decorated with profile_range(name) runs inside a torch profiler range
named "ekv/<name>" and a roctx range of the same name (torch.cuda.nvtx is
roctx on ROCm, so `rocprofv3 --marker-trace` shows it beside the kernels it
launched). Without the switch the decorator hands back the function itself
and imports nothing, so a timed run pays nothing; bench.py removes the switch
unless it is asked for ranges.
"""

from functools import wraps
import os

SWITCH = "EKV_PROFILE_RANGES"


def enabled():
    """Whether diagnostic ranges are on for modules imported from now on."""
    return os.environ.get(SWITCH) == "1"


def _unchanged(function):
    return function


def _marker():
    """torch.cuda.nvtx (roctx on ROCm) when this torch build has it, else None."""
    try:
        import torch
    except ImportError:
        return None
    nvtx = getattr(torch.cuda, "nvtx", None)
    return nvtx if nvtx is not None and hasattr(nvtx, "range_push") else None


def profile_range(name):
    """Decorator: run the callable inside the "ekv/<name>" ranges when the switch is on."""
    if not enabled():
        return _unchanged

    from torch.profiler import record_function

    label = f"ekv/{name}"
    marker = [_marker()]   # dropped after a marker call fails (a torch build without a marker library)

    def push():
        if marker[0] is None:
            return False
        try:
            marker[0].range_push(label)
            return True
        except RuntimeError:
            marker[0] = None
            return False

    def decorate(function):
        @wraps(function)
        def measured(*args, **kwargs):
            with record_function(label):
                if not push():
                    return function(*args, **kwargs)
                try:
                    return function(*args, **kwargs)
                finally:
                    marker[0].range_pop()

        return measured

    return decorate


# The serving engine's coordinator methods that end in this library's native
# calls (the reference marks the same two: profile_ranges.py:28-45).
_COORDINATOR_MODULE = "sglang.srt.managers.hisparse_coordinator"
_COORDINATOR_METHODS = (("map_last_loc_to_buffer", "native/map_latest"),
                        ("swap_in_selected_blocks", "native/swap"))


def install_native_profile_ranges():
    """Wrap the engine coordinator's native-backed methods once, when the switch is on.

    Imports the coordinator only with the switch on (a diagnostic worker runs
    inside the engine, where it is importable); calling it again is a no-op.
    """
    if not enabled():
        return
    import importlib

    cls = importlib.import_module(_COORDINATOR_MODULE).HiSparseCoordinator
    if getattr(cls, "_ekv_native_profile_ranges", False):
        return
    for method, name in _COORDINATOR_METHODS:
        setattr(cls, method, profile_range(name)(getattr(cls, method)))
    cls._ekv_native_profile_ranges = True
