"""ctypes binding of the ekv_* kernel entry points of libelastic_vmm.so.

torch tensors are described to the C ABI as (pointer, dtype code, shape,
element strides); nothing but plain values crosses the boundary. The
launch-bound entry points (the lookup, the row gather, the SGLang-convention
swap-in and the one-call decode step) are called through a small compiled
launch helper (launch_helper) that builds the same descriptors in C++. There
is no fallback: if the library or the helper cannot be loaded, every kernel
call raises.
"""

import ctypes as ct
import importlib.util
import os
import struct
import sysconfig
from pathlib import Path

import torch

from ._source_hash import source_hash
from .backing import _load_library, library_path

EKV_ABI_VERSION = 3

_DTYPE_CODES = {
    torch.int32: 1,
    torch.int64: 2,
    torch.uint8: 3,
    torch.int8: 4,
    torch.int16: 5,
    torch.bfloat16: 6,
    torch.float16: 7,
    torch.float32: 8,
}


class EkvTensor(ct.Structure):
    _fields_ = [
        ("data", ct.c_void_p),
        ("dtype", ct.c_int32),
        ("ndim", ct.c_int32),
        ("shape", ct.c_int64 * 4),
        ("stride", ct.c_int64 * 4),
    ]


class EkvPlanes(ct.Structure):
    _fields_ = [
        ("base", ct.c_void_p),
        ("layers", ct.c_int64),
        ("kv", ct.c_int64),
        ("layer_stride", ct.c_int64),
        ("kv_stride", ct.c_int64),
        ("row_stride", ct.c_int64),
        ("row_bytes", ct.c_int64),
        ("rows", ct.c_int64),
    ]


class EkvKvRows(ct.Structure):
    _fields_ = [
        ("data", ct.c_void_p),
        ("layer_stride", ct.c_int64),
        ("batch_stride", ct.c_int64),
        ("kv_stride", ct.c_int64),
        ("lane_stride", ct.c_int64),
    ]


_P_TENSOR = ct.POINTER(EkvTensor)
# The lookup entries take their descriptors as plain pointers, so the wrapper can
# hand over the bytes of packed() (a ctypes.byref(EkvTensor) is accepted as well).
_TENSOR_ADDRESS = ct.c_void_p
_SIGNATURES = {
    "ekv_abi_version": ([], ct.c_int),
    "ekv_source_hash": ([], ct.c_char_p),
    "ekv_resolve_resident": ([_TENSOR_ADDRESS] * 9 + [ct.c_int64, ct.c_void_p], ct.c_int),
    "ekv_resolve_resident_bits": ([_TENSOR_ADDRESS] * 3 + [ct.c_int64] + [_TENSOR_ADDRESS] * 6
                                  + [ct.c_int64, ct.c_void_p], ct.c_int),
    "ekv_resolve_resident_local": ([_TENSOR_ADDRESS] * 4 + [ct.c_int64] + [_TENSOR_ADDRESS] * 6
                                   + [ct.c_int64, ct.c_void_p], ct.c_int),
    "ekv_residency_bits": ([_P_TENSOR, _P_TENSOR, ct.c_int64, ct.c_void_p], ct.c_int),
    "ekv_gather_rows": ([_P_TENSOR] * 7 + [ct.c_int64, ct.c_int64, ct.c_int, ct.c_void_p], ct.c_int),
    "ekv_gather_kv": ([ct.POINTER(EkvPlanes), _P_TENSOR, ct.POINTER(EkvKvRows), ct.c_int64, ct.c_void_p],
                      ct.c_int),
    "ekv_scatter_kv": ([ct.POINTER(EkvPlanes), _P_TENSOR, ct.POINTER(EkvKvRows), ct.c_int64, ct.c_void_p],
                       ct.c_int),
    "ekv_swap_in": ([_P_TENSOR, ct.c_int64] + [_P_TENSOR] * 7 + [ct.c_int64] + [_P_TENSOR] * 7
                    + [ct.c_int64, _P_TENSOR, ct.c_void_p], ct.c_int),
    "ekv_swap_in_counted": ([_P_TENSOR, ct.c_int64] + [_P_TENSOR] * 7 + [ct.c_int64] + [_P_TENSOR] * 9
                            + [ct.c_void_p], ct.c_int),
    "ekv_move_kv": ([ct.POINTER(EkvPlanes), _P_TENSOR, ct.POINTER(EkvPlanes), _P_TENSOR, _P_TENSOR, ct.c_int64,
                     ct.c_void_p], ct.c_int),
    "ekv_compare_kv": ([ct.POINTER(EkvPlanes), _P_TENSOR, ct.POINTER(EkvPlanes), _P_TENSOR, _P_TENSOR,
                        ct.c_void_p], ct.c_int),
    "ekv_hisparse_swap_in": ([_P_TENSOR] * 4 + [ct.POINTER(EkvPlanes)] * 2 + [_P_TENSOR] * 4
                             + [ct.c_int64, ct.c_int64, _P_TENSOR, ct.c_void_p], ct.c_int),
    "ekv_host_device_pointer": ([ct.c_void_p, ct.POINTER(ct.c_void_p)], ct.c_int),
    "ekv_host_alloc": ([ct.c_uint64, ct.POINTER(ct.c_void_p), ct.POINTER(ct.c_void_p)], ct.c_int),
    "ekv_host_free": ([ct.c_void_p], ct.c_int),
    "ekv_stream_probe": ([ct.c_int, ct.c_void_p, ct.c_void_p, ct.c_uint64, ct.c_int, ct.c_void_p], ct.c_int),
    "ekv_decode_step_workspace_bytes": ([ct.c_int64, ct.c_int64, ct.c_int64], ct.c_uint64),
    "ekv_decode_step": ([ct.c_void_p, ct.c_void_p, ct.c_uint64, ct.c_void_p], ct.c_int),
    "ekv_decode_step_static": ([ct.c_void_p, ct.c_void_p], ct.c_int),
}
KERNEL_SYMBOLS = tuple(_SIGNATURES)


_TYPED = {}   # argument (or ELASTIC_VMM_LIBRARY, or None for the in-tree build) -> typed library


def kernel_library(library=None):
    """The native library with ekv_* signatures declared (cached per path argument).

    The cache is keyed on the path as given, so a call costs one dictionary
    lookup: resolving the path (file-system calls) happens on first use only.
    """
    key = library if library is not None else os.environ.get("ELASTIC_VMM_LIBRARY")
    lib = _TYPED.get(key)
    if lib is not None:
        return lib
    lib = _load_library(library_path(library))
    if not getattr(lib, "_ekv_typed", False):
        for name, (argtypes, restype) in _SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as exc:
                raise RuntimeError(
                    f"libelastic_vmm.so lacks {name}; rebuild it with "
                    "`python elastic-kv-vmm_amd/build_native.py`"
                ) from exc
            fn.argtypes = argtypes
            fn.restype = restype
        version = lib.ekv_abi_version()
        if version != EKV_ABI_VERSION:
            raise RuntimeError(f"libelastic_vmm.so kernel ABI {version} != {EKV_ABI_VERSION}; rebuild it")
        built, tree = lib.ekv_source_hash().decode(), source_hash()
        if tree is not None and built != tree:
            raise RuntimeError(
                f"libelastic_vmm.so was built from other sources (library {built}, tree {tree}); rebuild it "
                "with `python elastic-kv-vmm_amd/build_native.py`"
            )
        lib._ekv_typed = True
    _TYPED[key] = lib
    return lib


LAUNCHER_PATH = (Path(__file__).resolve().parents[1] / "lib"
                 / ("_ekv_launch" + sysconfig.get_config_var("EXT_SUFFIX")))
_LAUNCH = {}   # ELASTIC_VMM_LIBRARY key -> (launch helper module, {entry name: address})
# The entry points the launch helper calls (by address).
_LAUNCH_ENTRIES = ("ekv_resolve_resident", "ekv_resolve_resident_bits", "ekv_resolve_resident_local",
                   "ekv_gather_rows", "ekv_gather_kv", "ekv_scatter_kv", "ekv_move_kv", "ekv_swap_in",
                   "ekv_swap_in_counted", "ekv_hisparse_swap_in", "ekv_host_device_pointer", "ekv_decode_step")


_DEFAULT = object()   # _LAUNCH key of the helper bound on the first call without a library argument
_BOUND = {}           # _LAUNCH key -> the typed library whose entry points that helper calls


def launch_helper(library=None):
    """(module, entry addresses) for the launch-bound entry points (cached like kernel_library).

    Without a library argument the first call binds the helper to the
    library that ELASTIC_VMM_LIBRARY (or the in-tree default) names then, and
    later calls reuse it without reading the environment again: reading it
    cost about a microsecond, a sixth of a small lookup's launch.

    The module (lib/_ekv_launch*.so, built from csrc/py_launch.cpp by
    build_native.py) reads the tensors' descriptors in C++ and calls the
    entry point of kernel_library(library) whose address it is given: the
    lookup, the row gather, the per-layer SGLang-convention swap-in and a
    small decode step can take a few microseconds on the GPU, and describing
    their tensors from Python took longer than that. It is
    refused when missing or built from other sources, like the library.
    """
    if library is None:
        found = _LAUNCH.get(_DEFAULT)
        if found is not None:
            return found
    key = library if library is not None else os.environ.get("ELASTIC_VMM_LIBRARY")
    found = _LAUNCH.get(key)
    if found is not None:
        if library is None:
            _LAUNCH[_DEFAULT], _BOUND[_DEFAULT] = found, _BOUND.get(key)
        return found
    lib = kernel_library(library)
    if not LAUNCHER_PATH.exists():
        raise RuntimeError(f"the launch helper {LAUNCHER_PATH.name} is missing; build it with "
                           "`python elastic-kv-vmm_amd/build_native.py`")
    spec = importlib.util.spec_from_file_location("_ekv_launch", LAUNCHER_PATH)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    if module.abi_version() != EKV_ABI_VERSION:
        raise RuntimeError(f"{LAUNCHER_PATH.name} was built for kernel ABI {module.abi_version()}, "
                           f"not {EKV_ABI_VERSION}; rebuild it")
    tree = source_hash()
    if tree is not None and module.source_hash() != tree:
        raise RuntimeError(f"{LAUNCHER_PATH.name} was built from other sources (module {module.source_hash()}, "
                           f"tree {tree}); rebuild it with `python elastic-kv-vmm_amd/build_native.py`")
    entries = {name: ct.cast(getattr(lib, name), ct.c_void_p).value for name in _LAUNCH_ENTRIES}
    found = _LAUNCH[key] = (module, entries)
    _BOUND[key] = lib
    if library is None:
        _LAUNCH[_DEFAULT], _BOUND[_DEFAULT] = found, lib
    return found


def launch_check(status, what):
    """Raise for a failed call through the default launch helper, with the message of the library it called."""
    if status:
        check(_BOUND.get(_DEFAULT) or kernel_library(), status, what)


def describe(tensor, name="tensor"):
    """EkvTensor for a torch tensor (any strides, at most 4 dimensions)."""
    ndim = tensor.dim()
    if ndim > 4:
        raise ValueError(f"{name} has more than 4 dimensions")
    code = _DTYPE_CODES.get(tensor.dtype)
    if code is None:
        raise TypeError(f"{name} has unsupported dtype {tensor.dtype}")
    view = EkvTensor(tensor.data_ptr() if tensor.numel() else None, code, ndim)
    # Slice assignment: setting the extents one by one costs more host time per launch.
    view.shape[:ndim] = tensor.shape
    view.stride[:ndim] = tensor.stride()
    return view


# One struct.Struct per rank: pointer, dtype code, rank, the extents and the
# element strides, each padded with zero bytes to 4 entries (the EkvTensor layout).
_PACKERS = tuple(struct.Struct(f"<qii{n}q{8 * (4 - n)}x{n}q{8 * (4 - n)}x") for n in range(5))
assert all(p.size == ct.sizeof(EkvTensor) for p in _PACKERS)


def packed(tensor, name="tensor"):
    """The bytes of describe(tensor), built in one call: the lookup's launch is bound by host time.

    The data pointer goes over as it is also for an empty tensor (the entry points
    read no element of one).
    """
    shape = tensor.shape
    ndim = len(shape)
    code = _DTYPE_CODES.get(tensor.dtype)
    if code is None or ndim > 4:
        describe(tensor, name)   # raises the error that names the problem
    return _PACKERS[ndim].pack(tensor.data_ptr(), code, ndim, *shape, *tensor.stride())


def device_of(*tensors):
    """The single GPU device shared by every given tensor."""
    devices = {t.device for t in tensors if t is not None}
    if len(devices) != 1:
        raise ValueError(f"tensors must share one device, got {sorted(map(str, devices))}")
    device = devices.pop()
    if device.type != "cuda":
        raise ValueError("hot-path kernels need GPU tensors (no CPU fallback exists)")
    return device


# torch's raw current-stream query (the one its generated launch code uses) costs a
# tenth of building a torch.cuda.Stream object; the public call is the fallback.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device):
    """The hipStream_t of torch's current stream on `device`, for a launch."""
    if _RAW_STREAM is not None:
        return ct.c_void_p(_RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device()))
    return ct.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class _Current:
    """A no-op context: the device is already the current one."""

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_CURRENT = _Current()


def on_device(device):
    """Context that makes `device` current for a launch; no switch (and no cost) when it already is."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return _CURRENT if index == torch.cuda.current_device() else torch.cuda.device(index)


def check(lib, status, what):
    if status:
        message = lib.ev_error().decode("utf-8", errors="replace")
        raise RuntimeError(f"{what}: {message}")
