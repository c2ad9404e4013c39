"""The C-ABI library loads and exports what include/*.h declares (CPU only).

No compute call is made here: the error paths exercised below fail in host
validation before any HIP call.
"""

import ctypes as ct
import re
import subprocess

import pytest

from conftest import ROOT

HEADERS = sorted((ROOT / "include").glob("*.h"))
LIBRARY = ROOT / "elastic-kv-vmm_amd" / "lib" / "libelastic_vmm.so"


def declared_functions():
    names = []
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b((?:ev|ekv)_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not LIBRARY.exists():
        pytest.fail(f"{LIBRARY} is missing; run __graft_entry__.build()")
    import torch  # noqa: F401  (binds the HIP runtime torch ships, as in production)

    return ct.CDLL(str(LIBRARY))


def test_headers_declare_the_reference_abi_and_kernels():
    names = declared_functions()
    reference_abi = ["ev_backed", "ev_base", "ev_close", "ev_create", "ev_drop", "ev_ensure", "ev_error",
                     "ev_granularity", "ev_poisoned", "ev_precommit", "ev_reserved"]
    assert set(reference_abi) <= set(names)
    assert {"ekv_resolve_resident", "ekv_gather_rows", "ekv_gather_kv", "ekv_scatter_kv",
            "ekv_abi_version"} <= set(names)


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing


def test_python_bindings_cover_the_kernel_abi():
    from elastic_kv import _native

    declared = {name for name in declared_functions() if name.startswith("ekv_")}
    assert declared == set(_native.KERNEL_SYMBOLS)


def test_abi_version_matches_python(lib):
    from elastic_kv import _native

    lib.ekv_abi_version.restype = ct.c_int
    assert lib.ekv_abi_version() == _native.EKV_ABI_VERSION


def test_create_validation_error_is_reported_through_ev_error(lib):
    lib.ev_create.argtypes = [ct.c_int, ct.c_uint64, ct.c_uint64]
    lib.ev_create.restype = ct.c_void_p
    lib.ev_error.restype = ct.c_char_p
    assert lib.ev_create(0, 0, 2 << 20) is None
    assert b"positive" in lib.ev_error()
    assert lib.ev_create(0, 4 << 20, 17) is None
    assert b"multiple of 16" in lib.ev_error()


def test_null_handles_fail_cleanly(lib):
    lib.ev_error.restype = ct.c_char_p
    lib.ev_base.argtypes = [ct.c_void_p]
    lib.ev_base.restype = ct.c_uint64
    assert lib.ev_base(None) == (1 << 64) - 1
    assert b"null backing handle" in lib.ev_error()
    lib.ev_close.argtypes = [ct.c_void_p]
    assert lib.ev_close(None) == 0


def test_kernel_entry_points_validate_before_launch(lib):
    from elastic_kv import _native

    typed = _native.kernel_library(str(LIBRARY))

    def tensor(shape, dtype):
        t = _native.EkvTensor()
        t.data = 4096  # never dereferenced: validation fails first
        t.dtype = dtype
        t.ndim = len(shape)
        for i, extent in enumerate(shape):
            t.shape[i] = extent
            t.stride[i] = 1
        return t

    topk = tensor((1, 2, 4), 1)
    table = tensor((2, 8), 2)
    rows = tensor((2,), 2)
    lengths = tensor((2,), 1)
    bad_output = tensor((1, 2, 7), 1)
    status = typed.ekv_resolve_resident(ct.byref(topk), ct.byref(table), None, ct.byref(rows), ct.byref(lengths),
                                        ct.byref(rows), ct.byref(bad_output), None, None, 2, None)
    assert status == -1
    assert b"output dimension 2 is 7, expected 8" in typed.ev_error()
    status = typed.ekv_resolve_resident(None, ct.byref(table), None, ct.byref(rows), ct.byref(lengths),
                                        ct.byref(rows), ct.byref(bad_output), None, None, 2, None)
    assert status == -1 and b"topk is required" in typed.ev_error()
    planes = _native.EkvPlanes(4096, 1, 3, 0, 0, 16, 16, 4)
    slots = tensor((1, 1, 1), 1)
    rows_out = _native.EkvKvRows(4096, 0, 0, 0, 16)
    assert typed.ekv_gather_kv(ct.byref(planes), ct.byref(slots), ct.byref(rows_out), 1, None) == -1
    assert b"kv 1 or 2" in typed.ev_error()

    # HiSparse swap-in: 2 rows x 2 blocks of 4 tokens against an 8-slot hot buffer.
    pair = _native.EkvPlanes(4096, 1, 2, 0, 1 << 20, 256, 256, 64)
    blocks = tensor((2, 2), 1)
    state = dict(tokens=tensor((3, 9), 1), host_locs=tensor((3, 100), 2), dev_locs=tensor((3, 9), 1),
                 out=tensor((2, 8), 1), req=tensor((2,), 2), seq=tensor((2,), 1), lru=tensor((3, 8), 5))

    def swap(hot=8, bs=4, planes=pair, **changes):
        args = {**state, **changes}
        return typed.ekv_hisparse_swap_in(
            ct.byref(blocks), ct.byref(args["tokens"]), ct.byref(args["host_locs"]), ct.byref(args["dev_locs"]),
            ct.byref(planes), ct.byref(pair), ct.byref(args["out"]), ct.byref(args["req"]), ct.byref(args["seq"]),
            ct.byref(args["lru"]), hot, bs, None, None)

    assert swap(out=tensor((2, 7), 1)) == -1 and b"top_k_device_locs dimension 1 is 7" in typed.ev_error()
    assert swap(hot=7, lru=tensor((3, 7), 5)) == -1 and b"must not exceed hot_buffer_size" in typed.ev_error()
    assert swap(tokens=tensor((3, 8), 1)) == -1 and b"hot_buffer_size + 1 columns" in typed.ev_error()
    assert swap(lru=tensor((3, 8), 2)) == -1 and b"lru_slots must be int16 or int32" in typed.ev_error()
    assert swap(hot=5000) == -1 and b"hot_buffer_size must be 1..4096" in typed.ev_error()
    one_plane = _native.EkvPlanes(4096, 1, 1, 0, 0, 256, 256, 64)
    assert swap(planes=one_plane) == -1 and b"one layer of K and V planes" in typed.ev_error()
    assert typed.ekv_host_device_pointer(None, ct.byref(ct.c_void_p())) == -1
    assert typed.ekv_stream_probe(2 | 0x40, 4096, 4096, 1 << 20, 0, None) == -1
    assert b"unknown stream probe flags" in typed.ev_error()
    assert typed.ekv_stream_probe(3 | 0x10, 4096, 4096, 1 << 20, 0, None) == -1
    assert b"mode must be" in typed.ev_error()


def test_packed_descriptors_are_the_struct_bytes(lib):
    import torch

    from elastic_kv import _native

    typed = _native.kernel_library(str(LIBRARY))
    cases = [torch.zeros(1, 2, 8, dtype=torch.int32), torch.zeros(3, 4, 5, 6, dtype=torch.bfloat16)[:, 1:3],
             torch.zeros(2, 9, dtype=torch.int16).t(), torch.tensor(7, dtype=torch.int64),
             torch.zeros(4, dtype=torch.uint8)[::2]]
    for t in cases:
        assert _native.packed(t) == bytes(_native.describe(t)), (t.shape, t.stride())
    with pytest.raises(ValueError, match="topk has more than 4 dimensions"):
        _native.packed(torch.zeros(1, 1, 1, 1, 1, dtype=torch.int32), "topk")
    with pytest.raises(TypeError, match="rows has unsupported dtype"):
        _native.packed(torch.zeros(2, dtype=torch.float64), "rows")

    # The C side reads the packed bytes: the same validation error as through ctypes.byref.
    topk = _native.packed(torch.zeros(1, 2, 4, dtype=torch.int32))
    table = _native.packed(torch.zeros(2, 8, dtype=torch.int64))
    rows = _native.packed(torch.zeros(2, dtype=torch.int64))
    lengths = _native.packed(torch.zeros(2, dtype=torch.int32))
    bad_output = _native.packed(torch.zeros(1, 2, 7, dtype=torch.int32))
    status = typed.ekv_resolve_resident(topk, table, None, rows, lengths, rows, bad_output, None, None, 2, None)
    assert status == -1
    assert b"output dimension 2 is 7, expected 8" in typed.ev_error()


FASTDIV_TEST = r"""
#include "ekv_fastdiv.h"
#include <cstdio>
#include <cstdint>
int main() {
    const uint32_t divisors[] = {1, 2, 3, 5, 7, 16, 31, 32, 100, 128, 255, 256, 257, 2048, 4095, 65536,
                                 1000003, 0x7fffffffu};
    uint64_t state = 88172645463325252ull;
    for (uint32_t d : divisors) {
        ekv::FastDiv f(d);
        for (uint32_t n = 0; n < 200000; ++n) {
            if (f.div(n) != n / d) { std::printf("fail %u / %u\n", n, d); return 1; }
        }
        for (int i = 0; i < 200000; ++i) {
            state ^= state << 13; state ^= state >> 7; state ^= state << 17;
            const uint32_t n = static_cast<uint32_t>(state) & 0x7fffffffu;
            if (f.div(n) != n / d) { std::printf("fail %u / %u\n", n, d); return 1; }
        }
        if (f.div(0x7fffffffu) != 0x7fffffffu / d) { std::printf("fail max / %u\n", d); return 1; }
    }
    std::puts("ok");
    return 0;
}
"""


def test_fast_division_is_exact_below_2_pow_31(tmp_path):
    source = tmp_path / "fastdiv.cpp"
    source.write_text(FASTDIV_TEST)
    binary = tmp_path / "fastdiv"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "elastic-kv-vmm_amd" / "csrc"),
                    str(source), "-o", str(binary)], check=True)
    assert subprocess.run([str(binary)], capture_output=True, text=True).stdout.strip() == "ok"


def test_library_fingerprint_matches_the_sources(lib):
    from elastic_kv._source_hash import source_hash

    lib.ekv_source_hash.restype = ct.c_char_p
    assert lib.ekv_source_hash().decode() == source_hash()


def test_library_built_from_other_sources_is_refused(monkeypatch):
    from elastic_kv import _native, backing

    backing._load_library.cache_clear()
    try:
        monkeypatch.setattr(_native, "source_hash", lambda: "0" * 32)
        monkeypatch.setattr(_native, "_TYPED", {})   # forget the library typed by earlier tests
        with pytest.raises(RuntimeError, match="built from other sources"):
            _native.kernel_library()
    finally:
        backing._load_library.cache_clear()


def test_launch_helper_loads_and_matches_the_library(lib):
    import torch

    from elastic_kv import _native
    from elastic_kv._source_hash import source_hash

    helper, entries = _native.launch_helper()
    assert helper.abi_version() == _native.EKV_ABI_VERSION
    assert helper.source_hash() == source_hash()
    typed = _native.kernel_library()
    for name, address in entries.items():
        assert address == ct.cast(getattr(typed, name), ct.c_void_p).value, name
    # Host tensors are refused before any HIP call, with the ctypes path's messages.
    i32 = lambda *shape: torch.zeros(shape, dtype=torch.int32)  # noqa: E731
    with pytest.raises(ValueError, match="no CPU fallback"):
        helper.resolve(0, entries["ekv_resolve_resident"], i32(1, 2, 4), i32(2, 8), None, None, None, 0,
                       torch.arange(2), i32(2), torch.arange(2), i32(1, 2, 4), None, None, 1)
    with pytest.raises(ValueError, match="no CPU fallback"):
        helper.gather_rows(entries["ekv_gather_rows"], i32(64), i32(1, 2), i32(1), i32(1), None, None,
                           i32(1, 2, 8), 8, 0, 0)
    with pytest.raises(TypeError, match="rows must be a tensor"):
        helper.resolve(0, entries["ekv_resolve_resident"], i32(1, 2, 4), i32(2, 8), None, None, None, 0,
                       [0, 1], i32(2), torch.arange(2), i32(1, 2, 4), None, None, 1)
    with pytest.raises(TypeError, match="resolve takes 15 arguments"):
        helper.resolve(0)


def test_launch_helper_built_from_other_sources_is_refused(monkeypatch):
    from elastic_kv import _native

    monkeypatch.setattr(_native, "source_hash", lambda: "0" * 32)
    monkeypatch.setattr(_native, "_LAUNCH", {})
    monkeypatch.setattr(_native, "kernel_library", lambda library=None: None)
    with pytest.raises(RuntimeError, match="launch helper|built from other sources"):
        _native.launch_helper()
