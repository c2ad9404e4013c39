"""Failure paths of the native VMM backing on the CPU, under a fault-injecting driver.

csrc/vmm_core.h holds the backing's host logic with the driver as a template
parameter; tests/native/vmm_fault_driver.cpp is a driver that keeps its own
books, fails the k-th call of any operation and counts contract breaches.
Two builds with g++ (no GPU, no HIP):
  * tests/native/vmm_fault_cases.cpp + the driver, with AddressSanitizer and
    UBSan: every rollback, poison and retry case of the reference's
    native/elastic_vmm.cpp:97-215 through the ev_* ABI;
  * the driver alone as a shared library, loaded by the Python Backing
    (library=...), so its rollback / poison handling runs over the real native
    code - the cases of the reference's tests/test_backing.py:205-265 without
    the broker, which is not part of this library.
"""

import ctypes as ct
import shutil
import subprocess
from pathlib import Path

import pytest

from elastic_kv.backing import Backing, _load_library

ROOT = Path(__file__).resolve().parents[1]
NATIVE = Path(__file__).resolve().parent / "native"
CSRC = ROOT / "elastic-kv-vmm_amd" / "csrc"
BUILD = NATIVE / "_build"
CHUNK = 2 << 20
OPS = {name: i for i, name in enumerate(("reserve", "free", "open_stream", "close_stream", "create", "map",
                                          "set_access", "unmap", "release", "zero", "wait_zero", "sync"))}


def _gxx():
    compiler = shutil.which("g++")
    if compiler is None:
        pytest.fail("g++ is required for the native fault-injection tests")
    return compiler


def _compile(output, sources, flags):
    BUILD.mkdir(exist_ok=True)
    command = [_gxx(), "-std=c++17", "-g", "-Wall", "-Wextra", f"-I{CSRC}", *flags, *map(str, sources), "-o",
               str(output)]
    result = subprocess.run(command, capture_output=True, text=True, timeout=300)
    assert result.returncode == 0, result.stderr
    return output


def test_native_fault_cases_under_sanitizers():
    sanitizers = ["-O1", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
                  "-fno-sanitize-recover=undefined"]
    binary = _compile(BUILD / "vmm_fault_cases", [NATIVE / "vmm_fault_cases.cpp", NATIVE / "vmm_fault_driver.cpp"],
                      sanitizers)
    result = subprocess.run([str(binary)], capture_output=True, text=True, timeout=120,
                            env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0",
                                 "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert result.returncode == 0, result.stdout + result.stderr
    assert "all VMM fault cases passed" in result.stdout
    assert "contract violation" not in result.stderr


@pytest.fixture(scope="module")
def fake_library():
    path = _compile(BUILD / "libvmm_fault_driver.so", [NATIVE / "vmm_fault_driver.cpp"], ["-O1", "-shared", "-fPIC"])
    lib = ct.CDLL(str(path))
    lib.fake_fail.argtypes = [ct.c_int, ct.c_long, ct.c_int]
    lib.fake_set_chunk.argtypes = [ct.c_uint64]
    for name in ("fake_live_handles", "fake_live_maps", "fake_live_ranges", "fake_violations"):
        getattr(lib, name).restype = ct.c_long
    lib.fake_set_chunk(CHUNK)
    _load_library.cache_clear()
    yield str(path), lib
    _load_library.cache_clear()


def _open(fake_library, chunks=4):
    path, lib = fake_library
    lib.fake_reset()
    return Backing(chunks * CHUNK, CHUNK, 0, library=path), lib


def _clean(lib):
    return (lib.fake_live_handles(), lib.fake_live_maps(), lib.fake_live_ranges(), lib.fake_violations()) == (0,) * 4


def test_backing_bookkeeping_over_the_native_core(fake_library):
    backing, lib = _open(fake_library)
    assert backing.reserved_bytes == 4 * CHUNK and backing.chunk_count == 4
    assert backing.ensure([0, 1]) == 2 and backing.precommit([2, 1]) == 1
    assert backing.mapped_chunks == {0, 1} and backing.backed_bytes == 3 * CHUNK
    assert backing.ensure([2]) == 0 and backing.mapped_chunks == {0, 1, 2}
    assert backing.reclaim([1, 3], synchronize=False) == 1
    assert backing.metrics["backed_bytes"] == 2 * CHUNK and backing.metrics["reclaim_chunks"] == 1
    with pytest.raises(ValueError, match="outside reserved range"):
        backing.ensure([4])
    backing.close()
    assert _clean(lib)


def test_clean_native_rollback_allows_retry(fake_library):
    backing, lib = _open(fake_library)
    lib.fake_fail(OPS["map"], 2, 0)
    with pytest.raises(RuntimeError, match="hipMemMap"):
        backing.ensure([0, 1])
    assert backing.mapped_chunks == frozenset() and not backing._poisoned
    assert backing.backed_bytes == 0 and lib.fake_live_handles() == 0
    assert backing.metrics["ensure_calls"] == 0
    assert backing.ensure([0, 1]) == 2 and backing.mapped_chunks == {0, 1}
    backing.close()
    assert _clean(lib)


def test_partial_native_map_failure_poisons(fake_library):
    backing, lib = _open(fake_library)
    lib.fake_fail(OPS["set_access"], 2, 0)
    lib.fake_fail(OPS["unmap"], 1, 0)           # the rollback of chunk 1 fails
    with pytest.raises(RuntimeError, match="hipMemSetAccess"):
        backing.ensure([0, 1])
    assert backing._poisoned
    with pytest.raises(RuntimeError, match="closed or has encountered"):
        backing.ensure([2])
    backing.close()                              # teardown still releases what is left
    assert _clean(lib)


def test_partial_native_decommit_poisons_and_failed_close_retries(fake_library):
    backing, lib = _open(fake_library)
    backing.ensure([0, 1, 2])
    lib.fake_fail(OPS["release"], 2, 0)
    with pytest.raises(RuntimeError, match="decommit chunk"):
        backing.reclaim([0, 1, 2], synchronize=False)
    assert backing._poisoned
    lib.fake_reset()
    lib.fake_fail(OPS["sync"], 1, 0)
    with pytest.raises(RuntimeError, match="teardown failed"):
        backing.close()
    backing.close()
    assert _clean(lib)


def test_unreferenced_backing_releases_its_reservation(fake_library):
    import gc

    backing, lib = _open(fake_library)
    backing.ensure([0, 3])
    del backing
    gc.collect()
    assert _clean(lib)


def test_spare_pool_through_the_python_backing(fake_library):
    path, lib = fake_library
    lib.fake_reset()
    backing = Backing(4 * CHUNK, CHUNK, 0, library=path, spare_chunks=2)
    lib.fake_calls.restype = ct.c_long
    assert backing.ensure([0, 1, 2]) == 3 and lib.fake_calls(OPS["create"]) == 3
    assert backing.reclaim([0, 1, 2], synchronize=False) == 3
    assert backing.spare_bytes == 2 * CHUNK and backing.backed_bytes == 0
    assert lib.fake_calls(OPS["release"]) == 1 and lib.fake_live_handles() == 2
    metrics = backing.metrics                    # the kept chunks are still held, not released
    assert (metrics["spare_bytes"], metrics["backed_bytes"], metrics["held_bytes"]) == (2 * CHUNK, 0, 2 * CHUNK)
    assert backing.ensure([3, 2]) == 2 and lib.fake_calls(OPS["create"]) == 3     # both recycled
    assert backing.spare_bytes == 0 and backing.mapped_chunks == {2, 3}
    with pytest.raises(ValueError, match="spare_chunks"):
        backing.set_spare_chunks(5)
    backing.reclaim([2], synchronize=False)
    backing.set_spare_chunks(0)                  # gives the kept chunk back
    assert backing.spare_bytes == 0 and lib.fake_live_handles() == 1
    backing.close()
    assert _clean(lib)
