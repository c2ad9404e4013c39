"""Compile the native library libelastic_vmm.so for gfx950 with hipcc.

The library holds the HIP VMM backing (ev_* ABI) and the hot-path kernels
(ekv_* ABI). It is built in-tree so that it travels with the source tree:
    python elastic-kv-vmm_amd/build_native.py
This mirrors the reference's "compile the packaged native source" step
(elastic_kv/build_vmm.py:20-41), with hipcc in place of g++ + libcuda.
"""

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
if str(PACKAGE_ROOT) not in sys.path:
    sys.path.insert(0, str(PACKAGE_ROOT))

from elastic_kv._source_hash import source_hash  # noqa: E402
SOURCE_DIR = PACKAGE_ROOT / "csrc"
BUILD_DIR = PACKAGE_ROOT / "_build"
LIBRARY = PACKAGE_ROOT / "lib" / "libelastic_vmm.so"
# The launch helper module for the launch-bound entry points (csrc/py_launch.cpp).
LAUNCHER = PACKAGE_ROOT / "lib" / ("_ekv_launch" + sysconfig.get_config_var("EXT_SUFFIX"))
LAUNCHER_SOURCE = "py_launch.cpp"
SOURCES = ("vmm_backing.hip", "lookup.hip", "gather.hip", "swap_in.hip", "compare.hip", "hisparse_swap.hip",
           "stream_probe.hip", "decode_step.hip", "build_info.hip")
OFFLOAD_ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # Code-object v5 is loadable by the HIP runtime bundled with PyTorch as
    # well as by the system ROCm runtime.
    "-mcode-object-version=5",
    # Keep the compiler from forming packed-FP32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc():
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build libelastic_vmm.so")
    return found


def _compile(compiler, source, obj, verbose, extra=()):
    command = [compiler, *COMMON_FLAGS, *extra, "-c", str(source), "-o", str(obj)]
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stdout}\n{result.stderr}")
    return result.stderr


def _build_launcher(fingerprint, verbose):
    """Compile the launch helper module with the host compiler against torch's headers and libraries.

    It is host code only; the HIP platform macro selects the HIP flavour of torch's c10 stream headers.
    """
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    rocm = Path(hipcc()).resolve().parents[1]
    temporary = LAUNCHER.with_name(LAUNCHER.name + ".tmp")
    command = [os.environ.get("CXX", "g++"), "-O2", "-shared", "-fPIC", "-std=c++17", "-Wall",
               f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}", "-D__HIP_PLATFORM_AMD__=1",
               "-DUSE_ROCM=1", f"-DEKV_SOURCE_HASH={fingerprint}",
               *(f"-I{path}" for path in cpp_extension.include_paths()), f"-I{sysconfig.get_paths()['include']}",
               f"-I{rocm / 'include'}", str(SOURCE_DIR / LAUNCHER_SOURCE), "-o", str(temporary),
               f"-L{torch_lib}", "-ltorch_python", "-ltorch", "-lc10", "-lc10_hip", f"-Wl,-rpath,{torch_lib}"]
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"the launch helper failed to compile:\n{result.stdout}\n{result.stderr}")
    os.replace(temporary, LAUNCHER)
    return result.stderr


def build(verbose=False):
    """Compile every source, link lib/libelastic_vmm.so and build the launch helper; returns the library path."""
    compiler = hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    LIBRARY.parent.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), max(1, (os.cpu_count() or 1)))
    fingerprint = source_hash()
    objects = []
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        futures = []
        for name in SOURCES:
            source = SOURCE_DIR / name
            obj = BUILD_DIR / (Path(name).stem + ".o")
            objects.append(obj)
            extra = [f"-DEKV_SOURCE_HASH={fingerprint}"] if name == "build_info.hip" else []
            futures.append(pool.submit(_compile, compiler, source, obj, verbose, extra))
        futures.append(pool.submit(_build_launcher, fingerprint, verbose))
        for future in futures:
            warnings = future.result()
            if verbose and warnings.strip():
                print(warnings, file=sys.stderr)
    temporary = LIBRARY.with_suffix(".so.tmp")
    command = [compiler, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC",
               *map(str, objects), "-o", str(temporary)]
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(temporary, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
