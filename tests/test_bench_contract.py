"""CPU checks of the bench.py command-line contract and of loud failure
when the native kernels are missing."""

import subprocess
import sys
from types import SimpleNamespace
from unittest.mock import patch

import pytest

from conftest import ROOT


def test_bench_refuses_more_than_one_gpu():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1"],
                            capture_output=True, text=True, timeout=120)
    assert result.returncode == 2
    assert "one GPU only" in result.stderr
    assert result.stdout == ""


def test_kernel_library_without_kernels_raises():
    from elastic_kv import _native
    from elastic_kv.backing import _load_library

    names = ("ev_create", "ev_ensure", "ev_precommit", "ev_drop", "ev_base", "ev_backed", "ev_reserved",
             "ev_granularity", "ev_close", "ev_error", "ev_poisoned")
    library = SimpleNamespace(**{name: lambda *a: 0 for name in names})
    _load_library.cache_clear()
    try:
        with patch("elastic_kv.backing.ct.CDLL", return_value=library):
            with pytest.raises(RuntimeError, match="lacks ekv_"):
                _native.kernel_library("no-kernels-libelastic-vmm.so")
    finally:
        _load_library.cache_clear()


def test_product_code_never_imports_the_oracle():
    # The oracle is test infrastructure: the package must not import it (bench.py's
    # CPU-baseline leg and __graft_entry__.smoke are the only non-test users).
    import ast

    offenders = []
    for path in sorted((ROOT / "elastic-kv-vmm_amd").rglob("*.py")):
        tree = ast.parse(path.read_text(), filename=str(path))
        for node in ast.walk(tree):
            names = []
            if isinstance(node, ast.Import):
                names = [alias.name for alias in node.names]
            elif isinstance(node, ast.ImportFrom) and node.module:
                names = [node.module]
            if any(name == "oracle" or name.startswith("oracle.") for name in names):
                offenders.append(f"{path.relative_to(ROOT)}:{node.lineno}")
    assert offenders == []


def test_kernels_refuse_cpu_tensors():
    # No CPU fallback exists: every hot-path wrapper raises on host tensors.
    import torch

    from adaptive_sparse.kv_pool import KVPlanes
    from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
    from adaptive_sparse.sparse_read import gather_kv

    i32 = lambda *shape: torch.zeros(shape, dtype=torch.int32)  # noqa: E731
    with pytest.raises(ValueError, match="no CPU fallback"):
        resolve_resident(i32(1, 2, 4), i32(2, 8), None, torch.arange(2), i32(2), torch.arange(2), i32(1, 2, 4), 1)
    with pytest.raises(ValueError, match="no CPU fallback"):
        build_residency_bits(i32(2, 64))
    planes = KVPlanes(base=0, device=0, layers=1, kv=2, layer_stride=0, kv_stride=64, row_stride=8, row_bytes=8,
                      rows=8, owner=None)
    with pytest.raises(ValueError, match="no CPU fallback"):
        gather_kv(planes, i32(1, 2, 3), torch.zeros((2, 1, 2, 3, 8), dtype=torch.uint8))


def test_decode_inputs_reject_shapes_that_cannot_hold_the_picks():
    # A recent region smaller than the 80 % recent picks would make the index
    # gathers read past their sources; the generator refuses such shapes.
    import bench
    import torch

    with pytest.raises(ValueError, match="decode inputs need"):
        bench.decode_inputs(torch, torch.device("cpu"), 1, 1, 65536, 2048, 1024, 1024, 0)


def test_default_line_extras_name_real_workloads_and_options(monkeypatch):
    import bench

    monkeypatch.setattr(sys, "argv", ["bench.py"])
    defaults = vars(bench.parse_args())
    keys = [key for key, _, _ in bench.EXTRA_CONFIGS]
    assert len(keys) == len(set(keys))
    for key, workload, overrides in bench.EXTRA_CONFIGS:
        assert workload in bench.WORKLOADS, key
        assert set(overrides) <= set(defaults), (key, set(overrides) - set(defaults))
    assert {"config1_topk_gather", "config2_block_gather", "config4_migration", "config5_composite",
            "lookup_micro"} <= set(keys)
