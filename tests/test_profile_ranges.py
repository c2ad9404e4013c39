"""EKV_PROFILE_RANGES: off means the functions themselves and no imports; on
means nested "ekv/<name>" ranges that still raise what the call raises, the
hot path's entry points wrapped at import, and the engine coordinator marked
once. Follows the behaviour the reference tests in tests/test_profile_ranges.py."""

from contextlib import contextmanager
import importlib
import os
import sys
from types import ModuleType
from unittest.mock import patch

import pytest
import torch  # noqa: F401  (imported before any sys.modules patch, which would drop a first import on exit)

from adaptive_sparse import profile_ranges
from adaptive_sparse.profile_ranges import install_native_profile_ranges, profile_range


@contextmanager
def switched_on(events):
    """Switch on, with a torch.profiler whose record_function logs enter/exit."""

    @contextmanager
    def record_function(name):
        events.append(("enter", name))
        try:
            yield
        finally:
            events.append(("exit", name))

    fake = ModuleType("torch.profiler")
    fake.record_function = record_function
    with patch.dict(os.environ, {"EKV_PROFILE_RANGES": "1"}), patch.dict(sys.modules, {"torch.profiler": fake}):
        yield


@pytest.mark.parametrize("value", [None, "0", "true", ""])
def test_off_returns_the_function_and_imports_nothing(value):
    def original(x):
        return x + 1

    environment = {k: v for k, v in os.environ.items() if k != "EKV_PROFILE_RANGES"}
    if value is not None:
        environment["EKV_PROFILE_RANGES"] = value
    with patch.dict(os.environ, environment, clear=True):
        with patch("builtins.__import__", side_effect=AssertionError("imported while off")):
            wrapped = profile_range("test")(original)
            install_native_profile_ranges()
    assert wrapped is original and wrapped(1) == 2


def test_ranges_nest_and_pass_exceptions_through():
    events, failure = [], KeyError("lane 7")
    with switched_on(events):
        @profile_range("inner")
        def inner(*, fail):
            if fail:
                raise failure
            return "ok"

        @profile_range("outer")
        def outer(fail):
            return inner(fail=fail)

        assert outer(False) == "ok"
        with pytest.raises(KeyError) as caught:
            outer(True)
    assert caught.value is failure
    assert inner.__name__ == "inner" and outer.__wrapped__.__name__ == "outer"
    once = [("enter", "ekv/outer"), ("enter", "ekv/inner"), ("exit", "ekv/inner"), ("exit", "ekv/outer")]
    assert events == once * 2


def test_roctx_range_brackets_the_call():
    calls = []

    class Marker:
        def range_push(self, label):
            calls.append(("push", label))

        def range_pop(self):
            calls.append(("pop",))

    with switched_on([]), patch.object(profile_ranges, "_marker", return_value=Marker()):
        @profile_range("native/lookup")
        def lookup():
            calls.append(("call",))
            raise ValueError("bad")

        with pytest.raises(ValueError):
            lookup()
    assert calls == [("push", "ekv/native/lookup"), ("call",), ("pop",)]


def test_hot_path_entry_points_are_wrapped_only_when_on():
    names = {"adaptive_sparse.resident_lookup": "resolve_resident", "adaptive_sparse.swap_in": "swap_in",
             "adaptive_sparse.sparse_read": "gather_kv", "adaptive_sparse.decode_step": "decode_step",
             "adaptive_sparse.hisparse_swap": "load_blocks_to_device_buffer_mha"}
    modules = {name: importlib.import_module(name) for name in names}
    try:
        events = []
        with switched_on(events):
            for name, function in names.items():
                reloaded = importlib.reload(modules[name])
                assert hasattr(getattr(reloaded, function), "__wrapped__"), name
    finally:
        with patch.dict(os.environ, {"EKV_PROFILE_RANGES": "0"}):
            for name, function in names.items():
                reloaded = importlib.reload(modules[name])
                assert not hasattr(getattr(reloaded, function), "__wrapped__"), name


def test_coordinator_is_marked_once():
    class Coordinator:
        def map_last_loc_to_buffer(self, row):
            return row * 2

        def swap_in_selected_blocks(self, *, row):
            return row + 1

    module = ModuleType("sglang.srt.managers.hisparse_coordinator")
    module.HiSparseCoordinator = Coordinator
    events = []
    with switched_on(events), patch.dict(sys.modules, {module.__name__: module}):
        install_native_profile_ranges()
        first = (Coordinator.map_last_loc_to_buffer, Coordinator.swap_in_selected_blocks)
        install_native_profile_ranges()
        assert (Coordinator.map_last_loc_to_buffer, Coordinator.swap_in_selected_blocks) == first
        coordinator = Coordinator()
        assert coordinator.map_last_loc_to_buffer(5) == 10
        assert coordinator.swap_in_selected_blocks(row=6) == 7
    assert events == [("enter", "ekv/native/map_latest"), ("exit", "ekv/native/map_latest"),
                      ("enter", "ekv/native/swap"), ("exit", "ekv/native/swap")]


def test_bench_drops_the_switch_unless_asked():
    import bench

    environment = {"EKV_PROFILE_RANGES": "1", "HIP_VISIBLE_DEVICES": "0"}
    bench.apply_profile_switch(environment, False)
    assert environment == {"HIP_VISIBLE_DEVICES": "0"}
    bench.apply_profile_switch(environment, True)
    assert environment["EKV_PROFILE_RANGES"] == "1"
    assert bench.parse_args.__module__ == "bench"
