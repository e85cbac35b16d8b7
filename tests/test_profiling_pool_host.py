"""Host-side contracts of cx.profile() and cx.memory_pool() (reference
python/tensorcx/profiling.py:31-153, memory.py:24-90): argument validation,
single use, owning thread, nesting, report shape. No device is needed."""

from __future__ import annotations

import json
import threading

import pytest

import tensorcx as cx


@pytest.mark.parametrize("bad", [0, 100001, True, 1.5, "3"])
def test_profile_rejects_bad_limits(bad):
    with pytest.raises(ValueError):
        cx.profile(max_events=bad)


@pytest.mark.parametrize("bad", [1, None, "yes"])
def test_profile_device_timing_must_be_bool(bad):
    with pytest.raises(ValueError):
        cx.profile(device_timing=bad)


def test_profile_lifecycle_and_report(tmp_path):
    p = cx.profile(max_events=8)
    with pytest.raises(RuntimeError):
        p.report()
    with p:
        with pytest.raises(RuntimeError):
            with cx.profile():
                pass
    report = p.report()
    assert report["events"] == [] and report["device_events"] == []
    assert report["complete"] and report["host_complete"] and report["device_complete"] is None
    assert report["schema_version"] == 1 and report["device_clock"] == "hip_events_elapsed_ms"
    assert p.summary() == [] and p.device_summary() == []
    with pytest.raises(RuntimeError):
        with p:
            pass
    out = tmp_path / "trace.json"
    p.export_chrome_trace(out)
    assert json.loads(out.read_text())["traceEvents"] == []


def test_profile_exit_must_be_on_owner_thread():
    p = cx.profile()
    p.__enter__()
    errors = []

    def other():
        try:
            p.__exit__(None, None, None)
        except RuntimeError as error:
            errors.append(error)
    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert errors
    p.__exit__(None, None, None)


@pytest.mark.parametrize("kwargs", [{"max_cached_bytes": -1}, {"max_cached_blocks": 0},
                                    {"max_cached_blocks": 4097}, {"max_cached_bytes": True},
                                    {"max_cached_blocks": 2.5}])
def test_memory_pool_rejects_bad_limits(kwargs):
    with pytest.raises(ValueError):
        cx.memory_pool("hip", **kwargs)


def test_memory_pool_contract_on_the_host():
    pool = cx.memory_pool("hip", max_cached_bytes=1 << 20, max_cached_blocks=4)
    with pytest.raises(RuntimeError):
        pool.stats()
    with pytest.raises(RuntimeError):
        pool.trim()
    with pytest.raises(ValueError):
        with cx.memory_pool("cpu"):
            pass
    with pytest.raises(ValueError):
        cx.memory_pool("cuda")
    if not cx.is_available("hip"):
        with pytest.raises(RuntimeError):  # no device: the native pool is unavailable
            with pool:
                pass
