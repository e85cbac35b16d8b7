"""cx.profile() and cx.memory_pool() on the hip device: host spans from the
native backend, HIP-event device intervals per operation, pool reuse."""

from __future__ import annotations

import numpy as np
import pytest

from conftest import require_gpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def cx():
    require_gpu()
    import tensorcx
    return tensorcx


def test_profile_spans_and_device_intervals(cx):
    a = np.ones((256, 128), np.float32)
    b = np.ones((128, 64), np.float32)
    with cx.profile(device_timing=True) as p:
        x, y = cx.tensor(a, device="hip"), cx.tensor(b, device="hip")
        z = cx.softmax(cx.matmul(x, y), -1)
        host = z.numpy()
    assert np.allclose(host, 1 / 64)
    report = p.report()
    events = report["events"]
    by_id = {e["id"]: e for e in events}
    dispatch = [e for e in events if e["category"] == "dispatch"]
    assert [e["operation"] for e in dispatch] == ["matmul", "softmax"]
    copies = [e for e in events if e["category"] == "copy_api"]
    assert {e["name"] for e in copies} == {"host_to_device", "device_to_host"}
    assert sorted(e["bytes"] for e in copies) == sorted([64 * 256 * 4, 128 * 64 * 4, 256 * 128 * 4])
    allocations = [e for e in events if e["category"] == "allocation"]
    # The matmul and softmax outputs are allocated inside their dispatch spans.
    assert any(by_id.get(e["parent_id"], {}).get("operation") == "matmul" for e in allocations)
    for e in events:
        assert 0 <= e["self_ns"] <= e["duration_ns"]
    device = report["device_events"]
    assert [e["operation"] for e in device] == ["matmul", "softmax"]
    assert all(e["error"] is None and e["elapsed_ms"] > 0 for e in device)
    assert report["complete"] and report["device_complete"]
    assert {row["operation"] for row in p.device_summary()} == {"matmul", "softmax"}
    assert any(row["category"] == "synchronize" for row in p.summary())


def test_profile_bounded_and_drops_counted(cx):
    x = cx.tensor(np.ones((4, 4), np.float32), device="hip")
    with cx.profile(max_events=3, device_timing=True) as p:
        for _ in range(4):
            cx.exp(x)
    report = p.report()
    assert len(report["events"]) == 3 and report["dropped_events"] > 0
    assert not report["complete"]


def test_profile_off_records_nothing(cx):
    x = cx.tensor(np.ones((4, 4), np.float32), device="hip")
    cx.exp(x)  # no session: no spans anywhere
    with cx.profile() as p:
        pass
    assert p.report()["events"] == []


def test_memory_pool_lifecycle(cx):
    pool = cx.memory_pool("hip", max_cached_bytes=8 << 20, max_cached_blocks=4)
    with pool:
        x = cx.tensor(np.ones((128, 128), np.float32), device="hip")
        for _ in range(4):
            y = cx.exp(x)
            del y
        stats = pool.stats()
        assert stats["active"] and stats["hits"] >= 2 and stats["cached_blocks"] >= 1
        pool.trim()
        assert pool.stats()["cached_blocks"] == 0
        np.testing.assert_array_equal(x.numpy(), np.ones((128, 128), np.float32))  # live tensors stay
    assert not pool.stats()["active"]
    with pytest.raises(RuntimeError):
        with pool:
            pass
