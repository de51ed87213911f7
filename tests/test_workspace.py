"""Workspace buffers of the tensor API (host logic, CPU tensors): one
buffer per (device, stream, kind); growth releases buffers no captured
graph uses and keeps those that one does; a capture stream with no buffer
of its own borrows the device's largest."""
import pytest
import torch

from kuillm_amd import ops

CPU = torch.device("cpu")


@pytest.fixture
def fake_streams(monkeypatch):
    state = {"stream": 1, "capturing": False}
    monkeypatch.setattr(ops, "_WS", {})
    monkeypatch.setattr(ops, "_RETIRED", [])
    monkeypatch.setattr(ops, "_CAPTURED", set())
    monkeypatch.setattr(ops, "_stream_key", lambda device: state["stream"])
    monkeypatch.setattr(ops, "_capturing", lambda device: state["capturing"])
    return state


def test_two_streams_get_distinct_buffers(fake_streams):
    a = ops.workspace(CPU, 1000, "gemv")
    fake_streams["stream"] = 2
    b = ops.workspace(CPU, 1000, "gemv")
    assert a.data_ptr() != b.data_ptr()
    assert ops.workspace(CPU, 1000, "attn").data_ptr() not in (a.data_ptr(), b.data_ptr())
    fake_streams["stream"] = 1
    assert ops.workspace(CPU, 1000, "gemv") is a
    assert ops.workspace_buffer(CPU, "gemv") is a
    assert not a.any() and not b.any()              # counters start at zero


def test_growth_releases_uncaptured_and_keeps_captured(fake_streams):
    a = ops.workspace(CPU, 1000, "gemv")
    big = ops.workspace(CPU, 3 << 20, "gemv")
    assert big.numel() >= 3 << 20 and big is not a
    assert not ops._RETIRED                          # no graph used `a`
    fake_streams["capturing"] = True
    assert ops.workspace(CPU, 1000, "gemv") is big  # handed out during a capture
    fake_streams["capturing"] = False
    bigger = ops.workspace(CPU, 5 << 20, "gemv")
    assert bigger is not big and any(r is big for r in ops._RETIRED)


def test_capture_stream_borrows_and_refuses_growth(fake_streams):
    a = ops.workspace(CPU, 2 << 20, "attn")         # eager warm-up on stream 1
    fake_streams.update(stream=7, capturing=True)   # capture on another stream
    assert ops.workspace(CPU, 1 << 20, "attn") is a
    with pytest.raises(RuntimeError, match="during HIP graph capture"):
        ops.workspace(CPU, 4 << 20, "attn")
    fake_streams.update(stream=1, capturing=False)
    b = ops.workspace(CPU, 4 << 20, "attn")         # a larger eager call on stream 1
    fake_streams.update(stream=7, capturing=True)   # the capture stream's borrowed buffer is too small
    assert ops.workspace(CPU, 3 << 20, "attn") is b
    assert any(r is a for r in ops._RETIRED)        # `a` was handed to a capture: kept alive
    with pytest.raises(RuntimeError):
        ops.workspace(CPU, 16, "gemv")              # no buffer of that kind anywhere
