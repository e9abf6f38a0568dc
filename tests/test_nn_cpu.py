"""The switch module's host-side bookkeeping, without a GPU: the launchers'
once-checked stream record (kernels.CheckedStreams) is dropped whenever a
stream could have changed shape, dtype, device or address."""

from __future__ import annotations

import torch

from mlx_iqk_amd import kernels
from mlx_iqk_amd.nn import IqkSwitchLinear


def test_checked_streams_are_dropped_when_a_stream_changes():
    m = IqkSwitchLinear("iq2_ks", 4, 64, 2048)
    sentinel = object()
    object.__setattr__(m, "_checked_streams", sentinel)
    m.fused_prefill = False  # not a stream: kept
    assert m._checked_streams is sentinel
    m.qs = torch.zeros_like(m.qs)  # a stream reassigned
    assert m._checked_streams is None
    object.__setattr__(m, "_checked_streams", sentinel)
    m.to(torch.float32)  # a move or cast of the buffers
    assert m._checked_streams is None
    object.__setattr__(m, "_checked_streams", sentinel)
    m.load_state_dict(m.state_dict())  # copies in place: same tensors, same shapes
    assert m._checked_streams is sentinel
    assert "_checked_streams" not in m.state_dict() and "_stream_set" not in m.state_dict()


class _Recorder:
    """Stands in for kernels.CheckedStreams (which needs GPU tensors) and
    records the stream addresses of every record made."""

    made: list = []

    def __init__(self, member, streams, num_experts, out_features, in_features):
        self.ptrs = tuple(t.data_ptr() for t in streams)
        _Recorder.made.append(self.ptrs)


def test_checked_streams_follow_buffers_replaced_behind_setattr(monkeypatch):
    monkeypatch.setattr(kernels, "CheckedStreams", _Recorder)
    _Recorder.made = []
    m = IqkSwitchLinear("iq2_ks", 4, 64, 2048)
    first = m._checked()
    assert m._checked() is first and len(_Recorder.made) == 1  # unchanged streams: reused

    m.register_buffer("qs", torch.zeros_like(m.qs))  # bypasses __setattr__
    second = m._checked()
    assert second is not first and second.ptrs[0] == m.qs.data_ptr()

    m.qs.data = torch.zeros_like(m.qs)  # swaps the storage of the same Parameter/buffer object
    third = m._checked()
    assert third is not second and third.ptrs[0] == m.qs.data_ptr()

    m.scl.data = torch.zeros(m.scl.numel(), dtype=m.scl.dtype).view(m.scl.shape)  # a new storage
    fourth = m._checked()
    assert fourth is not third and fourth.ptrs[1] == m.scl.data_ptr()

    m.load_state_dict(m.state_dict())  # in-place copies: same addresses
    assert m._checked() is fourth
    assert len(_Recorder.made) == 4
