"""The switch module's host-side bookkeeping, without a GPU: the launchers'
once-checked stream record (kernels.CheckedStreams) is dropped whenever a
stream could have changed shape, dtype, device or address."""

from __future__ import annotations

import torch

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
