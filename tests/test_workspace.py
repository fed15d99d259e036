"""Device workspaces of the kernels' Python layer (CPU: the bookkeeping
only, no kernel runs)."""
import torch

from nanosglang_amd.kernels import AcceptWorkspace


def test_grown_workspace_keeps_the_replaced_buffers():
    """A HIP graph captured while a smaller buffer was current keeps its
    address: growing the workspace must not free that buffer, or later
    replays of the graph write into memory that other tensors now hold."""
    ws = AcceptWorkspace("cpu")
    a = ws.get(100)
    pa = a.data_ptr()
    del a
    b = ws.get(1000)
    assert b.numel() >= 1000 and b.data_ptr() != pa
    assert [t.data_ptr() for t in ws._retired] == [pa]
    c = ws.get(500)                      # fits: same buffer, nothing retired
    assert c.data_ptr() == b.data_ptr() and len(ws._retired) == 1
    assert int(ws.get(4000).sum()) == 0  # a new buffer starts zero
    assert len(ws._retired) == 2

