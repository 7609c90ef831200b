"""The drop-in's workspace policy (pgmoe.workspace.WorkspacePool), on the CPU.

One grow-only buffer per stream: token counts that fit reuse it (no allocation, no
zero-fill), a larger one allocates a buffer at least twice as big and retires the old one
without freeing it (a captured graph may still replay into it), and streams never share a
buffer (the MoE workspace keeps state between calls).
"""

import torch

from pgmoe.workspace import WorkspacePool


def test_grow_only_per_stream_and_retired_buffers_stay_alive():
    pool = WorkspacePool(torch.device("cpu"), zeroed=True)
    a = pool.get(1000, stream=1)
    assert a.numel() >= 1000 and a.data_ptr() % 256 == 0 and int(a.sum()) == 0
    a.fill_(7)  # state a forward would leave
    for n in (1, 10, 999, 1000, a.numel()):  # requests that fit: the same buffer, not re-zeroed
        b = pool.get(n, stream=1)
        assert b.data_ptr() == a.data_ptr() and int(b[0]) == 7
    c = pool.get(a.numel() + 1, stream=1)  # larger: a new zeroed buffer at least twice the old size
    assert c.data_ptr() != a.data_ptr() and c.numel() >= 2 * a.numel() and int(c.sum()) == 0
    assert c.data_ptr() % 256 == 0
    # the outgrown buffer is retired, not freed: its memory still holds what was written
    assert any(r.data_ptr() == a.data_ptr() for r in pool._retired)
    assert int(a[0]) == 7
    d = pool.get(500, stream=2)  # another stream: its own buffer
    assert d.data_ptr() not in (a.data_ptr(), c.data_ptr())
    assert pool.get(2000, stream=1).data_ptr() == c.data_ptr()
    c.fill_(3)
    pool.zero(1)  # after a failed forward
    assert int(pool.get(1, stream=1).sum()) == 0
    pool.release()
    assert not pool.buffers() and not pool._retired


def test_retired_total_is_below_current():
    pool = WorkspacePool(torch.device("cpu"), zeroed=False)
    for n in range(1, 5000, 37):  # many growing requests
        pool.get(n, stream=0)
    cur = pool.buffers()[0].numel()
    assert sum(r.numel() for r in pool._retired) < cur
    assert len(pool._retired) <= 13  # at least doubling each time from 256 bytes


def test_unzeroed_pool_for_stateless_workspaces():
    pool = WorkspacePool(torch.device("cpu"), zeroed=False)
    w = pool.get(300, stream=0)
    assert w.numel() >= 300 and w.data_ptr() % 256 == 0


def test_status_word_reaches_the_next_forward_without_a_sync():
    """The failure path: a kernel whose bounded wait gives up ORs PGMOE_STATUS_SPIN_TIMEOUT
    into the layer's host-mapped status word (pgmoe_layer.status_host); the next forward
    (or check_status) reads it with a plain host load, raises, and clears it.  Here the
    kernel's store is played by a host write to an unpinned CPU word."""
    import pytest

    from pgmoe import _lib
    from pgmoe.moe import raise_for_status
    from pgmoe.workspace import StatusWord

    w = StatusWord(pinned=False)
    assert w.ptr() != 0 and w.take() == 0
    raise_for_status(w.take())  # nothing set: no error
    w._t[0] = _lib.STATUS_SPIN_TIMEOUT
    with pytest.raises(RuntimeError, match="timed out"):
        raise_for_status(w.take())
    assert w.take() == 0  # cleared once reported
    w._t[0] = 0x40
    with pytest.raises(RuntimeError, match="0x40"):
        raise_for_status(w.take())
    # the layer struct carries the word's address to the C entry points
    L = _lib.Layer()
    L.status_host = w.ptr()
    assert L.status_host == w.ptr()
    assert _lib.Layer.status_host.offset > _lib.Layer.act.offset
