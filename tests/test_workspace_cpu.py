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
