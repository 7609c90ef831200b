"""Grow-only device workspaces for the C-ABI forwards, one per HIP stream.

The C entry points allocate nothing: the caller brings a workspace of
``pgmoe_*_workspace_bytes(M)`` bytes.  One buffer serves every token count up to the
largest seen so far (the C layer lays it out so that a workspace sized for the largest M
serves any smaller M), so an engine that alternates M = 1 decode with M = 2..8 verify
steps (pygguf_engine/model.py:1875, :2114) allocates and zero-fills only when a larger M
first appears.

Buffers are never freed while their owner lives: a HIP graph captured around a forward
keeps the workspace's address, so a buffer outgrown by a later, larger call stays
allocated (retired, not reused) for any graph that may still replay it.  Sizes grow at
least twofold, so the retired buffers of one stream total less than its current one.
``release()`` drops everything, for callers that know no graph holds a buffer.

Each stream has its own buffer: the MoE workspace keeps state between calls (the decode
router's self-resetting ready-tagged logits and the status word), so forwards on two
streams must not share one.  Calls on one stream are ordered by the stream itself.
"""

from __future__ import annotations

from typing import Dict, List

import torch

_ALIGN = 256


class WorkspacePool:
    def __init__(self, device: torch.device, zeroed: bool) -> None:
        self.device = device
        self.zeroed = zeroed  # zero-fill new buffers (the MoE workspace requires it)
        self._cur: Dict[int, torch.Tensor] = {}  # stream handle -> aligned buffer view
        self._retired: List[torch.Tensor] = []

    def get(self, nbytes: int, stream: int) -> torch.Tensor:
        """An aligned uint8 buffer of at least nbytes for `stream` (a hipStream_t handle)."""
        ws = self._cur.get(stream)
        if ws is not None and ws.numel() >= nbytes:
            return ws
        size = max(int(nbytes), 2 * ws.numel() if ws is not None else 0)
        size = (size + _ALIGN - 1) // _ALIGN * _ALIGN
        alloc = torch.zeros if self.zeroed else torch.empty
        raw = alloc(size + _ALIGN, dtype=torch.uint8, device=self.device)
        new = raw[(-raw.data_ptr()) % _ALIGN:][:size]
        if ws is not None:
            self._retired.append(ws)
        self._cur[stream] = new
        return new

    def zero(self, stream: int) -> None:
        """Zero the stream's buffer again (after a forward that failed part-way)."""
        ws = self._cur.get(stream)
        if ws is not None:
            ws.zero_()

    def buffers(self) -> Dict[int, torch.Tensor]:
        return dict(self._cur)

    def all_buffers(self) -> List[torch.Tensor]:
        """Every buffer still held: the streams' current ones and the retired ones that a
        captured graph may still replay into."""
        return list(self._cur.values()) + list(self._retired)

    def release(self) -> None:
        """Free every buffer.  Only safe when no captured graph still uses one."""
        self._cur.clear()
        self._retired.clear()

    def clone_empty(self) -> "WorkspacePool":
        return WorkspacePool(self.device, self.zeroed)


class StatusWord:
    """A host word the kernels can write (pinned, device-mapped memory on a GPU host): the
    MoE forward passes its address as ``pgmoe_layer.status_host``, and a kernel that sets a
    status bit in its workspace ORs the bit in here too.  Reading it is a plain host load,
    so a forward can check the word of the forwards before it without synchronising the
    stream (a bit set by a forward still running shows up at a later check)."""

    def __init__(self, pinned: bool = True) -> None:
        self._t = torch.zeros(1, dtype=torch.int32, pin_memory=pinned)

    def ptr(self) -> int:
        return self._t.data_ptr()

    def take(self) -> int:
        """The bits set so far, cleared."""
        v = int(self._t[0])
        if v:
            self._t[0] = 0
        return v
