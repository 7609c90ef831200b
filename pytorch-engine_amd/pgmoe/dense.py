"""HipDenseMLP: drop-in replacement for PyGGUF's GGUFDenseMLP on MI355X.

Reads the tensors GGUFDenseMLP.from_gguf reads (pygguf_engine/model.py:789-805):

    {prefix}.ffn_{gate,up}.weight   [I, H]
    {prefix}.ffn_down.weight        [H, I]

with prefix ``blk.{layer_idx}`` or ``prefix_override``, and computes
``forward(x) -> fp32`` = down(silu(gate x) * (up x)) (model.py:839-846) with the same HIP
kernels as the MoE experts: the weights stay in the 64-row tile layout of their GGUF
bits, and one C-ABI call (pgmoe_dense_forward) enqueues the gate/up + SwiGLU and down
products without a host sync.  gemma architectures take the reference's GeGLU (the
tanh-approximation GELU in place of SiLU), as HipSparseMoEMLP does.
"""

from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn as nn

from ._lib import ACT_GELU_TANH, ACT_SILU, Dense, check, lib
from .moe import _ExpertTensor, _load_lock, padded_inter
from .workspace import WorkspacePool


class HipDenseMLP(nn.Module):
    """Dense SwiGLU FFN (gate || up -> silu(gate) * up -> down) on GGUF weights."""

    def __init__(self, gguf_file: Any, config: Any, layer_idx: int, device: torch.device,
                 prefix_override: Optional[str] = None) -> None:
        super().__init__()
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("HipDenseMLP runs on a HIP device (torch.device('cuda', i))")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        lib()  # fail now, not at the first forward, when the HIP library is missing
        self.device = device
        self.use_gelu = str(config.arch).startswith("gemma")  # GeGLU (model.py:800)
        prefix = prefix_override or f"blk.{layer_idx}"
        with _load_lock, torch.cuda.device(device):
            inter, i_out = padded_inter(gguf_file, f"{prefix}.ffn_down.weight")  # zero padding of I
            self.gate_proj = _ExpertTensor(gguf_file, f"{prefix}.ffn_gate.weight", device, False, rows_out=i_out)
            self.up_proj = _ExpertTensor(gguf_file, f"{prefix}.ffn_up.weight", device, False, rows_out=i_out)
            self.down_proj = _ExpertTensor(gguf_file, f"{prefix}.ffn_down.weight", device, False, cols_out=i_out)
            self.down_proj.check_fp16_down(f"{prefix}.ffn_down.weight")
            torch.cuda.current_stream(device).synchronize()  # uploads done before host buffers go away
        g, u, d = self.gate_proj, self.up_proj, self.down_proj
        if g.cols != g.gguf_cols:
            raise ValueError(f"{prefix}: hidden size {g.gguf_cols} is not a multiple of 256")
        if (u.rows, u.cols) != (g.rows, g.cols) or (d.rows, d.cols) != (g.cols, g.rows):
            raise ValueError(f"{prefix}: gate {g.rows}x{g.cols}, up {u.rows}x{u.cols} and down "
                             f"{d.rows}x{d.cols} do not form an [I, H] / [H, I] FFN")
        self.hidden, self.inter, self.inter_padded = g.cols, inter, g.rows
        self._ws = WorkspacePool(device, zeroed=False)  # the dense workspace keeps no state
        self._dense = self._build()

    @classmethod
    def from_gguf(cls, gguf_file: Any, config: Any, layer_idx: int, device: torch.device,
                  prefix_override: Optional[str] = None) -> "HipDenseMLP":
        """The reference's factory (model.py:789-805), same arguments."""
        return cls(gguf_file, config, layer_idx, device, prefix_override)

    def _build(self) -> Dense:
        D = Dense()
        D.hidden = self.hidden
        D.gate = self.gate_proj.weights()
        D.up = self.up_proj.weights()
        D.down = self.down_proj.weights()
        D.act = ACT_GELU_TANH if self.use_gelu else ACT_SILU
        return D

    def workspace_bytes(self, M: int) -> int:
        n = lib().pgmoe_dense_workspace_bytes(self._dense, M)
        if n == 0 and M > 0:
            check(-1, "pgmoe_dense_workspace_bytes")
        return int(n)

    def _workspace(self, M: int) -> torch.Tensor:
        """The current stream's grow-only workspace (never freed while a graph may hold it;
        see pgmoe.workspace)."""
        return self._ws.get(self.workspace_bytes(M), torch.cuda.current_stream(self.device).cuda_stream)

    def release_workspaces(self) -> None:
        """Free the workspaces (only when no captured graph replays this layer any more)."""
        self._ws.release()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x_2d = x.reshape(-1, orig_shape[-1])
        if x_2d.shape[1] != self.hidden:
            raise ValueError(f"expected hidden size {self.hidden}, got {x_2d.shape[1]}")
        if x_2d.device != self.device:
            x_2d = x_2d.to(self.device, non_blocking=True)
        if x_2d.dtype != torch.float16:
            x_2d = x_2d.to(torch.float16)
        x_2d = x_2d.contiguous()
        M = x_2d.shape[0]
        out = torch.empty((M, self.hidden), dtype=torch.float32, device=self.device)
        if M:
            ws = self._workspace(M)
            stream = torch.cuda.current_stream(self.device).cuda_stream
            check(lib().pgmoe_dense_forward(self._dense, x_2d.data_ptr(), M, out.data_ptr(), ws.data_ptr(),
                                            ws.numel(), stream), "pgmoe_dense_forward")
        return out.reshape(orig_shape)

    def replica(self) -> "HipDenseMLP":
        """A copy with its own device copy of the weights (benchmarks rotate copies so that
        reads come from HBM, not the 256 MB MALL)."""
        import copy

        r = copy.copy(self)
        r._modules = dict(self._modules)
        for name in ("gate_proj", "up_proj", "down_proj"):
            t = getattr(self, name)
            c = copy.copy(t)
            c.buf = t.buf.clone()
            c.plane = t.plane.clone() if t.plane is not None else None
            object.__setattr__(r, name, c)
        r._ws = self._ws.clone_empty()
        r._dense = r._build()
        return r

    def weight_bytes(self) -> int:
        """GGUF bytes of the three matrices (what one decode step reads)."""
        return sum(t.gguf_bytes_per_mat for t in (self.gate_proj, self.up_proj, self.down_proj))
