"""HipSparseMoEMLP: drop-in replacement for PyGGUF's GGUFSparseMoEMLP on MI355X.

Same constructor ``(gguf_file, config, layer_idx, device)`` and ``forward(x) -> fp32`` as
pygguf_engine/model.py:849-937, reading the same tensors:

    blk.{i}.ffn_gate_inp.weight            router [E, H] (F32 / F16 / BF16)
    blk.{i}.ffn_{gate,up,down}_exps.weight  routed experts [E, I, H] / [E, H, I]
    blk.{i}.ffn_{gate,up,down}_shexp.weight optional shared expert
    blk.{i}.ffn_gate_inp_shexp.weight       optional shared-expert sigmoid gate [H]

and the config fields ``n_experts``, ``n_experts_used``, ``norm_topk_prob`` and ``arch``.
Expert weights stay in GGUF block form on the device (the same bits moved into 64-row
tiles; Q4_0 / Q5_0 stored with the same values as Q4_1 / Q8_0); the whole forward is one C-ABI call that
enqueues router, top-k, dispatch, expert products and combine without a host sync.
"""

from __future__ import annotations

import ctypes
import threading
from typing import Any, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from . import ops
from ._lib import (ACT_GELU_TANH, ACT_SILU, F16, FLOAT_QTYPES, REQUANT_W4_QTYPES, REQUANT_W8_QTYPES,
                   STATUS_SPIN_TIMEOUT, SUPPORTED_QTYPES, Layer, Weights, check, lib)
from .workspace import StatusWord, WorkspacePool

_F32, _F16, _BF16 = 0, 1, 30
_load_lock = threading.Lock()


def raise_for_status(bits: int) -> None:
    """RuntimeError for the PGMOE_STATUS_* bits a kernel set (0: nothing to report)."""
    if bits & STATUS_SPIN_TIMEOUT:
        raise RuntimeError("an earlier forward's wait for the router logits timed out: its output was wrong")
    if bits:
        raise RuntimeError(f"pgmoe status {bits:#x} from an earlier forward")


def load_float_tensor(gguf_file: Any, name: str, device: torch.device) -> torch.Tensor:
    """fp32 copy of a router / gate / norm tensor on ``device`` (quant_kernels.py:1095-1114):
    F32 / F16 / BF16 converted, and quantised ones (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, Q4_1, Q5_0; the
    reference's gguf.quants.dequantize branch) dequantised once on the device to the values
    the ggml block definitions give.  CPU targets take the float types only.  The formats
    the reference re-quantises for its matrix products (Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4, Q5_1)
    are not decoded here: its float tensors get their exact gguf-py values, which only the
    re-quantised form is built for."""
    info = gguf_file.tensors[name]
    raw = gguf_file.get_tensor_bytes(name)
    shape = tuple(int(s) for s in info.shape)
    if info.qtype == _F32:
        arr = torch.from_numpy(np.frombuffer(raw, dtype=np.float32).reshape(shape).copy())
    elif info.qtype == _F16:
        arr = torch.from_numpy(np.frombuffer(raw, dtype=np.float16).reshape(shape).copy()).float()
    elif info.qtype == _BF16:
        u16 = np.frombuffer(raw, dtype=np.uint16).reshape(shape).copy()
        arr = torch.from_numpy(u16.view(np.int16)).view(torch.bfloat16).float()
    elif (int(info.qtype) in SUPPORTED_QTYPES and int(info.qtype) not in REQUANT_W4_QTYPES + REQUANT_W8_QTYPES
          and torch.device(device).type == "cuda"):
        cols = shape[-1]
        rows = int(np.prod(shape[:-1])) if len(shape) > 1 else 1
        if cols % 256:
            raise NotImplementedError(f"{name}: quantised rows of {cols} weights (a multiple of 256 is needed)")
        src = torch.from_numpy(np.ascontiguousarray(np.asarray(raw)).view(np.uint8)).to(device)
        return ops.dequant_matrix(int(info.qtype), src, rows, cols).reshape(shape).contiguous()
    else:
        raise NotImplementedError(f"{name}: router/gate tensors of ggml type {info.qtype} are not supported")
    return arr.to(device=device, dtype=torch.float32).contiguous()


def padded_inter(gguf_file: Any, down_name: str) -> Tuple[int, int]:
    """(I, I_out) of an FFN whose down tensor is `down_name` ([E, H, I] or [H, I]): I_out = I
    when I is a multiple of 256; for a 32-weight down format (Q8_0, Q5_0, Q5_1, Q4_0, Q4_1, IQ4_NL, MXFP4) with I
    a multiple of 32 (e.g. 1408), I rounded up to one of 256: gate / up then get zero rows and
    down zero columns up to I_out, and the kernels compute the unpadded layer's values (zero
    rows give SwiGLU values of exactly 0, which meet zero weights)."""
    info = gguf_file.tensors[down_name]
    inter = int(info.shape[-1])
    io = ops.padded_width(int(info.qtype), inter)
    if io < 0:
        raise ValueError(f"{down_name}: {inter} input features (a multiple of 256, or of 32 for the 32-weight "
                         "formats Q8_0, Q5_0, Q5_1, Q4_0, Q4_1, IQ4_NL, MXFP4)")
    return inter, io


class _ExpertTensor:
    """One quantised weight tensor ([E, N, K] or [N, K]) held in the device layout, as
    [rows_out, cols_out] matrices when given (zero padding; see padded_inter)."""

    def __init__(self, gguf_file: Any, name: str, device: torch.device, three_d: bool,
                 rows_out: Optional[int] = None, cols_out: Optional[int] = None):
        info = gguf_file.tensors[name]
        shape = tuple(int(s) for s in info.shape)
        if three_d and len(shape) != 3:
            raise ValueError(f"Expected 3D MoE tensor for {name}, got shape={shape}")
        if not three_d and len(shape) != 2:
            raise ValueError(f"Expected 2D tensor for {name}, got shape={shape}")
        self.n_mats, self.gguf_rows, self.gguf_cols = (shape if three_d else (1,) + shape)
        self.gguf_qtype = int(info.qtype)
        self.qtype = ops.device_qtype(self.gguf_qtype)  # format of the device layout
        if self.gguf_qtype not in SUPPORTED_QTYPES:
            raise NotImplementedError(
                f"{name}: ggml type {info.qtype_name if hasattr(info, 'qtype_name') else self.qtype} "
                "has no HIP kernel (supported: Q4_K, Q5_K, Q6_K, Q8_0, Q4_1, Q4_0 / Q5_0 relaid out as Q4_1 / "
                "Q8_0, F16 / BF16 / F32 held as fp16, and Q2_K / Q3_K / IQ4_NL / IQ4_XS / MXFP4 re-quantised to "
                "Q4_1 as the reference's W4 repack does, Q5_1 to its W8 values held as fp16)")
        width = ops.padded_width(self.gguf_qtype, self.gguf_cols)
        if width < 0 or (cols_out is not None and cols_out < width):
            raise ValueError(f"{name}: {self.gguf_cols} input features is not a multiple of 256"
                             + (" (nor of 32 for a 32-weight format)" if width < 0 else ""))
        self.rows = self.gguf_rows if rows_out is None else int(rows_out)
        self.cols = width if cols_out is None else int(cols_out)
        if self.gguf_qtype in FLOAT_QTYPES:
            # fp16 weights, rounded from F32 / BF16 as the reference's fp16 expert mode loads
            # them (load_float_tensor(..., dtype=torch.float16), quant_kernels.py:1962-1964)
            w16 = load_float_tensor(gguf_file, name, device).to(torch.float16).contiguous()
            raw = w16.view(torch.uint8).reshape(-1)
            src_qtype = F16
        else:
            raw = torch.from_numpy(np.asarray(gguf_file.get_tensor_bytes(name))).to(device)  # H2D copy
            src_qtype = self.gguf_qtype
        self.buf = ops.relayout(src_qtype, raw, self.n_mats, self.gguf_rows, self.gguf_cols, self.rows, self.cols)
        del raw
        # K-quants: the sub-block scales decoded once for the prefill MFMA products
        self.plane = ops.scale_plane(self.qtype, self.buf, self.n_mats, self.rows, self.cols)

    def weights(self) -> Weights:
        return ops.make_weights(self.qtype, self.buf, self.n_mats, self.rows, self.cols, self.plane)

    def check_fp16_down(self, name: str) -> None:
        """fp16 down projections run on the fused decode down + combine, whose rows hold at
        most 32 super-blocks (8192 inputs); a longer fp16 row would fail at the first decode
        forward, so it is refused at load."""
        if self.qtype == F16 and self.cols > 8192:
            raise NotImplementedError(f"{name}: fp16 down projection of {self.cols} inputs (at most 8192)")

    @property
    def gguf_bytes_per_mat(self) -> int:
        per, bb = ops.GGUF_BLOCK[self.gguf_qtype]
        return self.gguf_rows * (self.gguf_cols // per) * bb


class HipSparseMoEMLP(nn.Module):
    """Sparse MoE FFN block (router -> top-k -> grouped GGUF expert SwiGLU -> combine)."""

    def __init__(self, gguf_file: Any, config: Any, layer_idx: int, device: torch.device) -> None:
        super().__init__()
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("HipSparseMoEMLP runs on a HIP device (torch.device('cuda', i))")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        lib()  # fail now, not at the first forward, when the HIP library is missing
        self.config = config
        self.device = device
        self.n_experts = int(config.n_experts)
        self.top_k = max(1, int(config.n_experts_used))
        self.norm_topk_prob = bool(config.norm_topk_prob)
        self.use_gelu = str(config.arch).startswith("gemma")  # GeGLU experts (model.py:868)

        prefix = f"blk.{layer_idx}"
        with _load_lock, torch.cuda.device(device):
            router = load_float_tensor(gguf_file, f"{prefix}.ffn_gate_inp.weight", device)
            self.register_buffer("router_weight", router, persistent=False)
            self.router_bias: Optional[torch.Tensor] = None
            # an intermediate size that is not a multiple of 256 is zero-padded (padded_inter)
            self.inter, self.inter_padded = padded_inter(gguf_file, f"{prefix}.ffn_down_exps.weight")
            i_out = self.inter_padded
            self.gate_exps = _ExpertTensor(gguf_file, f"{prefix}.ffn_gate_exps.weight", device, True, rows_out=i_out)
            self.up_exps = _ExpertTensor(gguf_file, f"{prefix}.ffn_up_exps.weight", device, True, rows_out=i_out)
            self.down_exps = _ExpertTensor(gguf_file, f"{prefix}.ffn_down_exps.weight", device, True,
                                           cols_out=i_out)
            self.down_exps.check_fp16_down(f"{prefix}.ffn_down_exps.weight")
            self.shared_gate = self.shared_up = self.shared_down = None
            self.shared_inp_gate: Optional[torch.Tensor] = None
            if f"{prefix}.ffn_gate_shexp.weight" in gguf_file.tensors:
                _, s_out = padded_inter(gguf_file, f"{prefix}.ffn_down_shexp.weight")
                self.shared_gate = _ExpertTensor(gguf_file, f"{prefix}.ffn_gate_shexp.weight", device, False,
                                                 rows_out=s_out)
                self.shared_up = _ExpertTensor(gguf_file, f"{prefix}.ffn_up_shexp.weight", device, False,
                                               rows_out=s_out)
                self.shared_down = _ExpertTensor(gguf_file, f"{prefix}.ffn_down_shexp.weight", device, False,
                                                 cols_out=s_out)
                self.shared_down.check_fp16_down(f"{prefix}.ffn_down_shexp.weight")
                gname = f"{prefix}.ffn_gate_inp_shexp.weight"
                if gname in gguf_file.tensors:
                    self.shared_inp_gate = load_float_tensor(gguf_file, gname, device).reshape(-1).contiguous()
            torch.cuda.current_stream(device).synchronize()  # uploads done before host buffers go away
        self.hidden = int(self.router_weight.shape[1])
        if self.gate_exps.cols != self.gate_exps.gguf_cols:
            raise ValueError(f"{prefix}: hidden size {self.gate_exps.gguf_cols} is not a multiple of 256")
        if self.router_weight.shape[0] != self.n_experts:
            raise ValueError(f"router has {self.router_weight.shape[0]} rows, config says {self.n_experts} experts")
        self._ws = WorkspacePool(device, zeroed=True)
        # host-mapped status word: the kernels' failure bits, readable without a stream sync
        self._status = StatusWord(pinned=True)
        self._layer = self._build_layer()

    # ------------------------------------------------------------------ plumbing
    def set_router_bias(self, bias: Optional[torch.Tensor]) -> None:
        """Harness-only extension: add bias[e] to the router logits before softmax."""
        if bias is not None:
            bias = bias.to(device=self.device, dtype=torch.float32).reshape(-1).contiguous()
            if bias.numel() != self.n_experts:
                raise ValueError("router bias must have n_experts entries")
        self.router_bias = bias
        self._layer = self._build_layer()

    def _build_layer(self) -> Layer:
        L = Layer()
        L.hidden = self.hidden
        L.n_experts = self.n_experts
        L.top_k = self.top_k
        L.norm_topk = int(self.norm_topk_prob)
        L.act = ACT_GELU_TANH if self.use_gelu else ACT_SILU
        L.router_w = self.router_weight.data_ptr()
        L.status_host = self._status.ptr()
        L.router_bias = self.router_bias.data_ptr() if self.router_bias is not None else None
        L.gate = self.gate_exps.weights()
        L.up = self.up_exps.weights()
        L.down = self.down_exps.weights()
        if self.shared_gate is not None:
            L.has_shared = 1
            L.sh_gate = self.shared_gate.weights()
            L.sh_up = self.shared_up.weights()
            L.sh_down = self.shared_down.weights()
            L.sh_inp_gate = self.shared_inp_gate.data_ptr() if self.shared_inp_gate is not None else None
        return L

    def workspace_bytes(self, M: int) -> int:
        n = lib().pgmoe_workspace_bytes(self._layer, M)
        if n == 0 and M > 0:
            check(-1, "pgmoe_workspace_bytes")
        return int(n)

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _workspace(self, M: int) -> torch.Tensor:
        """The current stream's workspace, grown (zero-filled) if M needs more bytes than it
        has.  It starts with the decode router's self-resetting ready-tagged logits and the
        status word, which must be zero when a buffer is new; see pgmoe.workspace."""
        return self._ws.get(self.workspace_bytes(M), self._stream())

    def release_workspaces(self) -> None:
        """Free the workspaces (only when no captured graph replays this layer any more)."""
        self._ws.release()

    def check_status(self, sync: bool = False) -> None:
        """Raise RuntimeError if a kernel of an earlier forward flagged its output as wrong (a
        decode wave's bounded wait for the router logits gave up), and clear the flags.

        Without ``sync`` this reads only the host-mapped status word the kernels also write:
        no stream synchronisation, so it suits every step of a loop that replays captured
        graphs (``forward`` itself checks it on entry).  With ``sync`` it also synchronises
        and reads the status word of every workspace this layer holds, including retired
        ones that captured graphs may still replay into."""
        bits = self._status.take()
        if sync:
            st = ctypes.c_int32()
            for ws in self._ws.all_buffers():
                check(lib().pgmoe_moe_status(self._layer, ws.data_ptr(), ws.numel(), ctypes.byref(st), 1,
                                             self._stream()), "pgmoe_moe_status")
                bits |= st.value
        raise_for_status(bits)

    def routing(self, M: int):
        """The routing the last forward of M tokens on the current stream produced, in sorted
        pair order: (offsets [E+1], expert [M*K], token [M*K], weight [M*K]) device tensors,
        read back from that forward's own workspace (pgmoe_moe_routing)."""
        ws = self._workspace(M)
        i32 = dict(dtype=torch.int32, device=self.device)
        P = M * self.top_k
        offsets = torch.empty(self.n_experts + 1, **i32)
        pe = torch.empty(max(P, 1), **i32)
        pt = torch.empty(max(P, 1), **i32)
        pw = torch.empty(max(P, 1), dtype=torch.float32, device=self.device)
        check(lib().pgmoe_moe_routing(self._layer, M, ws.data_ptr(), ws.numel(), offsets.data_ptr(),
                                      pe.data_ptr(), pt.data_ptr(), pw.data_ptr(), self._stream()),
              "pgmoe_moe_routing")
        return offsets, pe[:P], pt[:P], pw[:P]

    # ------------------------------------------------------------------ forward
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
        # an earlier forward's kernels may have flagged their output (a plain host read)
        raise_for_status(self._status.take())
        out = torch.empty((M, self.hidden), dtype=torch.float32, device=self.device)
        if M:
            ws = self._workspace(M)
            stream = self._stream()
            rc = lib().pgmoe_moe_forward(self._layer, x_2d.data_ptr(), M, out.data_ptr(), ws.data_ptr(),
                                         ws.numel(), stream)
            if rc:
                # a forward that stopped part-way may leave tagged router words set: the
                # workspace must be zero again before the next call
                self._ws.zero(stream)
                check(rc, "pgmoe_moe_forward")
        return out.reshape(orig_shape)

    def replica(self) -> "HipSparseMoEMLP":
        """A copy of this layer with its own device copy of every expert weight (used to
        rotate weight sets in benchmarks so reads come from HBM, not the 256 MB MALL)."""
        import copy

        r = copy.copy(self)
        r._modules = dict(self._modules)
        r._buffers = dict(self._buffers)
        for name in ("gate_exps", "up_exps", "down_exps", "shared_gate", "shared_up", "shared_down"):
            t = getattr(self, name)
            if t is not None:
                c = copy.copy(t)
                c.buf = t.buf.clone()
                c.plane = t.plane.clone() if t.plane is not None else None
                object.__setattr__(r, name, c)
        r._ws = self._ws.clone_empty()
        r._status = StatusWord(pinned=True)
        r._layer = r._build_layer()
        return r

    # ------------------------------------------------------------------ accounting
    def active_weight_bytes(self, n_distinct: int) -> int:
        """GGUF bytes of `n_distinct` routed experts (gate + up + down)."""
        per = sum(t.gguf_bytes_per_mat for t in (self.gate_exps, self.up_exps, self.down_exps))
        return n_distinct * per

    def shared_weight_bytes(self) -> int:
        if self.shared_gate is None:
            return 0
        return sum(t.gguf_bytes_per_mat for t in (self.shared_gate, self.shared_up, self.shared_down))
