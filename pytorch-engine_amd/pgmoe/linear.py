"""GGUFQuantLinear / FusedLinearPack on the HIP kernels (pgmoe_linear_forward).

Drop-ins for the reference's quantized linear (pygguf_engine/quant_kernels.py:1604-1915),
the module behind its attention projections, lm_head, embedding table and the shared
expert's fused gate||up:

    GGUFQuantLinear.from_gguf(gguf_file, weight_name, bias_name=None, device, workers=None)
    GGUFQuantLinear.forward(x)            -> x . W^T (+ bias), in x's dtype
    GGUFQuantLinear.embed_lookup(ids, dtype=torch.float16) -> the dequantised rows
    GGUFQuantLinear.fuse(linears)         -> one module, outputs concatenated
    FusedLinearPack(linears).forward(x) / .forward_single_concat(x)

The weights stay in GGUF block form on the device (the 64-row tile layout of the MoE
experts); M <= 8 tokens run the wavefront GEMV, more run the MFMA GEMM.  Unquantised
weights (F16 / F32 / BF16, the reference's "fp16" mode) run torch's fp16 F.linear on the
device, as in the reference.  There is no CPU path: quantised formats without a kernel,
rows whose width is not a multiple of 256, and CPU devices raise.  The reference's
tensor-parallel slicing (slice_output_rows / slice_input_blocks) is not provided: this
build runs on one GPU.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from ._lib import SUPPORTED_QTYPES, check, lib
from .moe import _load_lock, load_float_tensor
from .workspace import WorkspacePool

_F32, _F16, _BF16 = 0, 1, 30
_FLOAT_TYPES = (_F32, _F16, _BF16)
_W4_TYPES = (2, 3, 12)  # Q4_0, Q4_1, Q4_K: the reference's 4-bit "w4" mode
_OUT = {torch.float32: 0, torch.float16: 1}


class GGUFQuantLinear(nn.Module):
    """y = x . W^T (+ bias) with W in GGUF blocks on the device."""

    def __init__(self, mode: str, in_features: int, out_features: int, gguf_qtype: Optional[int] = None,
                 raw: Optional[np.ndarray] = None, weight: Optional[torch.Tensor] = None,
                 bias: Optional[torch.Tensor] = None, device: Optional[torch.device] = None) -> None:
        super().__init__()
        self.mode = mode  # "w4" / "w8" (quantised, by the reference's naming) or "fp16"
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.gguf_qtype = gguf_qtype
        dev = torch.device(device if device is not None else (weight.device if weight is not None else "cuda"))
        if dev.type != "cuda":
            raise ValueError("GGUFQuantLinear runs on a HIP device (torch.device('cuda', i))")
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self._raw = raw  # host GGUF bytes (mmap view): fuse() relays out their concatenation
        self.register_buffer("bias", None if bias is None else bias.to(dev, torch.float32).contiguous(),
                             persistent=False)
        self.register_buffer("weight", None, persistent=False)
        self.buf = self.plane = None
        self.cols = self.in_features
        if mode == "fp16":
            self.weight = weight.to(dev, torch.float16).contiguous()
            return
        if gguf_qtype not in SUPPORTED_QTYPES:
            raise NotImplementedError(f"ggml type {gguf_qtype} has no HIP kernel (supported: Q4_K, Q5_K, Q6_K, "
                                      "Q8_0, Q4_1, Q4_0 / Q5_0 relaid out as Q4_1 / Q8_0, and Q2_K / Q3_K / "
                                      "IQ4_NL / IQ4_XS / MXFP4 re-quantised to Q4_1 as the reference's W4 "
                                      "repack does, Q5_1 to its W8 values held as fp16)")
        # the device width: in_features, or for the 32-weight formats the next multiple of 256
        # (zero blocks appended to every row; forward appends as many zero inputs)
        self.cols = ops.padded_width(gguf_qtype, self.in_features)
        if self.cols < 0:
            raise NotImplementedError(f"{self.in_features} input features: the K-quant formats need a multiple "
                                      "of 256, the 32-weight formats a multiple of 32")
        self.qtype = ops.device_qtype(gguf_qtype)
        lib()
        with torch.cuda.device(dev):
            src = torch.from_numpy(np.ascontiguousarray(raw)).to(dev)
            self.buf = ops.relayout(gguf_qtype, src, 1, self.out_features, self.in_features, cols_out=self.cols)
            self.plane = ops.scale_plane(self.qtype, self.buf, 1, self.out_features, self.cols)
            torch.cuda.current_stream(dev).synchronize()  # the upload is done before `raw` may go away
        self._w = ops.make_weights(self.qtype, self.buf, 1, self.out_features, self.cols, self.plane)
        self._ws = WorkspacePool(dev, zeroed=False)

    # ------------------------------------------------------------------ construction
    @classmethod
    def from_gguf(cls, gguf_file: Any, weight_name: str, bias_name: Optional[str] = None,
                  device: torch.device = torch.device("cuda"), workers: Optional[int] = None) -> "GGUFQuantLinear":
        """The reference's loader (quant_kernels.py:1774-1812), same arguments (`workers` is
        accepted and unused: the relayout runs on the GPU)."""
        info = gguf_file.tensors[weight_name]
        out_features, in_features = int(info.shape[0]), int(info.shape[1])
        bias = None
        if bias_name and bias_name in gguf_file.tensors:
            # the reference keeps the bias in fp16 (load_float_tensor(..., dtype=torch.float16))
            bias = load_float_tensor(gguf_file, bias_name, torch.device("cpu")).to(torch.float16).float()
        qt = int(info.qtype)
        with _load_lock:
            if qt in _FLOAT_TYPES:
                w = load_float_tensor(gguf_file, weight_name, torch.device("cpu")).reshape(out_features, in_features)
                return cls("fp16", in_features, out_features, weight=w, bias=bias, device=device)
            mode = "w4" if qt in _W4_TYPES else "w8"
            raw = np.asarray(gguf_file.get_tensor_bytes(weight_name))
            return cls(mode, in_features, out_features, qt, raw=raw, bias=bias, device=device)

    @classmethod
    def fuse(cls, linears: Sequence["GGUFQuantLinear"]) -> "GGUFQuantLinear":
        """One module whose outputs are the concatenation of `linears`' (quant_kernels.py:1635):
        the GGUF rows are concatenated and relaid out once.  The members must share mode,
        input width, device and (for quantised ones) ggml type."""
        if len(linears) == 1:
            return linears[0]
        first = linears[0]
        for lin in linears[1:]:
            if (lin.mode != first.mode or lin.in_features != first.in_features or lin.device != first.device
                    or lin.gguf_qtype != first.gguf_qtype):
                raise ValueError("Cannot fuse GGUFQuantLinear modules with mismatched mode/in_features/device/qtype")
        total = sum(lin.out_features for lin in linears)
        bias = None
        if any(lin.bias is not None for lin in linears):
            bias = torch.cat([lin.bias.cpu() if lin.bias is not None else torch.zeros(lin.out_features)
                              for lin in linears])
        if first.mode == "fp16":
            w = torch.cat([lin.weight for lin in linears], dim=0)
            return cls("fp16", first.in_features, total, weight=w, bias=bias, device=first.device)
        raw = np.concatenate([np.asarray(lin._raw).reshape(-1) for lin in linears])
        return cls(first.mode, first.in_features, total, first.gguf_qtype, raw=raw, bias=bias, device=first.device)

    # ------------------------------------------------------------------ compute
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig_shape = x.shape
        x_2d = x.reshape(-1, self.in_features)
        if x_2d.device != self.device:
            x_2d = x_2d.to(self.device, non_blocking=True)
        if self.mode == "fp16":
            b = None if self.bias is None else self.bias.to(torch.float16)
            out = F.linear(x_2d.to(torch.float16), self.weight, b).to(x.dtype)
            return out.reshape(*orig_shape[:-1], self.out_features)
        xh = x_2d if x_2d.dtype == torch.float16 else x_2d.to(torch.float16)
        xh = xh.contiguous()
        if self.cols != self.in_features:  # zero inputs for the zero weight blocks
            xh = F.pad(xh, (0, self.cols - self.in_features))
        M = xh.shape[0]
        odt = x.dtype if x.dtype in _OUT else torch.float16
        out = torch.empty((M, self.out_features), dtype=odt, device=self.device)
        if M:
            stream = torch.cuda.current_stream(self.device).cuda_stream
            n = int(lib().pgmoe_linear_workspace_bytes(self._w, M, int(self.bias is not None), _OUT[odt]))
            ws = self._ws.get(max(n, 1), stream)
            check(lib().pgmoe_linear_forward(self._w, None if self.bias is None else self.bias.data_ptr(),
                                             xh.data_ptr(), M, out.data_ptr(), _OUT[odt], ws.data_ptr(), ws.numel(),
                                             stream), "pgmoe_linear_forward")
        if odt != x.dtype:
            out = out.to(x.dtype)
        return out.reshape(*orig_shape[:-1], self.out_features)

    def embed_lookup(self, token_ids: torch.Tensor, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """The rows of the given ids, dequantised (quant_kernels.py:1839): the embedding
        table lookup that lets one quantised buffer serve token_embd and a tied lm_head.

        Ids given on the host are range-checked there (IndexError, as the reference's
        index_select raises).  Ids already on the device are not read back: that would
        synchronise the stream every decode step and cannot run under graph capture (the
        reference captures this lookup in its decode graphs, model.py:1803, :2039); an id
        outside [0, N) gives a row of NaN instead."""
        if token_ids.device.type == "cpu" and token_ids.numel():
            ids_host = token_ids.reshape(-1)
            if bool(((ids_host < 0) | (ids_host >= self.out_features)).any()):
                raise IndexError(f"token id out of range [0, {self.out_features})")
        flat = token_ids.reshape(-1).to(self.device)
        K = self.in_features
        if self.mode == "fp16":
            rows = self.weight.index_select(0, flat.long()).to(dtype)
            return rows.reshape(*token_ids.shape, K)
        ids = flat.to(torch.int32).contiguous()
        odt = dtype if dtype in _OUT else torch.float32
        out = torch.empty((ids.numel(), self.cols), dtype=odt, device=self.device)
        if ids.numel():
            check(lib().pgmoe_dequant_rows(self._w, ids.data_ptr(), ids.numel(), out.data_ptr(), _OUT[odt],
                                           torch.cuda.current_stream(self.device).cuda_stream),
                  "pgmoe_dequant_rows")
        if self.cols != K:
            out = out[:, :K]
        return out.to(dtype).reshape(*token_ids.shape, K)


class FusedLinearPack(nn.Module):
    """Sibling projections sharing one input, fused into as few launches as their formats
    allow (quant_kernels.py:1867-1915): members are grouped by (mode, ggml type) in first-seen
    order and each group is one GGUFQuantLinear.fuse'd module."""

    def __init__(self, linears: Sequence[GGUFQuantLinear]) -> None:
        super().__init__()
        self.num_outputs = len(linears)
        self.out_sizes = [lin.out_features for lin in linears]
        key_to_idx: Dict[Tuple[str, Optional[int]], List[int]] = {}
        for i, lin in enumerate(linears):
            key_to_idx.setdefault((lin.mode, lin.gguf_qtype), []).append(i)
        self.groups = nn.ModuleList()
        self.group_slots: List[Tuple[List[int], List[int]]] = []
        for idxs in key_to_idx.values():
            self.groups.append(GGUFQuantLinear.fuse([linears[i] for i in idxs]))
            self.group_slots.append((idxs, [linears[i].out_features for i in idxs]))
        self.is_single_contiguous = len(self.groups) == 1 and self.group_slots[0][0] == list(range(self.num_outputs))

    def forward_single_concat(self, x: torch.Tensor) -> torch.Tensor:
        """All outputs fused into one matrix (e.g. [gate | up]): its output, concatenated."""
        assert self.is_single_contiguous
        return self.groups[0](x)

    def forward(self, x: torch.Tensor) -> List[torch.Tensor]:
        if self.is_single_contiguous:
            cat = self.groups[0](x)
            return [cat] if self.num_outputs == 1 else list(torch.split(cat, self.out_sizes, dim=-1))
        results: List[Optional[torch.Tensor]] = [None] * self.num_outputs
        for grp, (idxs, sizes) in zip(self.groups, self.group_slots):
            out = grp(x)
            if len(idxs) == 1:
                results[idxs[0]] = out
            else:
                for i, part in zip(idxs, torch.split(out, sizes, dim=-1)):
                    results[i] = part
        return [r for r in results if r is not None]


HipQuantLinear = GGUFQuantLinear
