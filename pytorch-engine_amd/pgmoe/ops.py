"""Tensor-level wrappers of the C ABI stages (device tensors in, device tensors out).

Each function enqueues work on the current HIP stream of the tensors' device and returns
without synchronising.  They mirror the steps of GGUFSparseMoEMLP.forward
(pygguf_engine/model.py:898-937) and exist for tests and for callers that want to fuse
around individual stages; ``HipSparseMoEMLP`` uses the one-call ``pgmoe_moe_forward``.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from ._lib import (BF16, F16, F32, FLOAT_QTYPES, IQ4_NL, IQ4_XS, MXFP4, Q2_K, Q3_K, Q4_0, Q4_1, Q4_K, Q5_0, Q5_1,
                   Q5_K, Q6_K, Q8_0, REQUANT_W4_QTYPES, REQUANT_W8_QTYPES, Weights, check, lib)

# (weights, bytes) of a GGUF block; the float types as 256-weight runs of a row
GGUF_BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34), Q4_0: (32, 18),
              Q4_1: (32, 20), Q5_0: (32, 22), F16: (256, 512), BF16: (256, 512), F32: (256, 1024),
              Q2_K: (256, 84), Q3_K: (256, 110), IQ4_NL: (32, 18), IQ4_XS: (256, 136), MXFP4: (32, 17),
              Q5_1: (32, 24)}


def device_qtype(qtype: int) -> int:
    """Format of the device layout the relayout of GGUF `qtype` produces: Q4_0 becomes Q4_1
    (d * (q - 8) = d q + m with m = -8d), Q5_0 becomes Q8_0 (d * (q - 16) is the Q8_0 value
    d * qs with qs = q - 16), F32 and BF16 become F16 (rounded to fp16 on the host, as the
    reference's fp16 expert mode loads them), Q2_K / Q3_K / IQ4_NL / IQ4_XS / MXFP4 become
    Q4_1 (the reference's W4 re-quantisation, requant_w4), Q5_1 becomes F16 (the reference's
    W8 re-quantisation, requant_w8_f16), the others keep theirs."""
    if qtype == Q4_0 or qtype in REQUANT_W4_QTYPES:
        return Q4_1
    return Q8_0 if qtype == Q5_0 else F16 if qtype in FLOAT_QTYPES + REQUANT_W8_QTYPES else qtype


def requant_w4(qtype: int, raw: torch.Tensor, n_rows: int, cols: int) -> torch.Tensor:
    """Q2_K / Q3_K / IQ4_NL / IQ4_XS / MXFP4 GGUF bytes of an n_rows x cols matrix on the
    device -> the Q4_1 GGUF bytes (uint8 [n_rows * cols / 32 * 20]) of the reference's W4
    re-quantisation (repack_gguf_to_w4a16, quant_kernels.py:906-942; pgmoe_requant_w4)."""
    dev = _need_cuda(raw)
    per, bb = GGUF_BLOCK[qtype]
    if cols % per or raw.numel() != n_rows * (cols // per) * bb:
        raise ValueError("raw byte count does not match the tensor shape")
    dst = torch.empty(n_rows * (cols // 32) * 20, dtype=torch.uint8, device=dev)
    check(lib().pgmoe_requant_w4(qtype, raw.data_ptr(), n_rows, cols, dst.data_ptr(), _stream(dev)),
          "pgmoe_requant_w4")
    return dst


def requant_w8_f16(qtype: int, raw: torch.Tensor, n_rows: int, cols: int, cols_out: Optional[int] = None) -> torch.Tensor:
    """Q5_1 GGUF bytes of an n_rows x cols matrix on the device -> fp16 weights (uint8
    [n_rows * cols_out * 2], zero past cols) with the reference's W8 values: per 16 weights
    sc = max|w| / 127, codes round(w / sc) in -127..127, weight fp16(fp16(sc) * code)
    (repack_gguf_to_w8a16's fallback, quant_kernels.py:1005-1025; pgmoe_requant_w8_f16)."""
    dev = _need_cuda(raw)
    co = cols if cols_out is None else cols_out
    per, bb = GGUF_BLOCK[qtype]
    if cols % per or raw.numel() != n_rows * (cols // per) * bb:
        raise ValueError("raw byte count does not match the tensor shape")
    dst = torch.empty(n_rows * co * 2, dtype=torch.uint8, device=dev)
    check(lib().pgmoe_requant_w8_f16(qtype, raw.data_ptr(), n_rows, cols, co, dst.data_ptr(), _stream(dev)),
          "pgmoe_requant_w8_f16")
    return dst


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _need_cuda(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("pgmoe kernels take device tensors")
        if not t.is_contiguous():
            raise ValueError("pgmoe kernels take contiguous tensors")
        dev = t.device
    assert dev is not None
    return dev


def weight_stride(qtype: int, rows: int, cols: int) -> int:
    n = lib().pgmoe_weight_bytes(qtype, rows, cols)
    if n < 0:
        raise ValueError(f"qtype {qtype} with {cols} columns is not supported by the HIP kernels")
    return int(n)


def relayout(qtype: int, raw: torch.Tensor, n_mats: int, rows: int, cols: int,
             rows_out: Optional[int] = None, cols_out: Optional[int] = None) -> torch.Tensor:
    """GGUF bytes on the device -> pgmoe device layout (uint8 [n_mats * stride]) of format
    device_qtype(qtype), of [rows_out, cols_out] matrices (default [rows, cols]) whose extra
    rows and columns are exact zeros (pgmoe_relayout_weights_padded)."""
    dev = _need_cuda(raw)
    ro = rows if rows_out is None else rows_out
    co = cols if cols_out is None else cols_out
    if qtype in REQUANT_W4_QTYPES:  # first to the Q4_1 blocks of the reference's W4 values
        raw = requant_w4(qtype, raw, n_mats * rows, cols)
        qtype = Q4_1
    elif qtype in REQUANT_W8_QTYPES:  # first to fp16 weights of the reference's W8 values, already co wide
        raw = requant_w8_f16(qtype, raw, n_mats * rows, cols, co)
        qtype, cols = F16, co
    stride = weight_stride(qtype, ro, co)
    per, bb = GGUF_BLOCK[qtype]
    if raw.numel() != n_mats * rows * (cols // per) * bb:
        raise ValueError("raw byte count does not match the tensor shape")
    if raw.data_ptr() % 16:  # the kernels read 16-byte aligned sources
        raw = raw.clone()
    dst = torch.empty(n_mats * stride, dtype=torch.uint8, device=dev)
    if (ro, co) == (rows, cols):
        check(lib().pgmoe_relayout_weights(qtype, raw.data_ptr(), n_mats, rows, cols, dst.data_ptr(),
                                           _stream(dev)), "pgmoe_relayout_weights")
    else:
        check(lib().pgmoe_relayout_weights_padded(qtype, raw.data_ptr(), n_mats, rows, cols, ro, co, dst.data_ptr(),
                                                  _stream(dev)), "pgmoe_relayout_weights_padded")
    return dst


def padded_width(qtype: int, cols: int) -> int:
    """The device width of a GGUF matrix with `cols` input features: cols itself when it is a
    multiple of 256; for the 32-weight formats (Q8_0, Q5_0, Q5_1, Q4_0, Q4_1, IQ4_NL, MXFP4) any
    multiple of 32 is padded up to one of 256 with zero blocks; -1 when the kernels cannot
    take it."""
    if cols % 256 == 0:
        return cols
    per, _ = GGUF_BLOCK.get(qtype, (256, 0))
    if per == 32 and cols % 32 == 0:
        return (cols + 255) // 256 * 256
    return -1


def scale_plane(qtype: int, buf: torch.Tensor, n_mats: int, rows: int, cols: int) -> Optional[torch.Tensor]:
    """The fp32 scale plane the MFMA (prefill) products read, built on the device from the
    device layout `buf` (uint8 [n_mats * plane bytes]); None for Q8_0, which has none."""
    dev = _need_cuda(buf)
    n = int(lib().pgmoe_scale_plane_bytes(qtype, rows, cols))
    if n < 0:
        raise ValueError(f"qtype {qtype} with {cols} columns is not supported by the HIP kernels")
    if n == 0:
        return None
    dst = torch.empty(n_mats * n, dtype=torch.uint8, device=dev)
    check(lib().pgmoe_build_scale_plane(qtype, buf.data_ptr(), n_mats, rows, cols, weight_stride(qtype, rows, cols),
                                        dst.data_ptr(), _stream(dev)), "pgmoe_build_scale_plane")
    return dst


def make_weights(qtype: int, buf: torch.Tensor, n_mats: int, rows: int, cols: int,
                 plane: Optional[torch.Tensor] = None) -> Weights:
    return Weights(qtype, rows, cols, n_mats, buf.data_ptr(), weight_stride(qtype, rows, cols),
                   plane.data_ptr() if plane is not None else None)


def dequant_rows(w: Weights, rows: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Rows `rows` (int32 device tensor) of the one-matrix weights `w`, dequantised on the device
    (pgmoe_dequant_rows): [len(rows), K] fp32 or fp16."""
    dev = _need_cuda(rows)
    code = {torch.float32: 0, torch.float16: 1}[out_dtype]
    out = torch.empty((rows.numel(), w.n_cols), dtype=out_dtype, device=dev)
    if rows.numel():
        check(lib().pgmoe_dequant_rows(w, rows.data_ptr(), rows.numel(), out.data_ptr(), code, _stream(dev)),
              "pgmoe_dequant_rows")
    return out


def dequant_matrix(qtype: int, raw: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """A whole GGUF matrix (raw bytes on the device) dequantised to fp32 [rows, cols] on the
    device: relaid out, then every row decoded."""
    buf = relayout(qtype, raw, 1, rows, cols)
    w = make_weights(device_qtype(qtype), buf, 1, rows, cols)
    ids = torch.arange(rows, dtype=torch.int32, device=raw.device)
    return dequant_rows(w, ids)


def router_topk(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor], k: int, norm: bool
                ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    dev = _need_cuda(x, w, bias)
    M, H = x.shape
    E = w.shape[0]
    logits = torch.empty((M, E), dtype=torch.float32, device=dev)
    idx = torch.empty((M, k), dtype=torch.int32, device=dev)
    tw = torch.empty((M, k), dtype=torch.float32, device=dev)
    check(lib().pgmoe_router_topk(x.data_ptr(), w.data_ptr(), _ptr(bias), M, H, E, k, int(norm),
                                  logits.data_ptr(), idx.data_ptr(), tw.data_ptr(), _stream(dev)),
          "pgmoe_router_topk")
    return logits, idx, tw


def dispatch(idx: torch.Tensor, n_experts: int, tile_rows: int = 256, blocks: str = "one"):
    """pgmoe_dispatch (blocks="one") or pgmoe_dispatch_ws with its scratch (blocks="many")."""
    dev = _need_cuda(idx)
    M, K = idx.shape
    P = M * K
    i32 = dict(dtype=torch.int32, device=dev)
    offsets = torch.empty(n_experts + 1, **i32)
    perm = torch.empty(max(P, 1), **i32)
    inv = torch.empty(max(P, 1), **i32)
    active = torch.empty(n_experts, **i32)
    n_active = torch.empty(1, **i32)
    tile_off = torch.empty(n_experts + 1, **i32)
    if blocks == "many":
        nws = int(lib().pgmoe_dispatch_ws_bytes(M, K, n_experts))
        ws = torch.empty(max(nws, 4), dtype=torch.uint8, device=dev)
        check(lib().pgmoe_dispatch_ws(idx.data_ptr(), M, K, n_experts, tile_rows, offsets.data_ptr(),
                                      perm.data_ptr(), inv.data_ptr(), active.data_ptr(), n_active.data_ptr(),
                                      tile_off.data_ptr(), ws.data_ptr(), ws.numel(), _stream(dev)),
              "pgmoe_dispatch_ws")
    else:
        check(lib().pgmoe_dispatch(idx.data_ptr(), M, K, n_experts, tile_rows, offsets.data_ptr(), perm.data_ptr(),
                                   inv.data_ptr(), active.data_ptr(), n_active.data_ptr(), tile_off.data_ptr(),
                                   _stream(dev)), "pgmoe_dispatch")
    return offsets, perm[:P], inv[:P], active, n_active, tile_off


def expert_gateup(gate: Weights, up: Weights, x: torch.Tensor, top_k: int, disp, mode: int) -> torch.Tensor:
    dev = _need_cuda(x)
    offsets, perm, inv, active, n_active, tile_off = disp
    M = x.shape[0]
    inter = torch.empty((M * top_k, gate.n_rows), dtype=torch.float32, device=dev)
    check(lib().pgmoe_expert_gateup(gate, up, x.data_ptr(), M, top_k, offsets.data_ptr(), perm.data_ptr(),
                                    active.data_ptr(), n_active.data_ptr(), tile_off.data_ptr(), mode,
                                    inter.data_ptr(), _stream(dev)), "pgmoe_expert_gateup")
    return inter


def expert_down(down: Weights, inter: torch.Tensor, M: int, top_k: int, disp, topk_w: torch.Tensor, mode: int,
                rowscale: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> torch.Tensor:
    """Weighted down partials [P, N].  mode 1 (MFMA): the row-scaled fp16 input and its
    scales go to `rowscale` = (a16 [P, K] fp16, rs [P] fp32) when given (else to scratch)."""
    dev = _need_cuda(inter, topk_w)
    offsets, perm, inv, active, n_active, tile_off = disp
    P = M * top_k
    partial = torch.empty((P, down.n_rows), dtype=torch.float32, device=dev)
    a16 = rs = None
    if mode == 1:
        a16, rs = rowscale if rowscale is not None else (
            torch.empty((P, down.n_cols), dtype=torch.float16, device=dev),
            torch.empty(P, dtype=torch.float32, device=dev))
    check(lib().pgmoe_expert_down(down, inter.data_ptr(), M, top_k, offsets.data_ptr(), perm.data_ptr(),
                                  active.data_ptr(), n_active.data_ptr(), tile_off.data_ptr(), topk_w.data_ptr(),
                                  mode, _ptr(a16), _ptr(rs), partial.data_ptr(), _stream(dev)),
          "pgmoe_expert_down")
    return partial


def combine(partial: torch.Tensor, inv: torch.Tensor, M: int, top_k: int,
            shared: Optional[torch.Tensor] = None, shared_logit: Optional[torch.Tensor] = None) -> torch.Tensor:
    dev = _need_cuda(partial, inv, shared, shared_logit)
    H = partial.shape[1]
    out = torch.empty((M, H), dtype=torch.float32, device=dev)
    check(lib().pgmoe_combine(partial.data_ptr(), inv.data_ptr(), M, top_k, H, _ptr(shared), _ptr(shared_logit),
                              out.data_ptr(), _stream(dev)), "pgmoe_combine")
    return out
