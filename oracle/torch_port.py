"""Torch-CPU restatement of the reference MoE block's CPU execution path.

TEST INFRASTRUCTURE ONLY (the timed ``cpu_baseline`` of bench.py and a second checker).
It reproduces what ``GGUFSparseMoEMLP.forward`` does when every ``exec_*`` helper takes
its PyTorch CPU branch:

* load-time repack of GGUF blocks into the reference's W4 / W8 structure-of-arrays
  (quant_kernels.py:854-904 for Q4_0 / Q4_1 / Q4_K -> W4, :945-1004 for Q8_0 / Q6_K / Q5_K
  -> W8), with the fp16 rounding of sub-block scale products;
* W4 / W8 matmul as chunked fp32 dequant (4096 rows) + fp32 ``F.linear``, result cast to
  the input dtype (quant_kernels.py:1276-1291, :1408-1420);
* SwiGLU (GeGLU for gemma) + dynamic row-scale with fp16 ``down_in`` (quant_kernels.py:1467-1475);
* the per-expert loop in ascending expert id with ``index_add_`` (model.py:898-937).

``faithful=True`` keeps the reference's fp16 casts (variant A: overflows to inf at
benchmark scale, exactly like the reference).  ``faithful=False`` keeps fp32 intermediates
and skips the fp16 casts (variant B).
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

from . import OracleLayer, Q4_0, Q4_1, Q4_K, Q5_K, Q6_K, Q8_0

W4_TYPES = (Q4_0, Q4_1, Q4_K)  # the reference's 4-bit repack (SUB_5BIT_W4_QTYPES)


def _k_scales(s12: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """6-bit (scale, min) pairs of K-quant headers: [n, 12] uint8 -> two [n, 8] arrays."""
    lo4 = s12[:, 0:4].astype(np.uint16)
    mid4 = s12[:, 4:8].astype(np.uint16)
    hi4 = s12[:, 8:12].astype(np.uint16)
    sc = np.concatenate([lo4 & 63, (hi4 & 15) | ((lo4 >> 2) & 48)], axis=1)
    mn = np.concatenate([mid4 & 63, (hi4 >> 4) | ((mid4 >> 2) & 48)], axis=1)
    return sc.astype(np.float32), mn.astype(np.float32)


def repack_w4(raw: np.ndarray, qtype: int, rows: int, cols: int):
    """Q4_0 / Q4_1 / Q4_K blocks -> (qweight u8 [rows, cols/2], scales f16 [rows, cols/32],
    zeros f16); byte i of a 32-weight group holds weight i (low nibble) and 16 + i (high)."""
    if qtype in (Q4_0, Q4_1):  # quant_kernels.py:864-875: scale d, zero 8d (Q4_0) / -m (Q4_1)
        bb = 18 if qtype == Q4_0 else 20
        blk = raw.reshape(-1, bb)
        d = blk[:, 0:2].copy().view(np.float16).reshape(rows, cols // 32)
        if qtype == Q4_0:
            z = (d.astype(np.float32) * 8.0).astype(np.float16)
        else:
            z = (-blk[:, 2:4].copy().view(np.float16).astype(np.float32)).astype(np.float16).reshape(rows, cols // 32)
        packed = np.ascontiguousarray(blk[:, bb - 16:bb]).reshape(rows, cols // 2)
        return torch.from_numpy(packed), torch.from_numpy(np.ascontiguousarray(d)), torch.from_numpy(z)
    if qtype != Q4_K:
        raise ValueError("W4 repack restated for Q4_0 / Q4_1 / Q4_K only")
    blk = raw.reshape(-1, 144)
    nb = blk.shape[0]
    d = blk[:, 0:4].copy().view(np.float16).astype(np.float32)  # [nb, 2] = (d, dmin)
    sc, mn = _k_scales(blk[:, 4:16])
    scales = (d[:, 0:1] * sc).astype(np.float16).reshape(rows, cols // 32)
    zeros = (d[:, 1:2] * mn).astype(np.float16).reshape(rows, cols // 32)
    qs = blk[:, 16:144].reshape(nb, 4, 32)
    nib = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32)  # sub-block 2c+hi
    packed = (nib[:, :, :16] | (nib[:, :, 16:] << 4)).astype(np.uint8).reshape(rows, cols // 2)
    return torch.from_numpy(packed), torch.from_numpy(scales), torch.from_numpy(zeros)


def repack_w8(raw: np.ndarray, qtype: int, rows: int, cols: int):
    """Q8_0 / Q6_K / Q5_K blocks -> (qweight i8 [rows, cols], scales f16 [rows, cols/16],
    zeros f16 [rows, cols/16] or None)."""
    zeros = None
    if qtype == Q8_0:
        blk = raw.reshape(-1, 34)
        d = blk[:, 0:2].copy().view(np.float16)  # [nb, 1]
        scales = np.repeat(d, 2, axis=1).reshape(rows, cols // 16)
        q = blk[:, 2:34].copy().view(np.int8).reshape(rows, cols)
    elif qtype == Q6_K:
        blk = raw.reshape(-1, 210)
        nb = blk.shape[0]
        ql = blk[:, 0:128].reshape(nb, 2, 64)
        qh = blk[:, 128:192].reshape(nb, 2, 32)
        lo = np.stack([ql & 15, ql >> 4], axis=2)  # [nb, h, 2, 64] -> element 128h + 64*sh + j
        hi = np.stack([(qh >> (2 * s)) & 3 for s in range(4)], axis=2)  # [nb, h, 4, 32]
        q = (lo.reshape(nb, 256).astype(np.int16) | (hi.reshape(nb, 256).astype(np.int16) << 4)) - 32
        q = q.astype(np.int8).reshape(rows, cols)
        sc = blk[:, 192:208].copy().view(np.int8).astype(np.float32)
        d = blk[:, 208:210].copy().view(np.float16).astype(np.float32)
        scales = (d * sc).astype(np.float16).reshape(rows, cols // 16)
    elif qtype == Q5_K:  # quant_kernels.py:984-1004: 5-bit codes 0..31, scale and zero per 32
        blk = raw.reshape(-1, 176)
        nb = blk.shape[0]
        d = blk[:, 0:4].copy().view(np.float16).astype(np.float32)  # [nb, 2] = (d, dmin)
        sc, mn = _k_scales(blk[:, 4:16])
        qh = blk[:, 16:48].reshape(nb, 1, 32)
        qs = blk[:, 48:176].reshape(nb, 4, 32)
        lo = np.stack([qs & 15, qs >> 4], axis=2).reshape(nb, 8, 32)  # sub-block 2c + nibble
        hi = (qh >> np.arange(8, dtype=np.uint8).reshape(1, 8, 1)) & 1  # sub-block s: bit s
        q = (lo | (hi << 4)).astype(np.int8).reshape(rows, cols)
        scales = np.repeat((d[:, 0:1] * sc).astype(np.float16), 2, axis=1).reshape(rows, cols // 16)
        zeros = np.repeat((d[:, 1:2] * mn).astype(np.float16), 2, axis=1).reshape(rows, cols // 16)
        zeros = torch.from_numpy(np.ascontiguousarray(zeros))
    else:
        raise ValueError("W8 repack restated for Q8_0 / Q6_K / Q5_K only")
    return torch.from_numpy(np.ascontiguousarray(q)), torch.from_numpy(np.ascontiguousarray(scales)), zeros


def w4_matmul(x: torch.Tensor, qw: torch.Tensor, sc: torch.Tensor, zr: torch.Tensor) -> torch.Tensor:
    M, K = x.shape
    N = qw.shape[0]
    xf = x.float()
    out = torch.empty((M, N), dtype=x.dtype)
    for r0 in range(0, N, 4096):
        r1 = min(N, r0 + 4096)
        p = qw[r0:r1].view(r1 - r0, K // 32, 16)
        q = torch.cat([(p & 15).float(), ((p >> 4) & 15).float()], dim=-1)
        w = (q * sc[r0:r1].float().unsqueeze(-1) - zr[r0:r1].float().unsqueeze(-1)).reshape(r1 - r0, K)
        out[:, r0:r1] = F.linear(xf, w).to(x.dtype)
    return out


def w8_matmul(x: torch.Tensor, qw: torch.Tensor, sc: torch.Tensor, zr: Optional[torch.Tensor] = None) -> torch.Tensor:
    M, K = x.shape
    N = qw.shape[0]
    xf = x.float()
    out = torch.empty((M, N), dtype=x.dtype)
    for r0 in range(0, N, 4096):
        r1 = min(N, r0 + 4096)
        w = qw[r0:r1].float().view(r1 - r0, K // 16, 16) * sc[r0:r1].float().unsqueeze(-1)
        if zr is not None:
            w = w - zr[r0:r1].float().unsqueeze(-1)
        out[:, r0:r1] = F.linear(xf, w.reshape(r1 - r0, K)).to(x.dtype)
    return out


def act_rowscale(g: torch.Tensor, u: torch.Tensor, faithful: bool, use_gelu: bool = False):
    act = F.gelu(g.float(), approximate="tanh") if use_gelu else F.silu(g.float())
    inter = act * u.float()
    rs = (inter.abs().amax(dim=-1, keepdim=True) / 16384.0).clamp(min=1.0)
    down_in = inter / rs
    if faithful:
        down_in = down_in.to(torch.float16)
    return down_in, rs


class _Proj:
    """One repacked projection (all experts, or a single shared matrix)."""

    def __init__(self, t: tuple, n_mats: int):
        qtype, n, k, raw = t
        self.qtype, self.n, self.k = qtype, n, k
        rows = n * n_mats
        if qtype in W4_TYPES:
            qw, sc, zr = repack_w4(raw, qtype, rows, k)
            self.w = (qw.view(n_mats, n, k // 2), sc.view(n_mats, n, k // 32), zr.view(n_mats, n, k // 32))
        else:
            qw, sc, zr = repack_w8(raw, qtype, rows, k)
            self.w = (qw.view(n_mats, n, k), sc.view(n_mats, n, k // 16),
                      None if zr is None else zr.view(n_mats, n, k // 16))

    def __call__(self, mat: int, x: torch.Tensor) -> torch.Tensor:
        if self.qtype in W4_TYPES:
            return w4_matmul(x, self.w[0][mat], self.w[1][mat], self.w[2][mat])
        return w8_matmul(x, self.w[0][mat], self.w[1][mat], None if self.w[2] is None else self.w[2][mat])


class PortMoE:
    """CPU restatement of GGUFSparseMoEMLP.forward (model.py:898-937)."""

    def __init__(self, layer: OracleLayer):
        self.L = layer
        E = layer.n_experts
        self.router = torch.from_numpy(layer.router_w)
        self.bias = None if layer.router_bias is None else torch.from_numpy(layer.router_bias)
        self.gate, self.up, self.down = _Proj(layer.gate, E), _Proj(layer.up, E), _Proj(layer.down, E)
        self.shared = None
        if layer.sh_gate is not None:
            self.shared = (_Proj(layer.sh_gate, 1), _Proj(layer.sh_up, 1), _Proj(layer.sh_down, 1))
        self.sh_inp = None if layer.sh_inp_gate is None else torch.from_numpy(layer.sh_inp_gate).view(1, -1)

    def forward(self, x: torch.Tensor, faithful: bool = True) -> torch.Tensor:
        L = self.L
        x2 = x.reshape(-1, x.shape[-1])
        xe_dtype = x2.dtype if faithful else torch.float32
        logits = F.linear(x2.float(), self.router)
        if self.bias is not None:
            logits = logits + self.bias
        probs = F.softmax(logits, dim=-1, dtype=torch.float32)
        tw, ti = torch.topk(probs, k=L.top_k, dim=-1)
        if L.norm_topk:
            tw = tw / tw.sum(dim=-1, keepdim=True).clamp(min=1e-20)
        out = torch.zeros_like(x2, dtype=torch.float32)
        for e in ti.unique().tolist():
            tok, slot = torch.where(ti == e)
            xe = x2.index_select(0, tok).to(xe_dtype)
            g = self.gate(e, xe)
            u = self.up(e, xe)
            din, rs = act_rowscale(g, u, faithful, bool(L.act))
            d = self.down(e, din.to(xe_dtype)).float() * rs
            out.index_add_(0, tok, d * tw[tok, slot].unsqueeze(-1))
        if self.shared is not None:
            sg, su, sd = self.shared
            xs = x2.to(xe_dtype)
            din, rs = act_rowscale(sg(0, xs), su(0, xs), faithful, bool(L.act))
            so = sd(0, din.to(xe_dtype)).float() * rs
            if self.sh_inp is not None:
                so = so * torch.sigmoid(F.linear(x2.float(), self.sh_inp))
            out = out + so
        return out.reshape(x.shape)

    def routing(self, x: torch.Tensor):
        logits = F.linear(x.reshape(-1, x.shape[-1]).float(), self.router)
        if self.bias is not None:
            logits = logits + self.bias
        return logits


def dense_weights(t: tuple, mat: int = 0, n_mats: Optional[int] = None) -> np.ndarray:
    """fp32 dense weights of one matrix as the W4/W8 repack defines them (q*s - z)."""
    p = _Proj(t, n_mats if n_mats is not None else 1)
    if p.qtype in W4_TYPES:
        qw, sc, zr = (a[mat] for a in p.w)
        n, k = p.n, p.k
        pk = qw.view(n, k // 32, 16)
        q = torch.cat([(pk & 15).float(), ((pk >> 4) & 15).float()], dim=-1)
        return (q * sc.float().unsqueeze(-1) - zr.float().unsqueeze(-1)).reshape(n, k).numpy()
    qw, sc = p.w[0][mat], p.w[1][mat]
    w = qw.float().view(p.n, p.k // 16, 16) * sc.float().unsqueeze(-1)
    if p.w[2] is not None:
        w = w - p.w[2][mat].float().unsqueeze(-1)
    return w.reshape(p.n, p.k).numpy()
