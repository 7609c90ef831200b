"""Residual add + RMSNorm on the HIP kernel (pgmoe_add_rmsnorm).

Drop-ins for the reference's norm operators (pygguf_engine/quant_kernels.py:1510-1597) and
its norm module (model.py:58-74), same names, arguments and results:

    exec_fused_rmsnorm(x, norm_weight, eps=1e-6, out_dtype=None) -> normed
    exec_fused_add_rmsnorm(x, delta, norm_weight, eps=1e-6, out_dtype=torch.float16)
        -> (h = x.float() + delta.float(), normed = RMSNorm(h) * w in out_dtype)
    GGUFRMSNorm(weight, eps).forward(x, out_dtype) / .forward_with_residual(x, delta, out_dtype)

``forward_with_residual`` is the call at model.py:1037 whose fp16 output is the MoE
block's input.  The reference falls back to PyTorch for dtypes its Triton kernel does
not take; here there is no CPU path: inputs must be fp32 / fp16 / bf16 CUDA tensors and
the output fp32 or fp16, anything else raises.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from ._lib import check, lib

_DT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 30}
_OUT = (torch.float32, torch.float16)


def _run(x: torch.Tensor, delta: Optional[torch.Tensor], norm_weight: torch.Tensor, eps: float,
         out_dtype: torch.dtype, want_h: bool):
    if x.device.type != "cuda":
        raise ValueError("pgmoe RMSNorm runs on a HIP device tensor")
    if x.dtype not in _DT or (delta is not None and delta.dtype not in _DT):
        raise NotImplementedError(f"RMSNorm inputs of dtype {x.dtype} / {None if delta is None else delta.dtype}")
    if out_dtype not in _OUT:
        raise NotImplementedError(f"RMSNorm output dtype {out_dtype} (fp32 or fp16)")
    orig_shape = x.shape
    D = orig_shape[-1]
    R = x.numel() // D if D else 0
    if norm_weight.numel() != D:
        raise ValueError(f"norm weight has {norm_weight.numel()} elements, rows have {D}")
    x_c = x.reshape(R, D).contiguous()
    d_c = None
    if delta is not None:
        if delta.shape != x.shape:
            raise ValueError(f"delta shape {tuple(delta.shape)} != x shape {tuple(orig_shape)}")
        d_c = delta.to(x.device).reshape(R, D).contiguous()
    w = norm_weight.to(device=x.device, dtype=torch.float32).contiguous()
    out = torch.empty((R, D), dtype=out_dtype, device=x.device)
    h = torch.empty((R, D), dtype=torch.float32, device=x.device) if want_h else None
    stream = torch.cuda.current_stream(x.device).cuda_stream
    check(lib().pgmoe_add_rmsnorm(x_c.data_ptr(), _DT[x.dtype], None if d_c is None else d_c.data_ptr(),
                                  _DT[d_c.dtype] if d_c is not None else 0, w.data_ptr(), R, D, float(eps),
                                  None if h is None else h.data_ptr(), out.data_ptr(), _DT[out_dtype], stream),
          "pgmoe_add_rmsnorm")
    return (None if h is None else h.reshape(orig_shape)), out.reshape(orig_shape)


def exec_fused_rmsnorm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float = 1e-6,
                       out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """RMSNorm(x.float(), norm_weight, eps).to(out_dtype or x.dtype) (quant_kernels.py:1510)."""
    target = out_dtype if out_dtype is not None else x.dtype
    return _run(x, None, norm_weight, eps, target, False)[1]


def exec_fused_add_rmsnorm(x: torch.Tensor, delta: torch.Tensor, norm_weight: torch.Tensor, eps: float = 1e-6,
                           out_dtype: torch.dtype = torch.float16) -> Tuple[torch.Tensor, torch.Tensor]:
    """(h fp32, RMSNorm(h) in out_dtype) with h = x.float() + delta.float()
    (quant_kernels.py:1552)."""
    h, out = _run(x, delta, norm_weight, eps, out_dtype, True)
    return h, out


class GGUFRMSNorm(nn.Module):
    """The reference's norm module (model.py:58-74) on the HIP kernel."""

    def __init__(self, weight: torch.Tensor, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.dim = int(weight.shape[-1])
        self.register_buffer("weight", weight.to(torch.float32).contiguous(), persistent=False)

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return exec_fused_rmsnorm(x, self.weight, self.eps, out_dtype=out_dtype)

    def forward_with_residual(self, x: torch.Tensor, delta: torch.Tensor,
                              out_dtype: torch.dtype = torch.float16) -> Tuple[torch.Tensor, torch.Tensor]:
        return exec_fused_add_rmsnorm(x, delta, self.weight, self.eps, out_dtype=out_dtype)


HipRMSNorm = GGUFRMSNorm
