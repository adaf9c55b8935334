"""Fused (residual add +) RMSNorm -> per-token e4m3, signatures of ``flashrec.kernel.rms_fp8``.

Reference: python/flashrec/kernel/rms_fp8.py:74-145.  The reference's CUDA
path is a Triton kernel that quantizes the fp32 normalised value; its CPU
path rounds the normalised row to the activation dtype (bf16 or fp16; fp32 rows
are not rounded) first (``rmsnorm`` then
``per_token_quant_fp8``, rms_fp8.py:128-130 / :141-145).  This kernel
reproduces the latter bit for bit, in one pass over HBM.
"""

from __future__ import annotations

from typing import Optional

import torch

from flashrec_amd._lib import DTYPE_CODE, call, require_device, stream_of
from flashrec_amd.kernel.sglops import _ACT

_FP8_MAX = 448.0


def _launch(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    residual: Optional[torch.Tensor],
) -> tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    if x.dtype not in _ACT or (residual is not None and residual.dtype != x.dtype):
        raise TypeError("rms_fp8 takes bf16, fp16 or fp32 activations (and a residual of the same dtype)")
    require_device(x, residual)
    orig = x.shape
    hidden = int(weight.numel())
    x2 = x.reshape(-1, hidden).contiguous()
    # the norm weight in the activations' dtype, as the reference's fused
    # path passes it (rms_fp8.py:86)
    w = weight.reshape(-1).to(device=x.device, dtype=x.dtype).contiguous()
    rows = int(x2.shape[0])
    r2 = None
    if residual is not None:
        r2 = residual.reshape(-1, hidden).contiguous()
        if r2.shape != x2.shape:
            raise ValueError(f"residual {tuple(residual.shape)} does not match x {tuple(orig)}")
    y = torch.empty(x2.shape, dtype=torch.float8_e4m3fn, device=x2.device)
    scale = torch.empty((rows, 1), dtype=torch.float32, device=x2.device)
    call("fr_rms_quant_fp8", x2.data_ptr(), DTYPE_CODE[x.dtype], x2.stride(0),
         None if r2 is None else r2.data_ptr(), 0 if r2 is None else r2.stride(0),
         w.data_ptr(), rows, hidden, float(eps), y.data_ptr(), scale.data_ptr(), stream_of(x))
    res_out = r2.reshape(residual.shape) if r2 is not None else None
    return y, scale, res_out


@torch.compiler.disable
def rmsnorm_per_token_quant_fp8(
    x: torch.Tensor, weight: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """RMSNorm(x)*weight -> (e4m3 [M,H], fp32 scale [M,1]) (rms_fp8.py:120-130)."""
    y, scale, _ = _launch(x, weight, eps, residual=None)
    return y, scale


@torch.compiler.disable
def fused_add_rmsnorm_per_token_quant_fp8(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``residual += x`` (bf16, in place), then RMSNorm -> e4m3 (rms_fp8.py:133-145)."""
    y, scale, res = _launch(x, weight, eps, residual=residual)
    return y, scale, res
