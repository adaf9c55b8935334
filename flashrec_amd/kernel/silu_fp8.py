"""Fused SiLU-and-mul -> per-token e4m3, signature of ``flashrec.kernel.silu_fp8``.

Reference: python/flashrec/kernel/silu_fp8.py:79-119.  Bit-for-bit the
reference's CPU composition ``per_token_quant_fp8(silu_and_mul(x))``
(bf16 rounding after ``silu`` and after the product), in one pass that reads
each input row once (the reference's Triton kernel reads it twice).
"""

from __future__ import annotations

import torch

from flashrec_amd._lib import DTYPE_CODE, call, require_device, stream_of
from flashrec_amd.kernel.sglops import _ACT

_FP8_MAX = 448.0


@torch.compiler.disable
def silu_and_mul_per_token_quant_fp8(
    x: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``silu(x[..., :d]) * x[..., d:]`` then per-token e4m3. ``d = last_dim // 2``."""
    if x.dtype not in _ACT:
        raise TypeError(f"silu_and_mul_per_token_quant_fp8 takes bf16, fp16 or fp32, got {x.dtype}")
    require_device(x)
    last = int(x.shape[-1])
    if last % 2 != 0:
        raise ValueError("silu_and_mul_per_token_quant_fp8 needs an even last dimension")
    d = last // 2
    x2 = x.reshape(-1, last).contiguous()
    rows = int(x2.shape[0])
    y = torch.empty((rows, d), dtype=torch.float8_e4m3fn, device=x2.device)
    scale = torch.empty((rows, 1), dtype=torch.float32, device=x2.device)
    call("fr_silu_quant_fp8", x2.data_ptr(), DTYPE_CODE[x.dtype], x2.stride(0), rows, d, y.data_ptr(),
         scale.data_ptr(), stream_of(x))
    return y, scale
