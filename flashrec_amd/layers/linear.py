"""Linear with W8A8 per-channel fp8, mirroring ``flashrec.layers.linear``.

Reference: python/flashrec/layers/linear.py.  Same public names and weight
layout: the fp8 weight is kept as a ``[K, N]`` column-major view of the
``[N, K]`` e4m3 matrix (``_fp8_weight``) with a ``[N]`` fp32 scale
(``_fp8_scale``).  Quantisation, activation quant and the GEMM run in HIP.
Difference from the reference: ``forward`` does not catch fp8 GEMM errors
and silently dequantise to a bf16 ``F.linear`` (linear.py:124-131); a failing
kernel raises.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from flashrec_amd._lib import DTYPE_CODE, call, require_device, stream_of
from flashrec_amd.kernel.sglops import fp8_scaled_mm, per_token_quant_fp8

_FP8_MAX = 448.0


def _is_fp8(dtype: torch.dtype) -> bool:
    return dtype in (
        torch.float8_e4m3fn,
        getattr(torch, "float8_e5m2", torch.float8_e4m3fn),
    )


def quantize_weight_fp8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-channel absmax quantize to e4m3. Returns (fp8 [N,K], scale [N]) (linear.py:26-32)."""
    require_device(weight)
    if weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"quantize_weight_fp8 takes bf16/fp16/fp32, got {weight.dtype}")
    w = weight if weight.stride(-1) == 1 else weight.contiguous()
    n, k = int(w.shape[0]), int(w.shape[1])
    q = torch.empty((n, k), dtype=torch.float8_e4m3fn, device=w.device)
    s = torch.empty((n,), dtype=torch.float32, device=w.device)
    call("fr_quantize_weight_fp8", w.data_ptr(), DTYPE_CODE[w.dtype], n, k,
         w.stride(0) if n > 1 else k, q.data_ptr(), s.data_ptr(), stream_of(w))
    return q, s


def as_channel_scale(
    scale: torch.Tensor,
    out_features: int,
    device: torch.device | None = None,
) -> torch.Tensor:
    """Per-tensor scale -> length ``out_features``; per-channel unchanged (linear.py:35-57)."""
    s = scale.detach().to(dtype=torch.float32).reshape(-1)
    if device is not None:
        s = s.to(device=device)
    n = int(s.numel())
    if n == 1:
        return s.expand(out_features).contiguous()
    if n == out_features:
        return s.contiguous()
    raise ValueError(
        f"FP8 weight_scale has {n} values, expected 1 (per-tensor) or "
        f"{out_features} (per-channel); block-wise scales are not supported"
    )


def _channel_scale(scale: torch.Tensor, out_features: int, device: torch.device) -> torch.Tensor:
    return as_channel_scale(scale, out_features, device)


class Linear(nn.Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = nn.Parameter(torch.empty(0), requires_grad=False)
        self.bias = (
            nn.Parameter(torch.empty(out_features), requires_grad=False) if bias else None
        )
        self._fp8_weight: Optional[torch.Tensor] = None  # [K, N] column-major
        self._fp8_scale: Optional[torch.Tensor] = None  # [N]
        self._use_fp8 = False

    def load(
        self,
        weight: torch.Tensor,
        bias: torch.Tensor | None = None,
        quantize_fp8: bool = False,
        weight_scale: torch.Tensor | None = None,
    ):
        """Load bf16 / fp8 weights (linear.py:81-116)."""
        device = weight.device
        if weight.dtype == torch.uint8 and weight_scale is not None:
            raise NotImplementedError(
                "NVFP4 Linear needs an official NVFP4 checkpoint "
                "(packed uint8 + block scale); online FP8->NVFP4 is not supported"
            )
        if _is_fp8(weight.dtype):
            if weight_scale is None:
                scale = torch.ones(self.out_features, dtype=torch.float32, device=device)
            else:
                scale = _channel_scale(weight_scale, self.out_features, device)
            self._fp8_weight = weight.t()
            self._fp8_scale = scale
            self._use_fp8 = True
        elif quantize_fp8:
            q, scale = quantize_weight_fp8(weight)
            self._fp8_weight = q.t()
            self._fp8_scale = scale.to(device=device)
            self._use_fp8 = True
        else:
            self.weight = nn.Parameter(weight, requires_grad=False)
            self._use_fp8 = False
        if bias is not None:
            self.bias = nn.Parameter(bias, requires_grad=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._use_fp8 and self._fp8_weight is not None and self._fp8_scale is not None:
            return self._fp8_forward(x)
        return F.linear(x, self.weight.to(dtype=x.dtype), self.bias)

    def forward_fp8(
        self,
        q: torch.Tensor,
        a_scale: torch.Tensor,
        orig_shape: tuple,
        out_dtype: torch.dtype,
    ) -> torch.Tensor:
        """GEMM from a pre-quantized activation. ``q`` is [M, K] e4m3 (linear.py:134-142)."""
        return self._fp8_mm(q, a_scale, orig_shape, out_dtype)

    def _fp8_forward(self, x: torch.Tensor) -> torch.Tensor:
        orig = x.shape
        x2 = x.reshape(-1, orig[-1]).contiguous()
        q, a_scale = per_token_quant_fp8(x2)
        out_dtype = x.dtype if x.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
        return self._fp8_mm(q, a_scale, orig, out_dtype)

    def _fp8_mm(
        self,
        q: torch.Tensor,
        a_scale: torch.Tensor,
        orig_shape: tuple,
        out_dtype: torch.dtype,
    ) -> torch.Tensor:
        b = self._fp8_weight
        b_scale = self._fp8_scale
        assert b is not None and b_scale is not None
        device = q.device
        if b.device != device:
            b = b.to(device=device)
            self._fp8_weight = b
        if b_scale.device != device:
            b_scale = b_scale.to(device=device)
            self._fp8_scale = b_scale
        bias = self.bias.to(dtype=out_dtype) if self.bias is not None else None
        out = fp8_scaled_mm(q, b, a_scale, b_scale, out_dtype, bias)
        return out.view(*orig_shape[:-1], self.out_features)
