"""W8A8 linear layer: a drop-in for ``flashrec.layers.linear`` on the fp8 path.

Interface kept from python/flashrec/layers/linear.py (what FlashRec's model
code and tests read):

* ``quantize_weight_fp8(w) -> (codes [N, K] e4m3, scale [N] fp32)`` (:26-32);
* ``as_channel_scale(scale, out_features, device=None)`` (:35-57): one value
  is broadcast to every output channel, ``out_features`` values are taken as
  they are, anything else (block-wise scales) is a ``ValueError``;
* ``Linear(in_features, out_features, bias=False)`` with ``load(weight, bias,
  quantize_fp8, weight_scale)``, ``forward(x)`` and ``forward_fp8(q, a_scale,
  orig_shape, out_dtype)`` (:66-151), and the attributes ``_use_fp8``,
  ``_fp8_weight`` (the ``[K, N]`` column-major view of the ``[N, K]`` codes)
  and ``_fp8_scale`` (``[N]`` fp32).

Layout here: the codes and their scales are registered buffers
(``w_codes`` ``[N, K]`` row-major, ``w_scale`` ``[N]``), so ``module.to()``
moves them with the module (a float cast of the module leaves them as they
are); ``_fp8_weight`` / ``_fp8_scale`` are views of them.  A call runs on the
HIP library only: per-token e4m3 quantisation of the activations, then the
W8A8 GEMM with both scales and the optional bias applied in its epilogue.
Beside the codes the layer keeps them once more in the prearranged GEMM's
layout (MFMA fragment order, built when the codes reach the GPU, about the
codes' size again): every bias-free call runs that kernel, which gives the
same bits as ``fp8_scaled_mm`` on the codes.

Behaviour that differs from the reference on purpose: a failing fp8 GEMM
raises instead of being retried as a dequantised bf16 ``F.linear``
(:124-131); a bias whose length is not ``out_features`` is refused at load.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from flashrec_amd._lib import DTYPE_CODE, call, require_device, stream_of
from flashrec_amd.kernel.sglops import (PrearrangedFp8Weight, fp8_scaled_mm, fp8_scaled_mm_prearranged,
                                        interleave_gate_up, per_token_quant_fp8, prearrange_fp8_weight)

_E4M3 = torch.float8_e4m3fn
_FP8_DTYPES = frozenset({torch.float8_e4m3fn, torch.float8_e5m2})
_HALF_DTYPES = (torch.bfloat16, torch.float16)


def quantize_weight_fp8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel absmax e4m3 codes of a ``[N, K]`` weight and their
    fp32 scales (amax / 448), in one HIP kernel (linear.py:26-32)."""
    require_device(weight)
    if weight.dim() != 2:
        raise ValueError(f"quantize_weight_fp8 takes a [N, K] matrix, got shape {tuple(weight.shape)}")
    if weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"quantize_weight_fp8 takes bf16/fp16/fp32, got {weight.dtype}")
    src = weight.contiguous() if weight.stride(-1) != 1 else weight
    rows, cols = src.shape
    codes = torch.empty((rows, cols), dtype=_E4M3, device=src.device)
    scale = torch.empty((rows,), dtype=torch.float32, device=src.device)
    row_stride = src.stride(0) if rows > 1 else cols
    call("fr_quantize_weight_fp8", src.data_ptr(), DTYPE_CODE[src.dtype], rows, cols, row_stride,
         codes.data_ptr(), scale.data_ptr(), stream_of(src))
    return codes, scale


def as_channel_scale(scale: torch.Tensor, out_features: int,
                     device: Optional[torch.device] = None) -> torch.Tensor:
    """A checkpoint's ``weight_scale`` as ``[out_features]`` fp32 (linear.py:35-57).

    Fused projections concatenate per-matrix scalars, so callers expand each
    source matrix's scale before concatenating (see ``flashrec_amd.weight``).
    """
    flat = scale.detach().reshape(-1).to(device=device, dtype=torch.float32)
    count = flat.numel()
    if count == out_features:
        return flat.contiguous()
    if count == 1:
        return flat.repeat(out_features)
    raise ValueError(
        f"weight_scale holds {count} values for a layer of {out_features} output channels: "
        "only a per-tensor (1) or per-channel scale is supported, not block-wise scales")


class Linear(nn.Module):
    """``y = x W^T (+ b)``, with ``W`` held as per-channel e4m3 codes when
    loaded from an fp8 checkpoint or with ``quantize_fp8=True``, otherwise as
    a plain ``weight`` parameter (the reference's unquantised layers)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.weight = nn.Parameter(torch.empty(0), requires_grad=False)
        self.bias = nn.Parameter(torch.empty(self.out_features), requires_grad=False) if bias else None
        self.register_buffer("w_codes", None)
        self.register_buffer("w_scale", None)

    # --- the attributes FlashRec's callers read ---------------------------------
    @property
    def _use_fp8(self) -> bool:
        return self.w_codes is not None

    @property
    def _fp8_weight(self) -> Optional[torch.Tensor]:
        """``[K, N]`` column-major view of the ``[N, K]`` codes."""
        return None if self.w_codes is None else self.w_codes.t()

    @property
    def _fp8_scale(self) -> Optional[torch.Tensor]:
        return self.w_scale

    def _prearranged(self) -> PrearrangedFp8Weight:
        """The codes in the prearranged GEMM's layout, built when first needed
        on the codes' device (and kept until the weights change or move)."""
        cached = self.__dict__.get("_pre")
        if cached is None or cached.data.device != self.w_codes.device:
            cached = prearrange_fp8_weight(self.w_codes.t())
            self.__dict__["_pre"] = cached
        return cached

    def _glu_operands(self):
        """The prearranged codes and the scales with gate/up rows interleaved
        for ``forward_fp8_silu`` (the interleaved codes themselves are not
        kept), built on first use."""
        cached = self.__dict__.get("_glu")
        if cached is None or cached[0].data.device != self.w_codes.device:
            cached = (prearrange_fp8_weight(interleave_gate_up(self.w_codes).t()), interleave_gate_up(self.w_scale))
            self.__dict__["_glu"] = cached
        return cached

    def prepare(self) -> None:
        """Build the prearranged weights now (eagerly, e.g. before a HIP graph
        is captured), for the plain and, for gate_up projections, the
        SiLU-and-mul forms."""
        if self.w_codes is not None and self.w_codes.is_cuda:
            self._prearranged()

    def _apply(self, fn, recurse=True):
        # Module.to() / .cuda() / .half() move the codes and scales to the new
        # device but never cast them: a float cast would destroy the e4m3 codes
        codes, scale = self.w_codes, self.w_scale
        self.w_codes = self.w_scale = None
        try:
            super()._apply(fn, recurse)
        finally:
            if codes is not None:
                dev = fn(torch.empty(0, device=codes.device)).device
                self.w_codes = codes.to(device=dev)
                self.w_scale = scale.to(device=dev)
        return self

    # --- loading ---------------------------------------------------------------
    def load(self, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
             quantize_fp8: bool = False, weight_scale: Optional[torch.Tensor] = None) -> None:
        """Take a ``[N, K]`` weight: fp8 codes (+ optional per-tensor or
        per-channel ``weight_scale``, default 1), or bf16/fp16/fp32 that is
        quantised here when ``quantize_fp8`` is set and kept as is otherwise
        (linear.py:81-116)."""
        if weight.dim() == 2 and weight.shape[0] != self.out_features:
            raise ValueError(f"weight has {weight.shape[0]} rows, layer has {self.out_features} outputs")
        if weight.dtype == torch.uint8 and weight_scale is not None:
            # packed 4-bit weights with block scales: a format this path does
            # not take (the reference refuses online conversion to it as well)
            raise NotImplementedError("packed uint8 weights with block scales (NVFP4) are not supported "
                                      "by the fp8 linear; load an fp8 or bf16 checkpoint")
        if weight.dtype in _FP8_DTYPES:
            if weight_scale is None:
                scale = torch.ones(self.out_features, dtype=torch.float32, device=weight.device)
            else:
                scale = as_channel_scale(weight_scale, self.out_features, weight.device)
            self._set_codes(weight, scale)
        elif quantize_fp8:
            self._set_codes(*quantize_weight_fp8(weight))
        else:
            self.weight = nn.Parameter(weight, requires_grad=False)
            self.w_codes = None
            self.w_scale = None
        if bias is not None:
            if bias.numel() != self.out_features:
                raise ValueError(f"bias has {bias.numel()} values, layer has {self.out_features} outputs")
            self.bias = nn.Parameter(bias.reshape(self.out_features), requires_grad=False)

    def _set_codes(self, codes: torch.Tensor, scale: torch.Tensor) -> None:
        # ``codes`` is the [N, K] matrix (a transposed [K, N] view stays a view)
        self.__dict__.pop("_glu", None)
        self.__dict__.pop("_pre", None)
        self.w_codes = codes
        self.w_scale = scale.to(device=codes.device, dtype=torch.float32).reshape(self.out_features)
        self.weight = nn.Parameter(torch.empty(0, device=codes.device), requires_grad=False)

    # --- calls -----------------------------------------------------------------
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.w_codes is None:
            return F.linear(x, self.weight.to(dtype=x.dtype), self.bias)
        rows = x.reshape(-1, x.shape[-1])
        if not rows.is_contiguous():
            rows = rows.contiguous()
        codes, scale = per_token_quant_fp8(rows)
        out_dtype = x.dtype if x.dtype in _HALF_DTYPES else torch.bfloat16
        return self.forward_fp8(codes, scale, tuple(x.shape), out_dtype)

    def forward_fp8(self, q: torch.Tensor, a_scale: torch.Tensor, orig_shape: tuple,
                    out_dtype: torch.dtype) -> torch.Tensor:
        """GEMM of already quantised ``[M, K]`` e4m3 rows with their ``[M, 1]``
        scales; the result has shape ``orig_shape[:-1] + (out_features,)``
        (linear.py:134-142, 153-172)."""
        if self.w_codes is None:
            raise RuntimeError("Linear.forward_fp8 needs fp8 weights (load an fp8 checkpoint "
                               "or pass quantize_fp8=True)")
        if self.w_codes.device != q.device:
            raise ValueError(f"activations on {q.device}, fp8 weights on {self.w_codes.device}: "
                             "move the module with .to() first")
        if self.bias is None:
            out = fp8_scaled_mm_prearranged(q, self._prearranged(), a_scale, self.w_scale, out_dtype)
        else:
            out = fp8_scaled_mm(q, self.w_codes.t(), a_scale, self.w_scale, out_dtype,
                                self.bias.to(dtype=out_dtype))
        return out.view(*tuple(orig_shape)[:-1], self.out_features)

    def forward_fp8_residual(self, q: torch.Tensor, a_scale: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """``residual += forward_fp8(q, a_scale, ...)`` with the add in the GEMM's
        epilogue (the product rounded to the residual's dtype, then the sum,
        as a separate add would round them); ``residual`` ``[M, out_features]``
        is updated in place and returned.  No bias (the layers this serves
        have none)."""
        if self.w_codes is None:
            raise RuntimeError("Linear.forward_fp8_residual needs fp8 weights")
        if self.bias is not None:
            raise ValueError("forward_fp8_residual takes a Linear without bias")
        if self.w_codes.device != q.device:
            raise ValueError(f"activations on {q.device}, fp8 weights on {self.w_codes.device}: "
                             "move the module with .to() first")
        return fp8_scaled_mm_prearranged(q, self._prearranged(), a_scale, self.w_scale, residual=residual)

    def forward_fp8_silu(self, q: torch.Tensor, a_scale: torch.Tensor, out: Optional[torch.Tensor] = None
                         ) -> torch.Tensor:
        """``silu_and_mul(forward_fp8(q, a_scale, ..., bf16))`` for a gate_up
        projection (gate rows, then up rows) with SiLU-and-mul in the GEMM's
        epilogue: ``[M, out_features / 2]`` bf16, bit-for-bit the two steps
        (qwen3.py:144-172 up to the per-token quant).  No bias."""
        if self.w_codes is None:
            raise RuntimeError("Linear.forward_fp8_silu needs fp8 weights")
        if self.bias is not None:
            raise ValueError("forward_fp8_silu takes a Linear without bias")
        if self.w_codes.device != q.device:
            raise ValueError(f"activations on {q.device}, fp8 weights on {self.w_codes.device}: "
                             "move the module with .to() first")
        pre, scale = self._glu_operands()
        return fp8_scaled_mm_prearranged(q, pre, a_scale, scale, out=out, silu=True)
