"""``RMSNorm`` module with the interface of ``flashrec.layers.norm.RMSNorm``
(python/flashrec/layers/norm.py:12-42): a ``weight`` parameter of ones, ``eps``
and ``hidden_size`` attributes, ``forward(x, residual=None)`` and
``quant_fp8(x, residual=None)``.

Both methods route to the HIP row kernels.  With a residual the add is
fused into the same pass and the residual stream is updated in place; the
``quant_fp8`` form writes e4m3 codes and a per-row fp32 scale instead of the
normalised rows, so the next linear reads one byte per element.
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch
import torch.nn as nn

from flashrec_amd.kernel.rms_fp8 import fused_add_rmsnorm_per_token_quant_fp8, rmsnorm_per_token_quant_fp8
from flashrec_amd.kernel.sglops import fused_add_rmsnorm, rmsnorm

_Pair = Tuple[torch.Tensor, torch.Tensor]
_Triple = Tuple[torch.Tensor, torch.Tensor, torch.Tensor]


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.hidden_size = int(hidden_size)
        self.eps = float(eps)
        self.weight = nn.Parameter(torch.ones(self.hidden_size), requires_grad=False)

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> Union[torch.Tensor, _Pair]:
        """Normalised rows in x's dtype; given a residual, ``(normalised,
        residual)`` after ``residual += x``."""
        if residual is not None:
            return fused_add_rmsnorm(x, residual, self.weight, self.eps)
        return rmsnorm(x, self.weight, self.eps)

    def quant_fp8(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None) -> Union[_Pair, _Triple]:
        """``(codes, scales)`` of the normalised rows as e4m3 with an
        ``[M, 1]`` fp32 scale; given a residual, ``(codes, scales, residual)``
        after ``residual += x``."""
        if residual is not None:
            return fused_add_rmsnorm_per_token_quant_fp8(x, residual, self.weight, self.eps)
        return rmsnorm_per_token_quant_fp8(x, self.weight, self.eps)
