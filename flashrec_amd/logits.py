"""SID-restricted lm_head mirroring ``flashrec.logits.RestrictedLMHead``.

Reference: python/flashrec/logits.py:11-166.  Same API (``bind``,
``bind_codebook``, ``compute``, ``compute_level``, ``compute_into``).  With
``fp8=True`` (the north-star upgrade; the reference always runs a bf16
``F.linear``), ``bind`` quantises the restricted weight slice per output
channel once, and every call runs per-token e4m3 quant of the hidden rows,
the W8A8 GEMM with fp32 logits, and an in-place fp32 log_softmax -- three HIP
kernels, no host sync, graph-capturable.  With ``fp8=False`` it behaves like
the reference (bf16 ``F.linear`` + fp32 ``log_softmax``).
"""

from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn.functional as F

from flashrec_amd.kernel.sglops import fp8_scaled_mm, log_softmax_f32, per_token_quant_fp8
from flashrec_amd.layers.linear import quantize_weight_fp8


class RestrictedLMHead:
    def __init__(
        self,
        special_token_ids: Optional[List[int]],
        enabled: bool = True,
        fp8: bool = False,
    ):
        self.ids = list(special_token_ids) if special_token_ids else None
        self.enabled = bool(enabled and self.ids)
        self.fp8 = bool(fp8)
        self._token_ids: Optional[torch.Tensor] = None
        self._weight: Optional[torch.Tensor] = None
        self._q_weight: Optional[torch.Tensor] = None  # [K, N] column-major e4m3
        self._q_scale: Optional[torch.Tensor] = None  # [N] fp32
        self._level_weights: Optional[List[torch.Tensor]] = None
        self._level_token_ids: Optional[List[torch.Tensor]] = None
        self._level_offsets: Optional[List[int]] = None
        self._codebook_sizes: Optional[List[int]] = None

    @property
    def token_ids(self) -> Optional[torch.Tensor]:
        return self._token_ids

    @property
    def num_tokens(self) -> Optional[int]:
        if self._token_ids is None:
            return None
        return int(self._token_ids.numel())

    @property
    def ready(self) -> bool:
        return bool(self.enabled and self._weight is not None and self._token_ids is not None)

    @property
    def per_codebook_ready(self) -> bool:
        return bool(self._level_weights is not None and len(self._level_weights) > 0)

    @property
    def num_levels(self) -> int:
        return len(self._level_weights) if self._level_weights else 0

    @property
    def max_codebook_k(self) -> int:
        if not self._codebook_sizes:
            return 0
        return max(self._codebook_sizes)

    def codebook_k(self, level: int) -> int:
        if not self._codebook_sizes or level < 0 or level >= len(self._codebook_sizes):
            return 0
        return self._codebook_sizes[level]

    def bind(self, lm_weight: torch.Tensor) -> None:
        """Slice (and with fp8, quantise) the restricted rows once after weight load."""
        if lm_weight is None:
            return
        self._ensure(lm_weight.device, lm_weight)

    def bind_codebook(self, codebook_sizes: List[int]) -> None:
        """Per-level zero-copy views of the bound slice (logits.py:66-90)."""
        if self._weight is None or not self.enabled:
            return
        total = sum(codebook_sizes)
        if total != self._weight.shape[0]:
            return
        self._codebook_sizes = list(codebook_sizes)
        self._level_weights = []
        self._level_token_ids = []
        self._level_offsets = []
        offset = 0
        ids = self.ids or []
        device = self._weight.device
        for size in codebook_sizes:
            self._level_weights.append(self._weight.narrow(0, offset, size))
            self._level_token_ids.append(
                torch.tensor(ids[offset : offset + size], dtype=torch.long, device=device)
            )
            self._level_offsets.append(offset)
            offset += size

    def _ensure(self, device: torch.device, lm_weight: torch.Tensor) -> None:
        """logits.py:92-116, plus the one-time fp8 quantisation of the slice."""
        if not self.enabled:
            return
        if self._token_ids is None or self._token_ids.device != device:
            vocab = int(lm_weight.shape[0])
            ids = self.ids or []
            if (not ids) or min(ids) < 0 or max(ids) >= vocab:
                raise ValueError(f"sid_token_range out of range for vocab {vocab}")
            self._token_ids = torch.tensor(ids, dtype=torch.long, device=device)
            self._weight = None
        if self._weight is None or self._weight.device != device:
            ids = self.ids or []
            lo, hi = int(ids[0]), int(ids[-1])
            contiguous = (
                len(ids) > 1
                and hi - lo == len(ids) - 1
                and all(b - a == 1 for a, b in zip(ids, ids[1:]))
            )
            if contiguous:
                self._weight = lm_weight.narrow(0, lo, len(ids))
            else:
                self._weight = torch.index_select(lm_weight, 0, self._token_ids)
            if self.fp8:
                q, s = quantize_weight_fp8(self._weight)
                self._q_weight = q.t()
                self._q_scale = s

    def _fp8_logprobs(self, hidden: torch.Tensor, lo: int, n: int,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
        assert self._q_weight is not None and self._q_scale is not None
        qa, sa = per_token_quant_fp8(hidden)
        w = self._q_weight.narrow(1, lo, n)
        s = self._q_scale.narrow(0, lo, n)
        logits = fp8_scaled_mm(qa, w, sa, s, torch.float32)
        return log_softmax_f32(logits, out=logits if out is None else out)

    def _restricted_logprobs(self, hidden: torch.Tensor) -> torch.Tensor:
        if self.fp8:
            return self._fp8_logprobs(hidden, 0, int(self._weight.shape[0]))
        logits = F.linear(hidden.to(dtype=self._weight.dtype), self._weight)
        return F.log_softmax(logits.float(), dim=-1)

    def compute_level(self, hidden: torch.Tensor, level: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Per-codebook logprobs: GEMM only against the level's slice (logits.py:122-138)."""
        weights = self._level_weights
        ids = self._level_token_ids
        if weights is None or ids is None or level < 0 or level >= len(weights):
            if self._weight is None or self._token_ids is None:
                raise RuntimeError("RestrictedLMHead.compute_level requires bind_codebook()")
            return self._restricted_logprobs(hidden), self._token_ids
        if self.fp8:
            assert self._level_offsets is not None
            lp = self._fp8_logprobs(hidden, self._level_offsets[level], int(weights[level].shape[0]))
            return lp, ids[level]
        w = weights[level]
        logits = F.linear(hidden.to(dtype=w.dtype), w)
        return F.log_softmax(logits.float(), dim=-1), ids[level]

    def compute_into(self, hidden: torch.Tensor, lm_weight: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """Write restricted logprobs into ``out`` [T, K] fp32 (logits.py:140-155)."""
        del lm_weight
        if self._weight is None or self._token_ids is None:
            raise RuntimeError("RestrictedLMHead.compute_into requires bind()")
        out.copy_(self._restricted_logprobs(hidden))
        return out

    def compute(self, hidden: torch.Tensor, lm_weight: torch.Tensor) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Return (logprobs [T, K or V], candidate_token_ids or None) (logits.py:157-166)."""
        device = hidden.device
        self._ensure(device, lm_weight)
        if self.enabled and self._weight is not None and self._token_ids is not None:
            return self._restricted_logprobs(hidden), self._token_ids
        logits = F.linear(hidden.to(dtype=lm_weight.dtype), lm_weight)
        return F.log_softmax(logits.float(), dim=-1), None
