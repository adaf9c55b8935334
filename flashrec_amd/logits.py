"""SID-restricted lm_head + log_softmax: a drop-in for ``flashrec.logits.RestrictedLMHead``
(python/flashrec/logits.py:11-166).

Interface kept: ``RestrictedLMHead(special_token_ids, enabled=True)``; the
properties ``token_ids``, ``num_tokens``, ``ready``, ``per_codebook_ready``,
``num_levels``, ``max_codebook_k``; ``codebook_k(level)``; ``bind(lm_weight)``
(ids checked against the vocabulary, ``ValueError`` when out of range),
``bind_codebook(sizes)`` (ignored unless the sizes add up to the bound
rows), ``compute(hidden, lm_weight)``, ``compute_level(hidden, level)`` (past
the last level: the whole restricted head) and ``compute_into(hidden,
lm_weight, out)`` (needs a prior ``bind``, ``RuntimeError`` otherwise; never
re-slices, so it can be graph-captured).  Results are fp32 log-probabilities
over the restricted rows, in the order of ``special_token_ids``.

Design here: the bound head is a ``_RowBlock`` -- the weight rows of the
restricted ids (a zero-copy ``narrow`` when the ids are one contiguous run,
a gathered copy otherwise), their ids on the device and, with ``fp8=True``,
their per-row e4m3 codes and fp32 scales, quantised once at bind time.  A
codebook level is a ``_RowBlock`` over a row range of the bound one (views
of the same weight, codes and scales).  With ``fp8=True`` (this build's
addition; the reference always runs a bf16 ``F.linear``) a call is three HIP
kernels: per-token e4m3 quant of the hidden rows, the W8A8 GEMM with fp32
logits, and a row-wise log_softmax written in place (or straight into
``compute_into``'s ``out``).  With ``fp8=False`` it is the reference's bf16
``F.linear`` + fp32 ``log_softmax``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from flashrec_amd.kernel.sglops import (PrearrangedFp8Weight, fp8_scaled_mm, fp8_scaled_mm_prearranged,
                                        log_softmax_f32, per_token_quant_fp8, prearrange_fp8_weight)
from flashrec_amd.layers.linear import quantize_weight_fp8


@dataclass
class _RowBlock:
    """Rows of the lm_head weight for a run of restricted ids."""

    weight: torch.Tensor  # [n, hidden]
    ids: torch.Tensor  # [n] int64, on the weight's device
    codes: Optional[torch.Tensor] = None  # [n, hidden] e4m3 (fp8 heads)
    scale: Optional[torch.Tensor] = None  # [n] fp32
    pre: Optional[PrearrangedFp8Weight] = None  # the codes prearranged (whole heads, not level cuts)

    @property
    def rows(self) -> int:
        return int(self.weight.shape[0])

    def sub(self, start: int, count: int) -> "_RowBlock":
        def cut(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
            return None if t is None else t.narrow(0, start, count)

        return _RowBlock(cut(self.weight), cut(self.ids), cut(self.codes), cut(self.scale))

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """fp32 logits [T, n] of these rows (before the log-softmax)."""
        if self.codes is None:
            return F.linear(hidden.to(dtype=self.weight.dtype), self.weight).float()
        rows = hidden.reshape(-1, hidden.shape[-1])
        return self.logits_fp8(*per_token_quant_fp8(rows))

    def logits_fp8(self, a_codes: torch.Tensor, a_scale: torch.Tensor) -> torch.Tensor:
        """fp32 logits from hidden rows already quantised per token (fp8 heads)."""
        if self.pre is not None:
            return fp8_scaled_mm_prearranged(a_codes, self.pre, a_scale, self.scale, torch.float32)
        return fp8_scaled_mm(a_codes, self.codes.t(), a_scale, self.scale, torch.float32)

    def logprobs(self, hidden: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        if self.codes is None:
            logits = F.linear(hidden.to(dtype=self.weight.dtype), self.weight)
            lp = F.log_softmax(logits.float(), dim=-1)
            return lp if out is None else out.copy_(lp)
        logits = self.logits(hidden)
        direct = (out is not None and out.dtype == torch.float32 and out.shape == logits.shape
                  and out.stride(1) == 1 and out.device == logits.device)
        if out is None or direct:
            return log_softmax_f32(logits, out=logits if out is None else out)
        return out.copy_(log_softmax_f32(logits, out=logits))


def _one_run(ids: Sequence[int]) -> bool:
    """True when the ids are lo, lo + 1, ..., lo + n - 1 (n > 1)."""
    return len(ids) > 1 and all(b == a + 1 for a, b in zip(ids, ids[1:]))


class RestrictedLMHead:
    def __init__(self, special_token_ids: Optional[Sequence[int]], enabled: bool = True,
                 fp8: bool = False):
        self.ids: Optional[List[int]] = [int(i) for i in special_token_ids] if special_token_ids else None
        self.enabled = bool(enabled) and self.ids is not None
        self.fp8 = bool(fp8)
        self._head: Optional[_RowBlock] = None
        self._levels: List[_RowBlock] = []

    # --- state -------------------------------------------------------------------
    @property
    def token_ids(self) -> Optional[torch.Tensor]:
        return None if self._head is None else self._head.ids

    @property
    def num_tokens(self) -> Optional[int]:
        return None if self._head is None else self._head.rows

    @property
    def ready(self) -> bool:
        return self.enabled and self._head is not None

    @property
    def per_codebook_ready(self) -> bool:
        return bool(self._levels)

    @property
    def num_levels(self) -> int:
        return len(self._levels)

    @property
    def max_codebook_k(self) -> int:
        return max((lv.rows for lv in self._levels), default=0)

    def codebook_k(self, level: int) -> int:
        return self._levels[level].rows if 0 <= level < len(self._levels) else 0

    # --- binding -------------------------------------------------------------------
    def _bound_to(self, lm_weight: torch.Tensor) -> bool:
        return self._head is not None and self._head.weight.device == lm_weight.device

    def bind(self, lm_weight: Optional[torch.Tensor]) -> None:
        """Select (and with fp8 quantise) the restricted rows once after weight load."""
        if lm_weight is None or not self.enabled or self._bound_to(lm_weight):
            return
        ids = self.ids or []
        vocab = int(lm_weight.shape[0])
        if min(ids) < 0 or max(ids) >= vocab:
            raise ValueError(f"sid_token_range out of range for vocab {vocab}")
        dev = lm_weight.device
        id_t = torch.tensor(ids, dtype=torch.int64, device=dev)
        rows = lm_weight.narrow(0, ids[0], len(ids)) if _one_run(ids) else lm_weight.index_select(0, id_t)
        head = _RowBlock(rows, id_t)
        if self.fp8:
            head.codes, head.scale = quantize_weight_fp8(rows)
            head.pre = prearrange_fp8_weight(head.codes.t())
        self._head = head
        self._levels = []

    def bind_codebook(self, codebook_sizes: Sequence[int]) -> None:
        """One level per codebook, each a zero-copy row range of the bound head."""
        if self._head is None or not self.enabled:
            return
        sizes = [int(n) for n in codebook_sizes]
        if sum(sizes) != self._head.rows:
            return
        starts = [sum(sizes[:i]) for i in range(len(sizes))]
        self._levels = [self._head.sub(s0, n) for s0, n in zip(starts, sizes)]

    # --- calls -------------------------------------------------------------------
    def compute(self, hidden: torch.Tensor, lm_weight: torch.Tensor
                ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """(logprobs ``[T, K]`` over the restricted ids, their ids), or over
        the full vocabulary with ``None`` when the head is disabled."""
        self.bind(lm_weight)
        if self.ready:
            return self._head.logprobs(hidden), self._head.ids
        logits = F.linear(hidden.to(dtype=lm_weight.dtype), lm_weight)
        return F.log_softmax(logits.float(), dim=-1), None

    def compute_logits(self, hidden: torch.Tensor, lm_weight: torch.Tensor
                       ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """``compute`` without the log-softmax: (fp32 logits, their ids), for a
        caller that folds the log-softmax into its top-k
        (``row_topk(..., log_softmax=True)``)."""
        self.bind(lm_weight)
        if self.ready:
            return self._head.logits(hidden), self._head.ids
        return F.linear(hidden.to(dtype=lm_weight.dtype), lm_weight).float(), None

    def compute_logits_fp8(self, a_codes: torch.Tensor, a_scale: torch.Tensor, lm_weight: torch.Tensor
                           ) -> Tuple[torch.Tensor, torch.Tensor]:
        """``compute_logits`` for hidden rows already quantised per token (e4m3
        codes [T, hidden], fp32 scales [T, 1]), e.g. by ``RMSNorm.quant_fp8``:
        the same logits as ``compute_logits`` on the bf16 rows they came from.
        fp8 heads only."""
        self.bind(lm_weight)
        if not self.ready or self._head.codes is None:
            raise RuntimeError("compute_logits_fp8 needs a bound fp8 head (RestrictedLMHead(..., fp8=True))")
        return self._head.logits_fp8(a_codes, a_scale), self._head.ids

    def compute_level(self, hidden: torch.Tensor, level: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Logprobs against one codebook level's rows only."""
        if 0 <= level < len(self._levels):
            block = self._levels[level]
            return block.logprobs(hidden), block.ids
        if self._head is None:
            raise RuntimeError("RestrictedLMHead.compute_level requires bind_codebook()")
        return self._head.logprobs(hidden), self._head.ids

    def compute_into(self, hidden: torch.Tensor, lm_weight: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
        """Restricted logprobs written into ``out`` ``[T, K]`` fp32."""
        del lm_weight  # already bound: nothing is sliced here
        if self._head is None:
            raise RuntimeError("RestrictedLMHead.compute_into requires bind()")
        return self._head.logprobs(hidden, out=out)
