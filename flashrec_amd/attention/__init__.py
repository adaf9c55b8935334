"""Paged fp8 attention over the KV pool (module path of ``flashrec.attention``)."""

from flashrec_amd.attention.paged import (AttentionBackend, attention_plan, paged_attention,
                                          paged_attention_quant_fp8, plan_size)

__all__ = ["AttentionBackend", "attention_plan", "paged_attention", "paged_attention_quant_fp8", "plan_size"]
