"""Paged fp8 attention over the KV pool (module path of ``flashrec.attention``)."""

from flashrec_amd.attention.paged import AttentionBackend, paged_attention

__all__ = ["AttentionBackend", "paged_attention"]
