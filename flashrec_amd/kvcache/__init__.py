"""Paged fp8 KV pool and request-slot pool (``flashrec.kvcache``)."""

from flashrec_amd.kvcache.pool import ReqToTokenPool, TokenToKVPool

__all__ = ["ReqToTokenPool", "TokenToKVPool"]
