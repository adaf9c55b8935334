"""Paged fp8 KV pool (``flashrec.kvcache``)."""
