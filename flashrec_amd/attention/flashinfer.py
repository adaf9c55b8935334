"""Import path of the reference's ``flashrec.attention.flashinfer``: the
backend class a model constructs (python/flashrec/attention/flashinfer.py:73).
Backed by the gfx950 paged kernel, not by FlashInfer."""

from flashrec_amd.attention.paged import AttentionBackend

__all__ = ["AttentionBackend"]
