"""flashrec_amd: FlashRec's FP8 quantized compute path, native to MI355X (gfx950).

Module layout mirrors the reference package ``flashrec`` for the operators
on this path, so callers switch imports only:

* ``flashrec_amd.kernel.sglops``      <- ``flashrec.kernel.sglops``
* ``flashrec_amd.kernel.rms_fp8``     <- ``flashrec.kernel.rms_fp8``
* ``flashrec_amd.kernel.silu_fp8``    <- ``flashrec.kernel.silu_fp8``
* ``flashrec_amd.kernel.qk_rope_kv``  <- ``flashrec.kernel.qk_rope_kv``
* ``flashrec_amd.layers.{linear,norm,rotary}`` <- ``flashrec.layers.*``
* ``flashrec_amd.kvcache.pool``       <- ``flashrec.kvcache.pool``
* ``flashrec_amd.logits``             <- ``flashrec.logits``

All compute runs in hand-written HIP kernels (``flashrec_amd/csrc``) behind
the C ABI in ``include/flashrec_amd.h``; there is no CPU or Triton path.
"""

__version__ = "0.1.0"
