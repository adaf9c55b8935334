"""Layer modules of the FP8 path (``flashrec.layers``)."""
