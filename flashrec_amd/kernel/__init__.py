"""Operator wrappers with the reference's Python signatures (``flashrec.kernel``)."""
