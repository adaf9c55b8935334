"""CPU oracle for the FP8 path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or the timed CPU
baseline), never as the thing measured or shipped.  The product package
``flashrec_amd`` never imports it.

* ``oracle.ops``    -- torch-CPU restatement of the reference's CPU fallback
  arithmetic for every operator on the path (each function cites the
  reference file:line it follows).
* ``oracle.e4m3``   -- an independent numpy float8_e4m3fn codec written from
  the OCP format definition, used to pin torch's conversion.
* ``oracle.inputs`` -- seeded synthetic inputs for the benchmark configs.

Pinning status (what checks each oracle function; see tests/test_oracle_*.py):
every function has at least one check that does not restate its own formula
(spec codec, exact rational arithmetic, float64 closed forms, integer-exact
matmuls, complex-rotation RoPE, permutation checks).  The reference ships no
golden vectors or known-answer tests for this path.
"""
