"""CPU oracle for the fused int4 x int8 linear-layer path (TEST INFRASTRUCTURE).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package.  It is the checker, never the thing measured or shipped: the
product path (webyiq_amd) has no CPU fallback and fails loudly when its HIP
library is missing.

  oracle.oracle     ctypes binding of the C restatement (q4q8_oracle.c):
                    RTN int4 quantiser/packer, activation quantiser, exact
                    integer group accumulators, canonical fp32 epilogue,
                    argmax with the reference tie rule.
  oracle.reference  the reference's torch fake-quant path
                    (tools/reference.py:35-48 + tools/convert.py:55-106),
                    seeded input generation, and the CPU baseline timer.
"""
