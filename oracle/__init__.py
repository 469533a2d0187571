"""CPU oracle for the CompactLogic hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithms on the CPU so that tests, the smoke check
and the benchmark's CPU-baseline leg can check the HIP kernels.  The product
(``compactlogic_amd``) never imports, links or calls anything here, and there is no code
path that substitutes the oracle for a missing HIP library.

Modules
  logic_np   float64 numpy restatement of the soft and discrete float paths (dense layer
             forward / backward / eval, inverse index, GroupSum, ConvLayer).
  packed     bit-packed evaluator (C in packed_ref.c, built by the Makefile here, with
             numpy fallbacks): pack, bitwise layer, group popcount, splitmix64 inputs.
  torch_cpu  pure-PyTorch CPU training step in the reference's CPU formulation, timed as
             the CPU baseline.

Pinning (what checks each function besides the HIP kernels) is listed in each module's
docstring; every function is pinned by a check in tests/ that does not restate it.
"""
