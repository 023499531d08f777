"""CPU oracle for the GPTQ-2D layer-quantization path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU, the reference algorithms
that the MI355X engine accelerates.  It is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The engine under ``gptq-2d_amd/`` never calls
into it and fails loudly when its HIP library is missing.

Modules and the reference code each one restates (IST-DASLab/GPTQ-2D):

- ``oracle.sweep``      -- ``direct_2d``, ``gptq_2d_torch`` and their super-entry
  variants, plus the antidiagonal geometry (gptq_2d.py:65-164, 1122-1292).
- ``oracle.algorithms`` -- paper Algorithms 1-7, super-entry Algorithms 1/3,
  D-sided Algorithms 2/4, YAQA_iterative, the LDL helpers and the
  vec(X) reference trajectory (gptq_2d_reference.py:24-382).
- ``oracle.quantize``   -- round / affine / INT abs-max quantizers
  (quantizer_int.py:18-134).
- ``oracle.trellis``    -- 1MAD / 3INST / HYB codes, the Viterbi search and the
  tail-biting trellis quantizer (quantizer_trellis.py:28-143, 344-369).

The seeded input generators of the benchmark configurations are not part of
the oracle (they compute no reference algorithm): ``gptq-2d_amd/instances.py``.

How each function is pinned (checked by something other than retyping it) is
listed in the module docstrings and exercised by ``tests/test_oracle_*.py``.
"""
