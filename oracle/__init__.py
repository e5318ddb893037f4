"""CPU oracle for the Walsh ternary structured-linear hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or as
the timed CPU baseline), never as the implementation under test.

Each function restates the reference algorithm from its source, cited as
``file:line`` relative to the reference repository root
(pulseofthemachine/Walsh-Research).  Integer/byte work (ternary codes,
2-bit packing, top-k selection) is numpy; floating-point work is numpy
float64/float32 or torch-CPU float32 where the reference's own CPU
arithmetic (torch) must be mirrored bit-for-bit (the absmean scale).

Pinning (what makes each function trustworthy, checked in
``tests/test_oracle_*.py``):

* ``ternary``  -- closed-form rounding cases (ties to even at +-0.5,
  clamping at +-1.5), brute force against a float64 restatement, the STE
  identity (value == code exactly), pack/unpack round trip and the
  published bit layout.
* ``hadamard`` -- Sylvester H against ``scipy.linalg.hadamard``, H = H^T,
  H.H = I, the two Rust known-answer tests of ``inference/src/hadamard.rs``
  (self-inverse on x[i]=i, norm preservation on x[i]=(i+1)/32), and the
  layer against a dense float64 C_out x C_in matrix built independently.
* ``octonion`` -- sign/index tables derived from an independent
  Cayley-Dickson doubling of the quaternions; the layer with in_o=out_o=1
  equals the octonion product; dense-equivalent matrix check.
* ``moe``      -- softmax/top-k against a brute-force sort with an explicit
  tie rule; experts against per-block brute force; aux loss closed form.
* ``mhc``      -- Sinkhorn invariants (row sums 1 after the last step,
  column sums -> 1, n=1 gives [[1]]), float64 closed-form iteration,
  sigmoid bounds, stream update with an identity layer.
* ``model``    -- assembled from the pinned pieces, and pinned end to end
  by the golden fixtures of ``tests/golden`` (written from the reference's
  own modules on the CPU by ``tests/golden/make_fixtures.py``): two small
  mHCWalsh models (SwiGLU with head mixing; MoE with channel modulation),
  HadamardMoE, the three stream mappings and one stream, Sinkhorn,
  HadamardLinear and the octonion layer (``tests/test_oracle_model.py``).
  Each method of ``Oracle`` is also checked against the function-level
  oracle of the same step.
"""
