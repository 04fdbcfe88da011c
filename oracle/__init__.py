"""CPU oracle for the ApexW optimizer-step hot path.  TEST INFRASTRUCTURE ONLY.

This package restates, with torch CPU tensor ops, the reference's own CPU
algorithm for the optimizer step, so that the HIP kernels can be checked
against it on the same seeded inputs.  The reference's CPU path *is* a sequence
of torch ops; restating it with the same ops reproduces its rounding points
(bf16 round-to-nearest-even after every foreach op, FMA in add/addcmul/lerp,
IEEE division in addcdiv) which is what the kernels must match.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or as the timed CPU
baseline).  The product package ``apexw_amd`` never imports it and has no CPU
fallback.

Modules and what pins them (golden vectors live in ``tests/golden``):

* ``quant``   -- NF4 / INT8 / log-uint8 blockwise quantizers and fp32->16-bit
  stochastic rounding.  Pinned by closed forms (codebook, LUT formula), brute
  force on tiny inputs, the reference's own known answers, and the 8-bit
  trajectories.
* ``compact`` -- compact-mode multi-tensor step.  Pinned by the compact golden
  trajectories (bit-exact, SR off).
* ``q8``      -- 8-bit step (NF4 m + quad log-u8 v, INT8 m + u8 v, tiny
  tensors).  Pinned by the 8-bit golden trajectories (bit-exact, SR off).
* ``clip``    -- global-L2 gradient clipping.  Pinned by ``clip_bf16.npz``.
* ``layout``  -- per-parameter state layout.  Pinned by ``layout.npz``.
* ``muon``    -- Newton-Schulz polar factor, Muon step and hybrid routing.
  Pinned by ``muon.npz`` and by the polar-factor invariants (SVD).
* ``optim``   -- ``OracleApexW`` / ``OracleHybrid``: the optimizer objects
  that drive the modules above the way the reference's ``ApexW.step`` does.

With stochastic rounding on, the oracle draws noise from torch's global RNG as
the reference does; SR results are compared statistically, never bit-wise.
"""
