"""CPU oracle of the SISA hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this package, and
only as the checker (or, for the baseline, as the timed CPU path). The product package ``sisa_amd`` never imports it.

Contents (``oracle.reference``): a plain-PyTorch restatement of the reference's algorithm (tlstngud/sisa 0.1.0) --
the attention formula, its fp64 truth with autograd, the delta-free analytic gradients, the FlashAttention-standard
rounding emulation, the prep glue (g, F, Phi, rotation) and its layout, the decay factors, and the chunked linear
cross-entropy -- plus the seeded input generators of the benchmark configurations. Every function cites the
reference file:line it restates. How each one is pinned (checks that a plausible mistake would fail) is listed in
the header of ``oracle/reference.py`` and exercised by ``tests/test_oracle.py``.
"""
