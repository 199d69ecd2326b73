"""CPU oracle for the fused chunked SSD scan — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or, for the CPU
baseline, as the thing timed on host cores). The product path
(``dhammic-ai_amd/kernels``) never imports it and has no CPU fallback.

Contents
--------
``ssd_chunked``    restatement of the reference's pure-PyTorch chunked path,
                   r2/dhammic-ai/src/kernels/ssd_scan.py:53-583 (segsum and
                   exp-clamp semantics with their strict backward masks, the
                   four contractions, the cache contract, the checkpointed
                   backward). Pinned by: the CES golden vectors, the ces-ssm
                   KAT, the sequential brute force, closed forms and
                   invariants, fp64 gradcheck (tests/test_oracle.py).
``ssd_sequential`` brute-force fp64 token-by-token recurrence (the exact
                   operator of stream/ces/ssd_reference/extract.py:13-63 and
                   stream/ces/ces-ssm/src/lib.rs:255-299).
``ssd_extended``   the composed operator (dt, per-head A, groups, D, gated
                   RMSNorm, initial/final state, packed varlen) that the
                   extended entry point computes; defined by composition over
                   ``ssd_chunked`` (no counterpart in the reference).
``trapezoidal``    the reference block's two SSD calls (gamma path, shifted beta path
                   reusing the cache, + D x, gated norm; mamba_base_engine.py:
                   152-191) over ``ssd_chunked``, and the same pair as two fp64
                   token recurrences that pin it (tests/test_trapz_oracle.py).
``inputs``         seeded input generators with BASELINE's distributions.
"""
