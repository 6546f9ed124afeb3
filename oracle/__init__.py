"""CPU oracle of the CVSA decode-step attention path -- TEST INFRASTRUCTURE ONLY.

A plain torch-on-CPU restatement of the reference's algorithm
(DJ-Melvin/coverage-verified-sparse-attention), used as the checker for the
HIP implementation.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product path in
``coverage-verified-sparse-attention_amd/cvsa`` never does.

Modules:
  cvsa_oracle     -- the per-op restatement (scoring, selection, coverage,
                     decode, complement, merge, KV append)
  backend_oracle  -- the CVSABackend scheduling state machine over those ops

Every function names the reference file:line it follows.  Where the HIP
contract deliberately differs from a reference quirk (empty selections give
the LSE-merge identity instead of NaN; top-k order is fixed instead of
unspecified) the oracle states the contract the HIP path is held to.
"""
