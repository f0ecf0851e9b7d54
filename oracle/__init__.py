"""CPU oracle for the KATA-SPD and chunked (gated) delta-rule hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``linatt_amd``)
imports, links or executes anything under ``oracle/``.  The only callers are
``tests/``, ``__graft_entry__.smoke()`` (as the checker) and the
``cpu_baseline`` leg of ``bench.py`` (timed beside the GPU path, never as the
thing measured).

The oracle restates the reference's algorithms in float64 PyTorch on the CPU:

* ``oracle.kata``   - KATA concat/sum/decay attention, its explicit backward,
  the psi-feature (linear-attention) form, and the O(T) prefill/decode state
  form.  Follows ``kata/parallel_kata_attn.py``, ``kata/kernels/parallel_kata.py``,
  ``kata/references/feature_maps.py`` and ``kata/spd/chunk_scan_cat.py`` of the
  reference (citations per function).
* ``oracle.delta``  - the DeltaNet / GatedDeltaNet delta rule: a naive per-token
  recurrence (ground truth) and the chunked WY/UT form.  The reference reaches
  this arithmetic only through the third-party ``flash-linear-attention==0.5.0``
  package (pinned at ``scripts/setup.sh:27``), which is absent; it is restated
  from the published algorithm (Yang et al., NeurIPS 2024; Yang, Kautz,
  Hatamizadeh, ICLR 2025).

How each function is pinned (closed forms, invariants, brute force, two
independent formulations checked against each other) is listed in
``tests/test_oracle_kata.py`` and ``tests/test_oracle_delta.py``.
"""
