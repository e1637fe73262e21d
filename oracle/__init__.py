"""CPU oracle for the scaled-FP8 paged KV path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker.  The product path in
``prism-infer_amd/`` never imports, links or executes anything from here.

Every function cites the reference (Prism-Infer) source it restates; pinning
evidence for each lives in ``tests/test_oracle_*.py``.  All functions are
pinned (none is "parity unpinned"):

* fp8 codec           -- exhaustive against torch's float8_e4m3fn cast.
* store (scaled/unit) -- reference test vectors (seed 20260717), closed forms
                         (absmax -> +-448, zero row -> floor scale, RNE error
                         bound, sign symmetry, float64 quotient rounding).
* decode              -- closed forms (ctx=1, identical keys, one dominant key),
                         invariants (page permutation, GQA mapping, ctx=0),
                         float64 brute force and torch SDPA on tiny shapes, the
                         reference's eager-vs-SDPA known-answer test (seed 20260718).
* compaction          -- torch index_select/index_copy_ and read-before-write
                         invariants under overlapping source/destination sets.
"""

from oracle.kv_oracle import *  # noqa: F401,F403
