"""CPU oracle of collab_infer's per-device attention / LSE / layer-op path.

TEST INFRASTRUCTURE ONLY.  This package restates, on the CPU and in PyTorch's CPU
operators, the algorithm the reference implements for this path, so the gfx950 kernels can
be checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the reference results to
compare with / the timed CPU baseline; the product package never imports, calls or falls back to it.

Modules:
* :mod:`oracle.attention_ref` - attention_with_lse / attention / merges
  (collab_infer/parallel/attention.py)
* :mod:`oracle.layers_ref` - RMSNorm, rotary, SiLU-gate with the reference's rounding
  points (collab_infer/models/llama.py:44-88, 305; models/config.py:165-189)
* :mod:`oracle.sp_ref` - per-rank ring / distributed-KV / Ulysses shares
  (collab_infer/parallel/sequence_parallel.py)

How each function is pinned (golden vectors, closed forms, library routines, invariants) is
listed in the tests that check it (tests/test_oracle_*.py).  The reference is pure Python
over torch: nothing of it is compiled, imported or executed; its own tests hold no stored
golden vectors, so the pins are its known-answer tests restated on seeded inputs plus the
mathematics.
"""
