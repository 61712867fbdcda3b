"""CPU oracle for the respect_amd kernels -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with numpy, the arithmetic of the reference
implementation (soonhong99/respect) for the trie-verification hot path, plus
float64 closed forms used to pin it.  It checks results; it is never the thing
that is measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``respect_amd``) never imports it and has no CPU fallback.

Modules (each function cites the reference file:line it follows):
  bf16       bf16 round-to-nearest-even helpers
  trie       build_trie / trie_ancestry / walk        (respect/candidates/trie.py, respect/decoding/acceptance.py)
  attention  attn_hyb (logical-order kernel), attn_blocked (negative control), attn_exact (fp64)
  norm       rmsnorm, rope, silu_mul at PyTorch rounding points, fp64 closed forms
  gen        seeded synthetic inputs for the five benchmark workloads

Pinning status is stated in each module's docstring.
"""
