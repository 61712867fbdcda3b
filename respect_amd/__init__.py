"""respect_amd -- MI355X (gfx950) deterministic trie-verification kernels.

Drop-in replacements for the kernels of soonhong99/respect: the Python call
signatures of ``respect.kernels`` (attention, rmsnorm, gemm) and of
``respect.system.fused`` (rope, silu_mul) are kept, and every call goes to a
hand-written HIP kernel in ``librespect_amd.so`` through its C ABI
(include/respect_amd.h).  There is no CPU or Triton fallback.
"""
__version__ = "0.1.0"
