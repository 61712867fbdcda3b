"""Kernel entry points with the signatures of ``respect.kernels`` (respect/kernels/*.py)."""
