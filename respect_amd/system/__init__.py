"""Elementwise kernels of ``respect.system.fused`` (respect/system/fused.py)."""
