"""Validating wrappers of the HIP entry points, one module per reference module
of ``gefen/kernels`` (same function names, checks and exception types)."""
