"""r9v_amd -- MI355X-native (gfx950) quantized-weight matrix path for R9V.

The product is the C-ABI library libr9vx.so (HIP kernels for CDNA4 plus the
host-side validation/dispatch layer), declared in include/r9vx.h.  The Python
modules here are thin ctypes/torch plumbing used by tests and the benchmark.
"""
