"""Native kernels: libffa.so (hand-written gfx950 HIP) behind the C ABI of include/ffa.h.

Sources live in ``kernels/hip/``; ``_lib`` is the ctypes binding. Nothing here imports
Triton or provides an alternative implementation.
"""
