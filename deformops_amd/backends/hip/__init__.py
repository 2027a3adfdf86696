"""The HIP backend: gfx950 kernels in libdeformops_amd.so, bound with ctypes."""
