"""The CPU backend: MSDA in torch operators, for CPU tensors only.

GPU tensors never run here: the registry's policy sends them to the HIP kernels,
and this backend declines any context whose device is not the CPU.
"""
