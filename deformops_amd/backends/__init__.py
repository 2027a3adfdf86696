"""Backend adapters: ``hip`` (the gfx950 kernels, GPU tensors) and ``eager`` (torch operators, CPU tensors)."""
