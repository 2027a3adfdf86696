"""Backend adapters. This build has one: ``hip``, the gfx950 kernels."""
