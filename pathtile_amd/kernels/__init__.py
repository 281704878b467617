"""Reference-named modules of the drop-in surface: ``warp_tiled`` (the frozen
Python API of kernels/warp_tiled.py) and ``warp_tiled_ampere`` (the
runtime/autograd names S4ConvD uses)."""
