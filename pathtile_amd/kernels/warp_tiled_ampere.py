"""The reference's ``kernels/warp_tiled_ampere.py`` runtime/autograd names
(the surface S4ConvD and the PathTile tuner call), backed by the MI355X
kernels. See ``pathtile_amd.runtime`` for the definitions."""

from ..runtime import *  # noqa: F401,F403
from ..runtime import __all__  # noqa: F401
