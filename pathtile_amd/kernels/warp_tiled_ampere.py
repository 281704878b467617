"""The reference's ``kernels/warp_tiled_ampere.py`` names: the runtime and
autograd surface S4ConvD and the PathTile tuner call, backed by the MI355X
kernels (definitions in ``pathtile_amd.runtime``), and the S4ConvD model
(definitions in ``pathtile_amd.s4convd``).

``TRAIN_CONV_BACKEND`` is the reference's backend switch (:1119): ``"warp"``
(the HIP path) or ``"pytorch"``; the S4ConvD modules read it from this module
on every forward call, so assigning it here switches them."""

from ..runtime import *  # noqa: F401,F403
from ..runtime import __all__ as _runtime_all
from ..s4convd import *  # noqa: F401,F403
from ..s4convd import __all__ as _s4_all

TRAIN_CONV_BACKEND = "warp"

__all__ = list(_runtime_all) + list(_s4_all) + ["TRAIN_CONV_BACKEND"]
