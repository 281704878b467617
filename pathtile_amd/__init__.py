"""MI355X-native depthwise Conv1D (FWD, dX, dK; L, K <= 48; FP32).

A hipcc-built C-ABI library (``libpathtile_hip.so``, ``include/pathtile_hip.h``)
behind the reference's Python surface:

* ``pathtile_amd.kernels.warp_tiled``         the kernels/warp_tiled.py API;
* ``pathtile_amd.kernels.warp_tiled_ampere``  runtime + autograd names used by
  S4ConvD (``DepthConvAmpere``, ``depthwise_conv_ampere``, ...), the S4ConvD
  model and its ``TRAIN_CONV_BACKEND`` switch;
* ``pathtile_amd.s4convd``                    the S4ConvD model, with each
  block's skip term fused into its convolution;
* ``pathtile_amd.tune``                       the PathTile offline tuner and
  its selector baselines;
* ``pathtile_amd.profiling``                  rocprofv3 result summaries.

Importing the package needs neither a GPU nor the built library; the first
launch loads the library and raises if it is missing.
"""

__version__ = "0.1.0"
