// Instantiates the channels-last DK kernels ([B, L, H] tensors, [K, H] dw).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// [row bucket]: 16 waves of two channels for rows up to 32 columns, 8 waves
// of four channels with two steps of loads in registers for 48.
const DkClFn kDkClTable[3] = {&dwconv_dk_cl_kernel<16>, &dwconv_dk_cl_kernel<32>,
                              &dwconv_dk_cl_kernel<48, kClWideChannels, 2>};
}  // namespace pt
