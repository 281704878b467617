// Instantiates the channels-last DK kernels ([B, L, H] tensors, [K, H] dw).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const DkClFn kDkClTable[3] = {&dwconv_dk_cl_kernel<16>,
                              &dwconv_dk_cl_kernel<32>,
                              &dwconv_dk_cl_kernel<48>};
}  // namespace pt
