// Instantiates the matrix-core DK kernels.
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const DkMfmaFn kDkMfmaTable[3] = {&dwconv_dk_mfma_kernel<16>,
                                  &dwconv_dk_mfma_kernel<32>,
                                  &dwconv_dk_mfma_kernel<48>};
}  // namespace pt
