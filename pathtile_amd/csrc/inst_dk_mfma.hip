// Instantiates the matrix-core DK kernels (per-channel and channel-group).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const DkMfmaFn kDkMfmaTable[3] = {&dwconv_dk_mfma_kernel<16>,
                                  &dwconv_dk_mfma_kernel<32>,
                                  &dwconv_dk_mfma_kernel<48>};
const DkCgFn kDkCgTable[3] = {&dwconv_dk_cg_kernel<16>,
                              &dwconv_dk_cg_kernel<32>,
                              &dwconv_dk_cg_kernel<48>};
const DkCgFn kDkCgTableNT[3] = {&dwconv_dk_cg_kernel<16, kCpolNT>,
                                &dwconv_dk_cg_kernel<32, kCpolNT>,
                                &dwconv_dk_cg_kernel<48, kCpolNT>};
}  // namespace pt
