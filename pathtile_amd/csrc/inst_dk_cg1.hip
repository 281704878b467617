// Instantiates the channel-group DK kernels that stage dwords (rows of any
// length, 4-byte aligned tensors) and the 48-bucket kernel with two channels
// per wave.
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const DkCgFn kDkCgTable1[3] = {&dwconv_dk_cg_kernel<16, kCpolNone, dk_cg_cpw(16), 1>,
                               &dwconv_dk_cg_kernel<32, kCpolNone, dk_cg_cpw(32), 1>,
                               &dwconv_dk_cg_kernel<48, kCpolNone, dk_cg_cpw(48), 1>};
const DkCgFn kDkCgTable1NT[3] = {&dwconv_dk_cg_kernel<16, kCpolNT, dk_cg_cpw(16), 1>,
                                 &dwconv_dk_cg_kernel<32, kCpolNT, dk_cg_cpw(32), 1>,
                                 &dwconv_dk_cg_kernel<48, kCpolNT, dk_cg_cpw(48), 1>};
const DkCgFn kDkCgPairNT = &dwconv_dk_cg_kernel<48, kCpolNT, 2, 4>;
}  // namespace pt
