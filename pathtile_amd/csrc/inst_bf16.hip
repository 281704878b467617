// Instantiates the BF16-I/O kernels (FWD / DX on the BF16 matrix cores, DK
// on the channel-group kernel).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// FWD / DX on the BF16 matrix cores, 8-channel groups
const RowsCgBf16Fn kRowsCgTableBf16[2][3] = {
    {&dwconv_rows_bf16mma_kernel<16, false, kRowsCgWaves>,
     &dwconv_rows_bf16mma_kernel<32, false, kRowsCgWaves>,
     &dwconv_rows_bf16mma_kernel<48, false, kRowsCgWaves>},
    {&dwconv_rows_bf16mma_kernel<16, true, kRowsCgWaves>,
     &dwconv_rows_bf16mma_kernel<32, true, kRowsCgWaves>,
     &dwconv_rows_bf16mma_kernel<48, true, kRowsCgWaves>}};
const DkCgBf16Fn kDkCgTableBf16[3] = {&dwconv_dk_cg_kernel<16, kCpolNone, uint16_t>,
                                      &dwconv_dk_cg_kernel<32, kCpolNone, uint16_t>,
                                      &dwconv_dk_cg_kernel<48, kCpolNone, uint16_t>};
const DkCgBf16Fn kDkCgTableBf16NT[3] = {&dwconv_dk_cg_kernel<16, kCpolNT, uint16_t>,
                                        &dwconv_dk_cg_kernel<32, kCpolNT, uint16_t>,
                                        &dwconv_dk_cg_kernel<48, kCpolNT, uint16_t>};
}  // namespace pt
