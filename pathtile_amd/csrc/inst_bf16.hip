// Instantiates the BF16-I/O channel-group kernels (FWD / DX and DK).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// Row bucket 48 uses 4-channel groups (4 waves, 50 KB of LDS, three
// workgroups per CU); 16 and 32 the 8-channel groups of the FP32 kernels.
const RowsCgBf16Fn kRowsCgTableBf16[2][3] = {
    {&dwconv_rows_cg_kernel<16, false, 2, uint16_t, 8>,
     &dwconv_rows_cg_kernel<32, false, 2, uint16_t, 8>,
     &dwconv_rows_cg_kernel<48, false, 2, uint16_t, kRowsCgBf16WavesL48>},
    {&dwconv_rows_cg_kernel<16, true, 2, uint16_t, 8>,
     &dwconv_rows_cg_kernel<32, true, 2, uint16_t, 8>,
     &dwconv_rows_cg_kernel<48, true, 2, uint16_t, kRowsCgBf16WavesL48>}};
const DkCgBf16Fn kDkCgTableBf16[3] = {&dwconv_dk_cg_kernel<16, kCpolNone, uint16_t>,
                                      &dwconv_dk_cg_kernel<32, kCpolNone, uint16_t>,
                                      &dwconv_dk_cg_kernel<48, kCpolNone, uint16_t>};
const DkCgBf16Fn kDkCgTableBf16NT[3] = {&dwconv_dk_cg_kernel<16, kCpolNT, uint16_t>,
                                        &dwconv_dk_cg_kernel<32, kCpolNT, uint16_t>,
                                        &dwconv_dk_cg_kernel<48, kCpolNT, uint16_t>};
}  // namespace pt
