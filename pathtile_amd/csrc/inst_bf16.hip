// Instantiates the BF16-I/O kernels (FWD / DX and DK on the BF16 matrix
// cores).
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
// DK on the BF16 matrix cores: plain and non-temporal loads
const DkBf16Fn kDkBf16mmaTable[3] = {&dwconv_dk_bf16mma_kernel<16, kCpolNone>,
                                       &dwconv_dk_bf16mma_kernel<32, kCpolNone>,
                                       &dwconv_dk_bf16mma_kernel<48, kCpolNone>};
const DkBf16Fn kDkBf16mmaTableNT[3] = {&dwconv_dk_bf16mma_kernel<16, kCpolNT>,
                                         &dwconv_dk_bf16mma_kernel<32, kCpolNT>,
                                         &dwconv_dk_bf16mma_kernel<48, kCpolNT>};
}  // namespace pt
