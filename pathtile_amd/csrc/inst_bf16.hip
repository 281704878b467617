// Instantiates the BF16-I/O kernels (FWD / DX and DK on the BF16 matrix
// cores).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// FWD / DX on the BF16 matrix cores: [dx][16-channel groups][row bucket]
const RowsCgBf16Fn kRowsCgTableBf16[2][2][3] = {
    {{&dwconv_rows_bf16mma_kernel<16, false, 8>,
      &dwconv_rows_bf16mma_kernel<32, false, 8>,
      &dwconv_rows_bf16mma_kernel<48, false, 8>},
     {&dwconv_rows_bf16mma_kernel<16, false, 16>,
      &dwconv_rows_bf16mma_kernel<32, false, 16>,
      &dwconv_rows_bf16mma_kernel<48, false, 16>}},
    {{&dwconv_rows_bf16mma_kernel<16, true, 8>,
      &dwconv_rows_bf16mma_kernel<32, true, 8>,
      &dwconv_rows_bf16mma_kernel<48, true, 8>},
     {&dwconv_rows_bf16mma_kernel<16, true, 16>,
      &dwconv_rows_bf16mma_kernel<32, true, 16>,
      &dwconv_rows_bf16mma_kernel<48, true, 16>}}};
// The same, 8-channel groups with plain (cached) input loads: [dx][row bucket]
const RowsCgBf16Fn kRowsCgTableBf16PL[2][3] = {
    {&dwconv_rows_bf16mma_kernel<16, false, 8, kCpolNone>,
     &dwconv_rows_bf16mma_kernel<32, false, 8, kCpolNone>,
     &dwconv_rows_bf16mma_kernel<48, false, 8, kCpolNone>},
    {&dwconv_rows_bf16mma_kernel<16, true, 8, kCpolNone>,
     &dwconv_rows_bf16mma_kernel<32, true, 8, kCpolNone>,
     &dwconv_rows_bf16mma_kernel<48, true, 8, kCpolNone>}};
// DK on the BF16 matrix cores: plain and non-temporal loads
const DkBf16Fn kDkBf16mmaTable[3] = {&dwconv_dk_bf16mma_kernel<16, kCpolNone>,
                                       &dwconv_dk_bf16mma_kernel<32, kCpolNone>,
                                       &dwconv_dk_bf16mma_kernel<48, kCpolNone>};
const DkBf16Fn kDkBf16mmaTableNT[3] = {&dwconv_dk_bf16mma_kernel<16, kCpolNT>,
                                         &dwconv_dk_bf16mma_kernel<32, kCpolNT>,
                                         &dwconv_dk_bf16mma_kernel<48, kCpolNT>};
}  // namespace pt
