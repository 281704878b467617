// Instantiates the DX kernels (dwordx4 row I/O).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const RowsFn kDxTableV[kNumLB][kNumKB] = {
    {&dwconv_rows_kernel<8, 4, true, true>, &dwconv_rows_kernel<8, 8, true, true>, &dwconv_rows_kernel<8, 16, true, true>, &dwconv_rows_kernel<8, 24, true, true>, &dwconv_rows_kernel<8, 32, true, true>, &dwconv_rows_kernel<8, 40, true, true>, &dwconv_rows_kernel<8, 48, true, true>},
    {&dwconv_rows_kernel<16, 4, true, true>, &dwconv_rows_kernel<16, 8, true, true>, &dwconv_rows_kernel<16, 16, true, true>, &dwconv_rows_kernel<16, 24, true, true>, &dwconv_rows_kernel<16, 32, true, true>, &dwconv_rows_kernel<16, 40, true, true>, &dwconv_rows_kernel<16, 48, true, true>},
    {&dwconv_rows_kernel<24, 4, true, true>, &dwconv_rows_kernel<24, 8, true, true>, &dwconv_rows_kernel<24, 16, true, true>, &dwconv_rows_kernel<24, 24, true, true>, &dwconv_rows_kernel<24, 32, true, true>, &dwconv_rows_kernel<24, 40, true, true>, &dwconv_rows_kernel<24, 48, true, true>},
    {&dwconv_rows_kernel<32, 4, true, true>, &dwconv_rows_kernel<32, 8, true, true>, &dwconv_rows_kernel<32, 16, true, true>, &dwconv_rows_kernel<32, 24, true, true>, &dwconv_rows_kernel<32, 32, true, true>, &dwconv_rows_kernel<32, 40, true, true>, &dwconv_rows_kernel<32, 48, true, true>},
    {&dwconv_rows_kernel<40, 4, true, true>, &dwconv_rows_kernel<40, 8, true, true>, &dwconv_rows_kernel<40, 16, true, true>, &dwconv_rows_kernel<40, 24, true, true>, &dwconv_rows_kernel<40, 32, true, true>, &dwconv_rows_kernel<40, 40, true, true>, &dwconv_rows_kernel<40, 48, true, true>},
    {&dwconv_rows_kernel<48, 4, true, true>, &dwconv_rows_kernel<48, 8, true, true>, &dwconv_rows_kernel<48, 16, true, true>, &dwconv_rows_kernel<48, 24, true, true>, &dwconv_rows_kernel<48, 32, true, true>, &dwconv_rows_kernel<48, 40, true, true>, &dwconv_rows_kernel<48, 48, true, true>}};
}  // namespace pt
