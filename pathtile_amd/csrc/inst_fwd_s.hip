// Instantiates the FWD kernels (dword row I/O).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const RowsFn kFwdTableS[kNumLB][kNumKB] = {
    {&dwconv_rows_kernel<8, 4, false, false>, &dwconv_rows_kernel<8, 8, false, false>, &dwconv_rows_kernel<8, 16, false, false>, &dwconv_rows_kernel<8, 24, false, false>, &dwconv_rows_kernel<8, 32, false, false>, &dwconv_rows_kernel<8, 40, false, false>, &dwconv_rows_kernel<8, 48, false, false>},
    {&dwconv_rows_kernel<16, 4, false, false>, &dwconv_rows_kernel<16, 8, false, false>, &dwconv_rows_kernel<16, 16, false, false>, &dwconv_rows_kernel<16, 24, false, false>, &dwconv_rows_kernel<16, 32, false, false>, &dwconv_rows_kernel<16, 40, false, false>, &dwconv_rows_kernel<16, 48, false, false>},
    {&dwconv_rows_kernel<24, 4, false, false>, &dwconv_rows_kernel<24, 8, false, false>, &dwconv_rows_kernel<24, 16, false, false>, &dwconv_rows_kernel<24, 24, false, false>, &dwconv_rows_kernel<24, 32, false, false>, &dwconv_rows_kernel<24, 40, false, false>, &dwconv_rows_kernel<24, 48, false, false>},
    {&dwconv_rows_kernel<32, 4, false, false>, &dwconv_rows_kernel<32, 8, false, false>, &dwconv_rows_kernel<32, 16, false, false>, &dwconv_rows_kernel<32, 24, false, false>, &dwconv_rows_kernel<32, 32, false, false>, &dwconv_rows_kernel<32, 40, false, false>, &dwconv_rows_kernel<32, 48, false, false>},
    {&dwconv_rows_kernel<40, 4, false, false>, &dwconv_rows_kernel<40, 8, false, false>, &dwconv_rows_kernel<40, 16, false, false>, &dwconv_rows_kernel<40, 24, false, false>, &dwconv_rows_kernel<40, 32, false, false>, &dwconv_rows_kernel<40, 40, false, false>, &dwconv_rows_kernel<40, 48, false, false>},
    {&dwconv_rows_kernel<48, 4, false, false>, &dwconv_rows_kernel<48, 8, false, false>, &dwconv_rows_kernel<48, 16, false, false>, &dwconv_rows_kernel<48, 24, false, false>, &dwconv_rows_kernel<48, 32, false, false>, &dwconv_rows_kernel<48, 40, false, false>, &dwconv_rows_kernel<48, 48, false, false>}};
}  // namespace pt
