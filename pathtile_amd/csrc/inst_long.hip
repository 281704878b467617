// Instantiates the long-row kernels (L up to 192, K up to 256; row buckets
// of 64).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// FWD / DX: [dx][row bucket][tap bucket]
const RowsLongFn kRowsLongTable[2][3][4] = {
    {
        {&dwconv_rows_long_kernel<64, 64, false>, &dwconv_rows_long_kernel<64, 128, false>, &dwconv_rows_long_kernel<64, 192, false>, &dwconv_rows_long_kernel<64, 256, false>},
        {&dwconv_rows_long_kernel<128, 64, false>, &dwconv_rows_long_kernel<128, 128, false>, &dwconv_rows_long_kernel<128, 192, false>, &dwconv_rows_long_kernel<128, 256, false>},
        {&dwconv_rows_long_kernel<192, 64, false>, &dwconv_rows_long_kernel<192, 128, false>, &dwconv_rows_long_kernel<192, 192, false>, &dwconv_rows_long_kernel<192, 256, false>},
    },
    {
        {&dwconv_rows_long_kernel<64, 64, true>, &dwconv_rows_long_kernel<64, 128, true>, &dwconv_rows_long_kernel<64, 192, true>, &dwconv_rows_long_kernel<64, 256, true>},
        {&dwconv_rows_long_kernel<128, 64, true>, &dwconv_rows_long_kernel<128, 128, true>, &dwconv_rows_long_kernel<128, 192, true>, &dwconv_rows_long_kernel<128, 256, true>},
        {&dwconv_rows_long_kernel<192, 64, true>, &dwconv_rows_long_kernel<192, 128, true>, &dwconv_rows_long_kernel<192, 192, true>, &dwconv_rows_long_kernel<192, 256, true>},
    },
};
const DkLongFn kDkLongTable[3] = {&dwconv_dk_long_kernel<64>, &dwconv_dk_long_kernel<128>,
                                  &dwconv_dk_long_kernel<192>};
}  // namespace pt
