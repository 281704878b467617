// Instantiates the long-row FWD / DX kernels on the BF16 matrix cores with
// three-way split operands, 16-byte row moves (L % 4 == 0, 16-byte
// aligned tensors; tap buckets of 32).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// [dx][row bucket][tap bucket]
const RowsLongFn kRowsLongS3TableVec[2][kNumLongLB][kNumLongS3KB] = {
    {
        {&dwconv_rows_long_s3_kernel<64, 32, false, true>, &dwconv_rows_long_s3_kernel<64, 64, false, true>, &dwconv_rows_long_s3_kernel<64, 96, false, true>, &dwconv_rows_long_s3_kernel<64, 128, false, true>, &dwconv_rows_long_s3_kernel<64, 160, false, true>, &dwconv_rows_long_s3_kernel<64, 192, false, true>, &dwconv_rows_long_s3_kernel<64, 224, false, true>, &dwconv_rows_long_s3_kernel<64, 256, false, true>},
        {&dwconv_rows_long_s3_kernel<96, 32, false, true>, &dwconv_rows_long_s3_kernel<96, 64, false, true>, &dwconv_rows_long_s3_kernel<96, 96, false, true>, &dwconv_rows_long_s3_kernel<96, 128, false, true>, &dwconv_rows_long_s3_kernel<96, 160, false, true>, &dwconv_rows_long_s3_kernel<96, 192, false, true>, &dwconv_rows_long_s3_kernel<96, 224, false, true>, &dwconv_rows_long_s3_kernel<96, 256, false, true>},
        {&dwconv_rows_long_s3_kernel<128, 32, false, true>, &dwconv_rows_long_s3_kernel<128, 64, false, true>, &dwconv_rows_long_s3_kernel<128, 96, false, true>, &dwconv_rows_long_s3_kernel<128, 128, false, true>, &dwconv_rows_long_s3_kernel<128, 160, false, true>, &dwconv_rows_long_s3_kernel<128, 192, false, true>, &dwconv_rows_long_s3_kernel<128, 224, false, true>, &dwconv_rows_long_s3_kernel<128, 256, false, true>},
        {&dwconv_rows_long_s3_kernel<160, 32, false, true>, &dwconv_rows_long_s3_kernel<160, 64, false, true>, &dwconv_rows_long_s3_kernel<160, 96, false, true>, &dwconv_rows_long_s3_kernel<160, 128, false, true>, &dwconv_rows_long_s3_kernel<160, 160, false, true>, &dwconv_rows_long_s3_kernel<160, 192, false, true>, &dwconv_rows_long_s3_kernel<160, 224, false, true>, &dwconv_rows_long_s3_kernel<160, 256, false, true>},
        {&dwconv_rows_long_s3_kernel<192, 32, false, true>, &dwconv_rows_long_s3_kernel<192, 64, false, true>, &dwconv_rows_long_s3_kernel<192, 96, false, true>, &dwconv_rows_long_s3_kernel<192, 128, false, true>, &dwconv_rows_long_s3_kernel<192, 160, false, true>, &dwconv_rows_long_s3_kernel<192, 192, false, true>, &dwconv_rows_long_s3_kernel<192, 224, false, true>, &dwconv_rows_long_s3_kernel<192, 256, false, true>},
    },
    {
        {&dwconv_rows_long_s3_kernel<64, 32, true, true>, &dwconv_rows_long_s3_kernel<64, 64, true, true>, &dwconv_rows_long_s3_kernel<64, 96, true, true>, &dwconv_rows_long_s3_kernel<64, 128, true, true>, &dwconv_rows_long_s3_kernel<64, 160, true, true>, &dwconv_rows_long_s3_kernel<64, 192, true, true>, &dwconv_rows_long_s3_kernel<64, 224, true, true>, &dwconv_rows_long_s3_kernel<64, 256, true, true>},
        {&dwconv_rows_long_s3_kernel<96, 32, true, true>, &dwconv_rows_long_s3_kernel<96, 64, true, true>, &dwconv_rows_long_s3_kernel<96, 96, true, true>, &dwconv_rows_long_s3_kernel<96, 128, true, true>, &dwconv_rows_long_s3_kernel<96, 160, true, true>, &dwconv_rows_long_s3_kernel<96, 192, true, true>, &dwconv_rows_long_s3_kernel<96, 224, true, true>, &dwconv_rows_long_s3_kernel<96, 256, true, true>},
        {&dwconv_rows_long_s3_kernel<128, 32, true, true>, &dwconv_rows_long_s3_kernel<128, 64, true, true>, &dwconv_rows_long_s3_kernel<128, 96, true, true>, &dwconv_rows_long_s3_kernel<128, 128, true, true>, &dwconv_rows_long_s3_kernel<128, 160, true, true>, &dwconv_rows_long_s3_kernel<128, 192, true, true>, &dwconv_rows_long_s3_kernel<128, 224, true, true>, &dwconv_rows_long_s3_kernel<128, 256, true, true>},
        {&dwconv_rows_long_s3_kernel<160, 32, true, true>, &dwconv_rows_long_s3_kernel<160, 64, true, true>, &dwconv_rows_long_s3_kernel<160, 96, true, true>, &dwconv_rows_long_s3_kernel<160, 128, true, true>, &dwconv_rows_long_s3_kernel<160, 160, true, true>, &dwconv_rows_long_s3_kernel<160, 192, true, true>, &dwconv_rows_long_s3_kernel<160, 224, true, true>, &dwconv_rows_long_s3_kernel<160, 256, true, true>},
        {&dwconv_rows_long_s3_kernel<192, 32, true, true>, &dwconv_rows_long_s3_kernel<192, 64, true, true>, &dwconv_rows_long_s3_kernel<192, 96, true, true>, &dwconv_rows_long_s3_kernel<192, 128, true, true>, &dwconv_rows_long_s3_kernel<192, 160, true, true>, &dwconv_rows_long_s3_kernel<192, 192, true, true>, &dwconv_rows_long_s3_kernel<192, 224, true, true>, &dwconv_rows_long_s3_kernel<192, 256, true, true>},
    },
};
}  // namespace pt
