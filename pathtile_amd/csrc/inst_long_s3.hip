// Instantiates the long-row FWD / DX kernels on the BF16 matrix cores with
// three-way split operands, dword row moves (tap buckets of 32).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// [dx][row bucket][tap bucket]
const RowsLongFn kRowsLongS3Table[2][kNumLongLB][kNumLongS3KB] = {
    {
        {&dwconv_rows_long_s3_kernel<64, 32, false, false>, &dwconv_rows_long_s3_kernel<64, 64, false, false>, &dwconv_rows_long_s3_kernel<64, 96, false, false>, &dwconv_rows_long_s3_kernel<64, 128, false, false>, &dwconv_rows_long_s3_kernel<64, 160, false, false>, &dwconv_rows_long_s3_kernel<64, 192, false, false>, &dwconv_rows_long_s3_kernel<64, 224, false, false>, &dwconv_rows_long_s3_kernel<64, 256, false, false>},
        {&dwconv_rows_long_s3_kernel<96, 32, false, false>, &dwconv_rows_long_s3_kernel<96, 64, false, false>, &dwconv_rows_long_s3_kernel<96, 96, false, false>, &dwconv_rows_long_s3_kernel<96, 128, false, false>, &dwconv_rows_long_s3_kernel<96, 160, false, false>, &dwconv_rows_long_s3_kernel<96, 192, false, false>, &dwconv_rows_long_s3_kernel<96, 224, false, false>, &dwconv_rows_long_s3_kernel<96, 256, false, false>},
        {&dwconv_rows_long_s3_kernel<128, 32, false, false>, &dwconv_rows_long_s3_kernel<128, 64, false, false>, &dwconv_rows_long_s3_kernel<128, 96, false, false>, &dwconv_rows_long_s3_kernel<128, 128, false, false>, &dwconv_rows_long_s3_kernel<128, 160, false, false>, &dwconv_rows_long_s3_kernel<128, 192, false, false>, &dwconv_rows_long_s3_kernel<128, 224, false, false>, &dwconv_rows_long_s3_kernel<128, 256, false, false>},
        {&dwconv_rows_long_s3_kernel<160, 32, false, false>, &dwconv_rows_long_s3_kernel<160, 64, false, false>, &dwconv_rows_long_s3_kernel<160, 96, false, false>, &dwconv_rows_long_s3_kernel<160, 128, false, false>, &dwconv_rows_long_s3_kernel<160, 160, false, false>, &dwconv_rows_long_s3_kernel<160, 192, false, false>, &dwconv_rows_long_s3_kernel<160, 224, false, false>, &dwconv_rows_long_s3_kernel<160, 256, false, false>},
        {&dwconv_rows_long_s3_kernel<192, 32, false, false>, &dwconv_rows_long_s3_kernel<192, 64, false, false>, &dwconv_rows_long_s3_kernel<192, 96, false, false>, &dwconv_rows_long_s3_kernel<192, 128, false, false>, &dwconv_rows_long_s3_kernel<192, 160, false, false>, &dwconv_rows_long_s3_kernel<192, 192, false, false>, &dwconv_rows_long_s3_kernel<192, 224, false, false>, &dwconv_rows_long_s3_kernel<192, 256, false, false>},
    },
    {
        {&dwconv_rows_long_s3_kernel<64, 32, true, false>, &dwconv_rows_long_s3_kernel<64, 64, true, false>, &dwconv_rows_long_s3_kernel<64, 96, true, false>, &dwconv_rows_long_s3_kernel<64, 128, true, false>, &dwconv_rows_long_s3_kernel<64, 160, true, false>, &dwconv_rows_long_s3_kernel<64, 192, true, false>, &dwconv_rows_long_s3_kernel<64, 224, true, false>, &dwconv_rows_long_s3_kernel<64, 256, true, false>},
        {&dwconv_rows_long_s3_kernel<96, 32, true, false>, &dwconv_rows_long_s3_kernel<96, 64, true, false>, &dwconv_rows_long_s3_kernel<96, 96, true, false>, &dwconv_rows_long_s3_kernel<96, 128, true, false>, &dwconv_rows_long_s3_kernel<96, 160, true, false>, &dwconv_rows_long_s3_kernel<96, 192, true, false>, &dwconv_rows_long_s3_kernel<96, 224, true, false>, &dwconv_rows_long_s3_kernel<96, 256, true, false>},
        {&dwconv_rows_long_s3_kernel<128, 32, true, false>, &dwconv_rows_long_s3_kernel<128, 64, true, false>, &dwconv_rows_long_s3_kernel<128, 96, true, false>, &dwconv_rows_long_s3_kernel<128, 128, true, false>, &dwconv_rows_long_s3_kernel<128, 160, true, false>, &dwconv_rows_long_s3_kernel<128, 192, true, false>, &dwconv_rows_long_s3_kernel<128, 224, true, false>, &dwconv_rows_long_s3_kernel<128, 256, true, false>},
        {&dwconv_rows_long_s3_kernel<160, 32, true, false>, &dwconv_rows_long_s3_kernel<160, 64, true, false>, &dwconv_rows_long_s3_kernel<160, 96, true, false>, &dwconv_rows_long_s3_kernel<160, 128, true, false>, &dwconv_rows_long_s3_kernel<160, 160, true, false>, &dwconv_rows_long_s3_kernel<160, 192, true, false>, &dwconv_rows_long_s3_kernel<160, 224, true, false>, &dwconv_rows_long_s3_kernel<160, 256, true, false>},
        {&dwconv_rows_long_s3_kernel<192, 32, true, false>, &dwconv_rows_long_s3_kernel<192, 64, true, false>, &dwconv_rows_long_s3_kernel<192, 96, true, false>, &dwconv_rows_long_s3_kernel<192, 128, true, false>, &dwconv_rows_long_s3_kernel<192, 160, true, false>, &dwconv_rows_long_s3_kernel<192, 192, true, false>, &dwconv_rows_long_s3_kernel<192, 224, true, false>, &dwconv_rows_long_s3_kernel<192, 256, true, false>},
    },
};
// dynamic LDS bytes: [dx][row bucket][tap bucket]
const size_t kRowsLongS3Lds[2][kNumLongLB][kNumLongS3KB] = {
    {
        {rows_long_s3_lds_bytes<64, 32, false>(), rows_long_s3_lds_bytes<64, 64, false>(), rows_long_s3_lds_bytes<64, 96, false>(), rows_long_s3_lds_bytes<64, 128, false>(), rows_long_s3_lds_bytes<64, 160, false>(), rows_long_s3_lds_bytes<64, 192, false>(), rows_long_s3_lds_bytes<64, 224, false>(), rows_long_s3_lds_bytes<64, 256, false>()},
        {rows_long_s3_lds_bytes<96, 32, false>(), rows_long_s3_lds_bytes<96, 64, false>(), rows_long_s3_lds_bytes<96, 96, false>(), rows_long_s3_lds_bytes<96, 128, false>(), rows_long_s3_lds_bytes<96, 160, false>(), rows_long_s3_lds_bytes<96, 192, false>(), rows_long_s3_lds_bytes<96, 224, false>(), rows_long_s3_lds_bytes<96, 256, false>()},
        {rows_long_s3_lds_bytes<128, 32, false>(), rows_long_s3_lds_bytes<128, 64, false>(), rows_long_s3_lds_bytes<128, 96, false>(), rows_long_s3_lds_bytes<128, 128, false>(), rows_long_s3_lds_bytes<128, 160, false>(), rows_long_s3_lds_bytes<128, 192, false>(), rows_long_s3_lds_bytes<128, 224, false>(), rows_long_s3_lds_bytes<128, 256, false>()},
        {rows_long_s3_lds_bytes<160, 32, false>(), rows_long_s3_lds_bytes<160, 64, false>(), rows_long_s3_lds_bytes<160, 96, false>(), rows_long_s3_lds_bytes<160, 128, false>(), rows_long_s3_lds_bytes<160, 160, false>(), rows_long_s3_lds_bytes<160, 192, false>(), rows_long_s3_lds_bytes<160, 224, false>(), rows_long_s3_lds_bytes<160, 256, false>()},
        {rows_long_s3_lds_bytes<192, 32, false>(), rows_long_s3_lds_bytes<192, 64, false>(), rows_long_s3_lds_bytes<192, 96, false>(), rows_long_s3_lds_bytes<192, 128, false>(), rows_long_s3_lds_bytes<192, 160, false>(), rows_long_s3_lds_bytes<192, 192, false>(), rows_long_s3_lds_bytes<192, 224, false>(), rows_long_s3_lds_bytes<192, 256, false>()},
    },
    {
        {rows_long_s3_lds_bytes<64, 32, true>(), rows_long_s3_lds_bytes<64, 64, true>(), rows_long_s3_lds_bytes<64, 96, true>(), rows_long_s3_lds_bytes<64, 128, true>(), rows_long_s3_lds_bytes<64, 160, true>(), rows_long_s3_lds_bytes<64, 192, true>(), rows_long_s3_lds_bytes<64, 224, true>(), rows_long_s3_lds_bytes<64, 256, true>()},
        {rows_long_s3_lds_bytes<96, 32, true>(), rows_long_s3_lds_bytes<96, 64, true>(), rows_long_s3_lds_bytes<96, 96, true>(), rows_long_s3_lds_bytes<96, 128, true>(), rows_long_s3_lds_bytes<96, 160, true>(), rows_long_s3_lds_bytes<96, 192, true>(), rows_long_s3_lds_bytes<96, 224, true>(), rows_long_s3_lds_bytes<96, 256, true>()},
        {rows_long_s3_lds_bytes<128, 32, true>(), rows_long_s3_lds_bytes<128, 64, true>(), rows_long_s3_lds_bytes<128, 96, true>(), rows_long_s3_lds_bytes<128, 128, true>(), rows_long_s3_lds_bytes<128, 160, true>(), rows_long_s3_lds_bytes<128, 192, true>(), rows_long_s3_lds_bytes<128, 224, true>(), rows_long_s3_lds_bytes<128, 256, true>()},
        {rows_long_s3_lds_bytes<160, 32, true>(), rows_long_s3_lds_bytes<160, 64, true>(), rows_long_s3_lds_bytes<160, 96, true>(), rows_long_s3_lds_bytes<160, 128, true>(), rows_long_s3_lds_bytes<160, 160, true>(), rows_long_s3_lds_bytes<160, 192, true>(), rows_long_s3_lds_bytes<160, 224, true>(), rows_long_s3_lds_bytes<160, 256, true>()},
        {rows_long_s3_lds_bytes<192, 32, true>(), rows_long_s3_lds_bytes<192, 64, true>(), rows_long_s3_lds_bytes<192, 96, true>(), rows_long_s3_lds_bytes<192, 128, true>(), rows_long_s3_lds_bytes<192, 160, true>(), rows_long_s3_lds_bytes<192, 192, true>(), rows_long_s3_lds_bytes<192, 224, true>(), rows_long_s3_lds_bytes<192, 256, true>()},
    },
};
}  // namespace pt
