// Instantiates the long-row kernels (L up to 192, K up to 256; row buckets
// of 32 from 64, tap buckets of 64).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
// FWD / DX with dword row moves: [dx][row bucket][tap bucket]
const RowsLongFn kRowsLongTable[2][kNumLongLB][4] = {
    {
        {&dwconv_rows_long_kernel<64, 64, false, false>, &dwconv_rows_long_kernel<64, 128, false, false>, &dwconv_rows_long_kernel<64, 192, false, false>, &dwconv_rows_long_kernel<64, 256, false, false>},
        {&dwconv_rows_long_kernel<96, 64, false, false>, &dwconv_rows_long_kernel<96, 128, false, false>, &dwconv_rows_long_kernel<96, 192, false, false>, &dwconv_rows_long_kernel<96, 256, false, false>},
        {&dwconv_rows_long_kernel<128, 64, false, false>, &dwconv_rows_long_kernel<128, 128, false, false>, &dwconv_rows_long_kernel<128, 192, false, false>, &dwconv_rows_long_kernel<128, 256, false, false>},
        {&dwconv_rows_long_kernel<160, 64, false, false>, &dwconv_rows_long_kernel<160, 128, false, false>, &dwconv_rows_long_kernel<160, 192, false, false>, &dwconv_rows_long_kernel<160, 256, false, false>},
        {&dwconv_rows_long_kernel<192, 64, false, false>, &dwconv_rows_long_kernel<192, 128, false, false>, &dwconv_rows_long_kernel<192, 192, false, false>, &dwconv_rows_long_kernel<192, 256, false, false>},
    },
    {
        {&dwconv_rows_long_kernel<64, 64, true, false>, &dwconv_rows_long_kernel<64, 128, true, false>, &dwconv_rows_long_kernel<64, 192, true, false>, &dwconv_rows_long_kernel<64, 256, true, false>},
        {&dwconv_rows_long_kernel<96, 64, true, false>, &dwconv_rows_long_kernel<96, 128, true, false>, &dwconv_rows_long_kernel<96, 192, true, false>, &dwconv_rows_long_kernel<96, 256, true, false>},
        {&dwconv_rows_long_kernel<128, 64, true, false>, &dwconv_rows_long_kernel<128, 128, true, false>, &dwconv_rows_long_kernel<128, 192, true, false>, &dwconv_rows_long_kernel<128, 256, true, false>},
        {&dwconv_rows_long_kernel<160, 64, true, false>, &dwconv_rows_long_kernel<160, 128, true, false>, &dwconv_rows_long_kernel<160, 192, true, false>, &dwconv_rows_long_kernel<160, 256, true, false>},
        {&dwconv_rows_long_kernel<192, 64, true, false>, &dwconv_rows_long_kernel<192, 128, true, false>, &dwconv_rows_long_kernel<192, 192, true, false>, &dwconv_rows_long_kernel<192, 256, true, false>},
    },
};
// DK: [16-byte staging][row bucket]
const DkLongFn kDkLongTable[2][kNumLongLB] = {
    {&dwconv_dk_long_kernel<64, false>, &dwconv_dk_long_kernel<96, false>, &dwconv_dk_long_kernel<128, false>, &dwconv_dk_long_kernel<160, false>, &dwconv_dk_long_kernel<192, false>},
    {&dwconv_dk_long_kernel<64, true>, &dwconv_dk_long_kernel<96, true>, &dwconv_dk_long_kernel<128, true>, &dwconv_dk_long_kernel<160, true>, &dwconv_dk_long_kernel<192, true>},
};
// Split DK, staged (row buckets 64 and 96): [16-byte staging][bucket]
const DkLongFn kDkLongS3Table[2][kNumLongDkStagedLB] = {
    {&dwconv_dk_long_s3_kernel<64, false>, &dwconv_dk_long_s3_kernel<96, false>},
    {&dwconv_dk_long_s3_kernel<64, true>, &dwconv_dk_long_s3_kernel<96, true>},
};
// Split DK, operands loaded in place (row buckets 128, 160, 192)
const DkLongFn kDkLongS3RTable[kNumLongLB - kNumLongDkStagedLB] = {
    &dwconv_dk_long_s3r_kernel<128>, &dwconv_dk_long_s3r_kernel<160>, &dwconv_dk_long_s3r_kernel<192>};
}  // namespace pt
