// Instantiates the short-tap streaming FWD / DX kernels (K = 1 .. 9).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const StreamFn kStreamTable[2][kStreamMaxK] = {
    {&dwconv_stream_kernel<1, false>, &dwconv_stream_kernel<2, false>, &dwconv_stream_kernel<3, false>,
     &dwconv_stream_kernel<4, false>, &dwconv_stream_kernel<5, false>, &dwconv_stream_kernel<6, false>,
     &dwconv_stream_kernel<7, false>, &dwconv_stream_kernel<8, false>, &dwconv_stream_kernel<9, false>},
    {&dwconv_stream_kernel<1, true>, &dwconv_stream_kernel<2, true>, &dwconv_stream_kernel<3, true>,
     &dwconv_stream_kernel<4, true>, &dwconv_stream_kernel<5, true>, &dwconv_stream_kernel<6, true>,
     &dwconv_stream_kernel<7, true>, &dwconv_stream_kernel<8, true>, &dwconv_stream_kernel<9, true>}};
const StreamFn kStreamTablePL[2][kStreamMaxK] = {
    {&dwconv_stream_kernel<1, false, kCpolNone>, &dwconv_stream_kernel<2, false, kCpolNone>, &dwconv_stream_kernel<3, false, kCpolNone>,
     &dwconv_stream_kernel<4, false, kCpolNone>, &dwconv_stream_kernel<5, false, kCpolNone>, &dwconv_stream_kernel<6, false, kCpolNone>,
     &dwconv_stream_kernel<7, false, kCpolNone>, &dwconv_stream_kernel<8, false, kCpolNone>, &dwconv_stream_kernel<9, false, kCpolNone>},
    {&dwconv_stream_kernel<1, true, kCpolNone>, &dwconv_stream_kernel<2, true, kCpolNone>, &dwconv_stream_kernel<3, true, kCpolNone>,
     &dwconv_stream_kernel<4, true, kCpolNone>, &dwconv_stream_kernel<5, true, kCpolNone>, &dwconv_stream_kernel<6, true, kCpolNone>,
     &dwconv_stream_kernel<7, true, kCpolNone>, &dwconv_stream_kernel<8, true, kCpolNone>, &dwconv_stream_kernel<9, true, kCpolNone>}};
}  // namespace pt
