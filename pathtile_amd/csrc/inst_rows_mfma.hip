// Instantiates the channel-group matrix-core FWD / DX kernels.
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
const RowsCgFn kRowsCgTable[2][3] = {
    {&dwconv_rows_cg_kernel<16, false, 2>, &dwconv_rows_cg_kernel<32, false, 2>,
     &dwconv_rows_cg_kernel<48, false, 2>},
    {&dwconv_rows_cg_kernel<16, true, 2>, &dwconv_rows_cg_kernel<32, true, 2>,
     &dwconv_rows_cg_kernel<48, true, 2>}};
const RowsCgFn kRowsCg16Table[2] = {&dwconv_rows_cg_kernel<48, false, 2, 16, 1>,
                                    &dwconv_rows_cg_kernel<48, true, 2, 16, 1>};
const RowsCgFn kRowsCgTablePL[2][3] = {
    {&dwconv_rows_cg_kernel<16, false, 2, kRowsCgWaves, 2, kCpolNone>,
     &dwconv_rows_cg_kernel<32, false, 2, kRowsCgWaves, 2, kCpolNone>,
     &dwconv_rows_cg_kernel<48, false, 2, kRowsCgWaves, 2, kCpolNone>},
    {&dwconv_rows_cg_kernel<16, true, 2, kRowsCgWaves, 2, kCpolNone>,
     &dwconv_rows_cg_kernel<32, true, 2, kRowsCgWaves, 2, kCpolNone>,
     &dwconv_rows_cg_kernel<48, true, 2, kRowsCgWaves, 2, kCpolNone>}};
const RowsCgFn kRowsCg16TablePL[2] = {&dwconv_rows_cg_kernel<48, false, 2, 16, 1, kCpolNone>,
                                      &dwconv_rows_cg_kernel<48, true, 2, 16, 1, kCpolNone>};
}  // namespace pt
