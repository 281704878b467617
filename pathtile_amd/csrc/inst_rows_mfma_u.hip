// Instantiates the channel-group matrix-core FWD / DX kernels for rows that
// are not whole float4s (L % 4 != 0).
#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"

namespace pt {
template <int LMAX, bool DX, int HC, int NIN, int CPOL>
constexpr RowsCgFn kU = &dwconv_rows_cg_kernel<LMAX, DX, 2, HC, NIN, CPOL, false>;

const RowsCgFn kRowsCgTableU[2][3] = {
    {kU<16, false, kRowsCgWaves, 2, kCpolNT>, kU<32, false, kRowsCgWaves, 2, kCpolNT>,
     kU<48, false, kRowsCgWaves, 2, kCpolNT>},
    {kU<16, true, kRowsCgWaves, 2, kCpolNT>, kU<32, true, kRowsCgWaves, 2, kCpolNT>,
     kU<48, true, kRowsCgWaves, 2, kCpolNT>}};
const RowsCgFn kRowsCgTableUPL[2][3] = {
    {kU<16, false, kRowsCgWaves, 2, kCpolNone>, kU<32, false, kRowsCgWaves, 2, kCpolNone>,
     kU<48, false, kRowsCgWaves, 2, kCpolNone>},
    {kU<16, true, kRowsCgWaves, 2, kCpolNone>, kU<32, true, kRowsCgWaves, 2, kCpolNone>,
     kU<48, true, kRowsCgWaves, 2, kCpolNone>}};
const RowsCgFn kRowsCg16TableU[2] = {kU<48, false, 16, 1, kCpolNT>, kU<48, true, 16, 1, kCpolNT>};
const RowsCgFn kRowsCg16TableUPL[2] = {kU<48, false, 16, 1, kCpolNone>,
                                       kU<48, true, 16, 1, kCpolNone>};
}  // namespace pt
