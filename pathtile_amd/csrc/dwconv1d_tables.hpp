// dwconv1d_tables.hpp — dispatch tables of the depthwise Conv1D kernels.
// Each table is defined (and its kernels instantiated) in its own
// translation unit so the build compiles them in parallel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pt {

constexpr int kNumLB = 6;  // row buckets 8, 16, ..., 48
constexpr int kNumKB = 7;  // tap buckets below
constexpr int kKBuckets[kNumKB] = {4, 8, 16, 24, 32, 40, 48};

using RowsFn = void (*)(const float*, const float*, float*, int, int, int,
                        uint32_t, uint32_t, uint32_t, uint32_t, uint32_t);
using DkFn = void (*)(const float*, const float*, float*, int, int, int, int,
                      int, int, uint32_t, int);
using DkMfmaFn = void (*)(const float*, const float*, float*, int, int, int,
                          int, int, int, uint32_t, int);

// [row bucket][tap bucket]; V = 16-byte aligned rows (dwordx4), S = dword.
extern const RowsFn kFwdTableV[kNumLB][kNumKB];
extern const RowsFn kFwdTableS[kNumLB][kNumKB];
extern const RowsFn kDxTableV[kNumLB][kNumKB];
extern const RowsFn kDxTableS[kNumLB][kNumKB];
// the V tables with plain (not non-temporal) input loads
extern const RowsFn kFwdTableVP[kNumLB][kNumKB];
extern const RowsFn kDxTableVP[kNumLB][kNumKB];
// short-tap streaming FWD / DX: [0 = FWD, 1 = DX][K - 1], K = 1 .. 9
using StreamFn = void (*)(const float*, const float*, float*, int, int, uint64_t,
                          uint64_t);
extern const StreamFn kStreamTable[2][9];
extern const StreamFn kStreamTablePL[2][9];  // plain input loads
extern const DkFn kDkTableV[kNumLB][kNumKB];
extern const DkFn kDkTableS[kNumLB][kNumKB];
// matrix-core DK by row bucket 16, 32, 48
extern const DkMfmaFn kDkMfmaTable[3];
using DkCgFn = void (*)(const float*, const float*, float*, int, int, int, int,
                        int, uint32_t, int);
// channel-group matrix-core DK by row bucket 16, 32, 48; NT: non-temporal
// loads (tensors of at least 256 MiB)
extern const DkCgFn kDkCgTable[3];
extern const DkCgFn kDkCgTableNT[3];
// the same staging dwords (any row length, 4-byte aligned tensors)
extern const DkCgFn kDkCgTable1[3];
extern const DkCgFn kDkCgTable1NT[3];
// row bucket 48 with two channels per wave, 16-byte chunks, non-temporal
extern const DkCgFn kDkCgPairNT;
using RowsCgFn = void (*)(const float*, const float*, float*, int, int, int,
                          int, int, uint32_t);
// channel-group matrix-core FWD / DX: [0 = FWD, 1 = DX][row bucket 16, 32, 48]
extern const RowsCgFn kRowsCgTable[2][3];
// 16-channel workgroups with one input stage, row bucket 48: [0 = FWD, 1 = DX]
extern const RowsCgFn kRowsCg16Table[2];
// the same with plain (not non-temporal) input loads
extern const RowsCgFn kRowsCgTablePL[2][3];
extern const RowsCgFn kRowsCg16TablePL[2];
// the four tables above for rows that are not whole float4s (L % 4 != 0)
extern const RowsCgFn kRowsCgTableU[2][3];
extern const RowsCgFn kRowsCg16TableU[2];
extern const RowsCgFn kRowsCgTableUPL[2][3];
extern const RowsCgFn kRowsCg16TableUPL[2];
// BF16 I/O (uint16_t bit patterns; FP32 taps, FP32 accumulation)
using RowsCgBf16Fn = void (*)(const uint16_t*, const float*, uint16_t*, int,
                              int, int, int, int, uint32_t);
using DkBf16Fn = void (*)(const uint16_t*, const uint16_t*, float*, int, int,
                            int, int, int, uint32_t, int);
extern const RowsCgBf16Fn kRowsCgTableBf16[2][2][3];
// 8-channel groups with plain input loads: [dx][row bucket]
extern const RowsCgBf16Fn kRowsCgTableBf16PL[2][3];
using DkClFn = void (*)(const float*, const float*, float*, int, int, int, int,
                       int, uint32_t);
extern const DkClFn kDkClTable[3];
using RowsLongFn = void (*)(const float*, const float*, float*, int, int, int, int);
using DkLongFn = void (*)(const float*, const float*, float*, int, int, int, int, int, int);
constexpr int kNumLongLB = 5;  // long-row buckets 64, 96, 128, 160, 192
extern const RowsLongFn kRowsLongTable[2][kNumLongLB][4];
extern const RowsLongFn kRowsLongTableVec[2][kNumLongLB][4];
constexpr int kNumLongS3KB = 8;  // split FWD / DX tap buckets 32, 64, ..., 256
extern const RowsLongFn kRowsLongS3Table[2][kNumLongLB][kNumLongS3KB];
extern const RowsLongFn kRowsLongS3TableVec[2][kNumLongLB][kNumLongS3KB];
extern const size_t kRowsLongS3Lds[2][kNumLongLB][kNumLongS3KB];
extern const DkLongFn kDkLongTable[2][kNumLongLB];
// Split DK: staged for row buckets 64 and 96 ([16-byte staging][bucket]),
// operands in place for 128, 160 and 192 ([bucket - 2]).
constexpr int kNumLongDkStagedLB = 2;
extern const DkLongFn kDkLongS3Table[2][kNumLongDkStagedLB];
extern const DkLongFn kDkLongS3RTable[kNumLongLB - kNumLongDkStagedLB];
extern const DkBf16Fn kDkBf16mmaTable[3];
extern const DkBf16Fn kDkBf16mmaTableNT[3];

}  // namespace pt
