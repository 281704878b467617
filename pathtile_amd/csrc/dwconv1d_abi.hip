// dwconv1d_abi.hip — host side of the depthwise Conv1D library: argument
// checks, launch geometry, dispatch and the C ABI of include/pathtile_hip.h.
// The kernels live in dwconv1d_kernels.hpp and are instantiated in the
// inst_*.hip translation units.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "dwconv1d_kernels.hpp"
#include "dwconv1d_tables.hpp"
#include "pathtile_hip.h"

namespace pt {

// Pass 2 of the deterministic DK: one wave per coefficient, lanes sum the
// batch-tile partials in a fixed order, then a fixed wave reduction.
__global__ __launch_bounds__(256) void dk_reduce_kernel(
    const float* __restrict__ partials, float* __restrict__ dk, int ncoef,
    int nbt) {
  const int lane = threadIdx.x & (kWave - 1);
  const int coef = blockIdx.x * (blockDim.x / kWave) + (int)(threadIdx.x / kWave);
  if (coef >= ncoef) return;
  const float* p = partials + (size_t)coef * (size_t)nbt;
  float acc = 0.0f;
  for (int q = lane; q < nbt; q += kWave) acc += p[q];
  acc = wave_sum(acc);
  if (lane == 0) dk[coef] = acc;
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p,
                                                        int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// Dispatch helpers
// ---------------------------------------------------------------------------
static int mfma_index(int L) { return (L + 15) / 16 - 1; }

// Static LDS of dwconv_dk_mfma_kernel<LMAX> (the workgroup's D, LMAX x
// (LMAX + 1) floats).
static int dk_mfma_static_lds(int L) {
  const int lmax = 16 * (mfma_index(L) + 1);
  return lmax * (lmax + 1) * (int)sizeof(float);
}

static int lbucket_index(int L) { return (L + 7) / 8 - 1; }
static int kbucket_index(int K) {
  for (int i = 0; i < kNumKB; ++i)
    if (K <= kKBuckets[i]) return i;
  return kNumKB - 1;
}

// ---------------------------------------------------------------------------
// Host-side validation and launch geometry
// ---------------------------------------------------------------------------
static int check_shape(int B, int H, int L, int K) {
  if (B < 0 || H < 0 || L < 1 || K < 1) return PT_ERR_SHAPE;
  if (L > kMaxL || K > kMaxK) return PT_ERR_SHAPE;
  const long long elems = (long long)B * (long long)H * (long long)L;
  if (elems >= (1LL << 31)) return PT_ERR_SHAPE;
  if ((long long)H * K * 4 >= (1LL << 31)) return PT_ERR_SHAPE;
  // a wave's 64-row tile must span < 2 GiB (buffer offsets, see kOob)
  if ((long long)kWave * H * L * 4 >= (1LL << 31)) return PT_ERR_SHAPE;
  return PT_OK;
}

static bool aligned(const void* p, uintptr_t a) {
  return ((uintptr_t)p & (a - 1)) == 0;
}

// --- device queries (cached per device / per kernel) -----------------------
// One device attribute of the current device, queried once per device.
// Entries are atomics because calls may come from several host threads;
// threads that race to fill an entry store the same value.
template <hipDeviceAttribute_t A>
static int device_attr(int fallback) {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    dev = 0;
  }
  const bool cached = dev >= 0 && dev < 64;
  if (cached) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, A, dev) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = fallback;
  }
  if (cached) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

static int num_cus() { return device_attr<hipDeviceAttributeMultiprocessorCount>(256); }

struct OccEntry {
  const void* fn;
  int block;
  size_t lds;
  int blocks;
};
static std::mutex g_occ_mu;
static OccEntry g_occ[512];
static int g_occ_n = 0;

// Resident workgroups per CU for (kernel, block size, dynamic LDS).
static int blocks_per_cu(const void* fn, int block, size_t lds) {
  {
    std::lock_guard<std::mutex> lk(g_occ_mu);
    for (int i = 0; i < g_occ_n; ++i)
      if (g_occ[i].fn == fn && g_occ[i].block == block && g_occ[i].lds == lds)
        return g_occ[i].blocks;
  }
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, block, lds) !=
          hipSuccess ||
      nb <= 0) {
    (void)hipGetLastError();
    nb = 1;
  }
  std::lock_guard<std::mutex> lk(g_occ_mu);
  if (g_occ_n < 512) g_occ[g_occ_n++] = OccEntry{fn, block, lds, nb};
  return nb;
}

// --- DK algorithm ----------------------------------------------------------
// Matrix-core (batch-contraction GEMM) kernel by default: it computes every
// (t, s) pair of the row window, which costs the matrix cores ~72 cycles per
// row at L = 48 whatever K is, well under the time the row takes to stream
// from HBM. The VALU lane-per-row kernel (the reference's structure) stays
// selectable with PATHTILE_DK_ALGO=valu for comparison.
enum DkAlgo { kDkValu = 0, kDkMfma = 1 };

static DkAlgo dk_algo(int L, int K) {
  const char* env = getenv("PATHTILE_DK_ALGO");
  (void)L;
  (void)K;
  if (env && strcmp(env, "valu") == 0) return kDkValu;
  return kDkMfma;
}

// A DK workgroup covers one channel and a batch tile of wpb waves x
// rows_per_wave samples. Rows per wave depend on the shape alone (not on the
// device), so the deterministic variant's workspace size needs no device:
// about 128 at large shapes (long per-wave runs stream worse, and the waves
// of the XCDs then stay within a compact address range), fewer at small
// shapes so the grid still fills the GPU.
constexpr long long kDkRowsDivisor = 16384;
constexpr double kDkMallBytes = 256.0 * 1024 * 1024;  // MI355X Infinity Cache

struct DkGeom {
  DkAlgo algo;
  bool cg;            // channel-group kernel
  bool nt;            // channel-group kernel with non-temporal loads
  int epc;            // channel-group kernel: floats per staging load (4 or 1)
  int cpw;            // channel-group kernel: channels per wave
  int wpb;
  int rows_per_wave;  // VALU: 64-sample chunks per wave; MFMA: samples;
                      // channel-group: samples per workgroup
  int nbt;            // partials per (h, j): batch tiles / sample ranges
  long long nblocks;  // workgroups
};

// Channel-group DK: groups of dk_cpw(L) channels per wave (one in the
// 48-column row bucket, two below; BF16 DK: two), at most 8 waves per
// workgroup. The FP32 kernel serves any row length (dk_cg_layout_ok); the
// BF16 one needs whole 16-byte aligned rows (dk_cg_ok, L % 4 == 0).
static int dk_cpw(int L) { return dk_cg_cpw(16 * (mfma_index(L) + 1)); }

static bool dk_cg_layout_ok(int H, int threads, int cpw) {
  const int wpb = threads / kWave;
  return wpb <= 8 && H % (cpw * wpb) == 0;
}

static bool dk_cg_ok(int H, int L, int threads, int cpw) {
  return L % 4 == 0 && dk_cg_layout_ok(H, threads, cpw);
}

// Staging width of the FP32 channel-group DK: 16-byte chunks when both
// tensors are 16-byte aligned and a group's segment (hc L floats) and a
// sample (H L floats) are whole chunks, dwords otherwise.
static int dk_cg_epc(int H, int L, int hc, bool vec16) {
  return vec16 && ((long long)hc * L) % 4 == 0 && ((long long)H * L) % 4 == 0 ? 4 : 1;
}

// Rows of 33-48 columns on tensors of at least 256 MiB (non-temporal
// loads): one channel per wave where a workgroup's segment (4 wpb L bytes)
// is a whole number of 64-byte units, else two channels per wave where H
// allows and the segments are then whole 16-byte chunks. Measured on MI355X over L = 33..48 at B16384
// H128 K48 with 128 threads (three interleaved rounds): one channel won at
// L = 40 and 48 (114.3 against 118.8 us, 122.7 against 125.7) and tied at
// 36; two won everywhere else, by up to 9% at even L (L38 111.8 against
// 119.6, L44 124.2 against 138.9, L46 125.3 against 137.1) and by 10-24%
// at odd L, where one channel per wave leaves dword staging (L37 115.7
// against 139.0, L41 122.8 against 155.7). Below 256 MiB one channel per
// wave stayed 5-7% faster at every L tried (B4096 H128 L33..47 K48).
static void dk_cg_staging(DkGeom& g, int H, int L, bool vec16) {
  g.cpw = dk_cpw(L);
  g.epc = dk_cg_epc(H, L, g.cpw * g.wpb, vec16);
  if (g.cpw == 1 && g.nt && ((long long)4 * g.wpb * L) % 64 != 0 &&
      H % (2 * g.wpb) == 0 && dk_cg_epc(H, L, 2 * g.wpb, vec16) == 4) {
    g.cpw = 2;
    g.epc = 4;
  }
}

static DkCgFn dk_cg_fn(bool nt, int epc, int cpw, int L) {
  if (cpw != dk_cpw(L)) return kDkCgPairNT;  // two channels per wave, 48 bucket
  const DkCgFn* t = epc == 4 ? (nt ? kDkCgTableNT : kDkCgTable)
                             : (nt ? kDkCgTable1NT : kDkCgTable1);
  return t[mfma_index(L)];
}

// Tensors of at least the 256 MiB MALL stream differently from smaller ones
// in the channel-group DK, so two settings depend on that size:
//  * loads: non-temporal from 256 MiB up (4-10% faster there, e.g. 128 vs
//    132 us at P), plain below (non-temporal loads cost small L = 16 / 32
//    shapes 11-20% in the tuner's per-launch protocol);
//  * interleaved sample ranges (a workgroup's successive steps lie nr steps
//    apart): from 256 MiB up, of the counts 2^k and 3 * 2^(k-1) in [8, 256]
//    the one nearest (by ratio; ties to the smaller) to 3 MiB / (bytes of one
//    4-sample step of one tensor). 3 MiB measured best at every row length;
//    at L = 16 and 32 it is 15-17% faster than the power of two nearest
//    2.5 MiB, and at L = 40, whose 3 MiB counts (38, 77) are neither form,
//    the neighbouring power of two is 4-8% faster than 38 or 77. Below
//    256 MiB: the power of two (8 .. 256) nearest to 2.5 MiB per step, which
//    keeps more steps per workgroup.
// Measured on MI355X over the 30 tuner shapes, P and S with the tuner's own
// protocol, both libraries on one box. Both depend on the shape only (not on
// the block size or the device).
static bool cg_large(int B, int H, int L) {
  return 4.0 * (double)B * (double)H * (double)L >= kDkMallBytes;
}

// Of the counts 2^k and 3 * 2^(k-1) in [8, 256], the one nearest (by ratio;
// ties to the smaller) to `want`.
static long long nearest_range_count(double want) {
  long long nr = 8;
  double best = 1e300;
  for (long long p = 8; p <= 256; p *= 2) {
    const long long cands[2] = {p, p + p / 2};
    for (long long c : cands) {
      if (c > 256) continue;
      const double d = fabs(log((double)c / want));
      if (d < best - 1e-12) {
        best = d;
        nr = c;
      }
    }
  }
  return nr;
}

static long long cg_ranges(int B, int H, int L) {
  const double step_bytes = (double)kCgStep * 4.0 * (double)H * (double)L;
  long long nr = 8;
  if (cg_large(B, H, L)) {
    nr = nearest_range_count(3.0 * 1024 * 1024 / step_bytes);
  } else {
    const double want = 2.5 * 1024 * 1024 / step_bytes;
    while (nr < 256 && (double)(nr * 2) <= want * 1.41421356) nr *= 2;
  }
  const long long tsteps = ((long long)B + kCgStep - 1) / kCgStep;
  if (nr > tsteps) nr = tsteps;
  return nr < 1 ? 1 : nr;
}

// BF16 DK on the BF16 matrix cores (16-sample steps):
//  * sample ranges: the 3 MiB count above for the 16-sample step, at every
//    tensor size (over the tuner's 30 shapes plus P, S and E2 in BF16 it was
//    1.4% faster in total than the 2.5 MiB power of two and 5% faster than
//    2 MiB);
//  * loads: non-temporal from 64 MiB per tensor up (4-9% faster there, e.g.
//    65 vs 69 us at P in BF16 and 234 vs 251 us at S), plain below (up to
//    20% faster on 32 MiB tensors).
// Measured on MI355X with interleaved rounds and a duplicate control.
constexpr double kBmNtBytes = 64.0 * 1024 * 1024;

static bool bm_nt(int B, int H, int L) {
  return 2.0 * (double)B * (double)H * (double)L >= kBmNtBytes;
}

static long long bm_ranges(int B, int H, int L) {
  const double step_bytes = (double)kBmStep * 2.0 * (double)H * (double)L;
  long long nr = nearest_range_count(3.0 * 1024 * 1024 / step_bytes);
  const long long tsteps = ((long long)B + kBmStep - 1) / kBmStep;
  if (nr > tsteps) nr = tsteps;
  return nr < 1 ? 1 : nr;
}

// Waves per workgroup of the channel-group DK: the caller's, raised at small
// K so that a workgroup's tap sums (cpw x waves channels x K taps) fill at
// least one 128-byte line, up to 8 waves and where H allows. Each workgroup
// adds its sums into dk with atomics, and every sample range adds into the
// same few lines: at B16384 H64 L16 K3 (dk is six lines, 128 ranges) two-wave
// workgroups took 25.2 us and eight-wave ones 23.0 (the deterministic
// variant, without atomics, 24.5-25.0 at every size); at B16384 H64 L24 K3
// 39.4 against 37.7, at B32768 H128 L40 K3 228.8 against 220.9, while at
// K = 8 the sizes tie (B16384 H64 L16 K8: 22.8-23.0 us). A wave's partial
// sums do not depend on its workgroup's size, so neither do the
// deterministic variant's bits.
static int dk_cg_waves(int H, int K, int cpw, int wpb) {
  const int want = (32 + cpw * K - 1) / (cpw * K);
  if (wpb >= want) return wpb;
  for (int w = want < 8 ? want : 8; w <= 8; ++w)
    if (H % (cpw * w) == 0) return w;
  for (int w = 8; w > wpb; --w)
    if (H % (cpw * w) == 0) return w;
  return wpb;
}

// device_cap: size the channel-group DK's ranges for the current device (a
// launch); without it the geometry depends on the shape alone and its
// range count bounds every launch's (the deterministic workspace size).
static DkGeom dk_geometry(int B, int H, int L, int K, int threads, bool vec16,
                          int esize = 4, bool device_cap = false) {
  DkGeom g;
  g.algo = dk_algo(L, K);
  g.wpb = threads / kWave;
  const long long wpb = g.wpb;
  const long long rows = (long long)B * H;
  g.cg = g.algo == kDkMfma && dk_cg_layout_ok(H, threads, dk_cpw(L));
  g.nt = g.cg && cg_large(B, H, L);
  g.epc = 4;
  g.cpw = dk_cpw(L);
  if (g.cg) {
    g.wpb = dk_cg_waves(H, K, g.cpw, g.wpb);
    dk_cg_staging(g, H, L, vec16);
    const long long ngroups = (long long)H / (g.cpw * g.wpb);
    long long nr = cg_ranges(B, H, L);
    // The stride rule was measured where its workgroups fill the resident
    // slots exactly (H a power of two). Where they overflow them, the few
    // left over run in a second round: B16384 H96 L48 K48 takes 128.8 us at
    // the rule's 48 ranges (2304 workgroups, 2048 slots) and 94.6 us at 42
    // (2016); B32768 H96 L48 K4 249 against 186 us. Cap at one round.
    if (device_cap) {
      const int mi = mfma_index(L);
      const DkCgFn fn = dk_cg_fn(g.nt, g.epc, g.cpw, L);
      const long long resident =
          (long long)blocks_per_cu((const void*)fn, g.wpb * kWave,
                                   cg_lds_bytes(16 * (mi + 1), g.wpb, L, g.cpw)) *
          num_cus();
      if (ngroups * nr > resident) nr = resident / ngroups;
      if (nr < 1) nr = 1;
    }
    g.rows_per_wave = 0;
    g.nbt = (int)nr;
    g.nblocks = ngroups * nr;
    return g;
  }
  long long rpw = (rows + kDkRowsDivisor - 1) / kDkRowsDivisor;
  long long tile;
  if (g.algo == kDkValu) {
    long long R = (rpw + kWave - 1) / kWave;  // 64-sample chunks per wave
    if (R < 1) R = 1;
    if (R > 2) R = 2;
    const long long chunks_per_h = ((long long)B + kWave - 1) / kWave;
    const long long rmax = (chunks_per_h + wpb - 1) / wpb;
    if (R > rmax) R = rmax < 1 ? 1 : rmax;
    g.rows_per_wave = (int)R;
    tile = wpb * R * kWave;
  } else {
    // Samples per load group of the MFMA kernel: 48 / 24 / 16 for row
    // buckets 16 / 32 / 48; rows per wave are whole groups.
    const long long grp = 48 / ((L + 15) / 16);
    const long long rcap = (128 + grp - 1) / grp * grp;
    rpw = (rpw + grp - 1) / grp * grp;
    if (rpw < grp) rpw = grp;
    if (rpw > rcap) rpw = rcap;
    const long long rmax = (((long long)B + wpb - 1) / wpb + grp - 1) / grp * grp;
    if (rpw > rmax) rpw = rmax;
    g.rows_per_wave = (int)rpw;
    tile = wpb * rpw;
  }
  g.nbt = (int)(((long long)B + tile - 1) / tile);
  if (g.nbt < 1) g.nbt = 1;
  g.nblocks = (long long)g.nbt * H;
  return g;
}

static bool valid_wpb(int wpb) {
  return wpb == 1 || wpb == 2 || wpb == 4 || wpb == 8 || wpb == 16;
}

static bool valid_dk_threads(int t) {
  return t >= kWave && t <= kMaxDkThreads && (t % kWave) == 0;
}

static int launch(const void* fn, uint32_t grid, uint32_t block, size_t lds,
                  void* stream, void** args) {
  hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(block), args, lds,
                                 (hipStream_t)stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return PT_ERR_HIP;
  }
  return PT_OK;
}

static int zero_fill(float* p, int n, void* stream) {
  if (n <= 0) return PT_OK;
  void* args[] = {&p, &n};
  const uint32_t grid = (uint32_t)((n + 255) / 256);
  return launch((const void*)&fill_zero_kernel, grid, 256, 0, stream, args);
}

// LDS of one FWD/DX wave: a 64-row tile at padded stride LMAX + 4.
static size_t rows_lds_per_wave(int L) {
  const int lmax = 8 * (lbucket_index(L) + 1);
  return (size_t)kWave * (size_t)(lmax + 4) * sizeof(float);
}

// 160 KiB: gfx950, the one target of this library.
static int max_lds_per_block() {
  return device_attr<hipDeviceAttributeMaxSharedMemoryPerBlock>(160 * 1024);
}

static int lds_per_cu() {
  return device_attr<hipDeviceAttributeMaxSharedMemoryPerMultiprocessor>(max_lds_per_block());
}

// Dynamic LDS that makes exactly `bpc` workgroups fit on a CU (at least
// `need` bytes, at most what one workgroup may allocate): the CU's LDS split
// bpc ways, in 1 KiB units so allocation granules never round bpc shares
// past the CU's capacity.
static size_t lds_for_blocks_per_cu(size_t need, size_t static_bytes, int bpc) {
  size_t share = (size_t)lds_per_cu() / (size_t)bpc / 1024 * 1024;
  if (share > (size_t)max_lds_per_block()) share = (size_t)max_lds_per_block();
  const size_t dyn = share > static_bytes ? share - static_bytes : 0;
  return dyn > need ? dyn : need;
}

// Useful FMAs of one row: sum over taps j of the outputs t whose input
// t + j - p lies in [0, L).
static long long useful_fma_per_row(int L, int K) {
  long long n = 0;
  const int p = K / 2;
  for (int j = 0; j < K; ++j) {
    const int s = j - p;
    const int lo = s < 0 ? -s : 0;
    const int hi = s > 0 ? L - s : L;
    if (hi > lo) n += hi - lo;
  }
  return n;
}

// Resident waves per CU for the FWD/DX tile kernel, measured on MI355X over
// every (row bucket, tap bucket) at B16384 H128: two waves per SIMD when the
// FMA chain is long (at least 0.7 L FMAs per element) so one wave's FMAs
// hide the other's memory time, or when tiles are small (L <= 16); one wave
// per SIMD otherwise, which streams HBM best. Waves per workgroup do not
// change this count, so they barely change the time. Small calls (at most
// eight tiles per CU) take two waves per SIMD whatever the chain, so every
// tile gets a wave in one round: B1000 H96 L37 K8 (1500 tiles) 16.4 against
// 11.1 us; at 4096 tiles the two counts tie, and from 8192 up one wave per
// SIMD stays faster (B8192 H128 L48 K4: 66.4 against 70.5 us).
static int rows_waves_per_cu(int L, int K, long long ntiles) {
  if (L <= 16 || ntiles <= 8LL * num_cus()) return 8;
  return 10 * useful_fma_per_row(L, K) >= 7LL * L * L ? 8 : 4;
}

// --- FWD / DX algorithm ----------------------------------------------------
// The channel-group matrix-core kernel costs the same whatever K is (it
// multiplies by the whole LMAX x LMAX band matrix of the row bucket); the VALU
// rows kernel's cost grows with the FMA chain. Rows of L % 4 == 0 from 16 to
// 48 columns take the matrix cores from the K of rows_mfma_min_k below;
// shorter ones once a row needs at least 10.5 (LMAX / L)^2 useful FMAs per
// output on average (LMAX = the row bucket 16, 32 or 48); below that the
// VALU kernel (bit-exact with the reference's fmaf chain) is as fast or
// faster. Rows of other lengths: kRowsOddMfmaRows below.
// Where the VALU serves, the tile kernel (a lane per row through an LDS
// transpose) runs, or the streaming kernel (float4 lanes, no LDS; rows of
// L % 4 == 0 floats, at most 9 taps) where the channel period would idle
// the tile kernel's grid (rows_path); both run the reference's chain bit
// for bit.
// PATHTILE_ROWS_ALGO=valu forces the VALU kernels everywhere (=tile: the
// tile kernel only, =stream: the streaming kernel wherever it can serve);
// =mfma forces the matrix cores wherever the layout allows them.
enum RowsAlgo { kRowsValu = 0, kRowsMfma = 1, kRowsTile = 2, kRowsStream = 3 };

// Input loads of the FWD / DX kernels: plain (cached) for tensors of at most
// 256 MiB, non-temporal above. Repeated calls on a tensor that small find
// part of it still in the 256 MiB MALL; measured on MI355X with
// back-to-back calls, plain loads were 8-14% faster there (matrix cores:
// B16384 H128 L32 K32 78.8 against 87.5 us, B8192 H128 L48 K48 61.8
// against 70.2; tile kernel: B16384 H128 L32 K8 78.1 against 87.4, B8192
// H128 L48 K4 60.3 against 67.7) and 2-7% slower from 320 MiB up (P 143.3
// against 136.1 us). Stores stay non-temporal: plain stores on top of plain
// loads were 1-25% slower at every size measured.
constexpr double kRowsPlainLoadBytes = 256.0 * 1024 * 1024;

static bool rows_plain_loads(int B, int H, int L) {
  return 4.0 * (double)B * (double)H * (double)L <= kRowsPlainLoadBytes;
}

// The matrix-core kernel stages the contiguous segments of kRowsCgWaves (or
// 16) channels in 16-byte chunks: with H % 8 == 0 a segment (HC L floats)
// and a sample (H L floats) are whole chunks at any L, so 16-byte aligned
// tensors are all it needs (rows of L % 4 != 0 take its A4 = false form).
static bool rows_cg_ok(int H, int L, const void* in, const void* out) {
  return H % kRowsCgWaves == 0 && aligned(in, 16) && aligned(out, 16) &&
         rows_cg_lds_bytes(L) <= (size_t)max_lds_per_block();
}

// Rows of L % 4 != 0 reach the VALU kernels a dword at a time; there the
// matrix cores measured 1.4-2.7x faster at every K from 2^18 rows (B * H)
// up (B16384 H128 L37 K4: 132 against 232 us; B4096 H64 L29 K4: 11.5
// against 23.9), and below that from 5 (LMAX / L)^2 useful FMAs per output
// (B1000 H96 L37: VALU 9.9 against 11.2 us at K = 4, a tie at K = 8, the
// matrix cores 0.89x at K = 12; B2048 H64 L45 likewise).
constexpr long long kRowsOddMfmaRows = 1LL << 18;

// Rows of L % 4 == 0 from 16 to 48 columns: the smallest K from which the
// matrix cores serve. Which kernel wins depends on how much of its row
// bucket L fills for each kernel (16, 32 or 48 columns for the matrix
// cores, steps of 8 for the VALU kernel), on the size of the call and, at
// 48 columns, on H and the load regime. Measured on MI355X (FWD,
// interleaved rounds, inputs rotated past the MALL below 256 MiB;
// matrix-core time / VALU time):
//  * calls of at least 2^17 rows (B x H): L16 K6 0.92-0.99; L20-32 and L44
//    K10-16 0.78-1.00 (K6-8 0.89-1.06); L36 and L40 K20 0.84-0.95 (K9-16
//    0.91-1.03 at L36, 1.00-1.13 at L40); L48 K10-16 0.91-0.98 on tensors
//    of at most 256 MiB with H <= 128, where above 256 MiB or at H = 256 the
//    two tie or the VALU kernel wins by up to 4%; K20 0.84-0.95 everywhere;
//  * smaller calls (B512 H128 to B1536 H96, 4-25 us), where the matrix
//    cores' fixed cost weighs more: L16 K12 0.90-0.98 (K9 up to 1.06), L20
//    K16 0.83-0.94, L24 K24 0.75-0.83 (K16 0.94-1.03), L28 and L32 K16
//    0.74-0.95 (K12 up to 1.10), L36 and L44 K24 0.71-0.94 (K16 up to
//    1.14), L40 K32 0.80-0.93 (K24 up to 1.07), L48 K24 0.79-0.97.
constexpr long long kRowsSmallCall = 1LL << 17;

static int rows_mfma_min_k(int L, int H, long long rows, bool plain) {
  const bool small = rows < kRowsSmallCall;
  switch (L) {
    case 16: return small ? 12 : 5;
    case 20: return small ? 16 : 9;
    case 24: return small ? 17 : 9;
    case 28:
    case 32: return small ? 13 : 9;
    case 36: return 17;
    case 40: return small ? 25 : 17;
    case 44: return small ? 17 : 9;
    default: return small || !plain || H > 128 ? 17 : 9;  // L = 48
  }
}

// forced: PT_ROWS_AUTO (the environment, then the rule), PT_ROWS_VALU or
// PT_ROWS_MATRIX (the caller's choice, over the environment).
static RowsAlgo rows_algo(int B, int H, int L, int K, int forced = PT_ROWS_AUTO) {
  if (forced == PT_ROWS_VALU) return kRowsValu;
  if (forced == PT_ROWS_MATRIX) return kRowsMfma;
  const char* env = getenv("PATHTILE_ROWS_ALGO");
  if (env && strcmp(env, "valu") == 0) return kRowsValu;
  if (env && strcmp(env, "tile") == 0) return kRowsTile;
  if (env && strcmp(env, "stream") == 0) return kRowsStream;
  if (env && strcmp(env, "mfma") == 0) return kRowsMfma;
  const long long lmax = 16LL * (mfma_index(L) + 1);
  const long long u2l = 2 * useful_fma_per_row(L, K) * L;
  if (L % 4 == 0) {
    if (L >= 16)
      return K >= rows_mfma_min_k(L, H, (long long)B * H, rows_plain_loads(B, H, L))
                 ? kRowsMfma : kRowsValu;
    // useful / L >= 10.5 (lmax / L)^2, in integers
    return u2l >= 21 * lmax * lmax ? kRowsMfma : kRowsValu;
  }
  if ((long long)B * H >= kRowsOddMfmaRows) return kRowsMfma;
  return u2l >= 10 * lmax * lmax ? kRowsMfma : kRowsValu;
}

// Launch of the channel-group kernel: one workgroup per (channel group,
// sample range), the ranges interleaved in 16-sample steps. As many ranges as
// fill the CUs with min(max_per_cu, resident) workgroups each (two 8-channel
// workgroups measured best where the LDS allows them, L <= 39; one above),
// rounded down: a grid a few workgroups past one round runs those few in a
// second round and nearly doubles the time (B16384 H160 L48 K48, 10
// channel groups: 26 ranges, 260 workgroups on 256 CUs, 276 us; 25 ranges
// fit one round).
// min_steps: fewer workgroups per CU while a workgroup would get fewer than
// this many steps (0: off). Two 8-channel FP32 workgroups per CU won from
// 4 steps each (B2048 H128 L24 K24 10.6 against 11.0 us, B4096 H96 L33 K40
// 26.5 against 28.9, B16384 H64 L35 K16 53.2 against 64.5), tied at 2 and
// lost below (E1 B1000 H96 L37 K48, 1.5 steps: 12.1 against 10.8; B1000
// H96 L36 K48 11.4 against 9.3; B2048 H64 L36 K48, 2 steps: 11.7 against
// 11.1), where one per CU runs each workgroup's steps back to back with no
// second workgroup competing for the CU.
// hc: channels (= waves) per workgroup; lds: dynamic LDS per workgroup;
// max_per_cu: workgroups per CU the range count is sized for (at most what
// fits).
template <typename T, typename Fn>
static int rows_cg_launch(Fn fn, const T* in, const float* w, T* out, int B,
                          int H, int L, int K, void* stream, int hc,
                          size_t lds, int max_per_cu, int min_steps = 0) {
  const int threads = hc * kWave;
  int per_cu = blocks_per_cu((const void*)fn, threads, lds);
  if (per_cu > max_per_cu) per_cu = max_per_cu;
  const long long ngroups = (long long)H / hc;
  const long long tsteps = ((long long)B + kRowsCgStep - 1) / kRowsCgStep;
  while (per_cu > 1 && tsteps < (long long)min_steps * (num_cus() * per_cu / ngroups)) --per_cu;
  long long nr = (long long)num_cus() * per_cu / ngroups;
  if (nr > tsteps) nr = tsteps;
  if (nr < 1) nr = 1;
  const long long nb = ngroups * nr;
  if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
  int nranges = (int)nr;
  uint32_t nblocks = (uint32_t)nb;
  void* args[] = {&in, &w, &out, &B, &H, &L, &K, &nranges, &nblocks};
  return launch((const void*)fn, nblocks, (uint32_t)threads, lds, stream, args);
}

// Channels (waves) per workgroup, whatever the caller's waves per block:
//  * rows of 33-48 columns with H % 16 == 0, on tensors above 256 MiB or
//    with at least 24 steps per CU, when L % 4 != 0 or the rows are long
//    and wide (L > 40 and H L above kRowsCg8MaxSampleFloats): 16, one per
//    CU, with one input and two output stages in LDS (148 KB at L = 48).
//    Each step then moves 16 segments of 3 KB instead of 1.5 KB: at
//    B16384 H256 L48 7-9% faster than 8 channels, B16384 H128 L37 K48
//    (the element-wise form) 11%. Since the 8-channel kernel issues its
//    next loads before the matrix work, 8 channels win elsewhere (FWD, 8
//    interleaved rounds, 8/16 time ratio: L40 0.91-0.94 at H64-256, L44
//    0.94-0.97 at H64-128, L36 0.96-0.98 at H128, P 0.97-0.99; B16384
//    H256 L44 1.01, L36 1.00);
//  * otherwise 8, two per CU where the LDS allows (two input and two output
//    stages) and each workgroup gets at least kRowsCgMinSteps steps, else
//    one (rows_cg_launch). Measured on MI355X at 1, 2, 4 and 8 channels, 8 was fastest
//    (at P: 227, 171, 156, 140 us). On tensors of at most 256 MiB (plain
//    loads) with fewer steps per CU the 16-channel grid gives the CUs
//    uneven step counts and fewer steps to overlap, and 8 channels measured
//    as fast or 2-20% faster (B16384 H64 L40 K40 55.8 against 58.7 us,
//    B4096 H128 L48 K48 33.4 against 35.8, B1000 H96 L37 K48 11.1 against
//    13.2; B4096 H256 L48 K48, 16 steps per CU, 63.4 against 62.3).
// The VALU kernel that serves the other shapes wants 1 to 4 waves per
// workgroup (at S: 553-568 us against 606 at 8), so one knob cannot serve
// both kernels.
// PATHTILE_ROWS_CHANNELS=8 or =16 forces the channel count where the layout
// allows it (16: rows of 33-48 columns, H % 16 == 0); the library reads the
// variable on every call.
// Steps per workgroup below which the 8-channel FP32 kernel runs one
// workgroup per CU (rows_cg_launch).
constexpr int kRowsCgMinSteps = 3;
// Floats per sample (H L) up to which rows of whole float4s keep 8-channel
// workgroups at any size (P: 128 x 48).
constexpr long long kRowsCg8MaxSampleFloats = 128LL * 48;

static int rows_cg_channels_env() {
  const char* env = getenv("PATHTILE_ROWS_CHANNELS");
  if (env && strcmp(env, "8") == 0) return 8;
  if (env && strcmp(env, "16") == 0) return 16;
  return 0;
}

static int rows_cg_path(bool dx, const float* in, const float* w, float* out,
                        int B, int H, int L, int K, void* stream,
                        int* probe = nullptr) {
  const bool plain = rows_plain_loads(B, H, L);
  const bool a4 = L % 4 == 0;
  const long long tsteps = ((long long)B + kRowsCgStep - 1) / kRowsCgStep;
  const int forced = rows_cg_channels_env();
  const bool want16 =
      forced ? forced == 16
             : (!plain || tsteps * (H / 16) >= 24LL * num_cus()) &&
                   (!a4 || (L > 40 && (long long)H * L > kRowsCg8MaxSampleFloats));
  if (mfma_index(L) == 2 && H % 16 == 0 && want16 &&
      rows_cg_lds_bytes(L, 16, 1) <= (size_t)max_lds_per_block()) {
    const RowsCgFn* t16 = a4 ? (plain ? kRowsCg16TablePL : kRowsCg16Table)
                             : (plain ? kRowsCg16TableUPL : kRowsCg16TableU);
    if (probe) {
      *probe = dx ? PT_KERNEL_DX_CG16 : PT_KERNEL_FWD_CG16;
      return PT_OK;
    }
    return rows_cg_launch(t16[dx ? 1 : 0], in, w, out, B, H, L, K, stream, 16,
                          rows_cg_lds_bytes(L, 16, 1), 1);
  }
  const RowsCgFn(*t8)[3] = a4 ? (plain ? kRowsCgTablePL : kRowsCgTable)
                              : (plain ? kRowsCgTableUPL : kRowsCgTableU);
  if (probe) {
    *probe = dx ? PT_KERNEL_DX_CG : PT_KERNEL_FWD_CG;
    return PT_OK;
  }
  return rows_cg_launch(t8[dx ? 1 : 0][mfma_index(L)], in, w, out, B, H, L, K,
                        stream, kRowsCgWaves, rows_cg_lds_bytes(L), 2, kRowsCgMinSteps);
}

static long long gcd_ll(long long a, long long b) {
  while (b) {
    const long long t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// The streaming kernel serves K <= 9 on whole float4 rows (16-byte aligned
// tensors), while a channel period H * L fits the 32-bit lane arithmetic.
static bool stream_ok(int H, int L, int K, const void* in, const void* out) {
  return K <= kStreamMaxK && L % 4 == 0 && aligned(in, 16) && aligned(out, 16) &&
         (long long)H * L < (1LL << 31);
}

// Grid of the streaming kernel: the resident waves, rounded to whole channel
// periods. Round r moves NW spans of 64 U float4s; when NW * 64 U is a
// multiple of H L / 4 every lane keeps its column and channel (and taps)
// from span to span. A period longer than the resident waves takes more
// workgroups than fit at once; if that is more waves than there are spans,
// every span gets its own wave instead.
static int stream_path(bool dx, const float* in, const float* w, float* out,
                       int B, int H, int L, int K, int wpb, void* stream,
                       int* probe = nullptr) {
  if (probe) {
    *probe = dx ? PT_KERNEL_DX_STREAM : PT_KERNEL_FWD_STREAM;
    return PT_OK;
  }
  const StreamFn fn =
      (rows_plain_loads(B, H, L) ? kStreamTablePL : kStreamTable)[dx ? 1 : 0][K - 1];
  const int threads = wpb * kWave;
  const unsigned long long nf4 = (unsigned long long)B * H * L / 4;
  const long long span = 64LL * kStreamU;
  const long long nspans = (long long)((nf4 + span - 1) / span);
  const long long need = (nspans + wpb - 1) / wpb;  // blocks for one span per wave
  const long long period = (long long)H * L / 4;
  const long long q = period / gcd_ll(period, span);  // waves per channel period
  const long long rq = q / gcd_ll(q, wpb);            // workgroups per period
  long long nb = (long long)blocks_per_cu((const void*)fn, threads, 0) * num_cus();
  nb = nb / rq * rq;
  if (nb < rq) nb = rq;
  if (nb > need) nb = need;
  if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
  uint32_t nblocks = (uint32_t)nb;
  uint64_t unf4 = nf4, uns = (uint64_t)nspans;
  void* args[] = {&in, &w, &out, &H, &L, &unf4, &uns};
  return launch((const void*)fn, nblocks, (uint32_t)threads, 0, stream, args);
}

// Fronts of the VALU tile kernel. With one front the whole grid walks one
// contiguous window of the input (and of the output, at the same offset),
// and the time then depends on where the two tensors lie relative to each
// other: at B32768 H256 L48 K4, with the output moved 0-512 MiB from the
// input inside one allocation, 552-633 us (FWD and DX alike), 32 MiB the
// worst. Two fronts, each half of the waves walking half of the tiles, ran
// 543-552 us at every one of those 17 offsets (mean 548 against 575), 4
// fronts 551-558, 8 563-566, 16 576-583, 32 602-609 (smaller windows per
// front). Across 18 shapes of this kernel, one placement each, two fronts
// measured 0.98-1.014x the time of one (B65536 H128 L16 K4 the 1.014).
// Returns the largest power of two up to the requested count
// (PATHTILE_ROWS_FRONTS, else 2) that divides the waves into equal sets
// whose step keeps each lane's channel (a multiple of `period` tiles), on
// grids that take more than one round; else 1.
static int rows_fronts(long long nwaves, long long ntiles, long long period) {
  int req = 2;
  const char* env = getenv("PATHTILE_ROWS_FRONTS");
  if (env) req = atoi(env);
  if (ntiles <= nwaves) return 1;
  int f = 1;
  while (2 * f <= req && nwaves % (2LL * f * period) == 0) f *= 2;
  return f;
}

// probe: when not NULL, nothing is launched; *probe receives the
// PT_KERNEL_* id of the kernel the call would launch (-1: none, B or H = 0).
static int rows_path(bool dx, const float* in, const float* w, float* out,
                     int B, int H, int L, int K, int wpb, void* stream,
                     int forced = PT_ROWS_AUTO, int* probe = nullptr) {
  int st = check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (!valid_wpb(wpb)) return PT_ERR_CONFIG;
  if (forced != PT_ROWS_AUTO && forced != PT_ROWS_VALU && forced != PT_ROWS_MATRIX)
    return PT_ERR_CONFIG;
  if (B == 0 || H == 0) {  // empty tensors may have NULL data
    if (probe) *probe = -1;
    return PT_OK;
  }
  if (!in || !w || !out) return PT_ERR_NULL;
  if (!aligned(in, 4) || !aligned(w, 4) || !aligned(out, 4))
    return PT_ERR_ALIGN;
  const RowsAlgo algo = rows_algo(B, H, L, K, forced);
  if (algo == kRowsMfma && rows_cg_ok(H, L, in, out))
    return rows_cg_path(dx, in, w, out, B, H, L, K, stream, probe);
  // The VALU tile kernel: one 64-row LDS tile per wave. Its limits on the
  // waves per workgroup hold for the streaming kernel too, so both VALU
  // kernels accept the same launch configurations.
  const size_t lds_need = (size_t)wpb * rows_lds_per_wave(L);
  if (lds_need > (size_t)max_lds_per_block()) return PT_ERR_CONFIG;
  const bool vec = (L % 4 == 0) && aligned(in, 16) && aligned(out, 16);
  if (wpb * kWave > rows_max_threads(8 * (lbucket_index(L) + 1), vec))
    return PT_ERR_CONFIG;
  if (algo == kRowsStream && stream_ok(H, L, K, in, out))
    return stream_path(dx, in, w, out, B, H, L, K, wpb, stream, probe);
  const long long R = (long long)B * H;
  const long long ntiles = (R + kWave - 1) / kWave;
  const int wpc = rows_waves_per_cu(L, K, ntiles);
  const size_t lds = lds_for_blocks_per_cu(lds_need, 0, wpb >= wpc ? 1 : wpc / wpb);
  const int li = lbucket_index(L), ki = kbucket_index(K);
  const bool plain = rows_plain_loads(B, H, L);
  RowsFn fn = dx ? (vec ? (plain ? kDxTableVP : kDxTableV) : kDxTableS)[li][ki]
                 : (vec ? (plain ? kFwdTableVP : kFwdTableV) : kFwdTableS)[li][ki];
  // Persistent grid: one round of resident workgroups, no more than there
  // are tiles. Wave g takes tiles g, g + G, ... (per front: rows_fronts);
  // lane i's channel stays fixed when G is a multiple of P = H / gcd(H, 64),
  // i.e. the workgroup count a multiple of Q = P / gcd(P, wpb), and with
  // fronts each front's share of G too. Rounding down to that idles
  // nb % Q workgroups; a lane whose channel changes reloads its taps every
  // tile, which measured 16% slower than idling 13% of the waves
  // (B30000 H37 L32 K8) and 25% faster than idling 49% (B2000 H131 L44 K9).
  // So: round when that idles at most a quarter of the workgroups; else the
  // streaming kernel (keeps its taps for any period, 33.6 -> 18.4 us at
  // B2000 H131 L44 K9) where it can serve, or tiles with tap reloads.
  long long nb = (long long)blocks_per_cu((const void*)fn, wpb * kWave, lds) *
                 num_cus();
  const long long need = (ntiles + wpb - 1) / wpb;
  if (nb > need) nb = need;
  const long long P = (long long)H / gcd_ll(H, kWave);
  const long long Q = P / gcd_ll(P, wpb);  // blocks per channel period
  const bool periodic = nb == need || Q <= 1 || (nb >= Q && 4 * (nb % Q) <= nb);
  if (!periodic && algo != kRowsTile && stream_ok(H, L, K, in, out))
    return stream_path(dx, in, w, out, B, H, L, K, wpb, stream, probe);
  if (probe) {
    *probe = dx ? PT_KERNEL_DX : PT_KERNEL_FWD;
    return PT_OK;
  }
  if (periodic && nb < need && Q > 1) nb = nb / Q * Q;
  if (nb < 1) nb = 1;
  if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
  uint32_t nblocks = (uint32_t)nb;
  uint32_t uR = (uint32_t)R, uT = (uint32_t)ntiles;
  uint32_t lmagic = (uint32_t)(((1u << 20) + (uint32_t)L - 1) / (uint32_t)L);
  uint32_t nfront = (uint32_t)rows_fronts(nb * wpb, ntiles, periodic ? P : 1);
  uint32_t chunk = (uint32_t)((ntiles + nfront - 1) / nfront);
  void* args[] = {&in, &w, &out, &H, &L, &K, &uR, &uT, &lmagic, &nfront, &chunk};
  return launch((const void*)fn, nblocks, (uint32_t)(wpb * kWave), lds, stream,
                args);
}

static int dk_path(bool det, const float* gy, const float* x, float* dst,
                   int B, int H, int L, int K, int threads, const DkGeom& g,
                   void* stream) {
  uint32_t nblocks = (uint32_t)g.nblocks;
  int rpw = g.rows_per_wave, nbt = g.nbt, d = det ? 1 : 0;
  if (g.cg) {
    DkCgFn fn = dk_cg_fn(g.nt, g.epc, g.cpw, L);
    const size_t lds = cg_lds_bytes(16 * (mfma_index(L) + 1), g.wpb, L, g.cpw);
    void* args[] = {&gy, &x, &dst, &B, &H, &L, &K, &nbt, &nblocks, &d};
    return launch((const void*)fn, nblocks, (uint32_t)(g.wpb * kWave), lds, stream,
                  args);
  }
  if (g.algo == kDkMfma) {
    DkMfmaFn fn = kDkMfmaTable[mfma_index(L)];
    // One-wave workgroups on inputs larger than the 256 MiB MALL stream HBM
    // best at 12 resident waves per CU (3 per SIMD) rather than the 16 the
    // registers allow; smaller inputs are latency-bound and keep them all.
    size_t lds = 0;
    const double bytes = 8.0 * (double)B * (double)H * (double)L;
    if (threads == kWave && bytes > kDkMallBytes) {
      const size_t stat = (size_t)dk_mfma_static_lds(L);
      lds = lds_for_blocks_per_cu(0, stat, 12);
    }
    void* args[] = {&gy, &x, &dst, &B, &H, &L, &K, &rpw, &nbt, &nblocks, &d};
    return launch((const void*)fn, nblocks, (uint32_t)threads, lds, stream,
                  args);
  }
  const bool vec = (L % 4 == 0) && aligned(gy, 16) && aligned(x, 16);
  DkFn fn = (vec ? kDkTableV : kDkTableS)[lbucket_index(L)][kbucket_index(K)];
  void* args[] = {&gy, &x, &dst, &B, &H, &L, &K, &rpw, &nbt, &nblocks, &d};
  return launch((const void*)fn, nblocks, (uint32_t)threads,
                (size_t)g.wpb * kStageBytes, stream, args);
}

// --- BF16 I/O --------------------------------------------------------------
// x, y, dy, dx are bfloat16 (uint16_t bit patterns), w and dk FP32. FWD / DX
// run on the BF16 matrix cores (FP32 taps as a hi + lo BF16 pair), DK on the
// channel-group kernel with BF16 widened to FP32 in LDS; both accumulate in
// FP32, and BF16 outputs are rounded to nearest-even. Layout: 4-value
// aligned row offsets (L % 4 == 0), 16-byte aligned tensors, H % 8 == 0
// (FWD / DX) or H % (2 * waves) == 0 with at most 8 waves (DK).
// BF16 FWD / DX: 16-channel workgroups where H % 16 == 0, else 8-channel
// ones; one pass of resident workgroups over the GPU (at most 2 per CU of
// 16 channels, 3 of 8). Measured on MI355X against 4 / 8 / 16 channels and
// 0.25x - 4x that many sample ranges: within 3% of the best at every shape
// tried (P, S, L = 16 / 24 / 32 / 40), and 8-16% faster than 8-channel
// groups at P, S, L = 40 and L = 16.
// Tensors of at most 256 MiB (2 B H L bytes) take plain (cached) input
// loads and 8-channel workgroups, one per CU for rows above 24 columns and
// two below: measured on MI355X 17-22% faster than the non-temporal
// 16-channel form at every row bucket (P in BF16 62.1 against 75.1 us,
// B16384 H128 L32 K32 39.9 against 48.8, L24 32.8 against 42.0, B32768
// H256 L16 K16 79.6 against 94.0, B4096 H128 L48 K48 22.1 against 26.1),
// the repeated calls finding part of their input still in the MALL;
// the best channel count and workgroups per CU varied by shape within 5% of
// this rule. Above 256 MiB the non-temporal 16-channel form stays faster
// (S in BF16 275.6 against 298.8 us for 8 channels with plain loads).
static int bf16_rows_path(bool dx, const void* in, const float* w, void* out,
                          int B, int H, int L, int K, void* stream) {
  int st = check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (L % 4 != 0 || H % 8 != 0) return PT_ERR_CONFIG;
  const bool plain = 2.0 * (double)B * (double)H * (double)L <= kRowsPlainLoadBytes;
  const bool wide = !plain && H % 16 == 0;
  const int hc = wide ? 16 : 8;
  const size_t lds = rows_bf16mma_lds_bytes(L, hc);
  if (lds > (size_t)max_lds_per_block()) return PT_ERR_CONFIG;
  if (B == 0 || H == 0) return PT_OK;
  if (!in || !w || !out) return PT_ERR_NULL;
  if (!aligned(in, 16) || !aligned(out, 16) || !aligned(w, 4)) return PT_ERR_ALIGN;
  const RowsCgBf16Fn fn = plain ? kRowsCgTableBf16PL[dx ? 1 : 0][mfma_index(L)]
                                : kRowsCgTableBf16[dx ? 1 : 0][wide ? 1 : 0][mfma_index(L)];
  const int per_cu = plain ? (L > 24 ? 1 : 2) : (wide ? 2 : 3);
  return rows_cg_launch(fn, (const uint16_t*)in, w, (uint16_t*)out, B, H, L, K,
                        stream, hc, lds, per_cu);
}

static int bf16_dk_check(int B, int H, int L, int K, int threads) {
  int st = check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (!valid_dk_threads(threads) || !dk_cg_ok(H, L, threads, kCgChannelsPerWave))
    return PT_ERR_CONFIG;
  return PT_OK;
}

// Geometry of the BF16 DK (one kernel: the shape checks of bf16_dk_check
// admit exactly the layouts it serves). device_cap: a launch, whose ranges
// are capped at one round of resident workgroups as in dk_geometry; the
// uncapped count bounds them (the deterministic workspace size).
static DkGeom bm_geometry(int B, int H, int L, int threads, bool device_cap = false) {
  DkGeom g;
  g.algo = kDkMfma;
  g.cg = true;
  g.nt = bm_nt(B, H, L);
  g.wpb = threads / kWave;
  g.rows_per_wave = 0;
  const long long ngroups = (long long)H / (kCgChannelsPerWave * g.wpb);
  long long nr = bm_ranges(B, H, L);
  if (device_cap) {
    const int mi = mfma_index(L);
    const DkBf16Fn fn = (g.nt ? kDkBf16mmaTableNT : kDkBf16mmaTable)[mi];
    const long long resident =
        (long long)blocks_per_cu((const void*)fn, threads,
                                 dk_bf16mma_lds_bytes(16 * (mi + 1), g.wpb)) *
        num_cus();
    if (ngroups * nr > resident) nr = resident / ngroups;
    if (nr < 1) nr = 1;
  }
  g.nbt = (int)nr;
  g.nblocks = ngroups * nr;
  return g;
}

static int bf16_dk_launch(bool det, const void* gy, const void* x, float* dst,
                          int B, int H, int L, int K, int threads,
                          const DkGeom& g, void* stream) {
  DkBf16Fn fn = (g.nt ? kDkBf16mmaTableNT : kDkBf16mmaTable)[mfma_index(L)];
  const size_t lds = dk_bf16mma_lds_bytes(16 * (mfma_index(L) + 1), g.wpb);
  const uint16_t* gyp = (const uint16_t*)gy;
  const uint16_t* xp = (const uint16_t*)x;
  uint32_t nblocks = (uint32_t)g.nblocks;
  int nbt = g.nbt, d = det ? 1 : 0;
  void* args[] = {&gyp, &xp, &dst, &B, &H, &L, &K, &nbt, &nblocks, &d};
  return launch((const void*)fn, nblocks, (uint32_t)threads, lds, stream, args);
}

// Channels-last DK: 32-channel workgroups (16 waves of two channels, or 8
// of four at 48 columns), one resident pass of them over the GPU (the sample ranges are the resident workgroups per
// channel group, rounded down so no workgroup waits for a second round),
// at most one range per 4-sample step.
static int dk_cl_launch(const float* x, const float* dy, float* dw, int B,
                        int H, int L, int K, void* stream) {
  const DkClFn fn = kDkClTable[mfma_index(L)];
  const int nw = dk_cl_waves(16 * (mfma_index(L) + 1));
  const size_t lds = dk_cl_lds_bytes(16 * (mfma_index(L) + 1), L, nw);
  if (lds > (size_t)max_lds_per_block()) return PT_ERR_CONFIG;
  const int threads = nw * kWave;
  const long long ngroups = (long long)H / kClChannels;
  const long long tsteps = ((long long)B + kCgStep - 1) / kCgStep;
  const long long slots = (long long)num_cus() * blocks_per_cu((const void*)fn, threads, lds);
  long long nr = slots / ngroups;
  if (nr > tsteps) nr = tsteps;
  if (nr < 1) nr = 1;
  const long long nb = ngroups * nr;
  if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
  int nranges = (int)nr;
  uint32_t nblocks = (uint32_t)nb;
  void* args[] = {&x, &dy, &dw, &B, &H, &L, &K, &nranges, &nblocks};
  return launch((const void*)fn, nblocks, (uint32_t)threads, lds, stream, args);
}

// --- long rows: L up to kLongMaxL, K up to kLongMaxK -----------------------
static int check_long_shape(int B, int H, int L, int K) {
  if (B < 0 || H < 0 || L < 1 || K < 1 || L > kLongMaxL || K > kLongMaxK)
    return PT_ERR_SHAPE;
  if ((long long)B * H * L >= (1LL << 31)) return PT_ERR_SHAPE;
  // a 16-sample tile spans < 2 GiB (buffer offsets, see kOob)
  if ((long long)16 * H * L * 4 >= (1LL << 31)) return PT_ERR_SHAPE;
  return PT_OK;
}

// Long-row buckets: LMAX = 64, 96, 128, 160, 192 (L > 64 takes the smallest
// multiple of 32 that holds it; the kernels' work grows with LMAX, not L).
static int long_index(int L) { return L <= 64 ? 0 : (L + 31) / 32 - 2; }
static int long_lmax(int li) { return 32 * (li + 2); }

// Long-row algorithm: the BF16 matrix cores on three-way split operands, or
// the FP32 matrix-core instructions. Both are within FP32 rounding of the
// exact sums. FWD / DX split everywhere (never slower on MI355X). DK splits
// from 40 taps up, and at L = 64 and 96 (full small buckets) for any K. With
// fewer taps a row meets few tiles, and the split kernel's fixed per-step
// work (gather, split, publish, two barriers, for every wave of the row
// bucket) made it 5-11% slower at (L, K) = (192, 33), (160, 33) and
// (52, 16) on MI355X; at L = 64 and 96 it was 8-25% faster for every K
// tried, and from K = 40 it won or came within 2.5%.
// PATHTILE_LONG_ALGO=fp32 forces the FP32 kernels, =split the split ones.
static int long_algo_env() {
  const char* env = getenv("PATHTILE_LONG_ALGO");
  if (env && strcmp(env, "fp32") == 0) return 0;
  if (env && strcmp(env, "split") == 0) return 1;
  return -1;
}

static bool long_split_algo() { return long_algo_env() != 0; }

static bool long_dk_split(int L, int K) {
  const int e = long_algo_env();
  return e < 0 ? (K >= 40 || L == 64 || L == 96) : e == 1;
}

// Split DK kernel of a row bucket: operands loaded in place (every wave
// loads its own column tile of both tensors straight into registers and
// publishes only the x parts) from LMAX = 128 up, the FP32 stage in LDS
// below. Measured on MI355X at B16384 H128 (us, in place against staged):
// L192 K192 790 / 858, L192 K96 640 / 703, L128 K64 382 / 452; L96 K48
// 337 / 301, L64 K64 215 / 181, L64 K16 213 / 169 (short rows give a
// wave's 64-byte row pieces too little work to hide their latency).
static bool long_dk_in_place(int li) { return li >= kNumLongDkStagedLB; }

static int rows_long_path(bool dx, const float* in, const float* w, float* out,
                          int B, int H, int L, int K, void* stream) {
  int st = check_long_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (B == 0 || H == 0) return PT_OK;
  if (!in || !w || !out) return PT_ERR_NULL;
  if (!aligned(in, 4) || !aligned(w, 4) || !aligned(out, 4)) return PT_ERR_ALIGN;
  const int li = long_index(L);
  const int ki = (K + 63) / 64 - 1;  // tap bucket of 64
  const int di = dx ? 1 : 0;
  const bool vec = L % 4 == 0 && aligned(in, 16) && aligned(out, 16);
  if (long_split_algo()) {
    // tap buckets of 32: the diagonal walk covers the bucket's whole band
    const int k3 = (K + 31) / 32 - 1;
    const long long nb = (long long)H * (((long long)B + kLongS3Waves * 16 - 1) / (kLongS3Waves * 16));
    if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
    void* args[] = {&in, &w, &out, &B, &H, &L, &K};
    return launch((const void*)(vec ? kRowsLongS3TableVec : kRowsLongS3Table)[di][li][k3],
                  (uint32_t)nb, kLongS3Waves * kWave, kRowsLongS3Lds[di][li][k3], stream, args);
  }
  const long long nb = (long long)H * (((long long)B + kLongRowsWaves * 16 - 1) / (kLongRowsWaves * 16));
  if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
  void* args[] = {&in, &w, &out, &B, &H, &L, &K};
  const size_t lds = rows_long_lds_bytes(long_lmax(li));
  return launch((const void*)(vec ? kRowsLongTableVec : kRowsLongTable)[di][li][ki], (uint32_t)nb,
                kLongRowsWaves * kWave, lds, stream, args);
}

// Long-row DK: one workgroup per (channel, interleaved range of sample
// steps); the range count aims at kLongDkTarget workgroups (two per CU of
// MI355X), at most one per 32 samples (the split kernel's step; the FP32
// kernel's 16-sample steps then number at least two per range), and depends
// on the shape only, so the workspace size does too. It is rounded down: a
// few workgroups past the target run in another round of their own.
constexpr long long kLongDkTarget = 512;

static long long long_dk_ranges(int B, int H) {
  long long nr = kLongDkTarget / (H > 0 ? H : 1);
  const long long tsteps = ((long long)B + 31) / 32;
  if (nr > tsteps) nr = tsteps;
  return nr < 1 ? 1 : nr;
}

// --- static scratch of the no-allocation deterministic DK -----------------
// The partials of pt_dwconv1d_dk_det_f32_noalloc live in this array instead
// of a caller's workspace. Each device holds its own copy for the life of
// the process. In host code `scratch` names a host-side stand-in, not device
// memory: kernels get the device address that hipGetSymbolAddress returns
// for the current device, looked up once per device and cached.
static __device__ __align__(256) float scratch[PT_DK_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxDevices];

static int scratch_address(float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return PT_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return PT_ERR_HIP;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return PT_ERR_HIP;
    }
    g_scratch_ptr[dev] = (float*)p;
  }
  *out = g_scratch_ptr[dev];
  return PT_OK;
}

// Deterministic DK into `partials` (H * K * g.nbt floats), then the
// fixed-order reduction that overwrites dk. Every partial is written by the
// first launch, so the buffer needs no clearing.
static int dk_det_launch(const float* dy, const float* x, float* dk,
                         float* partials, int B, int H, int L, int K,
                         int threads, const DkGeom& g, void* stream) {
  int st = dk_path(true, dy, x, partials, B, H, L, K, threads, g, stream);
  if (st != PT_OK) return st;
  int ncoef = H * K;
  int nbt = g.nbt;
  const float* cp = partials;
  void* args[] = {&cp, &dk, &ncoef, &nbt};
  const uint32_t grid = (uint32_t)((ncoef + 3) / 4);
  return launch((const void*)&dk_reduce_kernel, grid, 256, 0, stream, args);
}

static const void* kernel_for(int kernel_id, int L, int K) {
  if (L < 1 || L > kMaxL || K < 1 || K > kMaxK) return nullptr;
  const int li = lbucket_index(L), ki = kbucket_index(K);
  switch (kernel_id) {
    case PT_KERNEL_FWD: return (const void*)kFwdTableV[li][ki];
    case PT_KERNEL_DX: return (const void*)kDxTableV[li][ki];
    case PT_KERNEL_DK:
      return dk_algo(L, K) == kDkMfma ? (const void*)kDkMfmaTable[mfma_index(L)]
                                      : (const void*)kDkTableV[li][ki];
    case PT_KERNEL_DK_REDUCE: return (const void*)&dk_reduce_kernel;
    case PT_KERNEL_DK_CG: return (const void*)kDkCgTable[mfma_index(L)];
    case PT_KERNEL_FWD_CG:
    case PT_KERNEL_DX_CG:
      return (const void*)(L % 4 == 0 ? kRowsCgTable : kRowsCgTableU)
          [kernel_id == PT_KERNEL_DX_CG ? 1 : 0][mfma_index(L)];
    case PT_KERNEL_FWD_STREAM:
    case PT_KERNEL_DX_STREAM:
      if (K > kStreamMaxK || L % 4 != 0) return nullptr;
      return (const void*)kStreamTable[kernel_id == PT_KERNEL_DX_STREAM ? 1 : 0][K - 1];
    case PT_KERNEL_FWD_CG16:
    case PT_KERNEL_DX_CG16:
      if (mfma_index(L) != 2) return nullptr;
      return (const void*)(L % 4 == 0 ? kRowsCg16Table : kRowsCg16TableU)
          [kernel_id == PT_KERNEL_DX_CG16 ? 1 : 0];
    default: return nullptr;
  }
}

}  // namespace pt

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int pt_abi_version(void) { return PT_ABI_VERSION; }

const char* pt_status_string(int status) {
  switch (status) {
    case PT_OK: return "ok";
    case PT_ERR_NULL: return "null pointer argument";
    case PT_ERR_SHAPE: return "invalid shape (need B,H>=0, B*H*L<2^31, and L, K within the entry point's range: 1..48, or 1..192 and 1..256 for the long-row entry points)";
    case PT_ERR_CONFIG: return "unsupported launch configuration";
    case PT_ERR_WORKSPACE: return "workspace missing or too small";
    case PT_ERR_HIP: return "HIP runtime launch error";
    case PT_ERR_ALIGN: return "pointer not 4-byte aligned";
    case PT_ERR_SCRATCH: return "the call needs more partials than the library's static scratch holds (PT_DK_SCRATCH_BYTES); use pt_dwconv1d_dk_det_f32 with a workspace";
    default: return "unknown status";
  }
}

int pt_dwconv1d_fwd_f32(const float* x, const float* w, float* y, int B, int H,
                        int L, int K, int waves_per_block, void* stream) {
  return pt::rows_path(false, x, w, y, B, H, L, K, waves_per_block, stream);
}

int pt_dwconv1d_dx_f32(const float* dy, const float* w, float* dx, int B,
                       int H, int L, int K, int waves_per_block, void* stream) {
  return pt::rows_path(true, dy, w, dx, B, H, L, K, waves_per_block, stream);
}

int pt_dwconv1d_fwd_f32_algo(const float* x, const float* w, float* y, int B, int H,
                             int L, int K, int waves_per_block, int algo, void* stream) {
  return pt::rows_path(false, x, w, y, B, H, L, K, waves_per_block, stream, algo);
}

int pt_rows_kernel_id(int B, int H, int L, int K, int waves_per_block,
                      int algo, int aligned16, int dx, int* kernel_id) {
  if (!kernel_id) return PT_ERR_NULL;
  *kernel_id = -1;
  // Stand-in addresses with the requested alignment; the probe returns
  // before anything is launched, so they are never dereferenced.
  const float* p = reinterpret_cast<const float*>((uintptr_t)(aligned16 ? 256 : 260));
  return pt::rows_path(dx != 0, p, p, const_cast<float*>(p), B, H, L, K,
                       waves_per_block, nullptr, algo, kernel_id);
}

int pt_dwconv1d_dx_f32_algo(const float* dy, const float* w, float* dx, int B, int H,
                            int L, int K, int waves_per_block, int algo, void* stream) {
  return pt::rows_path(true, dy, w, dx, B, H, L, K, waves_per_block, stream, algo);
}

int pt_dwconv1d_dk_atomic_f32(const float* dy, const float* x, float* dk,
                              int B, int H, int L, int K,
                              int threads_per_block, int zero_first,
                              void* stream) {
  int st = pt::check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (!pt::valid_dk_threads(threads_per_block)) return PT_ERR_CONFIG;
  if (H == 0) return PT_OK;  // empty tensors may have NULL data
  if (!dk) return PT_ERR_NULL;
  if (!pt::aligned(dk, 4)) return PT_ERR_ALIGN;
  if (zero_first) {
    st = pt::zero_fill(dk, H * K, stream);
    if (st != PT_OK) return st;
  }
  if (B == 0) return PT_OK;
  if (!dy || !x) return PT_ERR_NULL;
  if (!pt::aligned(dy, 4) || !pt::aligned(x, 4)) return PT_ERR_ALIGN;
  const pt::DkGeom g =
      pt::dk_geometry(B, H, L, K, threads_per_block,
                      pt::aligned(dy, 16) && pt::aligned(x, 16), 4, true);
  if (g.nblocks >= (1LL << 31)) return PT_ERR_SHAPE;
  return pt::dk_path(false, dy, x, dk, B, H, L, K, threads_per_block, g,
                     stream);
}

int pt_dwconv1d_dk_det_workspace_bytes(int B, int H, int L, int K,
                                       int threads_per_block, size_t* bytes) {
  if (!bytes) return PT_ERR_NULL;
  int st = pt::check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (!pt::valid_dk_threads(threads_per_block)) return PT_ERR_CONFIG;
  if (B == 0 || H == 0) {
    *bytes = 0;
    return PT_OK;
  }
  // The kernel and its partial count follow from the shape and block size
  // (pointer alignment only sets the channel-group kernel's staging width).
  const pt::DkGeom g = pt::dk_geometry(B, H, L, K, threads_per_block, true);
  *bytes = (size_t)H * (size_t)K * (size_t)g.nbt * sizeof(float);
  return PT_OK;
}

int pt_dwconv1d_dk_det_f32(const float* dy, const float* x, float* dk,
                           void* workspace, size_t workspace_bytes, int B,
                           int H, int L, int K, int threads_per_block,
                           void* stream) {
  int st = pt::check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (!pt::valid_dk_threads(threads_per_block)) return PT_ERR_CONFIG;
  if (H == 0) return PT_OK;  // empty tensors may have NULL data
  if (!dk) return PT_ERR_NULL;
  if (!pt::aligned(dk, 4)) return PT_ERR_ALIGN;
  if (B == 0) return pt::zero_fill(dk, H * K, stream);
  if (!dy || !x) return PT_ERR_NULL;
  if (!pt::aligned(dy, 4) || !pt::aligned(x, 4)) return PT_ERR_ALIGN;
  const pt::DkGeom g =
      pt::dk_geometry(B, H, L, K, threads_per_block,
                      pt::aligned(dy, 16) && pt::aligned(x, 16), 4, true);
  if (g.nblocks >= (1LL << 31)) return PT_ERR_SHAPE;
  const size_t need = (size_t)H * (size_t)K * (size_t)g.nbt * sizeof(float);
  if (!workspace || workspace_bytes < need) return PT_ERR_WORKSPACE;
  if (!pt::aligned(workspace, 4)) return PT_ERR_ALIGN;
  return pt::dk_det_launch(dy, x, dk, (float*)workspace, B, H, L, K,
                           threads_per_block, g, stream);
}

int pt_dwconv1d_dk_det_f32_noalloc(const float* dy, const float* x, float* dk,
                                   int B, int H, int L, int K,
                                   int threads_per_block, void* stream) {
  int st = pt::check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (!pt::valid_dk_threads(threads_per_block)) return PT_ERR_CONFIG;
  if (H == 0) return PT_OK;  // empty tensors may have NULL data
  if (!dk) return PT_ERR_NULL;
  if (!pt::aligned(dk, 4)) return PT_ERR_ALIGN;
  if (B == 0) return pt::zero_fill(dk, H * K, stream);
  if (!dy || !x) return PT_ERR_NULL;
  if (!pt::aligned(dy, 4) || !pt::aligned(x, 4)) return PT_ERR_ALIGN;
  // The limit is the shape-only partial count (the size
  // pt_dwconv1d_dk_det_workspace_bytes reports), decided before any device
  // query; the launch's own count is at most that (the device cap only
  // lowers it), so the partials always fit.
  const pt::DkGeom g0 = pt::dk_geometry(B, H, L, K, threads_per_block, true);
  if ((size_t)H * (size_t)K * (size_t)g0.nbt * sizeof(float) > (size_t)PT_DK_SCRATCH_BYTES)
    return PT_ERR_SCRATCH;
  const pt::DkGeom g =
      pt::dk_geometry(B, H, L, K, threads_per_block,
                      pt::aligned(dy, 16) && pt::aligned(x, 16), 4, true);
  if (g.nblocks >= (1LL << 31)) return PT_ERR_SHAPE;
  float* partials = nullptr;
  st = pt::scratch_address(&partials);
  if (st != PT_OK) return st;
  return pt::dk_det_launch(dy, x, dk, partials, B, H, L, K, threads_per_block,
                           g, stream);
}

int pt_kernel_attributes(int kernel_id, int L, int K, int* regs,
                         int* lds_bytes, int* scratch_bytes,
                         int* max_threads) {
  const void* fn = pt::kernel_for(kernel_id, L, K);
  if (!fn) return PT_ERR_CONFIG;
  hipFuncAttributes a;
  if (hipFuncGetAttributes(&a, fn) != hipSuccess) {
    (void)hipGetLastError();
    return PT_ERR_HIP;
  }
  if (regs) *regs = a.numRegs;
  if (lds_bytes) *lds_bytes = (int)a.sharedSizeBytes;
  if (scratch_bytes) *scratch_bytes = (int)a.localSizeBytes;
  if (max_threads) *max_threads = a.maxThreadsPerBlock;
  return PT_OK;
}

int pt_dynamic_lds_bytes(int kernel_id, int L, int K, int block_config,
                         int* lds_bytes) {
  if (!lds_bytes) return PT_ERR_NULL;
  if (L < 1 || L > pt::kMaxL || K < 1 || K > pt::kMaxK) return PT_ERR_SHAPE;
  switch (kernel_id) {
    case PT_KERNEL_FWD:
    case PT_KERNEL_DX:
      if (!pt::valid_wpb(block_config)) return PT_ERR_CONFIG;
      *lds_bytes = (int)(block_config * pt::rows_lds_per_wave(L));
      return PT_OK;
    case PT_KERNEL_DK:
      if (!pt::valid_dk_threads(block_config)) return PT_ERR_CONFIG;
      *lds_bytes = pt::dk_algo(L, K) == pt::kDkMfma
                       ? 0  // the matrix-core DK uses static LDS only
                       : (int)((block_config / pt::kWave) * pt::kStageBytes);
      return PT_OK;
    case PT_KERNEL_DK_REDUCE:
      *lds_bytes = 0;
      return PT_OK;
    case PT_KERNEL_DK_CG:
      if (!pt::valid_dk_threads(block_config) || block_config > 8 * pt::kWave)
        return PT_ERR_CONFIG;
      *lds_bytes = (int)pt::cg_lds_bytes(16 * (pt::mfma_index(L) + 1),
                                         block_config / pt::kWave, L, pt::dk_cpw(L));
      return PT_OK;
    case PT_KERNEL_FWD_CG:
    case PT_KERNEL_DX_CG:
      // always kRowsCgWaves waves per workgroup, whatever the caller's config
      if (!pt::valid_wpb(block_config)) return PT_ERR_CONFIG;
      *lds_bytes = (int)pt::rows_cg_lds_bytes(L);
      return PT_OK;
    case PT_KERNEL_FWD_CG16:
    case PT_KERNEL_DX_CG16:
      // always 16 waves per workgroup, one input stage
      if (!pt::valid_wpb(block_config)) return PT_ERR_CONFIG;
      *lds_bytes = (int)pt::rows_cg_lds_bytes(L, 16, 1);
      return PT_OK;
    case PT_KERNEL_FWD_STREAM:
    case PT_KERNEL_DX_STREAM:
      if (!pt::valid_wpb(block_config)) return PT_ERR_CONFIG;
      *lds_bytes = 0;
      return PT_OK;
    default:
      return PT_ERR_CONFIG;
  }
}

int pt_dwconv1d_fwd_bf16(const void* x, const float* w, void* y, int B, int H,
                         int L, int K, void* stream) {
  return pt::bf16_rows_path(false, x, w, y, B, H, L, K, stream);
}

int pt_dwconv1d_dx_bf16(const void* dy, const float* w, void* dx, int B, int H,
                        int L, int K, void* stream) {
  return pt::bf16_rows_path(true, dy, w, dx, B, H, L, K, stream);
}

int pt_dwconv1d_dk_atomic_bf16(const void* dy, const void* x, float* dk, int B,
                               int H, int L, int K, int threads_per_block,
                               int zero_first, void* stream) {
  int st = pt::bf16_dk_check(B, H, L, K, threads_per_block);
  if (st != PT_OK) return st;
  if (H == 0) return PT_OK;
  if (!dk) return PT_ERR_NULL;
  if (!pt::aligned(dk, 4)) return PT_ERR_ALIGN;
  if (zero_first) {
    st = pt::zero_fill(dk, H * K, stream);
    if (st != PT_OK) return st;
  }
  if (B == 0) return PT_OK;
  if (!dy || !x) return PT_ERR_NULL;
  if (!pt::aligned(dy, 16) || !pt::aligned(x, 16)) return PT_ERR_ALIGN;
  const pt::DkGeom g = pt::bm_geometry(B, H, L, threads_per_block, true);
  if (g.nblocks >= (1LL << 31)) return PT_ERR_SHAPE;
  return pt::bf16_dk_launch(false, dy, x, dk, B, H, L, K, threads_per_block, g,
                            stream);
}

int pt_dwconv1d_dk_det_bf16_workspace_bytes(int B, int H, int L, int K,
                                            int threads_per_block,
                                            size_t* bytes) {
  if (!bytes) return PT_ERR_NULL;
  int st = pt::bf16_dk_check(B, H, L, K, threads_per_block);
  if (st != PT_OK) return st;
  if (B == 0 || H == 0) {
    *bytes = 0;
    return PT_OK;
  }
  const long long nr = pt::bm_ranges(B, H, L);
  *bytes = (size_t)H * (size_t)K * (size_t)nr * sizeof(float);
  return PT_OK;
}

int pt_dwconv1d_dk_det_bf16(const void* dy, const void* x, float* dk,
                            void* workspace, size_t workspace_bytes, int B,
                            int H, int L, int K, int threads_per_block,
                            void* stream) {
  int st = pt::bf16_dk_check(B, H, L, K, threads_per_block);
  if (st != PT_OK) return st;
  if (H == 0) return PT_OK;
  if (!dk) return PT_ERR_NULL;
  if (!pt::aligned(dk, 4)) return PT_ERR_ALIGN;
  if (B == 0) return pt::zero_fill(dk, H * K, stream);
  if (!dy || !x) return PT_ERR_NULL;
  if (!pt::aligned(dy, 16) || !pt::aligned(x, 16)) return PT_ERR_ALIGN;
  const pt::DkGeom g = pt::bm_geometry(B, H, L, threads_per_block, true);
  if (g.nblocks >= (1LL << 31)) return PT_ERR_SHAPE;
  const size_t need = (size_t)H * (size_t)K * (size_t)g.nbt * sizeof(float);
  if (!workspace || workspace_bytes < need) return PT_ERR_WORKSPACE;
  if (!pt::aligned(workspace, 4)) return PT_ERR_ALIGN;
  float* partials = (float*)workspace;
  st = pt::bf16_dk_launch(true, dy, x, partials, B, H, L, K, threads_per_block,
                          g, stream);
  if (st != PT_OK) return st;
  int ncoef = H * K;
  int nbt = g.nbt;
  const float* cp = partials;
  void* args[] = {&cp, &dk, &ncoef, &nbt};
  const uint32_t grid = (uint32_t)((ncoef + 3) / 4);
  return pt::launch((const void*)&pt::dk_reduce_kernel, grid, 256, 0, stream,
                    args);
}

int pt_dwconv1d_fwd_long_f32(const float* x, const float* w, float* y, int B,
                             int H, int L, int K, void* stream) {
  return pt::rows_long_path(false, x, w, y, B, H, L, K, stream);
}

int pt_dwconv1d_dx_long_f32(const float* dy, const float* w, float* dx, int B,
                            int H, int L, int K, void* stream) {
  return pt::rows_long_path(true, dy, w, dx, B, H, L, K, stream);
}

int pt_dwconv1d_dk_long_workspace_bytes(int B, int H, int L, int K,
                                        size_t* bytes) {
  if (!bytes) return PT_ERR_NULL;
  const int st = pt::check_long_shape(B, H, L, K);
  if (st != PT_OK) return st;
  *bytes = (B == 0 || H == 0)
               ? 0
               : (size_t)H * (size_t)K * (size_t)pt::long_dk_ranges(B, H) * sizeof(float);
  return PT_OK;
}

int pt_dwconv1d_dk_long_f32(const float* dy, const float* x, float* dk,
                            void* workspace, size_t workspace_bytes, int B,
                            int H, int L, int K, void* stream) {
  int st = pt::check_long_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (H == 0) return PT_OK;
  if (!dk) return PT_ERR_NULL;
  if (!pt::aligned(dk, 4)) return PT_ERR_ALIGN;
  if (B == 0) return pt::zero_fill(dk, H * K, stream);
  if (!dy || !x) return PT_ERR_NULL;
  if (!pt::aligned(dy, 4) || !pt::aligned(x, 4)) return PT_ERR_ALIGN;
  const long long nr = pt::long_dk_ranges(B, H);
  const size_t need = (size_t)H * (size_t)K * (size_t)nr * sizeof(float);
  if (!workspace || workspace_bytes < need) return PT_ERR_WORKSPACE;
  if (!pt::aligned(workspace, 4)) return PT_ERR_ALIGN;
  const long long nb = (long long)H * nr;
  if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
  const int li = pt::long_index(L);
  const int lmax = pt::long_lmax(li);
  float* partials = (float*)workspace;
  int nranges = (int)nr, det = 1;
  void* args[] = {&dy, &x, &partials, &B, &H, &L, &K, &nranges, &det};
  const bool vec = L % 4 == 0 && pt::aligned(dy, 16) && pt::aligned(x, 16);
  const bool split = pt::long_dk_split(L, K);
  if (split && pt::long_dk_in_place(li))
    st = pt::launch((const void*)pt::kDkLongS3RTable[li - pt::kNumLongDkStagedLB], (uint32_t)nb,
                    (uint32_t)((lmax / 16) * pt::kWave),
                    pt::dk_long_s3r_lds_bytes(lmax), stream, args);
  else if (split)
    st = pt::launch((const void*)pt::kDkLongS3Table[vec ? 1 : 0][li], (uint32_t)nb,
                    (uint32_t)((lmax / 16) * pt::kWave), pt::dk_long_s3_lds_bytes(lmax), stream, args);
  else
    st = pt::launch((const void*)pt::kDkLongTable[vec ? 1 : 0][li], (uint32_t)nb,
                    (uint32_t)((lmax / 16) * pt::kWave), pt::dk_long_lds_bytes(lmax), stream, args);
  if (st != PT_OK) return st;
  int ncoef = H * K;
  int nbt = nranges;
  const float* cp = partials;
  void* rargs[] = {&cp, &dk, &ncoef, &nbt};
  return pt::launch((const void*)&pt::dk_reduce_kernel, (uint32_t)((ncoef + 3) / 4), 256,
                    0, stream, rargs);
}

// The Flash-DWC dW bridge's C ABI (benchmark/flashdwc_fp32_bridge.cu:6-34):
// x and dy are [B, 1, L, H] FP32, dw is [1, K, H] and is accumulated into
// (the caller zeroes it). Returns 0, or -2 for the arguments the bridge
// rejects (NULL pointers; B, H, L, K, GZ <= 0; H % 32 != 0; B % GZ != 0;
// (B / GZ) % 16 != 0) and for the ones this library does not serve (L or K
// above 48, x or dy not 16-byte aligned, dw not 4-byte aligned), or
// PT_ERR_HIP if the launch fails. GZ, the bridge's batch split, changes
// nothing here: the kernel chooses its own sample ranges.
int flash_dk_fp32(const float* x, const float* dy, float* dw, int B, int H,
                  int L, int K, int GZ, void* stream) {
  if (!x || !dy || !dw || B <= 0 || H <= 0 || H % 32 != 0 || L <= 0 ||
      K <= 0 || GZ <= 0 || B % GZ != 0 || (B / GZ) % 16 != 0)
    return PT_ERR_SHAPE;
  if (pt::check_shape(B, H, L, K) != PT_OK) return PT_ERR_SHAPE;
  if (!pt::aligned(x, 16) || !pt::aligned(dy, 16) || !pt::aligned(dw, 4))
    return PT_ERR_SHAPE;
  const int st = pt::dk_cl_launch(x, dy, dw, B, H, L, K, stream);
  return st == PT_ERR_HIP ? PT_ERR_HIP : (st == PT_OK ? PT_OK : PT_ERR_SHAPE);
}

}  // extern "C"
