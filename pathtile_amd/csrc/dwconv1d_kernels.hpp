// dwconv1d_kernels.hpp — device code of the depthwise Conv1D for short rows (L <= 48, K <= 48), FP32,
// written for MI355X (gfx950, CDNA4, wave64).
//
// Paths (semantics of kernels/warp_tiled_ampere.py:372-619 in the reference):
//   FWD  y [b,h,t] = sum_j w[h,j] * x [b,h,t+j-p]          p = K/2
//   DX   dx[b,h,s] = sum_j w[h,j] * dy[b,h,s-j+p]
//   DK   dk[h,j]   = sum_b sum_t dy[b,h,t] * x[b,h,t+j-p]
// with zeros outside [0, L).
//
// Mapping (MI355X-first; the reference maps one row onto a 32-lane warp with
// one output per lane and re-reads taps and row elements per FMA):
//   * one LANE owns one whole (b,h) row, held in VGPRs, and computes all of
//     its outputs;
//   * FWD / DX (dwconv_rows_kernel): a WAVE owns a tile of 64 CONSECUTIVE
//     rows r = b*H + h of the flat [B*H, L] tensor (64*L*4 contiguous bytes),
//     so every HBM instruction of the wave moves 1 KiB of contiguous memory.
//     The tile passes through a per-wave LDS transpose (row stride LMAX + 4
//     floats, bank-conflict free for ds_read/ds_write_b128); each lane keeps
//     the taps of its own channel (r % H) in VGPRs across a persistent grid;
//   * DK contracts the batch on the matrix cores (v_mfma_f32_16x16x4_f32):
//     D_h[t][s] = sum_b dy[b,h,t] * x[b,h,s], and the taps are the diagonal
//     sums dk[h,j] = sum_t D_h[t][t + j - p]. dwconv_dk_cg_kernel (default
//     wherever H is a multiple of the channel group, any L) streams
//     contiguous channel-group segments [b, g*HC .. g*HC+HC, :] with each
//     wave owning one or two channels; dwconv_dk_mfma_kernel (every other
//     shape) gives a wave a run of samples of one channel;
//   * DK (dwconv_dk_kernel, PATHTILE_DK_ALGO=valu): a WAVE owns 64 samples of
//     one channel; a 16-column strided LDS transpose (TileIO) feeds each lane
//     its row pair and the lane accumulates every tap on the VALU;
//   * the inner loops are fully unrolled at compile time for a row bucket
//     LMAX (8..48) and a tap bucket KB (4..48). Taps outside [0,K) are zero
//     and row elements in [L, LMAX) are zero in VGPRs, so one instantiation
//     serves every (L, K) of its bucket and the unrolled FMA chain only
//     touches (t, m) pairs inside the LMAX window.
//
// FWD and DX run the reference's per-output fmaf chain in the reference's tap
// order (FWD: j ascending, kernels/warp_tiled_ampere.py:411-430; DX: j
// ascending, :479-498). Padded terms are exact no-ops (fma(0,w,a) == a,
// fma(x,0,a) == a for finite x), so outputs equal that chain bit for bit.
//
// DK reduces per workgroup, then either adds one global_atomic_add_f32 per
// tap per workgroup (atomic variant, kernels/warp_tiled_ampere.py:611-614)
// or stores one partial per tap into a [H, K, num_btiles] workspace that a
// fixed-order reduction kernel sums (deterministic variant,
// kernels/warp_tiled_noatomic_optimized.py:881-1160).

#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "pathtile_hip.h"

namespace pt {

constexpr int kWave = 64;                         // lanes per wavefront
constexpr int kChunk = 16;                        // columns per LDS pass
constexpr int kStride = 20;                       // floats per staged row
constexpr int kStageFloats = kWave * kStride;     // per-wave staging tile
constexpr int kStageBytes = kStageFloats * 4;     // 5120 B
constexpr int kNumXcd = 8;                        // MI355X: 8 XCDs
constexpr int kMaxWaves = 16;                     // 1024 threads
// DK keeps a 48-float row, 48 accumulators and a streamed dy chunk in VGPRs;
// 12 waves per CU (3 per SIMD) leave it 168 registers.
constexpr int kMaxDkThreads = 768;
constexpr int kMaxL = PT_MAX_L;
constexpr int kMaxK = PT_MAX_K;

// ---------------------------------------------------------------------------
// Compile-time helpers
// ---------------------------------------------------------------------------
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Tap window of a (row bucket, tap bucket, path). Lane-relative offsets
// m = s - t (FWD/DK: j = p + m; DX: j = p - m) lie in [lo, hi]. For K <= KB
// (KB even): FWD/DK need m in [-p, K-1-p] within [-KB/2, KB/2-1]; DX needs
// m in [-(K-1-p), p] within [-(KB/2-1), KB/2]. Offsets with |m| >= LMAX never
// meet a row element and are clipped.
template <int LMAX, int KB, bool DX>
struct Window {
  static constexpr int full_lo = DX ? -(KB / 2 - 1) : -(KB / 2);
  static constexpr int full_hi = full_lo + KB - 1;
  static constexpr int lo = full_lo > -(LMAX - 1) ? full_lo : -(LMAX - 1);
  static constexpr int hi = full_hi < (LMAX - 1) ? full_hi : (LMAX - 1);
  static constexpr int n = hi - lo + 1;
};

template <int LMAX>
struct RowGeo {
  static constexpr int nchunks = (LMAX + kChunk - 1) / kChunk;
  static constexpr int cols(int c) {
    return (LMAX - kChunk * c) >= kChunk ? kChunk : (LMAX - kChunk * c);
  }
};

// Orders the wave's own LDS accesses around a cross-lane exchange. LDS
// instructions of one wave execute in program order, so a compiler-level
// fence at wavefront scope is enough (no s_barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroups are dealt to the 8 XCDs round-robin (block p -> XCD p % 8).
// Renumber them so each XCD walks one contiguous range of logical tiles:
// neighbouring tiles (which share cache lines when rows are not 128-byte
// multiples) then meet in the same L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t p, uint32_t n) {
  const uint32_t q = n / kNumXcd;
  const uint32_t r = n % kNumXcd;
  const uint32_t xcd = p % kNumXcd;
  const uint32_t idx = p / kNumXcd;
  return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// ---------------------------------------------------------------------------
// Buffer addressing. A tile is reached through a wave-uniform buffer
// resource (base = the wave's row 0, in SGPRs), one 32-bit per-lane byte
// offset (VGPR) and, for loads only, a wave-uniform per-step byte offset
// (soffset; stores take their whole offset in the VGPR, see buf_store4). Lanes
// that must not touch memory use an offset past num_records: buffer loads
// then return 0 and buffer stores are dropped, so no branches are needed.
// The host guarantees 64 * H * L * 4 < 2^31 (a tile spans < 2 GiB).
// ---------------------------------------------------------------------------
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOob = 0x80000000u;         // >= num_records
constexpr int kNumRecords = 0x7fffffff;
constexpr int kRsrcWord3 = 0x00020000;         // gfx9: 32-bit data format
// Cache-policy bits of buffer instructions (gfx940+: bit 0 = sc0, bit 1 = nt,
// bit 4 = sc1). The streamed tensors are touched once per kernel, so their
// loads and stores are non-temporal: they neither displace other data nor
// leave dirty lines for the next kernel to write back.
constexpr int kCpolNone = 0;
constexpr int kCpolNT = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0,
                                           kNumRecords, kRsrcWord3);
}

template <int CPOL = kCpolNone>
__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r,
                                            uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, CPOL);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y),
                     __uint_as_float(v.z), __uint_as_float(v.w));
}

template <int CPOL = kCpolNone>
__device__ __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r,
                                           uint32_t voff, uint32_t soff) {
  return __uint_as_float(
      __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, CPOL));
}

// Stores take no SGPR offset (soffset is the constant 0). With a register
// in soffset the compiler inserts no wait states between a dwordx3/x4 store
// and a following VALU write of the store's data VGPRs; on gfx950 the store
// then wrote the VALU result in place of its first dword. The whole byte
// offset therefore travels in the VGPR offset.
template <int CPOL = kCpolNone>
__device__ __forceinline__ void buf_store4(float4 v, __amdgpu_buffer_rsrc_t r,
                                           uint32_t voff) {
  u32x4 u;
  u.x = __float_as_uint(v.x);
  u.y = __float_as_uint(v.y);
  u.z = __float_as_uint(v.z);
  u.w = __float_as_uint(v.w);
  __builtin_amdgcn_raw_buffer_store_b128(u, r, voff, 0, CPOL);
}

template <int CPOL = kCpolNone>
__device__ __forceinline__ void buf_store1(float v, __amdgpu_buffer_rsrc_t r,
                                           uint32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, 0, CPOL);
}

// ---------------------------------------------------------------------------
// Row tile staging: 64 rows (one per lane) <-> HBM, through per-wave LDS,
// one 16-column chunk C at a time. Row r of the tile starts r * rstride
// elements after the resource base. Step k of chunk C moves
//   rows (64/QPR)*k + lane/QPR, columns 16C + 4*(lane%QPR) .. +3,
// QPR = cols/4: one dwordx4 per lane when rows are 16-byte aligned
// (vec != 0), four dwords otherwise. Rows >= nrows and columns >= L are
// never accessed; lane-side copies of those elements are zero.
// ---------------------------------------------------------------------------
template <int LMAX>
struct TileIO {
  using G = RowGeo<LMAX>;

  template <int C>
  __device__ static __forceinline__ void load(__amdgpu_buffer_rsrc_t rs,
                                              uint32_t rstride, int nrows,
                                              int L, int lane, int vec,
                                              float4* buf) {
    constexpr int qpr = G::cols(C) / 4;
    constexpr int rpi = kWave / qpr;
    const int r0 = lane / qpr;
    const int col = kChunk * C + 4 * (lane % qpr);
    const uint32_t off = ((uint32_t)r0 * rstride + (uint32_t)col) * 4u;
#pragma unroll
    for (int k = 0; k < qpr; ++k) {
      const uint32_t soff = (uint32_t)(k * rpi) * rstride * 4u;
      const bool row_ok = r0 < nrows - k * rpi;
      if (vec) {
        buf[k] = buf_load4<kCpolNT>(rs, row_ok && col < L ? off : kOob, soff);
      } else {
        buf[k].x = buf_load1<kCpolNT>(rs, row_ok && col + 0 < L ? off + 0u : kOob, soff);
        buf[k].y = buf_load1<kCpolNT>(rs, row_ok && col + 1 < L ? off + 4u : kOob, soff);
        buf[k].z = buf_load1<kCpolNT>(rs, row_ok && col + 2 < L ? off + 8u : kOob, soff);
        buf[k].w = buf_load1<kCpolNT>(rs, row_ok && col + 3 < L ? off + 12u : kOob, soff);
      }
    }
  }

  // Lane r receives row r's columns [16C, 16C + cols) in dst[0 .. cols).
  template <int C>
  __device__ static __forceinline__ void transpose(float* stage, int lane,
                                                   const float4* buf,
                                                   float* dst) {
    constexpr int nc = G::cols(C);
    constexpr int qpr = nc / 4;
    constexpr int rpi = kWave / qpr;
    const int q = lane % qpr;
#pragma unroll
    for (int k = 0; k < qpr; ++k) {
      const int row = rpi * k + lane / qpr;
      *reinterpret_cast<float4*>(stage + row * kStride + 4 * q) = buf[k];
    }
    wave_lds_sync();
    read_own_row<nc>(stage, lane, dst);
  }

  template <int NC>
  __device__ static __forceinline__ void read_own_row(const float* stage,
                                                      int lane, float* dst) {
#pragma unroll
    for (int i = 0; i < NC / 4; ++i) {
      const float4 v =
          *reinterpret_cast<const float4*>(stage + lane * kStride + 4 * i);
      dst[4 * i + 0] = v.x;
      dst[4 * i + 1] = v.y;
      dst[4 * i + 2] = v.z;
      dst[4 * i + 3] = v.w;
    }
    wave_lds_sync();
  }

  // Whole tile HBM -> registers (all chunks' loads in flight at once).
  __device__ static __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t rs,
                                                   uint32_t rstride, int nrows,
                                                   int L, int lane, int vec,
                                                   float4* buf) {
    static_for<0, G::nchunks>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      load<c>(rs, rstride, nrows, L, lane, vec, buf + 4 * c);
    });
  }

  // Registers of load_tile -> lanes (row r -> lane r, dst[0 .. LMAX)).
  __device__ static __forceinline__ void transpose_tile(float* stage, int lane,
                                                        const float4* buf,
                                                        float* dst) {
    static_for<0, G::nchunks>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      transpose<c>(stage, lane, buf + 4 * c, dst + kChunk * c);
    });
  }

  // Whole tile HBM -> lanes.
  __device__ static __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rs,
                                                   uint32_t rstride, int nrows,
                                                   int L, int lane, int vec,
                                                   float* stage, float* dst) {
    float4 buf[LMAX / 4];
    load_tile(rs, rstride, nrows, L, lane, vec, buf);
    transpose_tile(stage, lane, buf, dst);
  }

  // One chunk HBM -> lanes.
  template <int C>
  __device__ static __forceinline__ void load_chunk(__amdgpu_buffer_rsrc_t rs,
                                                    uint32_t rstride,
                                                    int nrows, int L,
                                                    int lane, int vec,
                                                    float* stage, float* dst) {
    float4 buf[4];
    load<C>(rs, rstride, nrows, L, lane, vec, buf);
    transpose<C>(stage, lane, buf, dst);
  }
};

// Taps of channel h for window offsets m = LO .. LO+N-1, zero where the tap
// index j = p + m (FWD/DK) or p - m (DX) falls outside [0, K). Lane i loads
// window tap i with one buffer load (a masked lane reads 0), then each tap is
// broadcast with readlane, so the FMA chain takes it as a wave-uniform
// (SGPR) operand.
template <int LO, int N, bool DX>
__device__ __forceinline__ void load_taps(const float* __restrict__ w, int h,
                                          int H, int K, int lane, float* wt) {
  static_assert(N <= kWave, "tap window wider than a wave");
  const int p = K >> 1;
  const int m = LO + lane;
  const int j = DX ? (p - m) : (p + m);
  const bool ok = lane < N && (unsigned)j < (unsigned)K;
  const uint32_t off = ok ? (uint32_t)(h * K + j) * 4u : kOob;
  const float v = buf_load1(make_rsrc(w), off, 0);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    wt[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
  }
}

// ---------------------------------------------------------------------------
// FWD / DX on contiguous tiles. [B, H, L] is read as R = B*H consecutive
// rows of L floats; a tile is 64 consecutive rows (64*L*4 bytes, 256-byte
// aligned), one per lane, so every HBM load/store instruction of a wave
// covers 1 KiB of contiguous memory (dwordx4) and tiles never share a cache
// line. Lane i's row r0 + i belongs to channel (r0 + i) % H; its taps sit in
// VGPRs. The grid is persistent and walks the tiles in `nfront` fronts:
// the tiles split into nfront contiguous chunks, and wave g takes tiles
// c + g', c + g' + G', c + g' + 2G', ... of chunk g % nfront (start c,
// g' = g / nfront, G' = G / nfront), with G' a multiple of H / gcd(H, 64)
// where possible, so a lane keeps its channel (and its taps) for the whole
// kernel. With one front this is the order g, g + G, g + 2G, ...
//
// Per tile: flat loads -> LDS (padded row stride S = LMAX + 4 floats, so the
// ds_read_b128 of a lane's own row is bank-conflict free) -> own row into
// VGPRs -> fmaf chain -> own output row into LDS -> flat reads -> stores.
// The rows past the end of the tensor are outside the buffer resource's
// num_records: their loads read 0 and their stores are dropped.
// ---------------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_n(const float* base,
                                                              uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0,
                                           (int)bytes, kRsrcWord3);
}

// Row / column of flat element e (< 64 * 48) of a tile with row length L:
// row = floor(e * ceil(2^20 / L) / 2^20) is exact for e < 3072, L <= 48.
__device__ __forceinline__ void flat_rc(uint32_t e, uint32_t L, uint32_t lmagic,
                                        uint32_t& row, uint32_t& col) {
  row = (e * lmagic) >> 20;
  col = e - row * L;
}

// Lane-varying taps: lane's channel h, window offsets LO .. LO+N-1, zero
// where j = p + m (FWD) or p - m (DX) falls outside [0, K).
template <int LO, int N, bool DX>
__device__ __forceinline__ void load_lane_taps(const float* __restrict__ w,
                                               int h, int K, float* wt) {
  const int p = K >> 1;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(w);
  const uint32_t base = (uint32_t)h * (uint32_t)K;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int m = LO + i;
    const int j = DX ? (p - m) : (p + m);
    const bool ok = (unsigned)j < (unsigned)K;
    wt[i] = buf_load1(r, ok ? (base + (uint32_t)j) * 4u : kOob, 0);
  }
}

// Largest workgroup of the FWD/DX kernel. For LMAX >= 40 the LDS tile
// (64 * (LMAX + 4) floats per wave) caps a CU at 12 waves anyway, so the
// kernel may use the 168 VGPRs of 3 waves per SIMD (taps and row both live
// in VGPRs); the dword path (rows not 16-byte aligned, an edge case) gets the
// same budget for its per-element address arithmetic.
constexpr int rows_max_threads(int lmax, bool vec) {
  return (lmax >= 40 || !vec) ? 768 : 1024;
}

template <int LMAX, int KB, bool DX, bool VEC, int LOAD_CPOL = kCpolNT,
          int STORE_CPOL = kCpolNT>
__global__ __launch_bounds__(rows_max_threads(LMAX, VEC)) void dwconv_rows_kernel(
    const float* __restrict__ in, const float* __restrict__ w,
    float* __restrict__ out, int H, int L, int K, uint32_t R, uint32_t ntiles,
    uint32_t lmagic, uint32_t nfront, uint32_t chunk) {
  using W = Window<LMAX, KB, DX>;
  constexpr int S = LMAX + 4;     // padded LDS row stride (floats)
  constexpr int NV = LMAX / 4;    // dwordx4 steps per lane (vector path)
  extern __shared__ float lds[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t wpb = blockDim.x / kWave;
  // Wave-major numbering: consecutive tiles go to consecutive workgroups
  // (different CUs), whatever the workgroup size. Block-major numbering put
  // a workgroup's waves on adjacent tiles and measured 3-8% slower at 4 and
  // 8 waves per workgroup (B32768 H256 L48 K4: 573 against 555 us at 4).
  const uint32_t gwave = (uint32_t)wave * gridDim.x + blockIdx.x;
  const uint32_t nwaves = gridDim.x * wpb;
  const uint32_t uL = (uint32_t)L;
  const uint32_t tile_elems = (uint32_t)kWave * uL;
  float* tile = lds + wave * (kWave * S);

  float wt[W::n];
  int hcur = -1;
  bool tbad = false;  // a tap of this lane's channel is not finite
  // Padded terms (elements past L, taps outside [0, K) in the bucket's
  // window) are exact no-ops only for finite operands: 0 * Inf is NaN where
  // the reference skips the term. Without padding no such term exists.
  const bool padded = L != LMAX || K != KB;

  // Fronts: the tiles split into nfront chunks of `chunk` consecutive tiles
  // and the waves into nfront equal sets (nwaves % nfront == 0, set by the
  // host), wave g walking chunk g % nfront. nfront = 1, chunk = ntiles is
  // the plain order g, g + G, g + 2G, ...
  const uint32_t front = gwave % nfront;
  const uint32_t fstep = nwaves / nfront;
  const uint32_t tend = min(front * chunk + chunk, ntiles);
  for (uint32_t t0 = front * chunk + gwave / nfront; t0 < tend; t0 += fstep) {
    // readfirstlane keeps per-tile bases opaque to loop strength reduction.
    const uint32_t t = __builtin_amdgcn_readfirstlane(t0);
    const uint32_t r0 = t * kWave;
    const uint32_t nr = min((uint32_t)kWave, R - r0);
    const uint32_t vbytes = nr * uL * 4u;
    const size_t e0 = (size_t)r0 * (size_t)uL;
    const __amdgpu_buffer_rsrc_t rin = make_rsrc_n(in + e0, vbytes);
    const __amdgpu_buffer_rsrc_t rout = make_rsrc_n(out + e0, vbytes);

    // Flat loads (all in flight at once), then scatter into padded rows.
    if constexpr (VEC) {
      float4 v[NV];
#pragma unroll
      for (int k = 0; k < NV; ++k)
        v[k] = buf_load4<LOAD_CPOL>(rin, (uint32_t)(kWave * k + lane) * 16u, 0);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const uint32_t e = (uint32_t)(kWave * k + lane) * 4u;
        if (e < tile_elems) {
          uint32_t row, col;
          flat_rc(e, uL, lmagic, row, col);
          *reinterpret_cast<float4*>(tile + row * S + col) = v[k];
        }
      }
    } else {
      // dword path (rows not 16-byte aligned): groups of 16 loads, each
      // scattered before the next group is issued. The empty asm makes the
      // lane index opaque inside the tile loop, so the 2 * LMAX per-element
      // addresses are recomputed per tile instead of being hoisted out of the
      // loop and pinned in VGPRs.
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int g = 0; g < LMAX; g += 16) {
        constexpr int kG = 16;
        float v[kG];
#pragma unroll
        for (int k = 0; k < kG; ++k)
          if (g + k < LMAX)
            v[k] = buf_load1<LOAD_CPOL>(rin, (uint32_t)(kWave * (g + k) + ln) * 4u, 0);
#pragma unroll
        for (int k = 0; k < kG; ++k) {
          const uint32_t e = (uint32_t)(kWave * (g + k) + ln);
          if (g + k < LMAX && e < tile_elems) {
            uint32_t row, col;
            flat_rc(e, uL, lmagic, row, col);
            tile[row * S + col] = v[k];
          }
        }
      }
    }

    // Channel of this lane's row; reload the taps when any lane's changed.
    const int h = (int)((r0 + (uint32_t)lane) % (uint32_t)H);
    if (__builtin_amdgcn_ballot_w64(h != hcur)) {
      load_lane_taps<W::lo, W::n, DX>(w, h, K, wt);
      hcur = h;
      float ts = 0.0f;
#pragma unroll
      for (int i = 0; i < W::n; ++i) ts += wt[i];
      tbad = !__builtin_isfinite(ts);
    }

    wave_lds_sync();
    float xr[LMAX];
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      const float4 x4 = *reinterpret_cast<const float4*>(tile + lane * S + 4 * q);
      xr[4 * q + 0] = x4.x;
      xr[4 * q + 1] = x4.y;
      xr[4 * q + 2] = x4.z;
      xr[4 * q + 3] = x4.w;
    }
    if (L != LMAX) {  // columns >= L were not loaded in this tile
#pragma unroll
      for (int s = 0; s < LMAX; ++s) xr[s] = s < L ? xr[s] : 0.0f;
    }
    // A row with a non-finite element (or a lane with a non-finite tap)
    // meets a padded term: its sum is not finite.
    bool slow = false;
    if (padded) {
      float xs = 0.0f;
#pragma unroll
      for (int s = 0; s < LMAX; ++s) xs += xr[s];
      slow = tbad || !__builtin_isfinite(xs);
    }
    wave_lds_sync();

    if (__builtin_amdgcn_ballot_w64(slow)) {
      // The reference's chain with its skipped terms, every lane of the
      // wave (on finite rows it gives the fast path's bits). Elements come
      // from the input tensor (rows past R read 0 and are never stored) and
      // taps from memory, so the lane's LDS row can take each output as it
      // is made and the path holds no row in registers.
      const float* wh = w + (size_t)h * K;
      const int p = K >> 1;
      const uint32_t rowb = (uint32_t)lane * uL * 4u;
#pragma unroll 1
      for (int t = 0; t < L; ++t) {
        float acc = 0.0f;
#pragma unroll 1
        for (int j = 0; j < K; ++j) {
          const int e = DX ? t - j + p : t + j - p;
          if ((unsigned)e < (unsigned)L)
            acc = fmaf(buf_load1(rin, rowb + 4u * (uint32_t)e, 0), wh[j], acc);
        }
        tile[lane * S + t] = acc;
      }
    } else {
      // The reference's fmaf chain per output, taps in reference order
      // (FWD: j = p + m ascending <=> i ascending; DX: j = p - m ascending
      // <=> i descending); four outputs at a time (four independent chains)
      // go to the lane's own row.
#pragma unroll
      for (int t4 = 0; t4 < LMAX; t4 += 4) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ii = 0; ii < W::n; ++ii) {
          const int i = DX ? (W::n - 1 - ii) : ii;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int s = t4 + u + W::lo + i;
            if (s >= 0 && s < LMAX) acc[u] = fmaf(xr[s], wt[i], acc[u]);
          }
        }
        *reinterpret_cast<float4*>(tile + lane * S + t4) =
            make_float4(acc[0], acc[1], acc[2], acc[3]);
      }
    }
    wave_lds_sync();

    // Flat reads of the output rows, contiguous stores.
    if constexpr (VEC) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const uint32_t e = (uint32_t)(kWave * k + lane) * 4u;
        if (e < tile_elems) {
          uint32_t row, col;
          flat_rc(e, uL, lmagic, row, col);
          const float4 y4 = *reinterpret_cast<const float4*>(tile + row * S + col);
          buf_store4<STORE_CPOL>(y4, rout, e * 4u);
        }
      }
    } else {
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int k = 0; k < LMAX; ++k) {
        const uint32_t e = (uint32_t)(kWave * k + ln);
        if (e < tile_elems) {
          uint32_t row, col;
          flat_rc(e, uL, lmagic, row, col);
          buf_store1<STORE_CPOL>(tile[row * S + col], rout, e * 4u);
        }
      }
    }
    wave_lds_sync();
  }
}

// ---------------------------------------------------------------------------
// FWD / DX for short taps (K <= 9, so p = K/2 <= 4 and K-1-p <= 4) on rows of
// L % 4 == 0 floats, 16-byte aligned: a streaming kernel with no LDS.
//
// The tensor is read as F = B*H*L/4 float4s (a float4 never straddles two
// rows). A wave owns spans of 64*U consecutive float4s: lane i, register u
// holds float4 64u + i of the span, so every load and store instruction of
// the wave moves 1 KiB of contiguous memory, and U of them are in flight
// per wave. Each output needs at most 4 elements on either side, which lie
// in the neighbouring float4s: the lane to the left / right in the same
// register (DPP wave_shr:1 / wave_shl:1), lane 63 of register u-1 / lane 0
// of register u+1 at the register edges (readlane), and one float4 before
// and after the span at its edges (one load by lanes 0 and 1).
//
// A neighbouring float4 lies wholly inside or wholly outside the lane's row
// (column c0 of the lane's float4 is a multiple of 4): terms that reach
// into it are taken iff c0 >= 4 (left) or c0 + 4 < L (right), and skipped
// otherwise, exactly as the reference skips them; terms inside the lane's
// own float4 are always taken. Each output thus runs the reference's fmaf
// chain (start 0.0f, taps j = 0 .. K-1 ascending, the same skipped terms)
// bit for bit, for any values, non-finite ones included.
//
// The grid advances by NW spans per round (NW = waves in the grid); the host
// makes NW * 64U a multiple of H*L/4 float4s (or gives every span its own
// wave), so a lane's column and channel are the same in every span it takes:
// both, and the lane's U sets of K taps, are computed once per wave.
// ---------------------------------------------------------------------------
constexpr int kStreamMaxK = 9;
constexpr int kStreamU = 4;  // float4s per lane per span (spans of 4 KiB)

template <int CTRL>
__device__ __forceinline__ float dpp_shift(float v, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      __float_as_int(old), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_of(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float f4c(const float4& v, int c) {
  return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

// LOAD_CPOL: cache policy of the span loads (stores are non-temporal).
template <int K, bool DX, int LOAD_CPOL = kCpolNT, int U = kStreamU>
__global__ __launch_bounds__(1024) void dwconv_stream_kernel(
    const float* __restrict__ in, const float* __restrict__ w,
    float* __restrict__ out, int H, int L, uint64_t nf4, uint64_t nspans) {
  static_assert(K >= 1 && K <= kStreamMaxK, "stream kernel: K <= 9");
  constexpr int P = K / 2;
  // Window offsets d (output column - input column) of the chain: FWD
  // d = j - p, DX d = p - j; the left neighbour supplies d in [-4, -1],
  // the right one d in [4, 7] relative to the lane's first column.
  constexpr int NL = DX ? K - 1 - P : P;   // elements needed from the left
  constexpr int NR = DX ? P : K - 1 - P;   // elements needed from the right
  constexpr uint32_t kSpanBytes = 64u * U * 16u;

  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t wpb = blockDim.x / kWave;
  const uint64_t gw = (uint64_t)blockIdx.x * wpb + threadIdx.x / kWave;
  const uint64_t nw = (uint64_t)gridDim.x * wpb;
  if (gw >= nspans) return;

  // Column and channel of each of the lane's float4s (the same in every
  // span of this wave), and that channel's taps.
  const uint32_t HL = (uint32_t)H * (uint32_t)L;
  const uint32_t bmod = (uint32_t)((gw * (uint64_t)(64 * U) * 4u) % HL);
  int col[U];
  float wt[U][K];
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t r = (bmod + 4u * (uint32_t)(64 * u + lane)) % HL;
    const uint32_t h = r / (uint32_t)L;
    col[u] = (int)(r - h * (uint32_t)L);
#pragma unroll
    for (int j = 0; j < K; ++j) wt[u][j] = buf_load1(rw, (h * (uint32_t)K + (uint32_t)j) * 4u, 0);
  }

  for (uint64_t s = gw; s < nspans; s += nw) {
    const uint64_t f0 = s * (uint64_t)(64 * U);           // first float4 of the span
    const uint64_t hb = f0 ? f0 - 1 : 0;                  // first float4 the resource covers
    const uint32_t lead = (uint32_t)(f0 - hb) * 16u;      // bytes before the span (0 or 16)
    const uint64_t left = (nf4 - hb) * 16u;
    const uint32_t nrec = left < (uint64_t)(kSpanBytes + 32u) ? (uint32_t)left : kSpanBytes + 32u;
    const __amdgpu_buffer_rsrc_t rin = make_rsrc_n(in + 4 * hb, nrec);
    const uint64_t oleft = (nf4 - f0) * 16u;
    const __amdgpu_buffer_rsrc_t rout =
        make_rsrc_n(out + 4 * f0, oleft < (uint64_t)kSpanBytes ? (uint32_t)oleft : kSpanBytes);

    float4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      x[u] = buf_load4<LOAD_CPOL>(rin, lead + (uint32_t)(64 * u + lane) * 16u, 0);
    // Lane 0: the float4 before the span (none for the first span); lane 1:
    // the float4 after it (past the tensor's end it reads 0 and is unused).
    const uint32_t hoff = lane == 0 ? (f0 ? 0u : kOob) : lane == 1 ? lead + kSpanBytes : kOob;
    const float4 halo = buf_load4(rin, hoff, 0);

#pragma unroll
    for (int u = 0; u < U; ++u) {
      // win[4 + d] = element d of the row relative to the float4's column 0,
      // d in [-NL, 3 + NR].
      float win[12];
      win[4] = x[u].x;
      win[5] = x[u].y;
      win[6] = x[u].z;
      win[7] = x[u].w;
#pragma unroll
      for (int q = 0; q < NL; ++q) {   // left: component 3 - q of float4 - 1
        const int c = 3 - q;
        const float edge = u == 0 ? lane_of(f4c(halo, c), 0) : lane_of(f4c(x[u - 1], c), 63);
        win[c] = dpp_shift<0x138>(f4c(x[u], c), edge);       // wave_shr:1
      }
#pragma unroll
      for (int q = 0; q < NR; ++q) {   // right: component q of float4 + 1
        const float edge = u == U - 1 ? lane_of(f4c(halo, q), 1) : lane_of(f4c(x[u + 1], q), 0);
        win[8 + q] = dpp_shift<0x130>(f4c(x[u], q), edge);   // wave_shl:1
      }
      const bool lok = col[u] >= 4;
      const bool rok = col[u] + 4 < L;
      float acc[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < K; ++j) {
          const int idx = 4 + c + (DX ? P - j : j - P);
          const float f = fmaf(win[idx], wt[u][j], a);
          a = idx < 4 ? (lok ? f : a) : idx >= 8 ? (rok ? f : a) : f;
        }
        acc[c] = a;
      }
      buf_store4<kCpolNT>(make_float4(acc[0], acc[1], acc[2], acc[3]), rout,
                          (uint32_t)(64 * u + lane) * 16u);
    }
  }
}

// ---------------------------------------------------------------------------
// Wave reduction: DPP within 16-lane rows, ds_bpermute across rows. Every
// lane ends with the same total.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// ---------------------------------------------------------------------------
// DK: workgroup = (channel h, batch tile of wpb * R * 64 samples). Wave w
// takes the tile's 64-sample chunks w, w + wpb, ... (R of them); lane = one
// sample. The x row is register resident; dy arrives one 16-column chunk at
// a time and is consumed at once. det == 0: one atomic add per tap per
// workgroup into dk. det != 0: partials[(h*K + j) * nbt + bt] (no atomics).
// ---------------------------------------------------------------------------
template <int LMAX, int KB, bool VEC>
__global__ __launch_bounds__(kMaxDkThreads) void dwconv_dk_kernel(
    const float* __restrict__ gy, const float* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int R, int nbt,
    uint32_t nblocks, int det) {
  constexpr int vec = VEC ? 1 : 0;
  using W = Window<LMAX, KB, false>;
  using IO = TileIO<LMAX>;
  using G = RowGeo<LMAX>;
  extern __shared__ float lds[];
  __shared__ float red[kMaxWaves][W::n];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wpb = blockDim.x / kWave;
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int h = (int)(blk % (uint32_t)H);
  const int bt = (int)(blk / (uint32_t)H);
  const uint32_t rstride = (uint32_t)H * (uint32_t)L;
  float* stage = lds + wave * kStageFloats;

  float acc[W::n];
#pragma unroll
  for (int i = 0; i < W::n; ++i) acc[i] = 0.0f;

  const int tile0 = bt * wpb * R * kWave;
  for (int r = 0; r < R; ++r) {
    // readfirstlane keeps the chunk base opaque to loop strength reduction,
    // which would otherwise carry one 64-bit address per load across
    // iterations and spill them.
    const int b0 = __builtin_amdgcn_readfirstlane(tile0 + (wave + wpb * r) * kWave);
    if (b0 >= B) break;  // wave-uniform
    const int nrows = min(kWave, B - b0);
    const size_t row0 = ((size_t)b0 * (size_t)H + (size_t)h) * (size_t)L;

    float xr[LMAX];
    IO::load_rows(make_rsrc(x + row0), rstride, nrows, L, lane, vec, stage, xr);
    const __amdgpu_buffer_rsrc_t grsrc = make_rsrc(gy + row0);
    static_for<0, G::nchunks>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      constexpr int nc = G::cols(c);
      float g[kChunk];
      IO::template load_chunk<c>(grsrc, rstride, nrows, L, lane, vec, stage, g);
#pragma unroll
      for (int tt = 0; tt < nc; ++tt) {
        const int t = kChunk * c + tt;
#pragma unroll
        for (int i = 0; i < W::n; ++i) {
          const int s = t + W::lo + i;
          if (s >= 0 && s < LMAX) acc[i] = fmaf(g[tt], xr[s], acc[i]);
        }
      }
    });
  }

#pragma unroll
  for (int i = 0; i < W::n; ++i) acc[i] = wave_sum(acc[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < W::n; ++i) red[wave][i] = acc[i];
  }
  __syncthreads();

  // Threads 0..K-1: tap j; fixed summation order over waves.
  const int j = threadIdx.x;
  if (j < K) {
    const int m = j - (K >> 1);
    const bool in_window = m >= W::lo && m <= W::hi;
    float v = 0.0f;
    if (in_window) {
      for (int wv = 0; wv < wpb; ++wv) v += red[wv][m - W::lo];
    }
    if (det) {
      dst[((size_t)h * K + j) * (size_t)nbt + bt] = v;
    } else if (in_window) {
      atomicAdd(dst + (size_t)h * K + j, v);
    }
  }
}

// ---------------------------------------------------------------------------
// DK on the matrix cores. For channel h, D[t][s] = sum_b dy[b,t] * x[b,s] is
// a GEMM whose contraction runs over the batch, so v_mfma_f32_16x16x4_f32
// takes its operands straight from row-major HBM: for a step of 4 samples,
// lane l holds dy[b0 + l/16][16*tt + l%16] (A, 16 t x 4 b) and
// x[b0 + l/16][16*ts + l%16] (B, 4 b x 16 s); D is NT x NT tiles of 16 x 16
// (NT = LMAX/16), lane l, register r of a tile holding
// D[16*tt + 4*(l/16) + r][16*ts + l%16]. After its rows, a wave writes D to
// LDS and lane j sums the diagonal s - t = j - p over the valid t
// (benchmark/diagnose_dk_correctness.py:21), in a fixed order. Workgroup =
// (h, batch tile of wpb * rpw samples); then the same LDS reduction over
// waves and per-workgroup atomic / partial store as the VALU kernel.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int LMAX>
struct MfmaGeo {
  static constexpr int nt = (LMAX + 15) / 16;   // 16-wide tiles per side
  static constexpr int dim = 16 * nt;
  static constexpr int dstride = dim + 1;       // LDS row stride of D
  static constexpr int dfloats = dim * dstride; // per-wave D in LDS
};

template <int LMAX, int LOAD_CPOL = kCpolNone>
__global__ __launch_bounds__(1024) void dwconv_dk_mfma_kernel(
    const float* __restrict__ gy, const float* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int rpw, int nbt,
    uint32_t nblocks, int det) {
  using M = MfmaGeo<LMAX>;
  constexpr int NT = M::nt;
  // 4-sample steps per load group: 48 samples at LMAX = 16, 24 at 32, 16 at
  // 48, so a group moves about the same bytes whatever the row length (the
  // operand registers, 4 * kSteps * NT, stay at 48).
  constexpr int kSteps = 12 / NT;
  __shared__ float dsum[M::dfloats];  // workgroup sum of the waves' D

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wpb = blockDim.x / kWave;
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int h = (int)(blk % (uint32_t)H);
  const int bt = (int)(blk / (uint32_t)H);
  const uint32_t rstride = (uint32_t)H * (uint32_t)L;

  const int b_begin = bt * wpb * rpw + wave * rpw;
  const int b_end = min(B, b_begin + rpw);
  const int nrow = max(0, b_end - b_begin);

  f32x4 acc[NT][NT];
#pragma unroll
  for (int a = 0; a < NT; ++a)
#pragma unroll
    for (int b = 0; b < NT; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (nrow > 0) {
    const size_t row0 = ((size_t)b_begin * (size_t)H + (size_t)h) * (size_t)L;
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(gy + row0);
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + row0);
    const int kq = lane >> 4;   // sample within a 4-sample step
    const int col = lane & 15;  // column within a 16-wide tile
    const uint32_t off = ((uint32_t)kq * rstride + (uint32_t)col) * 4u;
    const uint32_t step_bytes = 4u * rstride * 4u;
    const int ngroups = (nrow + 4 * kSteps - 1) / (4 * kSteps);

    // Operands of one group of kSteps steps (4 * kSteps samples).
    auto load_group = [&](int g, float (&av)[kSteps][NT], float (&bv)[kSteps][NT]) {
#pragma unroll
      for (int u = 0; u < kSteps; ++u) {
        const int step = g * kSteps + u;
        const uint32_t soff = (uint32_t)step * step_bytes;
        const bool row_ok = step * 4 + kq < nrow;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
          const bool ok = row_ok && 16 * tt + col < L;
          const uint32_t o = ok ? off + 64u * tt : kOob;
          av[u][tt] = buf_load1<LOAD_CPOL>(gr, o, soff);
          bv[u][tt] = buf_load1<LOAD_CPOL>(xr, o, soff);
        }
      }
    };
    auto mfma_group = [&](const float (&av)[kSteps][NT], const float (&bv)[kSteps][NT]) {
#pragma unroll
      for (int u = 0; u < kSteps; ++u)
#pragma unroll
        for (int a = 0; a < NT; ++a)
#pragma unroll
          for (int b = 0; b < NT; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                av[u][a], bv[u][b], acc[a][b], 0, 0, 0);
    };

    // Two register buffers: the loads of group g + 1 are in flight while the
    // matrix cores consume group g.
    float a0[kSteps][NT], b0[kSteps][NT], a1[kSteps][NT], b1[kSteps][NT];
    load_group(0, a0, b0);
    for (int g0 = 0; g0 < ngroups; g0 += 2) {
      const int g = __builtin_amdgcn_readfirstlane(g0);
      if (g + 1 < ngroups) load_group(g + 1, a1, b1);
      mfma_group(a0, b0);
      if (g + 1 >= ngroups) break;
      if (g + 2 < ngroups) load_group(g + 2, a0, b0);
      mfma_group(a1, b1);
    }
  }

  // Sum the waves' D in a fixed order (wave 0, 1, ...), then one diagonal
  // reduction per workgroup: thread j sums D[t][t + j - p] over valid t.
  const int rq = 4 * (lane >> 4);
  const int cl = lane & 15;
  for (int wv = 0; wv < wpb; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int a = 0; a < NT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float* d = dsum + (16 * a + rq + r) * M::dstride + 16 * b + cl;
            *d = (wv == 0) ? acc[a][b][r] : *d + acc[a][b][r];
          }
    }
    __syncthreads();
  }

  const int j = threadIdx.x;
  if (j < K) {
    const int m = j - (K >> 1);
    const int t0 = max(0, -m);
    const int t1 = min(L, L - m);
    // Four independent partial sums (t = t0 + 4i + q), combined in a fixed
    // order: a shorter dependency chain, the same result every run.
    // D[t][t + m] = dsum[t * dstride + t + m] = diag[t * (dstride + 1)].
    float v4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float* diag = dsum + m;
    for (int t = t0; t < t1; t += 4) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (t + q < t1) v4[q] += diag[(t + q) * (M::dstride + 1)];
    }
    const float v = (v4[0] + v4[1]) + (v4[2] + v4[3]);
    if (det) {
      dst[((size_t)h * K + j) * (size_t)nbt + bt] = v;
    } else {
      atomicAdd(dst + (size_t)h * K + j, v);
    }
  }
}

// ---------------------------------------------------------------------------
// FWD / DX on channel-group tiles (matrix cores), for long FMA chains.
//   FWD: y [b,h,t] = sum_s x [b,h,s] * w[h, s - t + p]
//   DX : dx[b,h,t] = sum_s dy[b,h,s] * w[h, t - s + p]
// i.e. per channel a product of the [samples x L] rows with the banded
// Toeplitz matrix of the taps. Workgroup (g, r) owns channel group g (one
// channel per wave, HC = 8 or 16 waves) and the interleaved 16-sample steps
// r, r + nranges, ...; per step it stages the group's contiguous segments
// [b, g*HC .. g*HC+HC, :] through LDS (input and output stages, one or two
// barriers per step) and each wave runs v_mfma_f32_16x16x4_f32 with M = 16
// samples, N = 16 output columns, K = 4 input columns. K slot kk of MFMA step
// u is input column u + (LMAX/4) * kk, so a lane reads its A operands as
// LMAX/4 consecutive floats and its B operands (the taps) are loaded once.
// The sums run in the matrix cores' order, not the reference's fmaf chain:
// results agree with it to FP32 rounding (about 3e-7 max-abs-scaled).
// ---------------------------------------------------------------------------
constexpr int kRowsCgWaves = 8;    // one channel per wave
constexpr int kRowsCgStep = 16;    // samples per step (MFMA M)

// BF16 bit pattern of an FP32 value, round-to-nearest-even (a NaN stays a
// quiet NaN).
__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Two FP32 values as packed BF16 (a in the low half), round-to-nearest-even:
// one v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t bf16_pack2(float a, float b) {
  const uint32_t lo = __builtin_bit_cast(uint16_t, (__bf16)a);
  const uint32_t hi = __builtin_bit_cast(uint16_t, (__bf16)b);
  return lo | (hi << 16);
}

// A 16-byte chunk (4 FP32 values) between registers and LDS.
__device__ __forceinline__ void chunk_to_lds(float* dst, const u32x4 v) {
  *reinterpret_cast<float4*>(dst) =
      make_float4(__uint_as_float(v.x), __uint_as_float(v.y),
                  __uint_as_float(v.z), __uint_as_float(v.w));
}

__device__ __forceinline__ u32x4 lds_to_chunk(const float* src) {
  const float4 a = *reinterpret_cast<const float4*>(src);
  u32x4 v;
  v.x = __float_as_uint(a.x);
  v.y = __float_as_uint(a.y);
  v.z = __float_as_uint(a.z);
  v.w = __float_as_uint(a.w);
  return v;
}

template <int CPOL = kCpolNone>
__device__ __forceinline__ u32x4 buf_load_chunk(__amdgpu_buffer_rsrc_t r,
                                                uint32_t voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, CPOL);
}

template <int CPOL = kCpolNone>
__device__ __forceinline__ void buf_store_chunk(u32x4 v, __amdgpu_buffer_rsrc_t r,
                                                uint32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, CPOL);
}

template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_t(const T* base) {
  return make_rsrc(reinterpret_cast<const float*>(base));
}

__host__ __device__ constexpr size_t rows_cg_lds_bytes(int L, int hc = kRowsCgWaves,
                                                       int nin = 2) {
  // nin input + two output stages of 16 samples x (HC * L + 4) floats
  return (size_t)(nin + 2) * kRowsCgStep * (hc * L + 4) * sizeof(float);
}

// kDepth: steps in flight in registers; HC: channels (= waves) per
// workgroup; NIN: input stages in LDS. With two, one barrier per step
// separates the MFMAs of step s (and the input store of step s + 1) from
// the output flush of step s. With one (16 channels at L = 48, whose two
// input and two output stages would not fit), a second barrier per step
// keeps the input store of step s + 1 after every wave's reads of step s.
//
// Non-finite values. The band matrix multiplies every input column of a
// sample by every output column's taps, zeros included, so one Inf or NaN
// input turns every output of its sample (in that channel) into NaN, where
// the reference's fmaf chain touches an input only through the taps whose
// window holds it (kernels/warp_tiled_ampere.py:411-430, :479-498). Because
// every output's sum meets every input column, one output per lane shows
// it: a lane whose first output is not finite recomputes its outputs with
// the reference's chain (same start value, tap order and skipped terms)
// from the input stage, so those outputs are bit-exact with the reference.
// A non-finite tap needs no such care: band entries are the taps themselves
// where the window holds an element and exact zeros elsewhere, so a
// non-finite tap multiplies exactly the reference's terms, and a sum of
// terms of which some are infinite or NaN has the same non-finite value in
// any order (sums that overflow FP32 aside). A wave whose lanes all see
// finite first outputs skips the chain.
//
// LOAD_CPOL: cache policy of the input loads (stores are non-temporal).
//
// A4: rows are whole float4s (L % 4 == 0). Without it (any L; H % 8 == 0
// and 16-byte aligned tensors, so a segment of HC rows is still a whole
// number of 16-byte chunks and every sample's segments start 16-byte
// aligned), a channel's row starts at an arbitrary float in the stage: the
// lane reads its A operands and writes its outputs one float at a time, and
// an output chunk that straddles L is written element by element.
template <int LMAX, bool DX, int kDepth, int HC = kRowsCgWaves, int NIN = 2,
          int LOAD_CPOL = kCpolNT, bool A4 = true>
__global__ __launch_bounds__(HC * kWave) void dwconv_rows_cg_kernel(
    const float* __restrict__ in, const float* __restrict__ w,
    float* __restrict__ out, int B, int H, int L, int K, int nranges,
    uint32_t nblocks) {
  constexpr int NT = LMAX / 16;  // 16-wide output tiles
  constexpr int NU = LMAX / 4;   // MFMA steps over the input columns
  constexpr int EPC = 4;  // floats per 16-byte chunk
  constexpr int kNpt = (HC * LMAX * kRowsCgStep / EPC + HC * kWave - 1) / (HC * kWave);
  extern __shared__ float lds[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int ngroups = H / HC;
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int g = (int)(blk % (uint32_t)ngroups);
  const int r = (int)(blk / (uint32_t)ngroups);
  const int tsteps = (B + kRowsCgStep - 1) / kRowsCgStep;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;

  const int seg = HC * L, segc = seg / EPC;  // elements, chunks per sample
  const int sk = seg + 4;                 // LDS stride between samples
  const int sz = kRowsCgStep * sk;        // one stage
  const int per = kRowsCgStep * segc;     // chunks per stage
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 4u;
  const uint32_t grp_bytes = (uint32_t)g * (uint32_t)seg * 4u;
  float* inl = lds;                       // input stage(s)
  float* outl = lds + NIN * sz;           // output stages 0, 1

  // Loop-invariant part of each staged chunk (as in the DK kernel).
  int ek[kNpt];
  uint32_t eoff[kNpt], elds[kNpt];
#pragma unroll
  for (int i = 0; i < kNpt; ++i) {
    const int e = i * (HC * kWave) + (int)threadIdx.x;
    const int k = e < per ? e / segc : kRowsCgStep;
    const int q = e - (e / segc) * segc;
    ek[i] = k;
    eoff[i] = (uint32_t)k * row_bytes + grp_bytes + 16u * (uint32_t)q;
    elds[i] = (uint32_t)(k * sk + EPC * q);
  }
  u32x4 stg[kDepth][kNpt];
  auto load_step = [&](int s, u32x4 (&st)[kNpt]) {
    const int bs = (r + s * nranges) * kRowsCgStep;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(in + (size_t)bs * (size_t)H * (size_t)L);
    const int klim = min(kRowsCgStep, B - bs);
#pragma unroll
    for (int i = 0; i < kNpt; ++i)
      st[i] = buf_load_chunk<LOAD_CPOL>(rs, ek[i] < klim ? eoff[i] : kOob);
  };
  auto store_stage = [&](int buf, const u32x4 (&st)[kNpt]) {
#pragma unroll
    for (int i = 0; i < kNpt; ++i)
      if (ek[i] < kRowsCgStep) chunk_to_lds(inl + buf * sz + elds[i], st[i]);
  };
  auto flush_out = [&](int s) {
    const float* o = outl + (s & 1) * sz;
    const int bs = (r + s * nranges) * kRowsCgStep;
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(out + (size_t)bs * (size_t)H * (size_t)L);
    const int klim = min(kRowsCgStep, B - bs);
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      const u32x4 v = lds_to_chunk(o + (ek[i] < kRowsCgStep ? elds[i] : 0u));
      buf_store_chunk<kCpolNT>(v, ro, ek[i] < klim ? eoff[i] : kOob);
    }
  };

  // B operands: step u, tile tt, lane l -> input column s = u + NU*(l/16),
  // output column t = 16 tt + l % 16; zero outside the band and the row.
  const int kk = lane >> 4, jj = lane & 15;
  const int p = K >> 1;
  const int h = g * HC + wave;
  const float* wh = w + (size_t)h * K;
  float bt[NU][NT];
#pragma unroll
  for (int u = 0; u < NU; ++u)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int sc = u + NU * kk, tc = 16 * tt + jj;
      const int j = DX ? (tc - sc + p) : (sc - tc + p);
      const bool ok = j >= 0 && j < K && sc < L && tc < L;
      bt[u][tt] = ok ? wh[j] : 0.0f;
    }

  const int rq = 4 * kk;
  const int cb = wave * L;
  auto mfma_step = [&](int s) {
    const float* row = inl + (NIN == 2 ? (s & 1) : 0) * sz + jj * sk + cb;  // sample jj, this channel
    const float* src = row + NU * kk;
    float* orow = outl + (s & 1) * sz + jj * sk + cb;
    float a[NU];
    if constexpr (A4) {
#pragma unroll
      for (int q = 0; q < NU / 4; ++q) {
        const float4 v = *reinterpret_cast<const float4*>(src + 4 * q);
        a[4 * q + 0] = v.x;
        a[4 * q + 1] = v.y;
        a[4 * q + 2] = v.z;
        a[4 * q + 3] = v.w;
      }
      if (L != LMAX) {  // columns >= L belong to the next channel: zero them
#pragma unroll
        for (int u = 0; u < NU; ++u) a[u] = u + NU * kk < L ? a[u] : 0.0f;
      }
    } else {
      // Columns >= L are read where they lie (the next channel's row, or
      // past the input stage into the next stage of the allocation, which
      // always follows: at most LMAX - L - 5 floats past a stage, and which
      // other waves may be filling meanwhile) and zeroed, so their values
      // never matter. Reading in place keeps one base address for the whole row:
      // a per-column clamped address cost 21 VGPRs (129 against 108), which
      // held the 8-channel kernel to one workgroup per CU.
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const float v = src[u];
        a[u] = u + NU * kk < L ? v : 0.0f;
      }
    }
    // The MFMA computes the transposed tile (taps as A, rows as B; each lane
    // supplies the same values either way), so lane (jj, kk) holds output
    // columns 16 tt + 4 kk .. + 3 of sample jj: one 16-byte LDS write.
    bool bad = false;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < NU; ++u)
        d = __builtin_amdgcn_mfma_f32_16x16x4f32(bt[u][tt], a[u], d, 0, 0, 0);
      if (tt == 0) bad = !__builtin_isfinite(d[0]);
      const int t = 16 * tt + rq;
      if constexpr (A4) {  // L % 4 == 0: all four columns or none
        if (t < L) *reinterpret_cast<f32x4*>(orow + t) = d;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t + e < L) orow[t + e] = d[e];
      }
    }
    if (__builtin_amdgcn_ballot_w64(bad)) {
      if (bad) {
#pragma unroll 1
        for (int q = 0; q < 4 * NT; ++q) {
          const int t = 16 * (q >> 2) + rq + (q & 3);
          if (t < L) {
            float acc = 0.0f;
#pragma unroll 1
            for (int j = 0; j < K; ++j) {
              const int e = DX ? t - j + p : t + j - p;
              if ((unsigned)e < (unsigned)L) acc = fmaf(row[e], wh[j], acc);
            }
            orow[t] = acc;
          }
        }
      }
    }
  };

  if (nsteps > 0 && NIN == 2) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d)
      if (d < nsteps) load_step(d, stg[d]);
    store_stage(0, stg[0]);
    if (kDepth < nsteps) load_step(kDepth, stg[0]);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          // Input stage (s + 1) & 1 was last read by mfma_step(s - 1) and
          // output stage s & 1 by flush_out(s - 2), both finished by every
          // thread before the barrier of step s - 1. The next step's input
          // goes to LDS and the loads after it are issued before this
          // step's matrix work, so they overlap it: 3-9% faster than after
          // the MFMAs on medium and large calls (rows of 24-48 columns),
          // up to 3% slower on calls of a few microseconds.
          if (s + 1 < nsteps) {
            store_stage((s + 1) & 1, stg[(d + 1) % kDepth]);
            if (s + 1 + kDepth < nsteps)
              load_step(s + 1 + kDepth, stg[(d + 1) % kDepth]);
          }
          mfma_step(s);
          __syncthreads();
          flush_out(s);
        }
      }
    }
  } else if (nsteps > 0) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d)
      if (d < nsteps) load_step(d, stg[d]);
    for (int s0 = 0; s0 < nsteps; s0 += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          // The input stage was last read by mfma_step(s - 1), which every
          // thread finished before the second barrier of step s - 1; output
          // stage s & 1 was last read by flush_out(s - 2), finished before
          // the first barrier of step s - 1.
          store_stage(0, stg[d]);
          if (s + kDepth < nsteps) load_step(s + kDepth, stg[d]);
          __syncthreads();
          mfma_step(s);
          __syncthreads();
          flush_out(s);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// FWD / DX with BF16 I/O on the BF16 matrix cores. The channel-group tiling
// and pipeline of dwconv_rows_cg_kernel, with these differences:
//  * the input stages hold the BF16 values as they arrive (2 bytes each), and
//    a lane reads its A operands straight from them as 4-element BF16
//    vectors (no widening);
//  * v_mfma_f32_16x16x16_bf16 (M = 16 samples, N = 16 output columns,
//    K = 16 input columns) replaces four FP32 16x16x4 instructions; K slot
//    4 kg + i of MFMA u is input column (LMAX/4) kg + 4 u + i, so a lane's A
//    operands for all u are LMAX/4 consecutive values;
//  * the FP32 taps enter as two BF16 operands, hi = bf16(w) and
//    lo = bf16(w - hi), two MFMAs per chunk: the products x * hi + x * lo are
//    exact in FP32 and hi + lo differs from w by at most 2^-16 |w|, far
//    below the BF16 rounding of the outputs;
//  * each lane rounds its FP32 results to BF16 (nearest-even) as it writes
//    them to the output stage, which therefore holds BF16 values and is
//    copied out in 16-byte chunks;
//  * HC is 16 channels (1024 threads) where H allows: a workgroup then moves
//    1.5 KiB per sample at L = 48 instead of 768 bytes, which measured 8%
//    faster at P and 12% at S on MI355X.
typedef short s16x4 __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr size_t rows_bf16mma_lds_bytes(int L, int hc) {
  // two input and two output stages of 16 samples x (hc * L + 8) BF16 values
  return (size_t)4 * kRowsCgStep * (hc * L + 8) * sizeof(uint16_t);
}

template <int LMAX, bool DX, int HC, int LOAD_CPOL = kCpolNT>
__global__ __launch_bounds__(HC * kWave) void dwconv_rows_bf16mma_kernel(
    const uint16_t* __restrict__ in, const float* __restrict__ w,
    uint16_t* __restrict__ out, int B, int H, int L, int K, int nranges,
    uint32_t nblocks) {
  constexpr int NT = LMAX / 16;    // 16-wide output tiles
  constexpr int NUB = LMAX / 4;    // input columns per K group of a lane
  constexpr int NG = NUB / 4;      // MFMAs (16 input columns) per tile
  constexpr int kDepth = 2;        // steps in flight in registers
  constexpr int kNpt = (HC * LMAX * kRowsCgStep / 8 + HC * kWave - 1) / (HC * kWave);
  extern __shared__ float lds[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int ngroups = H / HC;
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int g = (int)(blk % (uint32_t)ngroups);
  const int r = (int)(blk / (uint32_t)ngroups);
  const int tsteps = (B + kRowsCgStep - 1) / kRowsCgStep;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;

  const int seg = HC * L, segc = seg / 8;   // BF16 values, 16-byte chunks
  const int ski = seg + 8;                  // input-stage stride (values)
  const int sko = seg + 8;                  // output-stage stride (values)
  const int per = kRowsCgStep * segc;       // chunks per stage
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 2u;
  const uint32_t grp_bytes = (uint32_t)g * (uint32_t)seg * 2u;
  uint16_t* inl = reinterpret_cast<uint16_t*>(lds);             // 2 stages
  uint16_t* outl = inl + 2 * kRowsCgStep * ski;                  // 2 stages
  const int szi = kRowsCgStep * ski, szo = kRowsCgStep * sko;

  int ek[kNpt];
  uint32_t eoff[kNpt], elds[kNpt], oelds[kNpt];
#pragma unroll
  for (int i = 0; i < kNpt; ++i) {
    const int e = i * (HC * kWave) + (int)threadIdx.x;
    const int k = e < per ? e / segc : kRowsCgStep;
    const int q = e - (e / segc) * segc;
    ek[i] = k;
    eoff[i] = (uint32_t)k * row_bytes + grp_bytes + 16u * (uint32_t)q;
    elds[i] = (uint32_t)(k * ski + 8 * q);   // in BF16 values
    oelds[i] = (uint32_t)(k * sko + 8 * q);
  }
  u32x4 stg[kDepth][kNpt];
  auto load_step = [&](int s, u32x4 (&st)[kNpt]) {
    const int bs = (r + s * nranges) * kRowsCgStep;
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc_t(in + (size_t)bs * (size_t)H * (size_t)L);
    const int klim = min(kRowsCgStep, B - bs);
#pragma unroll
    for (int i = 0; i < kNpt; ++i)
      st[i] = buf_load_chunk<LOAD_CPOL>(rs, ek[i] < klim ? eoff[i] : kOob);
  };
  auto store_stage = [&](int buf, const u32x4 (&st)[kNpt]) {
#pragma unroll
    for (int i = 0; i < kNpt; ++i)
      if (ek[i] < kRowsCgStep)
        *reinterpret_cast<u32x4*>(inl + buf * szi + elds[i]) = st[i];
  };
  auto flush_out = [&](int s) {
    const int bs = (r + s * nranges) * kRowsCgStep;
    const __amdgpu_buffer_rsrc_t ro =
        make_rsrc_t(out + (size_t)bs * (size_t)H * (size_t)L);
    const int klim = min(kRowsCgStep, B - bs);
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      const uint32_t oe = ek[i] < kRowsCgStep ? oelds[i] : 0u;
      const u32x4 v = *reinterpret_cast<const u32x4*>(outl + (s & 1) * szo + oe);
      buf_store_chunk<kCpolNT>(v, ro, ek[i] < klim ? eoff[i] : kOob);
    }
  };

  // B operands: MFMA u, tile tt, lane (n = l % 16, kg = l / 16), element i:
  // input column s = NUB kg + 4 u + i, output column t = 16 tt + n.
  const int kg = lane >> 4, jj = lane & 15;
  const int p = K >> 1;
  const int h = g * HC + wave;
  s16x4 bh[NG][NT], bl[NG][NT];
#pragma unroll
  for (int u = 0; u < NG; ++u)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int sc = NUB * kg + 4 * u + i, tc = 16 * tt + jj;
        const int j = DX ? (tc - sc + p) : (sc - tc + p);
        const bool ok = j >= 0 && j < K && sc < L && tc < L;
        const float wv = ok ? w[(size_t)h * K + j] : 0.0f;
        const uint32_t hi = bf16_bits_rne(wv);
        const uint32_t lo = bf16_bits_rne(wv - __uint_as_float(hi << 16));
        bh[u][tt][i] = (short)hi;
        bl[u][tt][i] = (short)lo;
      }

  const int rq = 4 * kg;
  const int cb = wave * L;
  auto mfma_step = [&](int s) {
    const uint16_t* src = inl + (s & 1) * szi + jj * ski + cb + NUB * kg;  // sample jj
    uint16_t* o = outl + (s & 1) * szo;
    s16x4 a[NG];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      a[u] = *reinterpret_cast<const s16x4*>(src + 4 * u);
      if (L != LMAX && NUB * kg + 4 * u >= L) a[u] = s16x4{0, 0, 0, 0};
    }
    // The MFMA computes the transposed tile (taps as A, rows as B; each lane
    // supplies the same values either way), so lane (jj, kg) holds output
    // columns 16 tt + 4 kg .. + 3 of sample jj: two packed conversions and
    // one 8-byte LDS write.
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < NG; ++u) {
        d = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bh[u][tt], a[u], d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bl[u][tt], a[u], d, 0, 0, 0);
      }
      const int t = 16 * tt + rq;  // L % 4 == 0: all four columns or none
      if (t < L) {
        u32x2 v;
        v.x = bf16_pack2(d[0], d[1]);
        v.y = bf16_pack2(d[2], d[3]);
        *reinterpret_cast<u32x2*>(o + jj * sko + cb + t) = v;
      }
    }
  };

  if (nsteps > 0) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d)
      if (d < nsteps) load_step(d, stg[d]);
    store_stage(0, stg[0]);
    if (kDepth < nsteps) load_step(kDepth, stg[0]);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          mfma_step(s);
          if (s + 1 < nsteps) {
            store_stage((s + 1) & 1, stg[(d + 1) % kDepth]);
            if (s + 1 + kDepth < nsteps)
              load_step(s + 1 + kDepth, stg[(d + 1) % kDepth]);
          }
          __syncthreads();
          flush_out(s);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// DK on channel-group tiles (matrix cores). For a sample b the rows of
// channels [g*HC, g*HC + HC) are one contiguous segment of HC * L floats, so
// a workgroup that owns channel group g streams whole segments instead of
// one 192-byte row per channel: full cache lines, and no line shared with a
// channel that another workgroup reads.
//
// Workgroup (g, r) owns channel group g of HC = CPW * wpb (CPW channels per
// wave: dk_cg_cpw(LMAX))
// channels and the interleaved steps r, r + nranges, r + 2 nranges, ... of
// 4 samples each. At any moment the running workgroups therefore cover one
// compact window of nranges steps of the whole [b, :, :] tensor; the host
// picks nranges so that a workgroup's successive steps lie about 2.5 MiB
// apart (contiguous per-workgroup sample ranges instead put every workgroup
// a fixed multi-MiB stride apart, and the time then swung by 30 % with that
// stride on MI355X).
//
// Per step the workgroup loads both tensors' segments (dwordx4 chunks where
// the tensors are 16-byte aligned and segments and samples are whole chunks,
// dwords otherwise: any L) into registers two steps ahead and into one
// of two LDS stages while the matrix cores consume the other; wave w
// accumulates D_c[t][s] = sum_b dy[b,c,t] * x[b,c,s] for its channels, then
// reduces the diagonals of each D_c (dk[c, j] = sum_t D_c[t][t + j - p])
// through a per-wave LDS tile: one atomic (or one partial) per tap and
// channel per workgroup.
// ---------------------------------------------------------------------------
constexpr int kCgChannelsPerWave = 2;

// Channels per wave of the FP32 row-major DK for a row bucket: one in the
// 48-column bucket (16 resident waves per CU with half the matrix work each,
// 3-7% faster at L = 40-48 with 256 or more threads per workgroup), two
// below (one per wave was 5-25% slower at L = 24 and H = 256).
__host__ __device__ constexpr int dk_cg_cpw(int lmax) { return lmax >= 48 ? 1 : 2; }
constexpr int kCgStep = 4;      // samples per stage (the MFMA K)
constexpr int kCgPad = 16;      // floats between the samples of a stage
constexpr int kCgDepth = 2;     // steps in flight in registers

template <int LMAX>
struct CgGeo {
  static constexpr int nt = LMAX / 16;
  static constexpr int dim = 16 * nt;
  static constexpr int dstride = dim + 1;
};

// Dynamic LDS of the channel-group DK kernel: two stages of both tensors,
// or, for the epilogue, one D tile per wave plus the workgroup's tap sums.
__host__ __device__ constexpr size_t cg_lds_bytes(int lmax, int wpb, int L,
                                                  int cpw) {
  const size_t stages =
      (size_t)2 * 2 * kCgStep * (cpw * wpb * L + kCgPad);
  const size_t dtile = (size_t)wpb * (16 * (lmax / 16)) * (16 * (lmax / 16) + 1) +
                       (size_t)cpw * wpb * kMaxK;
  return (stages > dtile ? stages : dtile) * sizeof(float);
}

// Epilogue shared by the channel-group DK kernels. Per wave: D_c through
// the wave's own LDS tile (the stages are free after the kernel's last
// barrier), then lane j < K sums D_c[t][t + j - p] over t in [t0, t1) in
// four fixed-order partial sums, all reads issued at once (the t loop is
// unrolled over the bucket, out-of-range terms masked). The workgroup's
// channels are consecutive, so its hc x K tap sums are one contiguous block
// of dk: they are collected in LDS and added with one coalesced atomic per
// element (a few cache lines per workgroup, not one line operation per wave
// and channel, which contended badly at small K). det: write the sums as
// partials [h][j][nranges] instead. CL: dk is [K][H] (the channels-last
// layout's dw), whose hc channels of one tap are contiguous; atomics only.
template <int LMAX, bool CL = false, int CPW = kCgChannelsPerWave>
__device__ __forceinline__ void dk_cg_epilogue(
    const f32x4 (&acc)[CPW][LMAX / 16][LMAX / 16], float* lds,
    float* __restrict__ dst, int wave, int wpb, int g, int r, int hc, int L,
    int K, int nranges, int det, int H = 0) {
  using G = CgGeo<LMAX>;
  constexpr int NT = G::nt;
  const int lane = threadIdx.x & (kWave - 1);
  const int nthreads = blockDim.x;
  float* dt = lds + wave * (G::dim * G::dstride);
  float* taps = lds + wpb * (G::dim * G::dstride);  // [hc][K]
  const int rq = 4 * (lane >> 4);
  const int cl = lane & 15;
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
#pragma unroll
    for (int a = 0; a < NT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          dt[(16 * a + rq + rr) * G::dstride + 16 * b + cl] = acc[c][a][b][rr];
    wave_lds_sync();
    const int hl = wave * CPW + c;  // channel within the group
    if (lane < K) {
      const int j = lane;
      const int m = j - (K >> 1);
      const int t0 = max(0, -m);
      const int t1 = min(L, L - m);
      float v4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < G::dim; ++t) {
        // D_c[t][t + m] = dt[m + t * (dstride + 1)]; masked terms read a
        // clamped in-tile address (a tap may have no valid t at all).
        int idx = m + t * (G::dstride + 1);
        idx = idx < 0 ? 0 : (idx < G::dim * G::dstride ? idx : G::dim * G::dstride - 1);
        const float d = dt[idx];
        v4[t & 3] += (t >= t0 && t < t1) ? d : 0.0f;
      }
      const float v = (v4[0] + v4[1]) + (v4[2] + v4[3]);
      if (det) {
        dst[((size_t)(g * hc + hl) * K + j) * (size_t)nranges + r] = v;
      } else {
        taps[hl * K + j] = v;
      }
    }
    wave_lds_sync();
  }
  if (!det) {
    __syncthreads();
    if constexpr (CL) {
      for (int e = threadIdx.x; e < hc * K; e += nthreads) {
        const int j = e / hc, c = e - j * hc;
        atomicAdd(dst + (size_t)j * H + (size_t)g * hc + c, taps[c * K + j]);
      }
    } else {
      float* out = dst + (size_t)g * hc * K;
      for (int e = threadIdx.x; e < hc * K; e += nthreads) atomicAdd(out + e, taps[e]);
    }
  }
}

// Staging units of the channel-group DK: EPC floats per lane and load (4:
// dwordx4 chunks, for 16-byte aligned tensors whose segments and samples are
// whole chunks; 1: dwords, for any row length and 4-byte aligned tensors).
template <int EPC> struct CgUnit;
template <> struct CgUnit<4> { using T = u32x4; };
template <> struct CgUnit<1> { using T = uint32_t; };

template <int EPC, int CPOL>
__device__ __forceinline__ typename CgUnit<EPC>::T buf_load_unit(__amdgpu_buffer_rsrc_t r,
                                                                 uint32_t voff) {
  if constexpr (EPC == 4)
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, CPOL);
  else
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, CPOL);
}

template <int EPC>
__device__ __forceinline__ void unit_to_lds(float* dst, const typename CgUnit<EPC>::T v) {
  if constexpr (EPC == 4)
    chunk_to_lds(dst, v);
  else
    *dst = __uint_as_float(v);
}

template <int LMAX, int LOAD_CPOL = kCpolNone, int CPW = dk_cg_cpw(LMAX), int EPC = 4>
__global__ __launch_bounds__(512) void dwconv_dk_cg_kernel(
    const float* __restrict__ gy, const float* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int nranges,
    uint32_t nblocks, int det) {
  using G = CgGeo<LMAX>;
  constexpr int NT = G::nt;
  constexpr int DEPTH = kCgDepth;
  extern __shared__ float lds[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wpb = blockDim.x / kWave;
  const int nthreads = blockDim.x;
  const int hc = CPW * wpb;
  const int ngroups = H / hc;
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int g = (int)(blk % (uint32_t)ngroups);
  const int r = (int)(blk / (uint32_t)ngroups);
  const int tsteps = (B + kCgStep - 1) / kCgStep;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;

  using U = typename CgUnit<EPC>::T;
  const int seg = hc * L;                     // elements per sample segment
  const int segc = seg / EPC;                 // chunks per segment
  const int sk = seg + kCgPad;                // LDS stride between samples
  const int sz = kCgStep * sk;                // one tensor's stage
  const int per = kCgStep * segc;             // chunks per stage and tensor
  constexpr int kNpt = (CPW * LMAX * 4 / EPC + kWave - 1) / kWave;  // per thread, tensor
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 4u;  // one sample
  const uint32_t grp_bytes = (uint32_t)g * (uint32_t)seg * 4u;

  // Loop-invariant part of each staged element: its sample within the
  // step, its byte offset from the step's first sample, its LDS offset.
  int ek[kNpt];
  uint32_t eoff[kNpt], elds[kNpt];
#pragma unroll
  for (int i = 0; i < kNpt; ++i) {
    const int e = i * nthreads + (int)threadIdx.x;
    const int k = e < per ? e / segc : kCgStep;  // kCgStep: no element
    const int q = e - (e / segc) * segc;
    ek[i] = k;
    eoff[i] = (uint32_t)k * row_bytes + grp_bytes + 4u * EPC * (uint32_t)q;
    elds[i] = (uint32_t)(k * sk + EPC * q);
  }

  // Global -> registers for local step s (global step r + s * nranges):
  // buffer resources rebased on the step's first sample; elements past the
  // stage or past B read 0 (no branch).
  U stg[DEPTH][2][kNpt];
  auto load_step = [&](int s, U (&st)[2][kNpt]) {
    const int bs = (r + s * nranges) * kCgStep;
    const size_t r0 = (size_t)bs * (size_t)H * (size_t)L;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(gy + r0);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0);
    const int klim = min(kCgStep, B - bs);
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      const uint32_t o = ek[i] < klim ? eoff[i] : kOob;
      st[0][i] = buf_load_unit<EPC, LOAD_CPOL>(rg, o);
      st[1][i] = buf_load_unit<EPC, LOAD_CPOL>(rx, o);
    }
  };
  auto store_stage = [&](int buf, const U (&st)[2][kNpt]) {
    float* base = lds + buf * 2 * sz;
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      if (ek[i] < kCgStep) {
        unit_to_lds<EPC>(base + elds[i], st[0][i]);
        unit_to_lds<EPC>(base + sz + elds[i], st[1][i]);
      }
    }
  };

  f32x4 acc[CPW][NT][NT];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int a = 0; a < NT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) acc[c][a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kq = lane >> 4;   // sample of the step
  const int col = lane & 15;  // column within a 16-wide tile
  auto mfma_step = [&](int s) {
    const float* gdy = lds + (s & 1) * 2 * sz + kq * sk;
    const float* gxx = gdy + sz;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const int cb = (wave * CPW + c) * L;
      float av[NT], bv[NT];
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        // Columns >= L (rows shorter than the bucket) read a clamped
        // address and are zeroed, without a branch.
        const int cc = 16 * tt + col;
        const int ca = cc < L ? cc : L - 1;
        const float va = gdy[cb + ca], vb = gxx[cb + ca];
        av[tt] = cc < L ? va : 0.f;
        bv[tt] = cc < L ? vb : 0.f;
      }
#pragma unroll
      for (int a = 0; a < NT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b)
          acc[c][a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[b],
                                                              acc[c][a][b], 0, 0, 0);
    }
  };

  if (nsteps > 0) {
    // Local step s lives in stg[s % DEPTH] until it is stored to LDS stage
    // s % 2; the loop is unrolled by DEPTH so register indices are static.
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if (d < nsteps) load_step(d, stg[d]);
    store_stage(0, stg[0]);
    if (DEPTH < nsteps) load_step(DEPTH, stg[0]);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += DEPTH) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          mfma_step(s);
          if (s + 1 < nsteps) {
            store_stage((s + 1) & 1, stg[(d + 1) % DEPTH]);
            if (s + 1 + DEPTH < nsteps) load_step(s + 1 + DEPTH, stg[(d + 1) % DEPTH]);
          }
          __syncthreads();
        }
      }
    }
  }

  dk_cg_epilogue<LMAX, false, CPW>(acc, lds, dst, wave, wpb, g, r, hc, L, K, nranges, det);
}

// ---------------------------------------------------------------------------
// Channel-group DK for BF16 tensors on the BF16 matrix cores.
//
// The channel-group DK above with three changes that keep its per-step
// pipeline off the critical path when the tensors are half as large:
//  * a step is 16 samples, the K of v_mfma_f32_16x16x16bf16_1k (4x fewer
//    barriers and LDS round trips per sample than 4-sample FP32 steps);
//  * the LDS stages keep the raw BF16 values (16-byte chunk copies, no
//    widening);
//  * each D_c tile is 16x16 BF16 products summed over 16 samples per
//    instruction. A product of two BF16 values is exact in FP32, so the
//    accumulation is the only rounding, as with widened operands.
// LDS is one region per wave, [stage][tensor][sample][kBmRow(LMAX)]: the
// wave's two channels (2 L values, a multiple of 8, so no 16-byte chunk
// straddles two waves) of each of the 16 samples. Every offset inside a
// region is a compile-time constant, so the operand gathers use one lane
// address per (channel, column tile) and immediate offsets.
// The MFMA's K index k = 4 * (lane / 16) + v (v = 0..3; lane l holds
// A[l % 16][k] and B[k][l % 16]) is mapped to sample kq + 4 v of the step
// (kq = lane / 16): any bijection gives the same sum over the step, and this
// one puts the four 16-lane groups of a wave one row apart; a row length of
// 16 (mod 32) values puts them in disjoint LDS banks.
// ---------------------------------------------------------------------------
constexpr int kBmStep = 16;  // samples per stage (the BF16 MFMA K)

// Values per sample row of a wave's region: at least the wave's two
// channels of the bucket, 16 (mod 32).
__host__ __device__ constexpr int kBmRow(int lmax) {
  return kCgChannelsPerWave * lmax + ((16 - (kCgChannelsPerWave * lmax) % 32) % 32 + 32) % 32;
}

// Dynamic LDS of the BF16 DK kernel: the wave regions (two stages of both
// tensors), or, for the epilogue, one D tile per wave plus the tap sums.
__host__ __device__ constexpr size_t dk_bf16mma_lds_bytes(int lmax, int wpb) {
  const size_t stages = (size_t)wpb * 2 * 2 * kBmStep * (size_t)kBmRow(lmax) * sizeof(uint16_t);
  const size_t dtile = ((size_t)wpb * (16 * (lmax / 16)) * (16 * (lmax / 16) + 1) +
                        (size_t)kCgChannelsPerWave * wpb * kMaxK) *
                       sizeof(float);
  return stages > dtile ? stages : dtile;
}

template <int LMAX, int LOAD_CPOL = kCpolNone>
__global__ __launch_bounds__(512) void dwconv_dk_bf16mma_kernel(
    const uint16_t* __restrict__ gy, const uint16_t* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int nranges,
    uint32_t nblocks, int det) {
  using G = CgGeo<LMAX>;
  constexpr int NT = G::nt;
  constexpr int CPW = kCgChannelsPerWave;
  constexpr int STEP = kBmStep;
  constexpr int EPC = 8;                     // BF16 values per 16-byte chunk
  constexpr int ROW = kBmRow(LMAX);
  constexpr int TSZ = STEP * ROW;            // one tensor's stage in a region
  constexpr int REGION = 2 * 2 * TSZ;        // one wave's region
  extern __shared__ float lds[];
  uint16_t* const l16 = reinterpret_cast<uint16_t*>(lds);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wpb = blockDim.x / kWave;
  const int nthreads = blockDim.x;
  const int hc = CPW * wpb;
  const int ngroups = H / hc;
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int g = (int)(blk % (uint32_t)ngroups);
  const int r = (int)(blk / (uint32_t)ngroups);
  const int tsteps = (B + STEP - 1) / STEP;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;

  const int seg = hc * L;                 // values per sample segment
  const int segc = seg / EPC;             // chunks per segment
  const int wseg = CPW * L;               // values of one wave per sample
  const int per = STEP * segc;            // chunks per stage and tensor
  constexpr int kNpt = (CPW * LMAX * STEP / EPC + kWave - 1) / kWave;
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 2u;  // one sample
  const uint32_t grp_bytes = (uint32_t)g * (uint32_t)seg * 2u;

  // Loop-invariant part of each staged chunk: its sample within the step,
  // its byte offset from the step's first sample, its place in LDS (the
  // region of the wave whose channels it holds).
  int ek[kNpt];
  uint32_t eoff[kNpt], elds[kNpt];
#pragma unroll
  for (int i = 0; i < kNpt; ++i) {
    const int e = i * nthreads + (int)threadIdx.x;
    const int k = e < per ? e / segc : STEP;  // STEP: no chunk
    const int q = e - (e / segc) * segc;
    const int w = (EPC * q) / wseg;
    ek[i] = k;
    eoff[i] = (uint32_t)k * row_bytes + grp_bytes + 16u * (uint32_t)q;
    elds[i] = (uint32_t)(w * REGION + k * ROW + (EPC * q - w * wseg));
  }

  // One step in flight in registers: a 16-sample step is 4x the bytes of
  // an FP32 channel-group step, and a second one measured no faster.
  u32x4 stg[2][kNpt];
  auto load_step = [&](int s, u32x4 (&st)[2][kNpt]) {
    const int bs = (r + s * nranges) * STEP;
    const size_t r0 = (size_t)bs * (size_t)H * (size_t)L;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc_t(gy + r0);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc_t(x + r0);
    const int klim = min(STEP, B - bs);
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      const uint32_t o = ek[i] < klim ? eoff[i] : kOob;
      st[0][i] = buf_load_chunk<LOAD_CPOL>(rg, o);
      st[1][i] = buf_load_chunk<LOAD_CPOL>(rx, o);
    }
  };
  auto store_stage = [&](int buf, const u32x4 (&st)[2][kNpt]) {
    uint16_t* base = l16 + buf * 2 * TSZ;
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      if (ek[i] < STEP) {
        *reinterpret_cast<u32x4*>(base + elds[i]) = st[0][i];
        *reinterpret_cast<u32x4*>(base + TSZ + elds[i]) = st[1][i];
      }
    }
  };

  f32x4 acc[CPW][NT][NT];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int a = 0; a < NT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) acc[c][a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Lane addresses of the operand gathers: sample kq of the step, column
  // 16 tt + (lane % 16) of channel c clamped to L - 1. Rows and columns at
  // or past L of D_c are never read by the epilogue, so the clamped values
  // need no masking.
  const int kq = lane >> 4;
  const int col = lane & 15;
  const uint16_t* lrow = l16 + wave * REGION + kq * ROW;
  int aoff[CPW][NT];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int cc = 16 * tt + col;
      aoff[c][tt] = c * L + (cc < L ? cc : L - 1);
    }
  auto mfma_step = [&](int buf) {
    const uint16_t* gdy = lrow + buf * 2 * TSZ;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      s16x4 av[NT], bv[NT];
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        const uint16_t* p = gdy + aoff[c][tt];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          av[tt][v] = (short)p[4 * v * ROW];
          bv[tt][v] = (short)p[TSZ + 4 * v * ROW];
        }
      }
#pragma unroll
      for (int a = 0; a < NT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b)
          acc[c][a][b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av[a], bv[b],
                                                                   acc[c][a][b], 0, 0, 0);
    }
  };

  if (nsteps > 0) {
    // Local step s is loaded into stg, stored to LDS stage s % 2 while step
    // s - 1 is consumed from the other stage, and consumed after the next
    // barrier; the loop is unrolled by 2 so the stage index is static.
    load_step(0, stg);
    store_stage(0, stg);
    if (1 < nsteps) load_step(1, stg);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          mfma_step(d);
          if (s + 1 < nsteps) {
            store_stage(d ^ 1, stg);
            if (s + 2 < nsteps) load_step(s + 2, stg);
          }
          __syncthreads();
        }
      }
    }
  }

  dk_cg_epilogue<LMAX>(acc, lds, dst, wave, wpb, g, r, hc, L, K, nranges, det);
}

// ---------------------------------------------------------------------------
// Channels-last DK: x and dy as [B][L][H] (the [B, 1, L, H] layout of the
// Flash-DWC dW kernel), dw as [K][H], dw += the taps' sums (the caller
// zeroes dw first).
//
// The channel-group contraction above with the staging transposed: a
// workgroup owns kClChannels = 32 consecutive channels (CPW per wave), so
// each (sample, t) row it loads is one whole 128-byte line of 32 channels. Rows land in LDS as [sample][t][kClChannels + 1]: a lane that
// gathers column t of channel c reads address t * 33 + c, so the 16 columns
// of a tile hit 16 distinct banks, and the sample stride is padded to
// 16 (mod 32) floats so the four 16-lane groups of a wave (four samples)
// use disjoint banks. Steps are 4 samples (the FP32 MFMA K); the epilogue
// is the shared one with the [K][H] output.
// ---------------------------------------------------------------------------
constexpr int kClChannels = 32;
constexpr int kClWaves = kClChannels / kCgChannelsPerWave;  // 16
// At 48 columns a wave takes four channels (8 waves, 226-250 VGPRs at two
// waves per SIMD), which leaves registers for two steps of loads: measured
// on MI355X 141.5 against 148.8 us at B16384 H128 K48 and 605 against 624
// us at B32768 H256 K4; at 16 and 32 columns it was 10-15% slower, so two
// channels per wave stay there.
constexpr int kClWideChannels = 4;

// Waves of the channels-last DK workgroup of row bucket lmax.
__host__ __device__ constexpr int dk_cl_waves(int lmax) {
  return lmax > 32 ? kClChannels / kClWideChannels : kClWaves;
}

// Floats between the samples of a channels-last stage: L rows of
// kClChannels + 1, rounded up to 16 (mod 32).
__host__ __device__ constexpr int cl_sample_stride(int L) {
  return L * (kClChannels + 1) + ((16 - (L * (kClChannels + 1)) % 32) % 32 + 32) % 32;
}

__host__ __device__ constexpr size_t dk_cl_lds_bytes(int lmax, int L, int waves = kClWaves) {
  const size_t stages = (size_t)2 * 2 * kCgStep * (size_t)cl_sample_stride(L) * sizeof(float);
  const size_t dtile = ((size_t)waves * (16 * (lmax / 16)) * (16 * (lmax / 16) + 1) +
                        (size_t)kClChannels * kMaxK) *
                       sizeof(float);
  return stages > dtile ? stages : dtile;
}

template <int LMAX, int CPW = kCgChannelsPerWave, int DEPTH = 1>
__global__ __launch_bounds__(kClChannels / CPW * kWave) void dwconv_dk_cl_kernel(
    const float* __restrict__ x, const float* __restrict__ gy,
    float* __restrict__ dw, int B, int H, int L, int K, int nranges,
    uint32_t nblocks) {
  using G = CgGeo<LMAX>;
  constexpr int NT = G::nt;
  constexpr int NW = kClChannels / CPW;
  constexpr int HC = kClChannels;
  constexpr int RW = HC + 1;           // LDS floats per (sample, t) row
  constexpr int CPR = HC / 4;          // 16-byte chunks per row
  constexpr int NTH = NW * kWave;
  constexpr int kNpt = (kCgStep * LMAX * CPR + NTH - 1) / NTH;
  extern __shared__ float lds[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int ngroups = H / HC;
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int g = (int)(blk % (uint32_t)ngroups);
  const int r = (int)(blk / (uint32_t)ngroups);
  const int tsteps = (B + kCgStep - 1) / kCgStep;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;

  const int sks = cl_sample_stride(L);   // LDS floats between samples
  const int sz = kCgStep * sks;          // one tensor's stage
  const int rows = L * CPR;              // chunks per sample
  const int per = kCgStep * rows;        // chunks per stage and tensor
  const uint32_t smp_bytes = (uint32_t)L * (uint32_t)H * 4u;

  // Loop-invariant part of each staged chunk: its sample within the step,
  // its byte offset from the step's first sample, its LDS offset.
  int ek[kNpt];
  uint32_t eoff[kNpt], elds[kNpt];
#pragma unroll
  for (int i = 0; i < kNpt; ++i) {
    const int e = i * NTH + (int)threadIdx.x;
    const int k = e < per ? e / rows : kCgStep;  // kCgStep: no chunk
    const int rem = e - (e / rows) * rows;
    const int t = rem / CPR, q = rem - (rem / CPR) * CPR;
    ek[i] = k;
    eoff[i] = (uint32_t)k * smp_bytes + ((uint32_t)t * (uint32_t)H + (uint32_t)(g * HC + 4 * q)) * 4u;
    elds[i] = (uint32_t)(k * sks + t * RW + 4 * q);
  }

  u32x4 stg[DEPTH][2][kNpt];
  auto load_step = [&](int s, u32x4 (&st)[2][kNpt]) {
    const int bs = (r + s * nranges) * kCgStep;
    const size_t r0 = (size_t)bs * (size_t)L * (size_t)H;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(gy + r0);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0);
    const int klim = min(kCgStep, B - bs);
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      const uint32_t o = ek[i] < klim ? eoff[i] : kOob;
      st[0][i] = buf_load_chunk<kCpolNT>(rg, o);
      st[1][i] = buf_load_chunk<kCpolNT>(rx, o);
    }
  };
  auto store_stage = [&](int buf, const u32x4 (&st)[2][kNpt]) {
    float* base = lds + buf * 2 * sz;
#pragma unroll
    for (int i = 0; i < kNpt; ++i) {
      if (ek[i] < kCgStep) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          base[elds[i] + v] = __uint_as_float(st[0][i][v]);
          base[sz + elds[i] + v] = __uint_as_float(st[1][i][v]);
        }
      }
    }
  };

  f32x4 acc[CPW][NT][NT];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int a = 0; a < NT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) acc[c][a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Lane offsets: sample kq of the step, column 16 tt + (lane % 16) clamped
  // to L - 1 (rows and columns of D_c at or past L are never read by the
  // epilogue), channel wave * CPW + c.
  const int kq = lane >> 4;
  const int col = lane & 15;
  int aoff[CPW][NT];
#pragma unroll
  for (int c = 0; c < CPW; ++c)
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int cc = 16 * tt + col;
      aoff[c][tt] = kq * sks + (cc < L ? cc : L - 1) * RW + wave * CPW + c;
    }
  auto mfma_step = [&](int buf) {
    const float* gdy = lds + buf * 2 * sz;
    const float* gxx = gdy + sz;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      float av[NT], bv[NT];
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        av[tt] = gdy[aoff[c][tt]];
        bv[tt] = gxx[aoff[c][tt]];
      }
#pragma unroll
      for (int a = 0; a < NT; ++a)
#pragma unroll
        for (int b = 0; b < NT; ++b)
          acc[c][a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[b], acc[c][a][b], 0, 0, 0);
    }
  };

  if (nsteps > 0 && DEPTH == 1) {
    // Local step s is loaded into stg, stored to LDS stage s % 2 while step
    // s - 1 is consumed from the other stage, and consumed after the next
    // barrier; the loop is unrolled by 2 so the stage index is static.
    load_step(0, stg[0]);
    store_stage(0, stg[0]);
    if (1 < nsteps) load_step(1, stg[0]);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          // Stage d ^ 1 was last read by mfma_step of step s - 1, finished
          // by every thread before the previous barrier: store step s + 1
          // and issue the loads of s + 2 before this step's matrix work
          // (1-2% faster than after it at every shape measured).
          if (s + 1 < nsteps) {
            store_stage(d ^ 1, stg[0]);
            if (s + 2 < nsteps) load_step(s + 2, stg[0]);
          }
          mfma_step(d);
          __syncthreads();
        }
      }
    }
  } else if (nsteps > 0) {
    // Two steps of loads in registers. Every step issues the same loads
    // (past the last step all out of bounds: no memory traffic), so the wait
    // before a stage store is for that step's loads only.
    load_step(0, stg[0]);
    load_step(1, stg[DEPTH - 1]);
    store_stage(0, stg[0]);
    load_step(2, stg[0]);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int s = s0 + d;
        store_stage(d ^ 1, stg[(d + 1) % DEPTH]);
        load_step(s + 3, stg[(d + 1) % DEPTH]);
        if (s < nsteps) mfma_step(d);
        __syncthreads();
      }
    }
  }

  dk_cg_epilogue<LMAX, true, CPW>(acc, lds, dw, wave, NW, g, r, HC, L, K, nranges, 0, H);
}

// ---------------------------------------------------------------------------
// Long rows (L up to kLongMaxL = 192, K up to kLongMaxK = 256): FWD / DX on
// the matrix cores.
//
// At L = K = 192 a path does B H L K / 2-ish useful multiply-adds (58 G at
// B16384 H128) against 3.2 GB of traffic, so it is bound by the FP32 matrix
// cores, not HBM. A wave owns one channel and 16 samples:
// v_mfma_f32_16x16x4_f32 with M = the 16 samples, N = 16 output columns and
// K = the 4 consecutive input columns 4u .. 4u + 3 (lane l holds A[l % 16]
// [l / 16] = x[sample l % 16][4u + l / 16] and B[l / 16][l % 16] = the tap
// that joins input column 4u + l / 16 to output column 16 tt + l % 16).
// Consecutive input columns per step make the band exact: step u and tile
// tt meet only if some (s, t) in them has a tap, a test that is the same for
// the whole wave, so out-of-band steps are skipped, not multiplied by zero.
// The taps sit in LDS as one zero-padded window per channel; a lane's tap
// for (u, tt) is window[lane base +/- (4u - 16tt)], an immediate offset.
// Every output tile accumulates at once (NT accumulators), so consecutive
// MFMAs never wait on each other. Rows go global -> LDS (the wave's own
// 16-row region, no block barrier), A is read per step from there, and the
// results return through the same region to coalesced stores.
// ---------------------------------------------------------------------------
// floor(a / b) for b > 0 and any sign of a.
__host__ __device__ constexpr int floor_div(int a, int b) {
  return a >= 0 ? a / b : -((-a + b - 1) / b);
}

constexpr int kLongMaxL = 192;         // largest L of the long path
constexpr int kLongMaxK = 256;         // largest K (taps past the row add 0)
constexpr int kLongRowsWaves = 4;      // waves (16-sample groups) per workgroup
constexpr int kLongTapPad = 20;        // zero taps on each side of the window

// Floats per LDS row of a wave's region: 4 (mod 64), so the 16 rows a wave
// reads at once (one per sample) start in different banks.
__host__ __device__ constexpr int long_row_stride(int lmax) { return lmax + 4; }

__host__ __device__ constexpr size_t rows_long_lds_bytes(int lmax) {
  return ((size_t)kLongRowsWaves * 16 * long_row_stride(lmax) +
          (size_t)(kLongMaxK + 2 * kLongTapPad)) *
         sizeof(float);
}

// A wave's 16 rows b0 .. b0 + 15 of channel h -> LDS rows xr[i * RS], columns
// >= L and rows >= B as zeros; VEC moves 16-byte chunks (L % 4 == 0 and
// 16-byte aligned tensors), otherwise dwords, both non-temporal.
template <int LMAX, bool VEC>
__device__ __forceinline__ void long_rows_to_lds(float* xr, const float* in, int b0,
                                                 int h, int B, int H, int L, int lane) {
  constexpr int RS = long_row_stride(LMAX);
  constexpr int NC = (LMAX + kWave - 1) / kWave;      // row chunks of 64 floats
  constexpr int kLongChunks = 16 * LMAX / 4 / kWave;  // 16-byte chunks per lane
  static_assert(LMAX % 16 == 0, "whole 16-byte chunks per lane");
  const int nrow = min(16, B - b0);
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(in + ((size_t)(b0 < B ? b0 : 0) * (size_t)H + (size_t)h) * (size_t)L);
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 4u;
  if constexpr (VEC) {
    u32x4 v[kLongChunks];
#pragma unroll
    for (int c = 0; c < kLongChunks; ++c) {
      const int e = c * kWave + lane;
      const int i = e / (LMAX / 4), q = e - i * (LMAX / 4);
      const uint32_t off = (i < nrow && 4 * q < L) ? (uint32_t)i * row_bytes + 16u * (uint32_t)q : kOob;
      v[c] = buf_load_chunk<kCpolNT>(rs, off);
    }
#pragma unroll
    for (int c = 0; c < kLongChunks; ++c) {
      const int e = c * kWave + lane;
      const int i = e / (LMAX / 4), q = e - i * (LMAX / 4);
      chunk_to_lds(xr + i * RS + 4 * q, v[c]);
    }
  } else {
    float v[16][NC];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = c * kWave + lane;
        const uint32_t off = (i < nrow && col < L) ? (uint32_t)i * row_bytes + 4u * (uint32_t)col : kOob;
        v[i][c] = buf_load1<kCpolNT>(rs, off, 0);
      }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (c * kWave + lane < LMAX) xr[i * RS + c * kWave + lane] = v[i][c];
  }
}

// The wave's 16 result rows in xr -> out (rows < B, columns < L), as the
// loads above. The caller orders its LDS writes before (wave_lds_sync).
template <int LMAX, bool VEC>
__device__ __forceinline__ void long_rows_from_lds(const float* xr, float* out, int b0,
                                                   int h, int B, int H, int L, int lane) {
  constexpr int RS = long_row_stride(LMAX);
  constexpr int NC = (LMAX + kWave - 1) / kWave;
  constexpr int kLongChunks = 16 * LMAX / 4 / kWave;
  const int nrow = min(16, B - b0);
  const __amdgpu_buffer_rsrc_t ro =
      make_rsrc(out + ((size_t)(b0 < B ? b0 : 0) * (size_t)H + (size_t)h) * (size_t)L);
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 4u;
  if constexpr (VEC) {
#pragma unroll
    for (int c = 0; c < kLongChunks; ++c) {
      const int e = c * kWave + lane;
      const int i = e / (LMAX / 4), q = e - i * (LMAX / 4);
      const uint32_t off = (i < nrow && 4 * q < L) ? (uint32_t)i * row_bytes + 16u * (uint32_t)q : kOob;
      buf_store_chunk<kCpolNT>(lds_to_chunk(xr + i * RS + 4 * q), ro, off);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int col = c * kWave + lane;
        const uint32_t off = (i < nrow && col < L) ? (uint32_t)i * row_bytes + 4u * (uint32_t)col : kOob;
        buf_store1<kCpolNT>(col < LMAX ? xr[i * RS + col] : 0.0f, ro, off);
      }
  }
}

// KB: tap-count bucket (K <= KB, a multiple of 64). VEC: rows move as
// 16-byte chunks (L % 4 == 0, 16-byte aligned tensors), else as dwords; both
// non-temporal (the rows are touched once). 16-byte moves measured 6-11%
// faster than dwords at L = 64 and 192 on MI355X.
template <int LMAX, int KB, bool DX, bool VEC>
__global__ __launch_bounds__(kLongRowsWaves * kWave) void dwconv_rows_long_kernel(
    const float* __restrict__ in, const float* __restrict__ w,
    float* __restrict__ out, int B, int H, int L, int K) {
  constexpr int NT = LMAX / 16;   // output tiles
  constexpr int NU = LMAX / 4;    // 4-column MFMA steps
  constexpr int RS = long_row_stride(LMAX);
  extern __shared__ float lds[];
  float* const wl = lds + kLongRowsWaves * 16 * RS;  // tap window

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int h = (int)(blockIdx.x % (uint32_t)H);
  const int b0 = (int)(blockIdx.x / (uint32_t)H) * (kLongRowsWaves * 16) + wave * 16;
  const int p = K >> 1;

  // Tap window: wl[kLongTapPad + j] = w[h][j], zero elsewhere.
  for (int i = threadIdx.x; i < K + 2 * kLongTapPad; i += kLongRowsWaves * kWave) {
    const int j = i - kLongTapPad;
    wl[i] = (j >= 0 && j < K) ? w[(size_t)h * K + j] : 0.0f;
  }

  // This wave's 16 rows: columns >= L (and rows past B) are zero.
  float* const xr = lds + wave * 16 * RS;
  long_rows_to_lds<LMAX, VEC>(xr, in, b0, h, B, H, L, lane);
  __syncthreads();  // taps and rows in place

  const int jj = lane & 15, kk = lane >> 4;
  // Lane's tap for step u and tile tt: FWD j = (4u + kk) - (16 tt + jj) + p,
  // DX j = (16 tt + jj) - (4u + kk) + p. Both depend on u and tt only through
  // the diagonal d = u - 4 tt, as does the band test, so the loop runs over
  // diagonals: one tap per diagonal, then one MFMA per output tile with step
  // u = d + 4 tt, a compile-time index into the lane's A values. The loop
  // covers every diagonal a tap count up to KB can reach (compile-time
  // bounds, no branch around any MFMA); a diagonal outside this call's band
  // multiplies by a zero tap. d is in the band when some (u, tt) on it
  // shares a tap:
  //   FWD 4d + 3 >= -p and 4d - 15 <= K - 1 - p,
  //   DX  15 - 4d >= -p and -4d - 3 <= K - 1 - p.
  // Taps read there stay in [-18, K + 17], inside the zero-padded window
  // (out-of-band diagonals read the band's nearest one, then select 0).
  // Columns at or past L are zeros in the rows, so steps past the row add 0.
  constexpr int PB = KB / 2;  // largest p of the bucket
  constexpr int DLO = DX ? floor_div(-PB + 1, 4) : floor_div(-PB, 4);
  constexpr int DHI = DX ? floor_div(PB + 15, 4) : floor_div(PB + 14, 4);
  constexpr int D0 = DLO > -(NU - 4) ? DLO : -(NU - 4);
  constexpr int D1 = DHI < NU - 1 ? DHI : NU - 1;
  const float* const wb = wl + kLongTapPad + (DX ? (jj - kk + p) : (kk - jj + p));
  const float* const ar = xr + jj * RS + kk;  // A: row jj, column 4u + kk
  const int dlo = DX ? floor_div(p - K - 2 + 3, 4) : floor_div(-p - 3 + 3, 4);
  const int dhi = DX ? floor_div(p + 15, 4) : floor_div(K + 14 - p, 4);
  float av[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) av[u] = ar[4 * u];
  f32x4 acc[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = D0; d <= D1; ++d) {
    const int dc = d < dlo ? dlo : (d > dhi ? dhi : d);  // uniform
    const float tap = wb[DX ? -4 * dc : 4 * dc];
    const float bv = d == dc ? tap : 0.0f;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int u = d + 4 * tt;
      if (u >= 0 && u < NU)  // compile-time
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], bv, acc[tt], 0, 0, 0);
    }
  }

  // Results back through this wave's region (its A reads are complete: LDS
  // operations of one wave run in order), then coalesced stores.
  const int rq = 4 * kk;
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) xr[(rq + r) * RS + 16 * tt + jj] = acc[tt][r];
  wave_lds_sync();
  long_rows_from_lds<LMAX, VEC>(xr, out, b0, h, B, H, L, lane);
}

// ---------------------------------------------------------------------------
// Long rows, FWD / DX on the BF16 matrix cores at FP32 accuracy.
//
// Every FP32 operand v (row element or tap) is split into three BF16 parts,
// hi = bf16(v), mid = bf16(v - hi), lo = bf16(v - hi - mid), each rounded to
// nearest even (8 significant bits, so each step leaves at most 2^-8 of the
// rest); both differences are exact in FP32, |mid| <= 2^-8 |v|,
// |lo| <= 2^-16 |v| and |v - hi - mid - lo| <= 2^-24 |v|. The six part
// products hi hi, hi mid, mid hi, mid mid, hi lo and lo hi leave out mid lo
// and lo mid (at most 2^-24 |x w| each) and lo lo (2^-32), so a product is
// off by at most about 2^-22 |x w|, the order of FP32 rounding. Each part
// product is exact in FP32 and the matrix cores sum them in FP32.
// This is the bf16x6 scheme of Henry, Tang and Heinecke, "Leveraging the
// bfloat16 artificial intelligence datatype for higher-precision
// computations" (ARITH 2019). On MI355X v_mfma_f32_16x16x32_bf16 measured
// 9.3x the multiply-adds per cycle of v_mfma_f32_16x16x4_f32 (independent
// accumulators, every SIMD busy), so six of them cost 1.5x less than the
// FP32 instructions for the same products.
//
// Mapping (per wave and tile: one channel, 16 samples): the MFMA computes
// the transposed tile, M = 16 output columns 16 tt + m, N = the 16 samples,
// K = 32 input columns. Lane l (m = l % 16, g = l / 16) gives its eight K
// slots i the input columns s_i = 32 c + 4 g + i (i < 4) and
// 32 c + 16 + 4 g + (i - 4) (i >= 4), two 16-byte LDS reads. Lane l
// supplies the taps joining s_i to output column 16 tt + m as A and
// x[sample m][s_i] as B, and receives output columns 16 tt + 4 g .. + 3 of
// sample m. A lane's tap index for slot i < 4 is
//   FWD j = 16 d + (4 g - m + p) + i,   DX j = -16 d + (m - 4 g + p) - i,
// with d = 2 c - tt, and 16 more (FWD) or less (DX) for slot i + 4. The walk
// runs over diagonals d: per diagonal and part two 8-byte LDS reads, then
// six MFMAs for each tile on it (tt = 2 c - d, compile-time). The taps are
// split once per workgroup into a zero-padded window held as four copies
// shifted by 0 .. 3 values, so each run of four consecutive taps is one
// aligned 8-byte vector of one copy.
// The diagonal range covers every tap count up to KB; the zero padding makes
// out-of-band diagonals multiply by zero without a branch around any MFMA.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Three-way BF16 split of eight FP32 values (round to nearest even). Values
// go in pairs: one v_cvt_pk_bf16_f32 rounds two, and widening a BF16 back to
// FP32 is a shift or a mask, so a pair costs 11 VALU instructions.
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split3_bf16x8(const float (&v)[8], bf16x8& hi,
                                              bf16x8& mid, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const f32x2v x = {v[i], v[i + 1]};
    const bf16x2v h = __builtin_convertvector(x, bf16x2v);
    const f32x2v r1 = x - __builtin_convertvector(h, f32x2v);
    const bf16x2v m = __builtin_convertvector(r1, bf16x2v);
    const f32x2v r2 = r1 - __builtin_convertvector(m, f32x2v);
    const bf16x2v l = __builtin_convertvector(r2, bf16x2v);
    hi[i] = h[0];
    hi[i + 1] = h[1];
    mid[i] = m[0];
    mid[i + 1] = m[1];
    lo[i] = l[0];
    lo[i + 1] = l[1];
  }
}

// Diagonal range of the split kernel for row bucket LMAX and tap bucket KB
// (p <= KB / 2, K <= KB). A diagonal is in a call's band when some lane
// and slot on it has 0 <= j < K:
//   FWD j in 16 d + p + [-15, 31],  DX j in -16 d + p + [-31, 15].
template <int LMAX, int KB, bool DX>
struct LongSplitDiag {
  static constexpr int NT = LMAX / 16, NC = LMAX / 32, PB = KB / 2;
  static constexpr int lo_band = DX ? floor_div(-PB - 15, 16) : floor_div(-PB - 16, 16);
  static constexpr int hi_band = DX ? floor_div(PB + 15, 16) : floor_div(PB + 14, 16);
  static constexpr int D0 = lo_band > -(NT - 1) ? lo_band : -(NT - 1);
  static constexpr int D1 = hi_band < 2 * (NC - 1) ? hi_band : 2 * (NC - 1);
  // The tap window spans taps j in [-WLO, WHI] (zero outside [0, K)): every
  // tap a lane reads on the diagonals [D0, D1].
  static constexpr int WLO = DX ? 16 * D1 + 31 : 15 - 16 * D0;
  static constexpr int WHI = DX ? -16 * D0 + 15 + PB : 16 * D1 + 31 + PB;
  static constexpr int WN = WLO + WHI + 1;
  // Copy length: a lane reads positions e0 .. e0 + 3 and e0 + 16 .. + 19
  // <= WN - 1 of copy e0 % 4 from index e0 - e0 % 4, so a copy spans WN + 3
  // values (rounded to whole 16-byte vectors).
  static constexpr int WNP = (WN + 3 + 7) / 8 * 8;
};

constexpr int kLongS3Waves = 4;  // waves per workgroup of the split kernel
constexpr int kLongS3MinWaves = 2;  // resident waves per SIMD the registers allow

// LDS of the split kernel: the rows of its waves, then the split tap window
// (3 parts x 4 copies).
template <int LMAX, int KB, bool DX>
__host__ __device__ constexpr size_t rows_long_s3_lds_bytes() {
  return (size_t)kLongS3Waves * 16 * long_row_stride(LMAX) * sizeof(float) +
         (size_t)3 * 4 * LongSplitDiag<LMAX, KB, DX>::WNP * sizeof(__bf16);
}

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// Slots 0 .. 3 from w[0 .. 3] and slots 4 .. 7 from w[16 .. 19] (8-byte
// aligned LDS reads).
__device__ __forceinline__ bf16x8 tap_runs(const __bf16* w) {
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(w);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(w + 16);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// A workgroup owns one channel and kLongS3Waves tiles of 16 samples (one per
// wave). Each wave stages its rows in LDS (whole-row 16-byte moves), takes
// its B operands from there, and returns the results through the same
// region to coalesced stores.
template <int LMAX, int KB, bool DX, bool VEC>
__global__ __launch_bounds__(kLongS3Waves * kWave, kLongS3MinWaves) void dwconv_rows_long_s3_kernel(
    const float* __restrict__ in, const float* __restrict__ w,
    float* __restrict__ out, int B, int H, int L, int K) {
  using G = LongSplitDiag<LMAX, KB, DX>;
  constexpr int NT = G::NT, NC = G::NC;
  constexpr int WNP = G::WNP;
  constexpr int RS = long_row_stride(LMAX);
  extern __shared__ float lds[];
  // Split tap window after the rows: part q (hi, mid, lo) of copy r holds
  // window position e + r at index e. FWD position e is tap e - WLO, DX
  // position e is tap WHI - e (reversed, so a lane's DX taps also run
  // upwards).
  __bf16* const wsp = reinterpret_cast<__bf16*>(lds + kLongS3Waves * 16 * RS);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int h = (int)(blockIdx.x % (uint32_t)H);
  const int b0 = (int)(blockIdx.x / (uint32_t)H) * (kLongS3Waves * 16) + wave * 16;
  const int p = K >> 1;

  for (int e = threadIdx.x; e < WNP; e += kLongS3Waves * kWave) {
    const int j = DX ? G::WHI - e : e - G::WLO;
    const float v = (e < G::WN && j >= 0 && j < K) ? w[(size_t)h * K + j] : 0.0f;
    const __bf16 hi = (__bf16)v;
    const float r1 = v - (float)hi;
    const __bf16 mid = (__bf16)r1;
    const __bf16 lo = (__bf16)(r1 - (float)mid);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (e - c >= 0) {
        wsp[(0 * 4 + c) * WNP + e - c] = hi;
        wsp[(1 * 4 + c) * WNP + e - c] = mid;
        wsp[(2 * 4 + c) * WNP + e - c] = lo;
      }
    }
  }
  float* const xr = lds + wave * 16 * RS;
  long_rows_to_lds<LMAX, VEC>(xr, in, b0, h, B, H, L, lane);
  __syncthreads();  // window and rows in place

  const int m = lane & 15, g = lane >> 4;
  // B operands: x[sample m][s_i], split once.
  bf16x8 xh[NC], xm[NC], xl[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float* src = xr + m * RS + 32 * c + 4 * g;
    const float4 v0 = *reinterpret_cast<const float4*>(src);
    const float4 v1 = *reinterpret_cast<const float4*>(src + 16);
    const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    split3_bf16x8(v, xh[c], xm[c], xl[c]);
  }
  // Window position of the lane's slot 0 on diagonal d: e0 = eb + 16 d (slot
  // 4: e0 + 16), read from copy eb % 4 (16 d is a multiple of 4) at the
  // 8-byte aligned index e0 - eb % 4.
  const int eb = DX ? G::WHI - (m - 4 * g + p) : G::WLO + (4 * g - m + p);
  const int rc = eb & 3;
  const __bf16* const wh = wsp + (0 * 4 + rc) * WNP + (eb - rc);
  const __bf16* const wm = wsp + (1 * 4 + rc) * WNP + (eb - rc);
  const __bf16* const wlo = wsp + (2 * 4 + rc) * WNP + (eb - rc);

  f32x4 acc[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int d = G::D0; d <= G::D1; ++d) {
    const bf16x8 th = tap_runs(wh + 16 * d);
    const bf16x8 tm = tap_runs(wm + 16 * d);
    const bf16x8 tl = tap_runs(wlo + 16 * d);
    // Six products per tile, each a pass over the diagonal's tiles
    // (independent accumulators back to back).
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      const bf16x8 av = (q == 0 || q == 1 || q == 4) ? th : (q == 5 ? tl : tm);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        const int c2 = d + tt;  // 2 c, compile-time
        if (c2 >= 0 && c2 < 2 * NC && (c2 & 1) == 0) {
          const int c = c2 >> 1;
          const bf16x8 bv = (q == 0 || q == 2 || q == 5) ? xh[c] : (q == 4 ? xl[c] : xm[c]);
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[tt], 0, 0, 0);
        }
      }
    }
  }

  // Lane l holds output columns 16 tt + 4 g .. + 3 of sample m: one 16-byte
  // LDS write per tile into this wave's region (its B reads are complete:
  // LDS operations of one wave run in order), then coalesced stores.
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
    *reinterpret_cast<f32x4*>(xr + m * RS + 16 * tt + 4 * g) = acc[tt];
  wave_lds_sync();
  long_rows_from_lds<LMAX, VEC>(xr, out, b0, h, B, H, L, lane);
}

// ---------------------------------------------------------------------------
// Long rows: DK on the matrix cores. For channel h, D[t][s] = sum_b
// dy[b,h,t] x[b,h,s] over the batch, then dk[h][j] = sum_t D[t][t + j - p].
// A workgroup owns one channel and the interleaved 16-sample steps r,
// r + nranges, ... of the batch; its NT = LMAX / 16 waves own one tile row
// of D each (t in [16a, 16a + 16)) and accumulate the tiles of that row that
// meet the band (v_mfma_f32_16x16x4_f32, K = 4 samples: lane l holds
// A[l % 16][l / 16] = dy[sample l / 16][16a + l % 16] and B[l / 16][l % 16] =
// x[sample l / 16][16 bb + l % 16]). Both tensors' 16 rows of a step are
// staged in LDS, double buffered, loaded a step ahead into registers; the
// stage rows are 16 (mod 64) floats apart so the four samples a wave reads
// at once sit in disjoint banks.
// Epilogue, in a fixed order: the waves' D rows go through the stage area
// four at a time; wave a sums its 16 rows' diagonals into part[a][j], and
// the workgroup adds part[0 .. NT)[j] in order. det: one partial per
// (h, j, range) for dk_reduce_kernel; otherwise one atomic per tap and
// workgroup.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int long_dk_row_stride(int lmax) { return lmax + 16; }

__host__ __device__ constexpr size_t dk_long_lds_bytes(int lmax) {
  return ((size_t)2 * 2 * 16 * long_dk_row_stride(lmax) + (size_t)(lmax / 16) * kLongMaxK) *
         sizeof(float);
}

// VEC: each thread stages one 16-byte chunk per tensor and step (L % 4 == 0,
// 16-byte aligned tensors), else four dwords.
template <int LMAX, bool VEC>
__global__ __launch_bounds__((LMAX / 16) * kWave) void dwconv_dk_long_kernel(
    const float* __restrict__ gy, const float* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int nranges, int det) {
  constexpr int NT = LMAX / 16;
  constexpr int NTH = NT * kWave;
  constexpr int RS = long_dk_row_stride(LMAX);
  constexpr int SZ = 16 * RS;                 // one tensor's stage
  constexpr int kNpt = 16 * LMAX / NTH;       // dwords per thread and tensor
  constexpr int DS = LMAX + 1;                // epilogue D-row stride
  constexpr int kRound = (4 * SZ) / (16 * DS);  // waves per epilogue round
  static_assert(16 * LMAX % NTH == 0, "whole rows per thread slice");
  static_assert(kRound >= 1, "stage area holds one wave's D rows");
  extern __shared__ float lds[];
  float* const part = lds + 4 * SZ;           // [NT][kLongMaxK]

  const int lane = threadIdx.x & (kWave - 1);
  const int a = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // tile row
  const int h = (int)(blockIdx.x % (uint32_t)H);
  const int r = (int)(blockIdx.x / (uint32_t)H);
  const int tsteps = (B + 15) / 16;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;
  const int p = K >> 1;
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 4u;

  // Loop-invariant part of each staged dword (or 16-byte chunk): sample
  // row, first column.
  constexpr int NE = VEC ? 1 : kNpt;       // loads per thread and tensor
  constexpr int EW = VEC ? 4 : 1;          // floats per load
  int erow[NE], ecol[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = i * NTH + (int)threadIdx.x;
    erow[i] = e / (LMAX / EW);
    ecol[i] = EW * (e - erow[i] * (LMAX / EW));
  }
  u32x4 stv[2][NE];  // VEC
  float stg[2][NE];  // dwords
  auto load_step = [&](int s) {
    const int bs = (r + s * nranges) * 16;
    const size_t r0 = ((size_t)bs * (size_t)H + (size_t)h) * (size_t)L;
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(gy + r0);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0);
    const int klim = min(16, B - bs);
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const uint32_t o = (erow[i] < klim && ecol[i] < L)
                             ? (uint32_t)erow[i] * row_bytes + 4u * (uint32_t)ecol[i]
                             : kOob;
      if constexpr (VEC) {
        stv[0][i] = buf_load_chunk<kCpolNT>(rg, o);
        stv[1][i] = buf_load_chunk<kCpolNT>(rx, o);
      } else {
        stg[0][i] = buf_load1<kCpolNT>(rg, o, 0);
        stg[1][i] = buf_load1<kCpolNT>(rx, o, 0);
      }
    }
  };
  auto store_stage = [&](int buf) {
    float* base = lds + buf * 2 * SZ;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      if constexpr (VEC) {
        chunk_to_lds(base + erow[i] * RS + ecol[i], stv[0][i]);
        chunk_to_lds(base + SZ + erow[i] * RS + ecol[i], stv[1][i]);
      } else {
        base[erow[i] * RS + ecol[i]] = stg[0][i];
        base[SZ + erow[i] * RS + ecol[i]] = stg[1][i];
      }
    }
  };

  // Tiles of row a that meet the band: s - t in 16 (bb - a) + [-15, 15]
  // against [-p, K - 1 - p] (the same for the whole wave).
  auto in_band = [&](int bb) {
    const int lo = 16 * (bb - a) - 15;
    return lo + 30 >= -p && lo <= K - 1 - p && 16 * bb < L && 16 * a < L;
  };
  f32x4 acc[NT];
#pragma unroll
  for (int bb = 0; bb < NT; ++bb) acc[bb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int kq = lane >> 4, col = lane & 15;
  auto mfma_step = [&](int buf) {
    const float* dyst = lds + buf * 2 * SZ;
    const float* xst = dyst + SZ;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const int row = (4 * k4 + kq) * RS;
      const float av = dyst[row + 16 * a + col];
#pragma unroll
      for (int bb = 0; bb < NT; ++bb)
        if (in_band(bb))
          acc[bb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, xst[row + 16 * bb + col], acc[bb], 0, 0, 0);
    }
  };

  if (nsteps > 0) {
    load_step(0);
    store_stage(0);
    if (1 < nsteps) load_step(1);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          mfma_step(d);
          if (s + 1 < nsteps) {
            store_stage(d ^ 1);
            if (s + 2 < nsteps) load_step(s + 2);
          }
          __syncthreads();
        }
      }
    }
  }

  // Epilogue rounds: waves [q, q + kRound) put their D rows in the stage
  // area (slot a - q), then sum their diagonals in order of t.
  for (int q = 0; q < NT; q += kRound) {
    const bool mine = a >= q && a < q + kRound;
    float* const blk = lds + (mine ? a - q : 0) * 16 * DS;
    if (mine) {
#pragma unroll
      for (int bb = 0; bb < NT; ++bb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) blk[(4 * kq + rr) * DS + 16 * bb + col] = acc[bb][rr];
    }
    __syncthreads();
    if (mine) {
      for (int jb = 0; jb < K; jb += kWave) {
        const int j = jb + lane;
        float v = 0.0f;
        for (int tr = 0; tr < 16; ++tr) {
          const int t = 16 * a + tr;
          const int sc = t + j - p;
          if (j < K && t < L && sc >= 0 && sc < L) v += blk[tr * DS + sc];
        }
        if (j < K) part[a * kLongMaxK + j] = v;
      }
    }
    __syncthreads();
  }
  for (int j = threadIdx.x; j < K; j += NTH) {
    float v = 0.0f;
    for (int aa = 0; aa < NT; ++aa) v += part[aa * kLongMaxK + j];
    if (det)
      dst[((size_t)h * K + j) * (size_t)nranges + r] = v;
    else
      atomicAdd(dst + (size_t)h * K + j, v);
  }
}

// ---------------------------------------------------------------------------
// Long rows: DK on the BF16 matrix cores at FP32 accuracy (the three-way
// split and six part products of the split FWD / DX kernel). D[t][s] =
// sum_b dy[b,h,t] x[b,h,s] with v_mfma_f32_16x16x32_bf16, K = 32 samples:
// lane (m, g) holds A[m][8 g + i] = dy[sample 8 g + i][16 a + m] and
// B[8 g + i][n] = x[sample 8 g + i][16 bb + n] (n = m = l % 16), and
// receives D[16 a + 4 g + r][16 bb + n], the layout of the FP32 kernel, so
// the epilogue is the same.
// A workgroup owns one channel and the interleaved 32-sample steps r,
// r + nranges, ...; wave a owns D tile row a. Both tensors' 32 rows of a
// step sit in LDS as FP32 (double buffered, coalesced 16-byte loads two
// steps ahead). Per step, wave a gathers column tile a of both, keeps the
// dy parts (its A operands) in registers and publishes the x parts in lane
// order for every wave (one split per element, not one per wave that uses
// it); after a barrier it multiplies by the published parts of the tiles of
// row a that meet the band. (Interleaving four tiles' MFMAs, or double
// buffering the publication behind a single stage, measured 10-12% slower
// on MI355X.)
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int long_dk_s3_row_stride(int lmax) { return lmax + 2; }

__host__ __device__ constexpr size_t dk_long_s3_lds_bytes(int lmax) {
  // stages [2][2 tensors][32][RS] floats, publication [3][LMAX / 16][64][8]
  // BF16, the epilogue's per-wave tap sums [LMAX / 16][kLongMaxK] floats
  return (size_t)2 * 2 * 32 * long_dk_s3_row_stride(lmax) * sizeof(float) +
         (size_t)3 * (lmax / 16) * 64 * 8 * sizeof(__bf16) +
         (size_t)(lmax / 16) * kLongMaxK * sizeof(float);
}

// VEC: rows move as 16-byte chunks (L % 4 == 0, 16-byte aligned tensors),
// else as dwords.
template <int LMAX, bool VEC>
__global__ __launch_bounds__((LMAX / 16) * kWave) void dwconv_dk_long_s3_kernel(
    const float* __restrict__ gy, const float* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int nranges, int det) {
  constexpr int NT = LMAX / 16;
  constexpr int NTH = NT * kWave;
  constexpr int RS = long_dk_s3_row_stride(LMAX);
  constexpr int SZ = 32 * RS;                 // one tensor's stage (floats)
  constexpr int PUB = 3 * NT * 64;            // the publication (bf16x8)
  constexpr int NE = VEC ? 2 : 8;             // loads per thread, tensor and step
  constexpr int EW = VEC ? 4 : 1;             // floats per load
  constexpr int DS = LMAX + 1;                // epilogue D-row stride
  // waves per epilogue round: D rows go through the stages and publication
  constexpr int kRound = (4 * SZ + PUB * 4) / (16 * DS);
  static_assert(32 * LMAX == NE * EW * NTH, "whole rows per thread slice");
  static_assert(16 % (32 / NE) == 0, "each load's rows lie in one half of the step");
  static_assert(kRound >= 1, "staging area holds one wave's D rows");
  extern __shared__ float lds[];
  bf16x8* const pub = reinterpret_cast<bf16x8*>(lds + 4 * SZ);  // [3][NT][64]
  float* const part = lds + 4 * SZ + PUB * 4;                   // [NT][kLongMaxK]

  const int lane = threadIdx.x & (kWave - 1);
  const int a = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // tile row
  const int h = (int)(blockIdx.x % (uint32_t)H);
  const int r = (int)(blockIdx.x / (uint32_t)H);
  const int tsteps = (B + 31) / 32;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;
  const int p = K >> 1;
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 4u;
  const int g = lane >> 4, col = lane & 15;

  // Staging: loop-invariant sample row and first column of each load.
  int erow[NE], ecol[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = i * NTH + (int)threadIdx.x;
    erow[i] = e / (LMAX / EW);
    ecol[i] = EW * (e - erow[i] * (LMAX / EW));
  }
  u32x4 stv[2][NE];  // VEC
  float stg[2][NE];  // dwords
  auto load_step = [&](int s) {
    const int bs = (r + s * nranges) * 32;
    const int klim = min(32, B - bs);
    // Load i covers rows [32 i / NE, 32 (i + 1) / NE), all in one half of
    // the step: offsets run from the half's base, so they span 16 rows.
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int half = (i * (32 / NE)) / 16;
      const size_t r0 = ((size_t)(bs + 16 * half) * (size_t)H + (size_t)h) * (size_t)L;
      const __amdgpu_buffer_rsrc_t rg = make_rsrc(gy + r0);
      const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0);
      const uint32_t o = (erow[i] < klim && ecol[i] < L)
                             ? (uint32_t)(erow[i] - 16 * half) * row_bytes + 4u * (uint32_t)ecol[i]
                             : kOob;
      if constexpr (VEC) {
        stv[0][i] = buf_load_chunk<kCpolNT>(rg, o);
        stv[1][i] = buf_load_chunk<kCpolNT>(rx, o);
      } else {
        stg[0][i] = buf_load1<kCpolNT>(rg, o, 0);
        stg[1][i] = buf_load1<kCpolNT>(rx, o, 0);
      }
    }
  };

  // Rows are 8-byte aligned (RS even): 16-byte chunks go in as two halves.
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NE; ++i) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float* d = lds + (2 * buf + t) * SZ + erow[i] * RS + ecol[i];
        if constexpr (VEC) {
          const u32x4 v = stv[t][i];
          *reinterpret_cast<float2*>(d) = make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
          *reinterpret_cast<float2*>(d + 2) = make_float2(__uint_as_float(v.z), __uint_as_float(v.w));
        } else {
          *d = stg[t][i];
        }
      }
    }
  };
  // Column 16 a + col of samples 8 g .. + 7 of tensor t in stage buf, split.
  auto gather_split = [&](int buf, int t, bf16x8& hi, bf16x8& mid, bf16x8& lo) {
    const float* src = lds + (2 * buf + t) * SZ + (8 * g) * RS + 16 * a + col;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = src[i * RS];
    split3_bf16x8(v, hi, mid, lo);
  };

  auto in_band = [&](int bb) {
    const int lo = 16 * (bb - a) - 15;
    return lo + 30 >= -p && lo <= K - 1 - p && 16 * bb < L && 16 * a < L;
  };
  f32x4 acc[NT];
#pragma unroll
  for (int bb = 0; bb < NT; ++bb) acc[bb] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mfma_step = [&](int buf) {
    bf16x8 ah, am, al;
    gather_split(buf, 0, ah, am, al);
    {
      bf16x8 xh, xm, xl;
      gather_split(buf, 1, xh, xm, xl);
      pub[(0 * NT + a) * 64 + lane] = xh;
      pub[(1 * NT + a) * 64 + lane] = xm;
      pub[(2 * NT + a) * 64 + lane] = xl;
    }
    __syncthreads();  // every wave's x parts published
#pragma unroll
    for (int bb = 0; bb < NT; ++bb) {
      if (in_band(bb)) {
        const bf16x8 bh = pub[(0 * NT + bb) * 64 + lane];
        const bf16x8 bm = pub[(1 * NT + bb) * 64 + lane];
        const bf16x8 bl = pub[(2 * NT + bb) * 64 + lane];
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bm, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bh, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bm, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc[bb], 0, 0, 0);
      }
    }
  };

  if (nsteps > 0) {
    load_step(0);
    store_stage(0);
    if (1 < nsteps) load_step(1);
    __syncthreads();
    for (int s0 = 0; s0 < nsteps; s0 += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int s = s0 + d;
        if (s < nsteps) {
          mfma_step(d);
          if (s + 1 < nsteps) {
            store_stage(d ^ 1);
            if (s + 2 < nsteps) load_step(s + 2);
          }
          // Stage s + 1 in place, and every wave's reads of the publication
          // of step s complete before step s + 1 overwrites it.
          __syncthreads();
        }
      }
    }
  }

  // Epilogue rounds: waves [q, q + kRound) put their D rows in the staging
  // area (slot a - q), then sum their diagonals in order of t.
  for (int q = 0; q < NT; q += kRound) {
    const bool mine = a >= q && a < q + kRound;
    float* const blk = lds + (mine ? a - q : 0) * 16 * DS;
    if (mine) {
#pragma unroll
      for (int bb = 0; bb < NT; ++bb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) blk[(4 * g + rr) * DS + 16 * bb + col] = acc[bb][rr];
    }
    __syncthreads();
    if (mine) {
      for (int jb = 0; jb < K; jb += kWave) {
        const int j = jb + lane;
        float v = 0.0f;
        for (int tr = 0; tr < 16; ++tr) {
          const int t = 16 * a + tr;
          const int sc = t + j - p;
          if (j < K && t < L && sc >= 0 && sc < L) v += blk[tr * DS + sc];
        }
        if (j < K) part[a * kLongMaxK + j] = v;
      }
    }
    __syncthreads();
  }
  for (int j = threadIdx.x; j < K; j += NTH) {
    float v = 0.0f;
    for (int aa = 0; aa < NT; ++aa) v += part[aa * kLongMaxK + j];
    if (det)
      dst[((size_t)h * K + j) * (size_t)nranges + r] = v;
    else
      atomicAdd(dst + (size_t)h * K + j, v);
  }
}


// ---------------------------------------------------------------------------
// Long rows: DK on the BF16 matrix cores with operands loaded in place.
// The contraction of the kernel above, without the FP32 staging: in step s
// (32 samples) lane (g, c) of wave a loads dy and x at column 16 a + c of
// samples 4 i + g, i = 0 .. 7, straight from HBM with dword loads (each
// instruction reads four 64-byte row pieces), which is the operand layout of
// v_mfma_f32_16x16x32_bf16 with the K index 8 g + i standing for sample
// 4 i + g (the same permutation on both operands, so D = dyᵀx is unchanged).
// The wave splits its values once: the dy parts stay in registers as its A
// operands, the x parts go to a double-buffered publication in LDS as the B
// operands of every wave whose tile row meets column tile a. One barrier per
// step: a publication buffer is written again two steps later, after every
// wave has passed the barrier that follows its reads. Loads run two steps
// ahead in registers, with the default cache policy (each 128-byte line is
// read by two waves; non-temporal loads measured 10% slower here). Buffer
// bases sit at sample 0 and 16 of the step, so a byte offset spans at most 16
// rows, and each buffer ends at the tensor's last byte, so samples past the
// batch read zero with no per-load mask. Against the staged kernel the split
// goes from every wave's gather of a stage to its own registers, LDS holds
// only the publication (74 KB at LMAX = 192 against 148 KB), and a step has
// one barrier instead of two.
// Measured and not kept (MI355X, L = K = 192): two tiles' accumulation
// chains interleaved (-1.5% time, +18 VGPRs, slower at K = 96); the next
// tile's parts read before this tile's MFMAs (+3%, 164 VGPRs); producer and
// consumer waves (4 producers split x for 12 consumers: +10%).
// ---------------------------------------------------------------------------
__host__ __device__ constexpr size_t dk_long_s3r_lds_bytes(int lmax) {
  // publication [2][3 parts][LMAX / 16][64] bf16x8; the epilogue reuses it
  return (size_t)2 * 3 * (lmax / 16) * 64 * 8 * sizeof(__bf16);
}

template <int LMAX>
__global__ __launch_bounds__((LMAX / 16) * kWave) void dwconv_dk_long_s3r_kernel(
    const float* __restrict__ gy, const float* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int nranges, int det) {
  constexpr int NT = LMAX / 16;
  constexpr int NTH = NT * kWave;
  constexpr int PUB = 3 * NT * 64;          // bf16x8 per publication buffer
  constexpr int AREA = 2 * PUB * 4;         // floats of the whole area
  constexpr int DS = LMAX + 1;              // epilogue D-row stride
  constexpr int PART = NT * kLongMaxK;      // epilogue tap sums (floats)
  constexpr int kRound = (AREA - PART) / (16 * DS);  // waves per epilogue round
  static_assert(kRound >= 1, "the area holds one wave's D rows and the tap sums");
  extern __shared__ float lds[];
  bf16x8* const pub = reinterpret_cast<bf16x8*>(lds);  // [2][3][NT][64]
  float* const part = lds + AREA - PART;               // [NT][kLongMaxK]

  const int lane = threadIdx.x & (kWave - 1);
  const int a = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // tile row
  const int h = (int)(blockIdx.x % (uint32_t)H);
  const int r = (int)(blockIdx.x / (uint32_t)H);
  const int tsteps = (B + 31) / 32;
  const int nsteps = r < tsteps ? (tsteps - 1 - r) / nranges + 1 : 0;
  const int p = K >> 1;
  const uint32_t row_bytes = (uint32_t)H * (uint32_t)L * 4u;
  const int g = lane >> 4, col = lane & 15;
  const int c = 16 * a + col;  // this lane's column
  // Byte offset of sample 4 i + g (i < 4) from the base of its half-step,
  // out of bounds past the row. Samples past the batch are out of bounds
  // through the buffer's size: it ends at the tensor's last byte.
  uint32_t voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    voff[i] = c < L ? (uint32_t)(4 * i + g) * row_bytes + 4u * (uint32_t)c : kOob;
  const long long total = (long long)B * H * L;

  float vy[2][8], vx[2][8];
  auto load_step = [&](int s, float (&ty)[8], float (&tx)[8]) {
    const int bs = (r + s * nranges) * 32;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const long long r0 = ((long long)(bs + 16 * half) * H + h) * L;
      const long long rem = total - r0;
      const uint32_t nrec = rem <= 0 ? 0u : (uint32_t)min(4 * rem, (long long)kNumRecords);
      const __amdgpu_buffer_rsrc_t rg = make_rsrc_n(gy + r0, nrec);
      const __amdgpu_buffer_rsrc_t rx = make_rsrc_n(x + r0, nrec);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ty[4 * half + i] = buf_load1<kCpolNone>(rg, voff[i], 0);
        tx[4 * half + i] = buf_load1<kCpolNone>(rx, voff[i], 0);
      }
    }
  };
  bf16x8 ah, am, al;  // this wave's A operands (dy parts) of the current step
  auto publish = [&](int buf, const float (&ty)[8], const float (&tx)[8]) {
    split3_bf16x8(ty, ah, am, al);
    bf16x8 xh, xm, xl;
    split3_bf16x8(tx, xh, xm, xl);
    pub[((3 * buf + 0) * NT + a) * 64 + lane] = xh;
    pub[((3 * buf + 1) * NT + a) * 64 + lane] = xm;
    pub[((3 * buf + 2) * NT + a) * 64 + lane] = xl;
  };
  auto in_band = [&](int bb) {
    const int lo = 16 * (bb - a) - 15;
    return lo + 30 >= -p && lo <= K - 1 - p && 16 * bb < L && 16 * a < L;
  };
  f32x4 acc[NT];
#pragma unroll
  for (int bb = 0; bb < NT; ++bb) acc[bb] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mfma_step = [&](int buf) {
    const bf16x8* const q = pub + 3 * buf * NT * 64 + lane;
#pragma unroll
    for (int bb = 0; bb < NT; ++bb) {
      if (in_band(bb)) {
        const bf16x8 bh = q[(0 * NT + bb) * 64], bm = q[(1 * NT + bb) * 64], bl = q[(2 * NT + bb) * 64];
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bm, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bh, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bm, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc[bb], 0, 0, 0);
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc[bb], 0, 0, 0);
      }
    }
  };

  // Steps run in pairs and every step issues the same loads (an odd count
  // gets one more step, and loads past the last step are all out of bounds:
  // zeros, no memory access, and zero products leave the sums unchanged),
  // so on every path the wait before a step's use is for the loads issued
  // before the next step's, not for those too.
  if (nsteps > 0) {
    load_step(0, vy[0], vx[0]);
    load_step(1, vy[1], vx[1]);
    for (int s0 = 0; s0 < nsteps; s0 += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        publish(d, vy[d], vx[d]);
        load_step(s0 + d + 2, vy[d], vx[d]);
        __syncthreads();  // every wave's x parts of step s0 + d published
        mfma_step(d);
      }
    }
  }
  __syncthreads();  // the last step's publication is read before reuse

  // Epilogue rounds: waves [q, q + kRound) put their D rows in the area
  // (slot a - q), then sum their diagonals in order of t.
  for (int q = 0; q < NT; q += kRound) {
    const bool mine = a >= q && a < q + kRound;
    float* const blk = lds + (mine ? a - q : 0) * 16 * DS;
    if (mine) {
#pragma unroll
      for (int bb = 0; bb < NT; ++bb)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) blk[(4 * g + rr) * DS + 16 * bb + col] = acc[bb][rr];
    }
    __syncthreads();
    if (mine) {
      for (int jb = 0; jb < K; jb += kWave) {
        const int j = jb + lane;
        float v = 0.0f;
        for (int tr = 0; tr < 16; ++tr) {
          const int t = 16 * a + tr;
          const int sc = t + j - p;
          if (j < K && t < L && sc >= 0 && sc < L) v += blk[tr * DS + sc];
        }
        if (j < K) part[a * kLongMaxK + j] = v;
      }
    }
    __syncthreads();
  }
  for (int j = threadIdx.x; j < K; j += NTH) {
    float v = 0.0f;
    for (int aa = 0; aa < NT; ++aa) v += part[aa * kLongMaxK + j];
    if (det)
      dst[((size_t)h * K + j) * (size_t)nranges + r] = v;
    else
      atomicAdd(dst + (size_t)h * K + j, v);
  }
}


}  // namespace pt
