// dwconv1d.hip — depthwise Conv1D for short rows (L <= 48, K <= 48), FP32,
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
//   * one LANE owns one whole (b,h) row, held in VGPRs;
//   * one WAVE owns 64 rows of one channel h (64 consecutive b), so the taps
//     of h are wave-uniform and live in SGPRs;
//   * a row tile is moved between HBM and the lanes through a 5 KiB per-wave
//     LDS transpose, 16 columns at a time: HBM side dwordx4 loads/stores
//     where rows are 16-byte aligned (L % 4 == 0), dword otherwise; lane side
//     ds_read/ds_write_b128 on a padded stride (20 floats) that is free of
//     bank conflicts;
//   * the inner loops are fully unrolled at compile time for a row bucket
//     LMAX (8..48) and a tap bucket KB (4..48). Taps outside [0,K) are zero
//     in SGPRs and row elements in [L, LMAX) are zero in VGPRs, so one
//     instantiation serves every (L, K) of its bucket and the unrolled FMA
//     chain only touches (t, m) pairs inside the LMAX window.
//
// FWD and DX run the reference's per-output fmaf chain in the reference's tap
// order (FWD: j ascending, kernels/warp_tiled_ampere.py:411-430; DX: j
// ascending, :479-498). Padded terms are exact no-ops (fma(0,w,a) == a,
// fma(x,0,a) == a for finite x), so outputs equal that chain bit for bit.
//
// DK: every lane accumulates all taps of its channel over the rows it owns
// (the reference's 4-tap packing, :548-584, taken to the full window since
// both rows are register resident), a DPP + bpermute wave reduction, an LDS
// reduction across the waves of the workgroup, then either one
// global_atomic_add_f32 per tap per workgroup (atomic variant, :611-614) or
// one store per tap into a [H, K, num_btiles] workspace followed by a
// fixed-order reduction kernel (deterministic variant,
// kernels/warp_tiled_noatomic_optimized.py:881-1160).

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
// offset (VGPR) and a wave-uniform per-step byte offset (soffset). Lanes
// that must not touch memory use an offset past num_records: buffer loads
// then return 0 and buffer stores are dropped, so no branches are needed.
// The host guarantees 64 * H * L * 4 < 2^31 (a tile spans < 2 GiB).
// ---------------------------------------------------------------------------
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOob = 0x80000000u;         // >= num_records
constexpr int kNumRecords = 0x7fffffff;
constexpr int kRsrcWord3 = 0x00020000;         // gfx9: 32-bit data format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0,
                                           kNumRecords, kRsrcWord3);
}

__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r,
                                            uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y),
                     __uint_as_float(v.z), __uint_as_float(v.w));
}

__device__ __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r,
                                           uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

__device__ __forceinline__ void buf_store4(float4 v, __amdgpu_buffer_rsrc_t r,
                                           uint32_t voff, uint32_t soff) {
  u32x4 u;
  u.x = __float_as_uint(v.x);
  u.y = __float_as_uint(v.y);
  u.z = __float_as_uint(v.z);
  u.w = __float_as_uint(v.w);
  __builtin_amdgcn_raw_buffer_store_b128(u, r, voff, soff, 0);
}

__device__ __forceinline__ void buf_store1(float v, __amdgpu_buffer_rsrc_t r,
                                           uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 0);
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
        buf[k] = buf_load4(rs, row_ok && col < L ? off : kOob, soff);
      } else {
        buf[k].x = buf_load1(rs, row_ok && col + 0 < L ? off + 0u : kOob, soff);
        buf[k].y = buf_load1(rs, row_ok && col + 1 < L ? off + 4u : kOob, soff);
        buf[k].z = buf_load1(rs, row_ok && col + 2 < L ? off + 8u : kOob, soff);
        buf[k].w = buf_load1(rs, row_ok && col + 3 < L ? off + 12u : kOob, soff);
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

  // Lane r holds columns [16C, 16C + cols) of row r in src[0 .. cols);
  // write rows [0, nrows), columns < L to HBM with coalesced stores.
  template <int C>
  __device__ static __forceinline__ void store(__amdgpu_buffer_rsrc_t rs,
                                               uint32_t rstride, int nrows,
                                               int L, int lane, int vec,
                                               float* stage, const float* src) {
    constexpr int nc = G::cols(C);
#pragma unroll
    for (int i = 0; i < nc / 4; ++i) {
      *reinterpret_cast<float4*>(stage + lane * kStride + 4 * i) =
          make_float4(src[4 * i + 0], src[4 * i + 1], src[4 * i + 2],
                      src[4 * i + 3]);
    }
    wave_lds_sync();
    constexpr int qpr = nc / 4;
    constexpr int rpi = kWave / qpr;
    const int r0 = lane / qpr;
    const int q = lane % qpr;
    const int col = kChunk * C + 4 * q;
    const uint32_t off = ((uint32_t)r0 * rstride + (uint32_t)col) * 4u;
#pragma unroll
    for (int k = 0; k < qpr; ++k) {
      const float4 v = *reinterpret_cast<const float4*>(
          stage + (rpi * k + r0) * kStride + 4 * q);
      const uint32_t soff = (uint32_t)(k * rpi) * rstride * 4u;
      const bool row_ok = r0 < nrows - k * rpi;
      if (vec) {
        buf_store4(v, rs, row_ok && col < L ? off : kOob, soff);
      } else {
        buf_store1(v.x, rs, row_ok && col + 0 < L ? off + 0u : kOob, soff);
        buf_store1(v.y, rs, row_ok && col + 1 < L ? off + 4u : kOob, soff);
        buf_store1(v.z, rs, row_ok && col + 2 < L ? off + 8u : kOob, soff);
        buf_store1(v.w, rs, row_ok && col + 3 < L ? off + 12u : kOob, soff);
      }
    }
    wave_lds_sync();
  }

  // Whole tile HBM -> lanes (row r -> lane r, dst[0 .. LMAX)).
  __device__ static __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rs,
                                                   uint32_t rstride, int nrows,
                                                   int L, int lane, int vec,
                                                   float* stage, float* dst) {
    float4 buf[LMAX / 4];
    static_for<0, G::nchunks>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      load<c>(rs, rstride, nrows, L, lane, vec, buf + 4 * c);
    });
    static_for<0, G::nchunks>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      transpose<c>(stage, lane, buf + 4 * c, dst + kChunk * c);
    });
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
// FWD / DX: one 64-row tile per wave. Workgroup = `wpb` waves on consecutive
// channels of the same 64-sample batch chunk; grid = ceil(H/wpb) channel
// groups x ceil(B/64) chunks, flattened and XCD-remapped.
// ---------------------------------------------------------------------------
template <int LMAX, int KB, bool DX>
__global__ __launch_bounds__(1024) void dwconv_rows_kernel(
    const float* __restrict__ in, const float* __restrict__ w,
    float* __restrict__ out, int B, int H, int L, int K, int wpb, int ngroups,
    uint32_t nblocks, int vec) {
  using W = Window<LMAX, KB, DX>;
  using IO = TileIO<LMAX>;
  using G = RowGeo<LMAX>;
  extern __shared__ float lds[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t blk = xcd_remap(blockIdx.x, nblocks);
  const int group = (int)(blk % (uint32_t)ngroups);
  const int chunk = (int)(blk / (uint32_t)ngroups);
  const int h = group * wpb + wave;
  if (h >= H) return;  // wave-uniform; no workgroup barrier below
  const int b0 = chunk * kWave;
  const int nrows = min(kWave, B - b0);
  const uint32_t rstride = (uint32_t)H * (uint32_t)L;
  const size_t row0 = ((size_t)b0 * (size_t)H + (size_t)h) * (size_t)L;
  float* stage = lds + wave * kStageFloats;

  float wt[W::n];
  load_taps<W::lo, W::n, DX>(w, h, H, K, lane, wt);

  float xr[LMAX];
  IO::load_rows(make_rsrc(in + row0), rstride, nrows, L, lane, vec, stage, xr);

  const __amdgpu_buffer_rsrc_t orsrc = make_rsrc(out + row0);
  // Per output: the reference's fmaf chain, taps in reference order
  // (FWD: j = p + m ascending <=> i ascending; DX: j = p - m ascending <=>
  // i descending). Computed and stored one 16-column chunk at a time.
  static_for<0, G::nchunks>([&](auto cc) {
    constexpr int c = decltype(cc)::value;
    constexpr int nc = G::cols(c);
    float yc[kChunk];
#pragma unroll
    for (int tt = 0; tt < nc; ++tt) {
      const int t = kChunk * c + tt;
      float acc = 0.0f;
#pragma unroll
      for (int ii = 0; ii < W::n; ++ii) {
        const int i = DX ? (W::n - 1 - ii) : ii;
        const int s = t + W::lo + i;
        if (s >= 0 && s < LMAX) acc = fmaf(xr[s], wt[i], acc);
      }
      yc[tt] = acc;
    }
    IO::template store<c>(orsrc, rstride, nrows, L, lane, vec, stage, yc);
  });
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
template <int LMAX, int KB>
__global__ __launch_bounds__(kMaxDkThreads) void dwconv_dk_kernel(
    const float* __restrict__ gy, const float* __restrict__ x,
    float* __restrict__ dst, int B, int H, int L, int K, int R, int nbt,
    uint32_t nblocks, int vec, int det) {
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
// Dispatch tables: row buckets 8..48 (step 8) x tap buckets below.
// ---------------------------------------------------------------------------
constexpr int kNumLB = 6;
constexpr int kNumKB = 7;
constexpr int kKBuckets[kNumKB] = {4, 8, 16, 24, 32, 40, 48};

using RowsFn = void (*)(const float*, const float*, float*, int, int, int, int,
                        int, int, uint32_t, int);
using DkFn = void (*)(const float*, const float*, float*, int, int, int, int,
                      int, int, uint32_t, int, int);

#define PT_ROWS_ROW(LM, DX)                                                   \
  {                                                                           \
    &dwconv_rows_kernel<LM, 4, DX>, &dwconv_rows_kernel<LM, 8, DX>,           \
        &dwconv_rows_kernel<LM, 16, DX>, &dwconv_rows_kernel<LM, 24, DX>,     \
        &dwconv_rows_kernel<LM, 32, DX>, &dwconv_rows_kernel<LM, 40, DX>,     \
        &dwconv_rows_kernel<LM, 48, DX>                                       \
  }
#define PT_ROWS_TABLE(DX)                                                     \
  {                                                                           \
    PT_ROWS_ROW(8, DX), PT_ROWS_ROW(16, DX), PT_ROWS_ROW(24, DX),             \
        PT_ROWS_ROW(32, DX), PT_ROWS_ROW(40, DX), PT_ROWS_ROW(48, DX)         \
  }
#define PT_DK_ROW(LM)                                                         \
  {                                                                           \
    &dwconv_dk_kernel<LM, 4>, &dwconv_dk_kernel<LM, 8>,                       \
        &dwconv_dk_kernel<LM, 16>, &dwconv_dk_kernel<LM, 24>,                 \
        &dwconv_dk_kernel<LM, 32>, &dwconv_dk_kernel<LM, 40>,                 \
        &dwconv_dk_kernel<LM, 48>                                             \
  }

static const RowsFn kFwdTable[kNumLB][kNumKB] = PT_ROWS_TABLE(false);
static const RowsFn kDxTable[kNumLB][kNumKB] = PT_ROWS_TABLE(true);
static const DkFn kDkTable[kNumLB][kNumKB] = {PT_DK_ROW(8),  PT_DK_ROW(16),
                                              PT_DK_ROW(24), PT_DK_ROW(32),
                                              PT_DK_ROW(40), PT_DK_ROW(48)};

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

// Samples per wave chunk is 64; a DK workgroup covers wpb * R chunks. R is
// chosen from the shape so that the grid holds about 2048 workgroups' worth
// of chunks (8 per CU), which keeps atomics per tap low (H * nbt * K total)
// without starving the 256 CUs.
struct DkGeom {
  int wpb, R, nbt;
  long long nblocks;
};

static DkGeom dk_geometry(int B, int H, int threads) {
  DkGeom g;
  g.wpb = threads / kWave;
  const long long chunks_per_h = ((long long)B + kWave - 1) / kWave;
  const long long total = chunks_per_h * (long long)H;
  long long R = total / ((long long)g.wpb * 2048);
  if (R < 1) R = 1;
  if (R > 16) R = 16;
  const long long per_wg = (long long)g.wpb * R;
  if (R > (chunks_per_h + g.wpb - 1) / g.wpb) {
    R = (chunks_per_h + g.wpb - 1) / g.wpb;
    if (R < 1) R = 1;
  }
  (void)per_wg;
  g.R = (int)R;
  const long long tile = (long long)g.wpb * g.R * kWave;
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

static int rows_path(bool dx, const float* in, const float* w, float* out,
                     int B, int H, int L, int K, int wpb, void* stream) {
  int st = check_shape(B, H, L, K);
  if (st != PT_OK) return st;
  if (!valid_wpb(wpb)) return PT_ERR_CONFIG;
  if (B == 0 || H == 0) return PT_OK;  // empty tensors may have NULL data
  if (!in || !w || !out) return PT_ERR_NULL;
  if (!aligned(in, 4) || !aligned(w, 4) || !aligned(out, 4))
    return PT_ERR_ALIGN;
  const int ngroups = (H + wpb - 1) / wpb;
  const long long nchunks = ((long long)B + kWave - 1) / kWave;
  const long long nb = nchunks * ngroups;
  if (nb >= (1LL << 31)) return PT_ERR_SHAPE;
  uint32_t nblocks = (uint32_t)nb;
  int vec = (L % 4 == 0) && aligned(in, 16) && aligned(out, 16);
  RowsFn fn = (dx ? kDxTable : kFwdTable)[lbucket_index(L)][kbucket_index(K)];
  void* args[] = {&in, &w, &out, &B, &H, &L, &K, &wpb, (void*)&ngroups,
                  &nblocks, &vec};
  return launch((const void*)fn, nblocks, (uint32_t)(wpb * kWave),
                (size_t)wpb * kStageBytes, stream, args);
}

static int dk_path(bool det, const float* gy, const float* x, float* dst,
                   int B, int H, int L, int K, int threads, const DkGeom& g,
                   void* stream) {
  uint32_t nblocks = (uint32_t)g.nblocks;
  int vec = (L % 4 == 0) && aligned(gy, 16) && aligned(x, 16);
  int R = g.R, nbt = g.nbt, d = det ? 1 : 0;
  DkFn fn = kDkTable[lbucket_index(L)][kbucket_index(K)];
  void* args[] = {&gy, &x, &dst, &B, &H, &L, &K, &R, &nbt, &nblocks, &vec, &d};
  return launch((const void*)fn, nblocks, (uint32_t)threads,
                (size_t)g.wpb * kStageBytes, stream, args);
}

static const void* kernel_for(int kernel_id, int L, int K) {
  if (L < 1 || L > kMaxL || K < 1 || K > kMaxK) return nullptr;
  const int li = lbucket_index(L), ki = kbucket_index(K);
  switch (kernel_id) {
    case PT_KERNEL_FWD: return (const void*)kFwdTable[li][ki];
    case PT_KERNEL_DX: return (const void*)kDxTable[li][ki];
    case PT_KERNEL_DK: return (const void*)kDkTable[li][ki];
    case PT_KERNEL_DK_REDUCE: return (const void*)&dk_reduce_kernel;
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
    case PT_ERR_SHAPE: return "invalid shape (need 1<=L<=48, 1<=K<=48, B,H>=0, B*H*L<2^31)";
    case PT_ERR_CONFIG: return "unsupported launch configuration";
    case PT_ERR_WORKSPACE: return "workspace missing or too small";
    case PT_ERR_HIP: return "HIP runtime launch error";
    case PT_ERR_ALIGN: return "pointer not 4-byte aligned";
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
  const pt::DkGeom g = pt::dk_geometry(B, H, threads_per_block);
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
  const pt::DkGeom g = pt::dk_geometry(B, H, threads_per_block);
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
  const pt::DkGeom g = pt::dk_geometry(B, H, threads_per_block);
  if (g.nblocks >= (1LL << 31)) return PT_ERR_SHAPE;
  const size_t need = (size_t)H * (size_t)K * (size_t)g.nbt * sizeof(float);
  if (!workspace || workspace_bytes < need) return PT_ERR_WORKSPACE;
  if (!pt::aligned(workspace, 4)) return PT_ERR_ALIGN;
  float* partials = (float*)workspace;
  st = pt::dk_path(true, dy, x, partials, B, H, L, K, threads_per_block, g,
                   stream);
  if (st != PT_OK) return st;
  int ncoef = H * K;
  int nbt = g.nbt;
  const float* cp = partials;
  void* args[] = {&cp, &dk, &ncoef, &nbt};
  const uint32_t grid = (uint32_t)((ncoef + 3) / 4);
  return pt::launch((const void*)&pt::dk_reduce_kernel, grid, 256, 0, stream,
                    args);
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
      *lds_bytes = block_config * pt::kStageBytes;
      return PT_OK;
    case PT_KERNEL_DK:
      if (!pt::valid_dk_threads(block_config)) return PT_ERR_CONFIG;
      *lds_bytes = (block_config / pt::kWave) * pt::kStageBytes;
      return PT_OK;
    case PT_KERNEL_DK_REDUCE:
      *lds_bytes = 0;
      return PT_OK;
    default:
      return PT_ERR_CONFIG;
  }
}

}  // extern "C"
