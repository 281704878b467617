/*
 * pathtile_hip.h — C ABI of the MI355X (gfx950) depthwise Conv1D library.
 *
 * Semantics shared by every entry point (FP32, contiguous row-major tensors):
 *   x, y, dy, dx : [B, H, L]      w, dk : [H, K]      p = K / 2 (floor)
 *   y [b,h,t] = sum_{j<K} w[h,j] * x [b,h,t+j-p]      (zero outside [0, L))
 *   dx[b,h,s] = sum_{j<K} w[h,j] * dy[b,h,s-j+p]
 *   dk[h,j]   = sum_b sum_t dy[b,h,t] * x[b,h,t+j-p]
 * i.e. cross-correlation, "same" length with asymmetric padding (left p,
 * right K-1-p), as in the reference kernels
 * kernels/warp_tiled_ampere.py:372-434 (fwd), :440-502 (dx), :509-619 (dk)
 * and the PyTorch boundary benchmark/benchmark_shape_sweep_ampere.py:220-239.
 *
 * Limits: 1 <= L <= 48, 1 <= K <= 48 (the reference rejects L>48 or K>48 at
 * kernels/warp_tiled_ampere.py:715-716), B >= 0, H >= 0, B*H*L < 2^31.
 *
 * Every entry point:
 *   - never allocates device memory and never throws across the boundary;
 *   - enqueues work on `stream` (a hipStream_t, NULL = default stream) of the
 *     device that is current on the calling thread, and returns without
 *     synchronising;
 *   - returns PT_OK or a negative PT_ERR_* code (the reference's only C ABI,
 *     benchmark/flashdwc_fp32_bridge.cu:14-19, returns -2 for bad arguments;
 *     PT_ERR_SHAPE keeps that value).
 */
#ifndef PATHTILE_HIP_H
#define PATHTILE_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PT_ABI_VERSION 1

#define PT_OK 0
#define PT_ERR_NULL (-1)       /* a required pointer is NULL                 */
#define PT_ERR_SHAPE (-2)      /* B,H,L,K outside the supported range        */
#define PT_ERR_CONFIG (-3)     /* launch configuration not supported         */
#define PT_ERR_WORKSPACE (-4)  /* workspace missing or too small             */
#define PT_ERR_HIP (-5)        /* the HIP runtime reported a launch error    */
#define PT_ERR_ALIGN (-6)      /* pointer not 4-byte aligned                 */
#define PT_ERR_SCRATCH (-7)    /* the static scratch is too small (noalloc)  */

/* Bytes of the static device scratch of pt_dwconv1d_dk_det_f32_noalloc. */
#define PT_DK_SCRATCH_BYTES (8u << 20)

#define PT_MAX_L 48
#define PT_MAX_K 48

/* Kernel identifiers for pt_kernel_attributes. */
#define PT_KERNEL_FWD 0
#define PT_KERNEL_DX 1
#define PT_KERNEL_DK 2
#define PT_KERNEL_DK_REDUCE 3
#define PT_KERNEL_DK_CG 4      /* channel-group DK (H a multiple of channels per wave x waves) */
#define PT_KERNEL_FWD_CG 5     /* channel-group matrix-core FWD (H % 8 == 0) */
#define PT_KERNEL_DX_CG 6      /* channel-group matrix-core DX  (H % 8 == 0) */
#define PT_KERNEL_FWD_STREAM 7 /* short-tap streaming FWD (K <= 9, L % 4 == 0) */
#define PT_KERNEL_DX_STREAM 8  /* short-tap streaming DX  (K <= 9, L % 4 == 0) */
#define PT_KERNEL_FWD_CG16 9   /* 16-channel matrix-core FWD (33 <= L <= 48, H % 16 == 0) */
#define PT_KERNEL_DX_CG16 10   /* 16-channel matrix-core DX  (33 <= L <= 48, H % 16 == 0) */

/* Version of this ABI (PT_ABI_VERSION). */
int pt_abi_version(void);

/* Static text for a status code ("ok", "invalid shape", ...). */
const char* pt_status_string(int status);

/*
 * Forward pass y = conv(x, w).
 * Replaces the launch of dwconv1d_warptile_fwd in
 * AmpereWarpRuntime.launch_fwd (kernels/warp_tiled_ampere.py:723-747).
 * waves_per_block: 64-lane wavefronts per workgroup, one of 1,2,4,8,16 (the
 * MI355X counterpart of WARPS_PER_BLOCK, kernels/warp_tiled_ampere.py:643-644).
 *
 * Two kernels serve FWD and DX. The lane-per-row VALU kernel reproduces the
 * reference's fmaf chain bit for bit and honours waves_per_block; its
 * workgroup holds a 64-row LDS tile per wave, so 16 waves fit only rows up
 * to 32 (PT_ERR_CONFIG for longer rows on this kernel). Where the FMA chain
 * is long enough and the layout allows it (H % 8 == 0, x and y 16-byte
 * aligned; any L), the channel-group matrix-core kernel runs instead. For
 * rows of L % 4 == 0 from 16 to 48 columns "long enough" means K at least
 * 5 (L = 16), 9 (L = 20-32, 44; L = 48 on tensors of at most 256 MiB with
 * H <= 128) or 17 (L = 36, 40; L = 48 otherwise), higher on calls of fewer
 * than 2^17 rows (B x H); shorter rows need 10.5 (16 / L)^2 useful FMAs per
 * output; rows of other lengths take it from 2^18 rows at any K, and below
 * that from 5 (LMAX / L)^2 useful FMAs per output (LMAX = 16 ceil(L / 16)).
 * It runs 8 waves (channels) per workgroup, or 16 on large calls (tensors
 * above 256 MiB or at least 24 16-sample steps per CU) with H % 16 == 0 for
 * rows of 33-47 columns with L % 4 != 0 and for rows of more than 40
 * columns with H L > 128 x 48, whatever waves_per_block says, so every
 * value is accepted there and gives the same bits; it sums in the
 * matrix cores' order (within FP32 rounding of the reference: about 3e-7
 * max-abs-scaled against FP64). On both kernels an Inf or NaN input or tap
 * reaches exactly the outputs whose reference window holds it (those
 * outputs follow the reference's chain). The environment variable
 * PATHTILE_ROWS_ALGO=valu selects the VALU kernel everywhere, =mfma the
 * matrix-core kernel wherever the layout allows; PATHTILE_ROWS_CHANNELS=8
 * or =16 forces the matrix-core kernel's channels per workgroup where the
 * layout allows; both are read on every call.
 */
int pt_dwconv1d_fwd_f32(const float* x, const float* w, float* y, int B, int H,
                        int L, int K, int waves_per_block, void* stream);

/*
 * pt_dwconv1d_fwd_f32 / pt_dwconv1d_dx_f32 with the kernel chosen by the
 * caller: PT_ROWS_AUTO as those entry points (PATHTILE_ROWS_ALGO, then the
 * library's rule), PT_ROWS_VALU the VALU kernels (the reference's fmaf
 * chain bit for bit, any layout), PT_ROWS_MATRIX the matrix-core kernel
 * wherever the layout allows it (else the VALU kernels). An explicit choice
 * takes precedence over PATHTILE_ROWS_ALGO; any other value of algo is
 * PT_ERR_CONFIG. No counterpart in the reference, whose one kernel per path
 * leaves nothing to choose: for a caller that needs the reference's bits
 * (or the matrix cores) in one runtime, not in the whole process.
 */
#define PT_ROWS_AUTO 0
#define PT_ROWS_VALU 1
#define PT_ROWS_MATRIX 2
int pt_dwconv1d_fwd_f32_algo(const float* x, const float* w, float* y, int B, int H,
                             int L, int K, int waves_per_block, int algo, void* stream);
int pt_dwconv1d_dx_f32_algo(const float* dy, const float* w, float* dx, int B, int H,
                            int L, int K, int waves_per_block, int algo, void* stream);

/*
 * Which kernel pt_dwconv1d_fwd_f32_algo (dx = 0) or pt_dwconv1d_dx_f32_algo
 * (dx != 0) would launch for this call on the current device, with tensors
 * 16-byte aligned (aligned16 != 0) or only 4-byte aligned: *kernel_id
 * receives PT_KERNEL_FWD / _DX (VALU tile kernel), _FWD_STREAM / _DX_STREAM,
 * _FWD_CG / _DX_CG (8-channel matrix cores) or _FWD_CG16 / _DX_CG16, or -1
 * when B or H is 0. The same dispatch code runs as in a launch (environment
 * variables included) and stops before launching; the return value is the
 * status that call would return. No counterpart in the reference, which has
 * one kernel per path: for harnesses that name or report the kernel.
 */
int pt_rows_kernel_id(int B, int H, int L, int K, int waves_per_block,
                      int algo, int aligned16, int dx, int* kernel_id);

/*
 * Input gradient dx = conv^T(dy, w).
 * Replaces dwconv1d_warptile_bwd_input in AmpereWarpRuntime.launch_bwd_input
 * (kernels/warp_tiled_ampere.py:749-770). Kernel choice as for the forward
 * pass (dy and dx 16-byte aligned for the matrix-core kernel).
 */
int pt_dwconv1d_dx_f32(const float* dy, const float* w, float* dx, int B,
                       int H, int L, int K, int waves_per_block, void* stream);

/*
 * Weight gradient, atomic variant: dk += sum over batch tiles.
 * Replaces dwconv1d_warptile_bwd_weight in AmpereWarpRuntime.launch_bwd_weight
 * (kernels/warp_tiled_ampere.py:772-812). The reference requires the caller
 * to zero dk first (:890-893); zero_first != 0 clears dk on `stream` with a
 * fill kernel before the accumulation, so "dK including zero-init" is one
 * call. threads_per_block: a multiple of 64 in [64, 768] (the counterpart of
 * BWDK_BLOCK, :645-649). Summation order across workgroups is not fixed.
 */
int pt_dwconv1d_dk_atomic_f32(const float* dy, const float* x, float* dk,
                              int B, int H, int L, int K,
                              int threads_per_block, int zero_first,
                              void* stream);

/*
 * Bytes of workspace pt_dwconv1d_dk_det_f32 needs for this shape/config
 * (the [H, K, num_btiles] partials of
 * kernels/warp_tiled_noatomic_optimized.py:1448-1471).
 */
int pt_dwconv1d_dk_det_workspace_bytes(int B, int H, int L, int K,
                                       int threads_per_block, size_t* bytes);

/*
 * Weight gradient, deterministic two-pass variant: per-batch-tile partials
 * into `workspace`, then a fixed-order reduction that overwrites dk (no
 * zero-init needed). Bitwise reproducible for a fixed shape,
 * threads_per_block and input alignment (16-byte aligned or not) on a
 * given device. Replaces dwconv1d_warptile_bwd_weight_partials +
 * dwconv1d_warptile_reduce_partials
 * (kernels/warp_tiled_noatomic_optimized.py:881,1116; launch :1473-1554).
 */
int pt_dwconv1d_dk_det_f32(const float* dy, const float* x, float* dk,
                           void* workspace, size_t workspace_bytes, int B,
                           int H, int L, int K, int threads_per_block,
                           void* stream);

/*
 * Deterministic weight gradient that allocates nothing and takes no
 * workspace. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same kernels, partial order and
 * result bits as pt_dwconv1d_dk_det_f32 with the same threads_per_block;
 * the partials go to a static device array of PT_DK_SCRATCH_BYTES (8 MiB)
 * that each device holds until the process ends. A call for which
 * pt_dwconv1d_dk_det_workspace_bytes reports more than that returns
 * PT_ERR_SCRATCH; the limit follows from the shape and threads_per_block
 * alone and is checked before any device query. Every call on a device
 * shares that device's array: calls that overlap on one device (two
 * streams, two host threads) race and must be ordered by the caller. Each
 * call overwrites every partial it reads, so nothing needs clearing
 * between calls. The first call on a device looks up the array's address
 * and the kernels' occupancy (HIP queries that are not stream work): make
 * one call on each device before capturing calls into a HIP graph.
 */
int pt_dwconv1d_dk_det_f32_noalloc(const float* dy, const float* x, float* dk,
                                   int B, int H, int L, int K,
                                   int threads_per_block, void* stream);

/*
 * BF16 I/O variants (no counterpart in the reference, which is FP32 only).
 * x, y, dy, dx are bfloat16 tensors passed as their 16-bit patterns; w and dk
 * stay FP32. The kernels multiply on the BF16 matrix cores with FP32
 * accumulation (FWD/DX split each FP32 tap into a hi + lo BF16 pair; DK
 * products of two BF16 values are exact in FP32) and round FP32 outputs to
 * BF16 to nearest-even. They halve the bytes the paths move. Only the
 * channel-group layout is served: L % 4 == 0 and, for FWD/DX, H % 8 == 0,
 * for DK, threads_per_block <= 512 with H % (2 * threads_per_block / 64) == 0
 * (PT_ERR_CONFIG otherwise); BF16 tensors must be 16-byte aligned
 * (PT_ERR_ALIGN). DK semantics match the FP32 entry points (atomic with
 * optional zero_first; deterministic two-pass with its own workspace size).
 */
int pt_dwconv1d_fwd_bf16(const void* x, const float* w, void* y, int B, int H,
                         int L, int K, void* stream);
int pt_dwconv1d_dx_bf16(const void* dy, const float* w, void* dx, int B, int H,
                        int L, int K, void* stream);
int pt_dwconv1d_dk_atomic_bf16(const void* dy, const void* x, float* dk, int B,
                               int H, int L, int K, int threads_per_block,
                               int zero_first, void* stream);
int pt_dwconv1d_dk_det_bf16_workspace_bytes(int B, int H, int L, int K,
                                            int threads_per_block,
                                            size_t* bytes);
int pt_dwconv1d_dk_det_bf16(const void* dy, const void* x, float* dk,
                            void* workspace, size_t workspace_bytes, int B,
                            int H, int L, int K, int threads_per_block,
                            void* stream);

/*
 * Long rows: L up to 192 and K up to 256 (taps past the row add nothing),
 * the regime of the
 * reference's kernels/shared_l192.py (DepthwiseConvShared, benchmarked at
 * L = K = 192 by benchmark/benchmark_gmc_vs_shared_l192.py:14-17), whose
 * forward / backward call the same three paths as the specialised API:
 *   FWD  y[b,h,t]  = sum_j w[h,j] x[b,h,t+j-K/2]      (kernels/shared_l192.py
 *   DX   gx[b,h,s] = sum_j w[h,j] gy[b,h,s-j+K/2]      :130-626, launched at
 *   DK   gk[h,j]   = sum_b sum_t gy[b,h,t] x[b,h,t+j-K/2]  :840-1005)
 * FP32 accuracy on the matrix cores: by default the BF16 instructions on
 * FP32 operands split three ways (six part products, each exact in FP32;
 * DK from 40 taps up and at L = 64, 96), else the FP32 instructions; PATHTILE_LONG_ALGO=fp32
 * or =split forces one kind. FWD/DX need only 4-byte aligned tensors. DK is
 * deterministic (fixed-order partials plus a reduction, as
 * pt_dwconv1d_dk_det_f32) and overwrites dk; its workspace size depends on
 * (B, H) only. B * H * L < 2^31 and 16 * H * L * 4 < 2^31 (PT_ERR_SHAPE).
 */
int pt_dwconv1d_fwd_long_f32(const float* x, const float* w, float* y, int B,
                             int H, int L, int K, void* stream);
int pt_dwconv1d_dx_long_f32(const float* dy, const float* w, float* dx, int B,
                            int H, int L, int K, void* stream);
int pt_dwconv1d_dk_long_workspace_bytes(int B, int H, int L, int K,
                                        size_t* bytes);
int pt_dwconv1d_dk_long_f32(const float* dy, const float* x, float* dk,
                            void* workspace, size_t workspace_bytes, int B,
                            int H, int L, int K, void* stream);

/*
 * Channels-last DK with the C ABI of the Flash-DWC dW bridge the reference
 * binds through ctypes (benchmark/flashdwc_fp32_bridge.cu:6-34; called from
 * benchmark/check_dk_fp64_comparison.py:16-65). x and dy are [B, 1, L, H]
 * FP32, dw is [1, K, H]:
 *   dw[j][h] += sum_b sum_t dy[b][t][h] * x[b][t + j - K/2][h]
 * (x zero outside [0, L)); the caller zeroes dw first. Returns 0, or -2 for
 * the arguments the bridge rejects (NULL pointers; B, H, L, K or GZ <= 0;
 * H % 32 != 0; B % GZ != 0; (B / GZ) % 16 != 0) and for the ones this
 * library does not serve (L or K above 48; x or dy not 16-byte aligned, dw
 * not 4-byte aligned), or PT_ERR_HIP. GZ, the bridge's batch split, is
 * validated as the bridge does and otherwise ignored.
 */
int flash_dk_fp32(const float* x, const float* dy, float* dw, int B, int H,
                  int L, int K, int GZ, void* stream);

/*
 * Compiled resources of the kernel that serves (L, K) for `kernel_id`
 * (PT_KERNEL_*), as hipFuncGetAttributes reports them on the current device:
 * registers per lane, static LDS bytes, scratch (private) bytes per lane and
 * max threads per block. Any output pointer may be NULL. Counterpart of the
 * PyCUDA attributes read by AmpereWarpRuntime.resource_report
 * (kernels/warp_tiled_ampere.py:814-833). Needs a device.
 */
int pt_kernel_attributes(int kernel_id, int L, int K, int* regs,
                         int* lds_bytes, int* scratch_bytes, int* max_threads);

/* Dynamic LDS bytes one workgroup of `kernel_id` uses at this launch config. */
int pt_dynamic_lds_bytes(int kernel_id, int L, int K, int block_config,
                         int* lds_bytes);

#ifdef __cplusplus
}
#endif

#endif /* PATHTILE_HIP_H */
