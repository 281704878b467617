/*
 * dwconv1d_oracle.c — CPU restatement of the reference's depthwise Conv1D
 * (FWD, dX, dK): the FP32 reference chains for L, K <= 48 (the range of the
 * reference kernels they restate), the FP64 sums for L, K <= 256 (the same
 * formulas, which the reference's long-row module kernels/shared_l192.py
 * computes for L = K = 192).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker. The product (pathtile_amd) never links, loads or calls it.
 *
 * Layouts: x, y, dy, dx [B,H,L] and w, dk [H,K], contiguous FP32.
 * p = K/2 (floor); zeros outside [0, L).
 *
 * Two families:
 *  - *_f32_refchain: the reference kernels' exact per-output FP32 fmaf chain
 *    (same start value 0.0f, same tap order, same skipped terms), so a
 *    correct implementation of that chain matches bit for bit:
 *      fwd  kernels/warp_tiled_ampere.py:404-433 (acc0 = fmaf(sX[xi0], kval,
 *           acc0) for kk = 0..K-1, xi0 = t + kk - pad, skipped outside [0,L))
 *      dx   kernels/warp_tiled_ampere.py:472-501 (tout = t - kk + pad)
 *  - *_f64: double accumulation of the exact float products (every
 *    float x float product is exact in double), in a fixed order:
 *      fwd/dx as above, dk as benchmark/check_dk_fp64_comparison.py:29-39
 *      (dK[h,k] = sum_{b,t} dy[b,h,t] * x_pad[b,h,t+k]) and
 *      benchmark/diagnose_dk_correctness.py:21 (valid t range per tap).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define ORACLE_MAX_CHAIN 48
#define ORACLE_MAX 256

int oracle_abi_version(void) { return 1; }

static int bad_limit(int B, int H, int L, int K, int lim) {
  return B < 0 || H < 0 || L < 1 || K < 1 || L > lim || K > lim;
}
static int bad_chain(int B, int H, int L, int K) {
  return bad_limit(B, H, L, K, ORACLE_MAX_CHAIN);
}
static int bad(int B, int H, int L, int K) {
  return bad_limit(B, H, L, K, ORACLE_MAX);
}

/* kernels/warp_tiled_ampere.py:372-434 */
int oracle_fwd_f32_refchain(const float* x, const float* w, float* y, int B,
                            int H, int L, int K) {
  if (bad_chain(B, H, L, K)) return -2;
  const int pad = K >> 1;
  const long long rows = (long long)B * H;
#pragma omp parallel for schedule(static)
  for (long long bh = 0; bh < rows; ++bh) {
    const int h = (int)(bh % H);
    const float* xr = x + bh * L;
    const float* kr = w + (long long)h * K;
    float* yr = y + bh * L;
    for (int t = 0; t < L; ++t) {
      float acc = 0.0f;
      for (int kk = 0; kk < K; ++kk) {
        const int xi = t + kk - pad;
        if ((unsigned)xi < (unsigned)L) acc = fmaf(xr[xi], kr[kk], acc);
      }
      yr[t] = acc;
    }
  }
  return 0;
}

/* kernels/warp_tiled_ampere.py:440-502 */
int oracle_dx_f32_refchain(const float* dy, const float* w, float* dx, int B,
                           int H, int L, int K) {
  if (bad_chain(B, H, L, K)) return -2;
  const int pad = K >> 1;
  const long long rows = (long long)B * H;
#pragma omp parallel for schedule(static)
  for (long long bh = 0; bh < rows; ++bh) {
    const int h = (int)(bh % H);
    const float* gr = dy + bh * L;
    const float* kr = w + (long long)h * K;
    float* xr = dx + bh * L;
    for (int t = 0; t < L; ++t) {
      float acc = 0.0f;
      for (int kk = 0; kk < K; ++kk) {
        const int tout = t - kk + pad;
        if ((unsigned)tout < (unsigned)L) acc = fmaf(gr[tout], kr[kk], acc);
      }
      xr[t] = acc;
    }
  }
  return 0;
}

int oracle_fwd_f64(const float* x, const float* w, double* y, int B, int H,
                   int L, int K) {
  if (bad(B, H, L, K)) return -2;
  const int pad = K >> 1;
  const long long rows = (long long)B * H;
#pragma omp parallel for schedule(static)
  for (long long bh = 0; bh < rows; ++bh) {
    const int h = (int)(bh % H);
    const float* xr = x + bh * L;
    const float* kr = w + (long long)h * K;
    double* yr = y + bh * L;
    for (int t = 0; t < L; ++t) {
      double acc = 0.0;
      for (int j = 0; j < K; ++j) {
        const int s = t + j - pad;
        if ((unsigned)s < (unsigned)L) acc += (double)xr[s] * (double)kr[j];
      }
      yr[t] = acc;
    }
  }
  return 0;
}

int oracle_dx_f64(const float* dy, const float* w, double* dx, int B, int H,
                  int L, int K) {
  if (bad(B, H, L, K)) return -2;
  const int pad = K >> 1;
  const long long rows = (long long)B * H;
#pragma omp parallel for schedule(static)
  for (long long bh = 0; bh < rows; ++bh) {
    const int h = (int)(bh % H);
    const float* gr = dy + bh * L;
    const float* kr = w + (long long)h * K;
    double* out = dx + bh * L;
    for (int s = 0; s < L; ++s) {
      double acc = 0.0;
      for (int j = 0; j < K; ++j) {
        const int t = s - j + pad;
        if ((unsigned)t < (unsigned)L) acc += (double)gr[t] * (double)kr[j];
      }
      out[s] = acc;
    }
  }
  return 0;
}

/*
 * dK in FP64: for each channel (one thread per channel, fixed order b, t).
 * Tap j meets t in [lo_j, hi_j) = [max(0, p-j), min(L, L+p-j)); taps with an
 * empty range are exactly 0 (benchmark/diagnose_dk_correctness.py:21).
 */
int oracle_dk_f64(const float* dy, const float* x, double* dk, int B, int H,
                  int L, int K) {
  if (bad(B, H, L, K)) return -2;
  const int pad = K >> 1;
#pragma omp parallel for schedule(static)
  for (int h = 0; h < H; ++h) {
    double acc[ORACLE_MAX];
    for (int j = 0; j < K; ++j) acc[j] = 0.0;
    for (int b = 0; b < B; ++b) {
      const long long row = ((long long)b * H + h) * L;
      const float* gr = dy + row;
      const float* xr = x + row;
      for (int j = 0; j < K; ++j) {
        const int lo = pad - j > 0 ? pad - j : 0;
        const int hi = L + pad - j < L ? L + pad - j : L;
        double a = 0.0;
        for (int t = lo; t < hi; ++t)
          a += (double)gr[t] * (double)xr[t + j - pad];
        acc[j] += a;
      }
    }
    for (int j = 0; j < K; ++j) dk[(long long)h * K + j] = acc[j];
  }
  return 0;
}
