// Device helpers shared by the gfx950 kernel files: complex arithmetic, wave
// and block reductions, and the LDS Stockham FFT.  Internal; not part of the
// C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>

#include "tsne_device.h"

namespace fehip {
namespace {

constexpr int kWave = 64;

// Instruction-issue priority of the iteration's latency-bound chain
// (statistics, binning, spreading, transforms, finalizes, update) over the
// attraction that shares its CUs when the two overlap: s_setprio raises this
// wave's priority in the CU's issue arbiter (0..3).  It does not touch queue
// or stream priorities.
__device__ __forceinline__ void chain_priority() { __builtin_amdgcn_s_setprio(3); }

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
__device__ __forceinline__ float2 cmul(float2 a, float2 b) {
  return make_float2(a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x);
}
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }
__device__ __forceinline__ float2 conjf2(float2 a) { return make_float2(a.x, -a.y); }
// i * a
__device__ __forceinline__ float2 mul_i(float2 a) { return make_float2(-a.y, a.x); }

// ---------------------------------------------------------------------------
// Reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ void combine(BlockStats& a, const BlockStats& b) {
  a.min_x = fminf(a.min_x, b.min_x);
  a.max_x = fmaxf(a.max_x, b.max_x);
  a.min_y = fminf(a.min_y, b.min_y);
  a.max_y = fmaxf(a.max_y, b.max_y);
  a.sum_x += b.sum_x;
  a.sum_y += b.sum_y;
}

__device__ __forceinline__ BlockStats stats_identity() {
  BlockStats s;
  s.min_x = FLT_MAX;
  s.max_x = -FLT_MAX;
  s.min_y = FLT_MAX;
  s.max_y = -FLT_MAX;
  s.sum_x = 0.0;
  s.sum_y = 0.0;
  return s;
}

__device__ __forceinline__ BlockStats wave_stats(BlockStats s) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    BlockStats o;
    o.min_x = __shfl_xor(s.min_x, off, kWave);
    o.max_x = __shfl_xor(s.max_x, off, kWave);
    o.min_y = __shfl_xor(s.min_y, off, kWave);
    o.max_y = __shfl_xor(s.max_y, off, kWave);
    o.sum_x = __shfl_xor(s.sum_x, off, kWave);
    o.sum_y = __shfl_xor(s.sum_y, off, kWave);
    combine(s, o);
  }
  return s;
}

// Block-wide reduction; the result is valid in thread 0.  Fixed order, so the
// result is deterministic for a fixed launch shape.
template <int NT>
__device__ BlockStats block_stats(BlockStats s) {
  __shared__ BlockStats part[NT / kWave];
  s = wave_stats(s);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) part[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    BlockStats t = part[0];
    for (int w = 1; w < NT / kWave; ++w) combine(t, part[w]);
    s = t;
  }
  __syncthreads();
  return s;
}

template <int NT>
__device__ double block_sum(double v) {
  __shared__ double part[NT / kWave];
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) part[wave] = v;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0) {
    for (int w = 0; w < NT / kWave; ++w) t += part[w];
  }
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------
// LDS Stockham FFT
//
// NSEQ sequences of length F, sequence q at s + q * F, transformed in place by
// NT threads.  Radix-4 stages (Ns = 1, 4, 16, ...) then one radix-2 stage
// when log2(F) is odd; every stage reads its inputs to registers, barriers,
// and writes the Stockham-permuted outputs, so the result is in natural order.
// Twiddles come from a 4096-entry table of e^{-2 pi i m / 4096} (computed in
// fp64 on the host); INV conjugates them and leaves the result unscaled.
// ---------------------------------------------------------------------------
template <bool INV>
__device__ __forceinline__ float2 twiddle(const float2* __restrict__ tw, int m) {
  const float2 w = tw[m];
  return INV ? make_float2(w.x, -w.y) : w;
}

// Copies the F twiddles e^{-2 pi i j / F} of the global 4096-entry table into
// LDS (the caller's next barrier publishes them); transforms then read their
// twiddles from LDS (TWS = 1) instead of from the cache hierarchy.
template <int F, int NT>
__device__ __forceinline__ void stage_twiddles(float2* lds_tw, const float2* __restrict__ tw) {
  constexpr int STRIDE = kTwiddleLen / F;
  for (int j = threadIdx.x; j < F; j += NT) lds_tw[j] = tw[j * STRIDE];
}

// tw holds e^{-2 pi i j / (F * TWS)}: the global table (TWS = 4096 / F) or
// one staged in LDS (TWS = 1).
template <int F, int NSEQ, int NT, bool INV, int TWS = kTwiddleLen / F>
__device__ __forceinline__ void fft_lds(float2* s, const float2* __restrict__ tw) {
  constexpr int LOG2F = ilog2(F);
  constexpr int Q = F / 4;
  constexpr int TOT = NSEQ * Q;
  constexpr int BPT = (TOT + NT - 1) / NT;
#pragma unroll
  for (int stage = 0; stage < LOG2F / 2; ++stage) {
    const int ns = 1 << (2 * stage);
    float2 v[BPT][4];
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const int t = threadIdx.x + b * NT;
      if (TOT % NT == 0 || t < TOT) {
        const int q = t / Q;
        const int j = t - q * Q;
        const float2* src = s + q * F;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[b][r] = src[j + r * Q];
        const int kk = j & (ns - 1);
        const int step = (F / (4 * ns)) * kk * TWS;
        v[b][1] = cmul(v[b][1], twiddle<INV>(tw, step));
        v[b][2] = cmul(v[b][2], twiddle<INV>(tw, 2 * step));
        v[b][3] = cmul(v[b][3], twiddle<INV>(tw, 3 * step));
        const float2 a = cadd(v[b][0], v[b][2]);
        const float2 c = csub(v[b][0], v[b][2]);
        const float2 d = cadd(v[b][1], v[b][3]);
        const float2 e = csub(v[b][1], v[b][3]);
        // forward: (-i) * e, inverse: (+i) * e
        const float2 er = INV ? make_float2(-e.y, e.x) : make_float2(e.y, -e.x);
        v[b][0] = cadd(a, d);
        v[b][1] = cadd(c, er);
        v[b][2] = csub(a, d);
        v[b][3] = csub(c, er);
      }
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const int t = threadIdx.x + b * NT;
      if (TOT % NT == 0 || t < TOT) {
        const int q = t / Q;
        const int j = t - q * Q;
        const int kk = j & (ns - 1);
        float2* dst = s + q * F + (j - kk) * 4 + kk;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r * ns] = v[b][r];
      }
    }
    __syncthreads();
  }
  if (LOG2F & 1) {
    constexpr int H2 = F / 2;
    constexpr int TOT2 = NSEQ * H2;
#pragma unroll
    for (int b = 0; b < (TOT2 + NT - 1) / NT; ++b) {
      const int t = threadIdx.x + b * NT;
      if (TOT2 % NT == 0 || t < TOT2) {
        const int q = t / H2;
        const int j = t - q * H2;
        float2* base = s + q * F;
        const float2 v0 = base[j];
        const float2 v1 = cmul(base[j + H2], twiddle<INV>(tw, j * TWS));
        base[j] = cadd(v0, v1);
        base[j + H2] = csub(v0, v1);
      }
    }
    __syncthreads();
  }
}

template <int F>
struct Shape {
  static constexpr int G = F / 2;
  static constexpr int H = F / 2 + 1;
  static constexpr int KROWS = F >= 1024 ? 1 : 1024 / F;  // single-sequence rows per block
  static constexpr int CROWS = F >= 512 ? 1 : 512 / F;    // two-sequence rows per block
  static constexpr int CCOLS = F >= 256 ? 1 : 256 / F;    // four-buffer columns per block
  static constexpr int NT = 256;
};

// ---------------------------------------------------------------------------
// FIt-SNE interpolation grid: box of a point and its order-3 Lagrange weights
// on the nodes (j + 1/2) / 3 of the unit box (Linderman et al. 2019).
// ---------------------------------------------------------------------------
struct LgPoint {
  int bx, by;
  float ux, uy;  // position inside the box, in box widths
};

// The box is found in fp64, (p - lo) / w correctly rounded, as FIt-SNE does:
// interpolation is discontinuous across box edges, and in fp32 a coordinate
// hundreds of boxes from the corner is only known to ~1e-4 of a box width.
__device__ __forceinline__ LgPoint lg_locate(float px, float py, const DeviceScalars& s) {
#pragma clang fp contract(off)
  const double lo = static_cast<double>(s.lg_lo);
  const double rx = (static_cast<double>(px) - lo) / s.lg_box_wd;
  const double ry = (static_cast<double>(py) - lo) / s.lg_box_wd;
  LgPoint b;
  b.bx = max(0, min(s.lg_boxes - 1, static_cast<int>(floor(rx))));
  b.by = max(0, min(s.lg_boxes - 1, static_cast<int>(floor(ry))));
  b.ux = static_cast<float>(rx - static_cast<double>(b.bx));
  b.uy = static_cast<float>(ry - static_cast<double>(b.by));
  return b;
}

// L_0(u) = (u - 1/2)(u - 5/6) / (2/9), L_1(u) = (u - 1/6)(u - 5/6) / (-1/9),
// L_2(u) = (u - 1/6)(u - 1/2) / (2/9).
__device__ __forceinline__ void lg_weights3(float u, float* w) {
#pragma clang fp contract(off)
  const float a = u - (1.0f / 6.0f);
  const float b = u - 0.5f;
  const float c = u - (5.0f / 6.0f);
  w[0] = 4.5f * (b * c);
  w[1] = -9.0f * (a * c);
  w[2] = 4.5f * (a * b);
}

}  // namespace
}  // namespace fehip
