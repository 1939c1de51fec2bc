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

// Exclusive scans of two arrays held PER consecutive entries per thread by a
// block of NT threads (entry q of thread t is element t * PER + q): the
// thread sums are scanned within each wave by shuffles and across the
// block's waves through part (2 * NT / kWave ints; one barrier).  total_a and
// total_b receive the sums over the block.
template <int PER, int NT>
__device__ __forceinline__ void block_exclusive_scan2(int (&a)[PER], int (&b)[PER], int* part, int& total_a,
                                                      int& total_b) {
  constexpr int kWaves = NT / kWave;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int wave = t / kWave;
  int sa = 0, sb = 0;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    sa += a[q];
    sb += b[q];
  }
  int ia = sa, ib = sb;  // inclusive scans over the wave
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int xa = __shfl_up(ia, off, kWave);
    const int xb = __shfl_up(ib, off, kWave);
    if (lane >= off) {
      ia += xa;
      ib += xb;
    }
  }
  if (lane == kWave - 1) {
    part[wave] = ia;
    part[kWaves + wave] = ib;
  }
  __syncthreads();
  int ba = 0, bb = 0;  // the sums of the waves before this one
  total_a = 0;
  total_b = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) {
      ba += part[w];
      bb += part[kWaves + w];
    }
    total_a += part[w];
    total_b += part[kWaves + w];
  }
  int ra = ba + ia - sa, rb = bb + ib - sb;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int ca = a[q], cb = b[q];
    a[q] = ra;
    b[q] = rb;
    ra += ca;
    rb += cb;
  }
}

// ---------------------------------------------------------------------------
// LDS Stockham FFT
//
// NSEQ sequences of length F = 2^a or 3 * 2^a in LDS, transformed in place
// by NT threads.  One radix-3 stage first when 3 divides F, then radix-16
// stages while 16 divides what is left, then one stage of radix 8, 4 or 2
// for the rest (F = 2048: 16, 16, 8; 768: 3, 16, 16).  A stage of radix R
// entered after Ns points are transformed (Ns = the product of the earlier
// radices) takes, for each j < F / R, the inputs j + r F / R, twiddles them
// by e^{-2 pi i r k / (Ns R)} with k = j mod Ns, and writes their R-point DFT
// (taken in registers) to (j - k) R + k + r Ns, so the result is in natural
// order.  Every stage reads its inputs to registers, barriers, then writes.
// Twiddles e^{-2 pi i j / F}, j < F / 2, are staged in LDS from the global
// table (computed in fp64 on the host), the other half taken by negation;
// INV conjugates them and leaves the result unscaled.
//
// LDS layout: sequence q starts at q * FftPad<F>::kStride and element i sits
// at i + i / 32 (fft_at): one pad element per 32 keeps the strided writes of
// the early stages (stride R elements) from falling into one LDS bank.
// ---------------------------------------------------------------------------
template <int F>
struct FftPad {
  static constexpr int kStride = F + F / 32;
};
__device__ __forceinline__ int fft_pad(int i) { return i + (i >> 5); }
template <int F>
__device__ __forceinline__ int fft_at(int q, int i) {
  return q * FftPad<F>::kStride + fft_pad(i);
}

// e^{-2 pi i m / F} (forward) or its conjugate, m < F, from the half table
// tw[j] = e^{-2 pi i j / F}, j < F / 2 (e^{-2 pi i (j + F/2) / F} = -tw[j]).
template <bool INV, int F>
__device__ __forceinline__ float2 twiddle(const float2* __restrict__ tw, int m) {
  const bool hi = m >= F / 2;
  const float2 w = tw[hi ? m - F / 2 : m];
  const float sx = hi ? -1.0f : 1.0f;
  return make_float2(sx * w.x, (INV ? -sx : sx) * w.y);
}

// Copies the F / 2 twiddles e^{-2 pi i j / F}, j < F / 2, of the global table
// into LDS (the caller's next barrier publishes them; twiddle() makes the
// other half by negation); transforms then read their twiddles from LDS
// (TWS = 1) instead of from the cache hierarchy.  Half a table keeps the
// transforms' LDS small enough to fit beside other kernels' workgroups.
template <int F, int NT>
__device__ __forceinline__ void stage_twiddles(float2* lds_tw, const float2* __restrict__ tw) {
  constexpr bool kR3 = F % 3 == 0;
  constexpr int BASE = kR3 ? kTwiddlePow2 : 0;
  constexpr int LEN = kR3 ? kTwiddlePow3 : kTwiddlePow2;
  static_assert(LEN % F == 0, "F divides its part of the twiddle table");
  constexpr int STRIDE = LEN / F;
  for (int j = threadIdx.x; j < F / 2; j += NT) lds_tw[j] = tw[BASE + j * STRIDE];
}

template <int F>
struct FftRadices {
  static constexpr bool kR3 = F % 3 == 0;
  static constexpr int kPow2 = kR3 ? F / 3 : F;
  static_assert(kPow2 >= 4 && (kPow2 & (kPow2 - 1)) == 0, "F = 2^a or 3 * 2^a");
};

// The first stage when 3 divides F (Ns = 1: no twiddles).  With
// c = cos(2 pi / 3) = -1/2 and s = sin(2 pi / 3), the DFT of (a, b, d) is
// (a + b + d, a + c (b + d) -+ i s (b - d), a + c (b + d) +- i s (b - d)),
// the upper signs forward.
template <int F, int NSEQ, int NT, bool INV>
__device__ __forceinline__ void fft_stage_r3(float2* s) {
  constexpr int T = F / 3;
  constexpr int TOT = NSEQ * T;
  constexpr int BPT = (TOT + NT - 1) / NT;
  constexpr float kSin = 0.866025403784438646763723f;
  float2 v[BPT][3];
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    const int t = threadIdx.x + b * NT;
    if (TOT % NT == 0 || t < TOT) {
      const int q = t / T;
      const int j = t - q * T;
#pragma unroll
      for (int r = 0; r < 3; ++r) v[b][r] = s[fft_at<F>(q, j + r * T)];
      const float2 sum = cadd(v[b][1], v[b][2]);
      const float2 dif = csub(v[b][1], v[b][2]);
      const float2 mid = make_float2(v[b][0].x - 0.5f * sum.x, v[b][0].y - 0.5f * sum.y);
      // forward: -i s (b - d), inverse: +i s (b - d)
      const float2 rot = INV ? make_float2(-kSin * dif.y, kSin * dif.x) : make_float2(kSin * dif.y, -kSin * dif.x);
      v[b][0] = cadd(v[b][0], sum);
      v[b][1] = cadd(mid, rot);
      v[b][2] = csub(mid, rot);
    }
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    const int t = threadIdx.x + b * NT;
    if (TOT % NT == 0 || t < TOT) {
      const int q = t / T;
      const int j = t - q * T;
#pragma unroll
      for (int r = 0; r < 3; ++r) s[fft_at<F>(q, 3 * j + r)] = v[b][r];
    }
  }
  __syncthreads();
}

// -i v (forward) or +i v (inverse).
template <bool INV>
__device__ __forceinline__ float2 rot_i(float2 v) {
  return INV ? make_float2(-v.y, v.x) : make_float2(v.y, -v.x);
}

// 4-point DFT in place, natural order.
template <bool INV>
__device__ __forceinline__ void dft4(float2& a0, float2& a1, float2& a2, float2& a3) {
  const float2 a = cadd(a0, a2);
  const float2 c = csub(a0, a2);
  const float2 d = cadd(a1, a3);
  const float2 e = rot_i<INV>(csub(a1, a3));
  a0 = cadd(a, d);
  a1 = cadd(c, e);
  a2 = csub(a, d);
  a3 = csub(c, e);
}

// e^{-2 pi i m / N} (forward) or its conjugate, m < N, for the radix-8 and
// radix-16 DFTs' internal twiddles (exact constants).
template <bool INV>
__device__ __forceinline__ float2 w16(int m) {
  constexpr float c1 = 0.923879532511286756128f;  // cos(pi / 8)
  constexpr float s1 = 0.382683432365089771728f;  // sin(pi / 8)
  constexpr float h = 0.707106781186547524401f;   // cos(pi / 4)
  float2 w;
  switch (m) {
    case 1: w = make_float2(c1, -s1); break;
    case 2: w = make_float2(h, -h); break;
    case 3: w = make_float2(s1, -c1); break;
    case 6: w = make_float2(-h, -h); break;
    case 9: w = make_float2(-c1, s1); break;
    default: w = make_float2(1.0f, 0.0f); break;
  }
  return INV ? make_float2(w.x, -w.y) : w;
}

// R-point DFT in registers (R = 2, 4, 8, 16).  With n = (R / 4) n1 + n2 and
// k = k1 + 4 k2: 4-point DFTs over n1, twiddles e^{-2 pi i n2 k1 / R}, then
// (R / 4)-point DFTs over n2.  X[k] ends in v[dft_slot<R>(k)].
template <int R>
__device__ __forceinline__ constexpr int dft_slot(int k) {
  return R <= 4 ? k : (R / 4) * (k & 3) + (k >> 2);
}
template <int R, bool INV>
__device__ __forceinline__ void dft_r(float2 (&v)[R]) {
  if constexpr (R == 2) {
    const float2 a = v[0];
    v[0] = cadd(a, v[1]);
    v[1] = csub(a, v[1]);
  } else if constexpr (R == 4) {
    dft4<INV>(v[0], v[1], v[2], v[3]);
  } else if constexpr (R == 8) {
    dft4<INV>(v[0], v[2], v[4], v[6]);
    dft4<INV>(v[1], v[3], v[5], v[7]);
    v[3] = cmul(v[3], w16<INV>(2));  // e^{-2 pi i / 8}
    v[5] = rot_i<INV>(v[5]);         // e^{-2 pi i 2 / 8}
    v[7] = cmul(v[7], w16<INV>(6));  // e^{-2 pi i 3 / 8}
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) {
      const float2 a = v[2 * k1];
      v[2 * k1] = cadd(a, v[2 * k1 + 1]);
      v[2 * k1 + 1] = csub(a, v[2 * k1 + 1]);
    }
  } else {
    static_assert(R == 16, "radix 2, 4, 8 or 16");
#pragma unroll
    for (int n2 = 0; n2 < 4; ++n2) dft4<INV>(v[n2], v[4 + n2], v[8 + n2], v[12 + n2]);
#pragma unroll
    for (int k1 = 1; k1 < 4; ++k1) {
#pragma unroll
      for (int n2 = 1; n2 < 4; ++n2) {
        float2& x = v[4 * k1 + n2];
        x = (n2 * k1 == 4) ? rot_i<INV>(x) : cmul(x, w16<INV>(n2 * k1));
      }
    }
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) dft4<INV>(v[4 * k1], v[4 * k1 + 1], v[4 * k1 + 2], v[4 * k1 + 3]);
  }
}

// One radix-R stage from Ns = NS.
template <int R, int F, int NS, int NSEQ, int NT, bool INV, int TWS>
__device__ __forceinline__ void fft_stage(float2* s, const float2* __restrict__ tw) {
  constexpr int Q = F / R;
  constexpr int TOT = NSEQ * Q;
  constexpr int BPT = (TOT + NT - 1) / NT;
  float2 v[BPT][R];
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    const int t = threadIdx.x + b * NT;
    if (TOT % NT == 0 || t < TOT) {
      const int q = t / Q;
      const int j = t - q * Q;
#pragma unroll
      for (int r = 0; r < R; ++r) v[b][r] = s[fft_at<F>(q, j + r * Q)];
      if constexpr (NS > 1) {
        const int kk = static_cast<int>(static_cast<unsigned int>(j) % NS);
        const int step = (F / (R * NS)) * kk * TWS;
#pragma unroll
        for (int r = 1; r < R; ++r) v[b][r] = cmul(v[b][r], twiddle<INV, F * TWS>(tw, r * step));
      }
      dft_r<R, INV>(v[b]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < BPT; ++b) {
    const int t = threadIdx.x + b * NT;
    if (TOT % NT == 0 || t < TOT) {
      const int q = t / Q;
      const int j = t - q * Q;
      const int kk = static_cast<int>(static_cast<unsigned int>(j) % NS);
      const int base = (j - kk) * R + kk;
#pragma unroll
      for (int r = 0; r < R; ++r) s[fft_at<F>(q, base + r * NS)] = v[b][dft_slot<R>(r)];
    }
  }
  __syncthreads();
}

// The power-of-two stages from Ns = NS: radix 16 while 16 divides F / Ns,
// then one stage of what is left (8, 4 or 2).
template <int F, int NS, int NSEQ, int NT, bool INV, int TWS>
__device__ __forceinline__ void fft_stages_pow2(float2* s, const float2* __restrict__ tw) {
  constexpr int REM = F / NS;
  if constexpr (REM > 1) {
    constexpr int R = REM % 16 == 0 ? 16 : REM;
    static_assert(R == 16 || R == 8 || R == 4 || R == 2, "radix plan ends at F");
    fft_stage<R, F, NS, NSEQ, NT, INV, TWS>(s, tw);
    fft_stages_pow2<F, NS * R, NSEQ, NT, INV, TWS>(s, tw);
  }
}

// tw holds e^{-2 pi i j / (F * TWS)} for j < F * TWS / 2 (staged in LDS by
// stage_twiddles: TWS = 1).  s holds NSEQ sequences in the fft_at layout.
template <int F, int NSEQ, int NT, bool INV, int TWS = 1>
__device__ __forceinline__ void fft_lds(float2* s, const float2* __restrict__ tw) {
  if constexpr (FftRadices<F>::kR3) {
    fft_stage_r3<F, NSEQ, NT, INV>(s);
    fft_stages_pow2<F, 3, NSEQ, NT, INV, TWS>(s, tw);
  } else {
    fft_stages_pow2<F, 1, NSEQ, NT, INV, TWS>(s, tw);
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
// The quotient is taken as q0 = x (1/w), then q0 + r (1/w) with the exact
// remainder r = x - q0 w (FMA): with 1/w correctly rounded and q0 within an
// ulp, that is the correctly rounded x / w (Markstein, IBM J. Res. Dev. 34,
// 111 (1990)) for any x that does not underflow, and x here is 0 or a
// difference of two floats (|x| >= 2^-149, a normal double).  Three fp64
// operations instead of the ~10 of the division sequence; checked equal to
// the IEEE division on 2e8 random and 1.4e7 near-multiple pairs.
__device__ __forceinline__ double lg_box_quotient(double x, const DeviceScalars& s) {
  const double q0 = x * s.lg_inv_box_wd;
  const double r = fma(-q0, s.lg_box_wd, x);
  return fma(r, s.lg_inv_box_wd, q0);
}
__device__ __forceinline__ LgPoint lg_locate(float px, float py, const DeviceScalars& s) {
#pragma clang fp contract(off)
  const double lo = static_cast<double>(s.lg_lo);
  const double rx = lg_box_quotient(static_cast<double>(px) - lo, s);
  const double ry = lg_box_quotient(static_cast<double>(py) - lo, s);
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
