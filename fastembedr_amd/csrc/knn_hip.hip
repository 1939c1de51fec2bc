// Exact k-nearest neighbours (Euclidean) on gfx950 (CDNA4), producing the
// device-resident KNN contract of the reference's GPU route
// (src/native_knn_cuda_impl.cpp:427-466: column-major query-by-k, 1-based
// int32 indices, float32 distances, self excluded on request).  The
// reference's exact route is a third-party brute force (cuVS / FAISS GPU,
// src/native_knn_cuda_impl.cpp:549, :704) finished by
// src/embedding_cuda_kernels.cpp:1412-1464 (k + 1 searched, self dropped,
// sqrt of the squared L2 distance); its tests define exact KNN as a dense
// squared-distance matrix ordered per row, ties by index
// (tests/testthat/helper-knn.R:5-38).
//
// Three steps, all on the device:
//  1. prep: column means in fp64, centred copy of the data padded to an even
//     width (xc, fp32), squared norms of the centred rows and their maximum.
//  2. scan (k_knn_scan, MFMA-bound): a workgroup holds 128 queries (32 per
//     wave) in LDS and streams every reference in tiles of 64 through LDS.
//     v_mfma_f32_32x32x2f32 gives 32 x 32 dot products per wave and step;
//     d2 = |q|^2 + |r|^2 - 2 q.r.  Each query keeps a threshold (the kp-th
//     smallest d2 seen so far, +inf until kp were seen) and a candidate
//     buffer of B entries in global memory; a wave owns its 32 queries, so
//     slots come from ballots, not atomics.  When a buffer could overflow in
//     the next tile, the wave sorts it (bitonic, across its 64 lanes) and
//     keeps the kp best.
//  3. finalize (k_knn_finalize): per query, the kp candidates' squared
//     distances are recomputed exactly enough (fp64 differences of the
//     input rows), sorted by (d2, index), and the first k written.  The
//     result is certified when no rejected reference can beat the k-th: every
//     rejected reference had an fp32 d2 >= the final threshold T, and the
//     fp32 expansion is within eps = (D + 12) 2^-23 (|q|^2 + max |r|^2) of
//     the exact value, so T - eps > d2_k suffices.  Uncertified queries are
//     listed for a rerun with a larger kp.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <string>
#include <vector>

#include "device_common.h"
#include "knn_device.h"

namespace fehip {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kKnnThreads = 256;  // 4 waves
constexpr int kKnnWaves = kKnnThreads / kWave;
constexpr int kKnnWaveQueries = 32;
constexpr int kKnnQueryBlock = kKnnWaves * kKnnWaveQueries;  // 128
constexpr int kKnnRefTile = 64;                               // two 32-column MFMA blocks
constexpr int kKnnPitch = kKnnRefTile + 1;                    // LDS row pitch of a reference tile
constexpr int kPrepThreads = 256;

// ---- 1. prep --------------------------------------------------------------------

// partial[b * d + c] = sum over rows [b * rows_per, (b + 1) * rows_per) of x[., c] in fp64.
__global__ __launch_bounds__(kPrepThreads) void k_knn_col_partials(const float* __restrict__ x, int n, int d,
                                                                    Strides st, int rows_per,
                                                                    double* __restrict__ partial) {
  const int r0 = static_cast<int>(blockIdx.x) * rows_per;
  const int r1 = min(n, r0 + rows_per);
  for (int c = threadIdx.x; c < d; c += kPrepThreads) {
    double s = 0.0;
    for (int r = r0; r < r1; ++r) s += static_cast<double>(x[st.at(r, c)]);
    partial[static_cast<long long>(blockIdx.x) * d + c] = s;
  }
}

__global__ __launch_bounds__(kPrepThreads) void k_knn_col_means(const double* __restrict__ partial, int blocks, int d,
                                                                 int n, double* __restrict__ mean) {
  for (int c = threadIdx.x; c < d; c += kPrepThreads) {
    double s = 0.0;
    for (int b = 0; b < blocks; ++b) s += partial[static_cast<long long>(b) * d + c];
    mean[c] = s / static_cast<double>(n);
  }
}

// One row per thread: xc = fl32(x - mean), zero in the padding; the squared
// norm of the stored fp32 row, summed in fp64; the norms' maximum (bits of a
// non-negative float compare as unsigned); rows holding a NaN or an infinity
// (or whose centred norm overflows fp32) are counted in bad_rows.  Rows n to
// n_pad - 1 (the rest of the last 64-row tile) are zero.
__global__ __launch_bounds__(kPrepThreads) void k_knn_center(const float* __restrict__ x, int n, int n_pad, int d,
                                                              Strides st, int D, const double* __restrict__ mean,
                                                              float* __restrict__ xc,
                                                              float* __restrict__ nrm,
                                                              unsigned int* __restrict__ nrm_max_bits,
                                                              int* __restrict__ bad_rows) {
  const int r = static_cast<int>(blockIdx.x) * kPrepThreads + threadIdx.x;
  float local = 0.0f;
  if (r < n) {
    double s = 0.0;
    for (int c = 0; c < D; ++c) {
      const float v = c < d ? static_cast<float>(static_cast<double>(x[st.at(r, c)]) - mean[c]) : 0.0f;
      xc[static_cast<long long>(r) * D + c] = v;
      s += static_cast<double>(v) * static_cast<double>(v);
    }
    local = static_cast<float>(s);
    if (!isfinite(local)) {  // NaN/inf input, or a norm beyond fp32
      atomicAdd(bad_rows, 1);
      local = 0.0f;
    }
    nrm[r] = local;
  } else if (r < n_pad) {  // padding rows of the last reference tile
    for (int c = 0; c < D; ++c) xc[static_cast<long long>(r) * D + c] = 0.0f;
    nrm[r] = 0.0f;
  }
  // wave maximum, then one atomic per wave
  for (int off = kWave / 2; off > 0; off >>= 1) local = fmaxf(local, __shfl_xor(local, off));
  if ((threadIdx.x & (kWave - 1)) == 0) atomicMax(nrm_max_bits, __float_as_uint(local));
}

// ---- sorting inside one wave ------------------------------------------------------
// PER keys per lane; element E = j * 64 + lane (j = register).  Ascending
// bitonic sort of the 64 * PER keys.

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int mask) {
  const int lo = __shfl_xor(static_cast<int>(v & 0xffffffffull), mask);
  const int hi = __shfl_xor(static_cast<int>(v >> 32), mask);
  return (static_cast<unsigned long long>(static_cast<unsigned int>(hi)) << 32) | static_cast<unsigned int>(lo);
}

// The stage loops stay rolled (size and distance are wave-uniform); only
// the per-register work is unrolled, with the in-lane distance a template
// argument so that registers are never indexed at run time.
template <int PER, int JD>
__device__ __forceinline__ void inlane_step_u64(unsigned long long (&key)[PER], int lane, int size) {
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if ((j & JD) == 0) {
      const bool asc = ((j * kWave + lane) & size) == 0;
      const unsigned long long a = key[j], b = key[j | JD];
      const bool swap = asc ? (a > b) : (a < b);
      key[j] = swap ? b : a;
      key[j | JD] = swap ? a : b;
    }
  }
}

template <int PER>
__device__ __forceinline__ void wave_sort_u64(unsigned long long (&key)[PER], int lane) {
  constexpr int N = PER * kWave;
  for (int size = 2; size <= N; size <<= 1) {
    for (int dist = size >> 1; dist > 0; dist >>= 1) {
      if (dist >= kWave) {
        switch (dist / kWave) {
          case 1: if constexpr (PER > 1) inlane_step_u64<PER, 1>(key, lane, size); break;
          case 2: if constexpr (PER > 2) inlane_step_u64<PER, 2>(key, lane, size); break;
          case 4: if constexpr (PER > 4) inlane_step_u64<PER, 4>(key, lane, size); break;
          case 8: if constexpr (PER > 8) inlane_step_u64<PER, 8>(key, lane, size); break;
          default: break;
        }
      } else {
        const bool lower = (lane & dist) == 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const unsigned long long other = shfl_xor_u64(key[j], dist);
          const bool keep_min = lower == (((j * kWave + lane) & size) == 0);
          key[j] = keep_min ? (other < key[j] ? other : key[j]) : (other > key[j] ? other : key[j]);
        }
      }
    }
  }
}

// (d2, index) pairs in fp64 / int: same network, lexicographic order.
template <int PER, int JD>
__device__ __forceinline__ void inlane_step_pairs(double (&d2)[PER], int (&id)[PER], int lane, int size) {
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if ((j & JD) == 0) {
      const bool asc = ((j * kWave + lane) & size) == 0;
      const double a = d2[j], b = d2[j | JD];
      const int ia = id[j], ib = id[j | JD];
      const bool a_gt = a > b || (a == b && ia > ib);
      const bool swap = asc ? a_gt : !a_gt;
      d2[j] = swap ? b : a;
      d2[j | JD] = swap ? a : b;
      id[j] = swap ? ib : ia;
      id[j | JD] = swap ? ia : ib;
    }
  }
}

template <int PER>
__device__ __forceinline__ void wave_sort_pairs(double (&d2)[PER], int (&id)[PER], int lane) {
  constexpr int N = PER * kWave;
  for (int size = 2; size <= N; size <<= 1) {
    for (int dist = size >> 1; dist > 0; dist >>= 1) {
      if (dist >= kWave) {
        switch (dist / kWave) {
          case 1: if constexpr (PER > 1) inlane_step_pairs<PER, 1>(d2, id, lane, size); break;
          case 2: if constexpr (PER > 2) inlane_step_pairs<PER, 2>(d2, id, lane, size); break;
          case 4: if constexpr (PER > 4) inlane_step_pairs<PER, 4>(d2, id, lane, size); break;
          case 8: if constexpr (PER > 8) inlane_step_pairs<PER, 8>(d2, id, lane, size); break;
          default: break;
        }
      } else {
        const bool lower = (lane & dist) == 0;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const double od = __shfl_xor(d2[j], dist);
          const int oi = __shfl_xor(id[j], dist);
          const bool keep_min = lower == (((j * kWave + lane) & size) == 0);
          const bool other_less = od < d2[j] || (od == d2[j] && oi < id[j]);
          const bool take = keep_min ? other_less : !other_less;
          d2[j] = take ? od : d2[j];
          id[j] = take ? oi : id[j];
        }
      }
    }
  }
}

// ---- 2. scan ----------------------------------------------------------------------

__device__ __forceinline__ unsigned long long cand_key(uint2 c) {
  return (static_cast<unsigned long long>(c.x) << 32) | c.y;
}

// Sorts the row's buffer and keeps its kp best (in order at its front);
// returns the new count, and the new threshold through thr when kp were
// seen.
template <int B>
__device__ __noinline__ int compact_row(uint2* __restrict__ row_buf, int cnt, int kp, int lane, float* thr) {
  constexpr int PER = B / kWave;
  // The entries were stored by other lanes of this wave: wait until those
  // stores are done (the CU's L1 is shared by the workgroup).
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  unsigned long long key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    key[j] = e < cnt ? cand_key(row_buf[e]) : ~0ull;
  }
  wave_sort_u64<PER>(key, lane);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    if (e < kp && e < cnt)
      row_buf[e] = make_uint2(static_cast<unsigned int>(key[j] >> 32), static_cast<unsigned int>(key[j]));
  }
  if (cnt >= kp) {
    // element kp - 1 sits in lane (kp - 1) % 64, register (kp - 1) / 64
    unsigned int bits = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (j == (kp - 1) / kWave) bits = static_cast<unsigned int>(key[j] >> 32);
    bits = __shfl(static_cast<int>(bits), (kp - 1) % kWave);
    *thr = __uint_as_float(bits);
  }
  return min(cnt, kp);
}

// Query list position p -> point index.
__device__ __forceinline__ int query_id(const int* __restrict__ qlist, int q_offset, int p) {
  return qlist != nullptr ? qlist[p] : q_offset + p;
}

// A reference tile's values for one thread: elements e = tid + 256 s of the
// 64 x D tile, which is contiguous in the row-padded xc, and the norm of row
// tid (tid < 64).
template <int MAXD>
struct TileRegs {
  float v[MAXD / 4];
  float norm;
};

template <int MAXD>
__device__ __forceinline__ void knn_load_tile(TileRegs<MAXD>& r, const float* __restrict__ xc,
                                              const float* __restrict__ nrm, int t, int D, int tid) {
  const float* const src = xc + static_cast<long long>(t) * kKnnRefTile * D;
#pragma unroll
  for (int s = 0; s < MAXD / 4; ++s) {
    const int e = tid + s * kKnnThreads;
    r.v[s] = e < kKnnRefTile * D ? src[e] : 0.0f;
  }
  r.norm = tid < kKnnRefTile ? nrm[t * kKnnRefTile + tid] : 0.0f;
}

// Where element e = tid + 256 s goes: row e / D and column e % D, stepped
// from (row0, col0) = (tid / D, tid % D) by (256 / D, 256 % D) with a carry,
// so that no division is done per tile.
struct TileWalk {
  int row0, col0, dq, dr;
};

// Transposed into LDS: dst[k * 65 + c] (pitch 65: conflict-free), norms in
// row D.
template <int MAXD>
__device__ __forceinline__ void knn_store_tile(const TileRegs<MAXD>& r, float* dst, int D, const TileWalk& w,
                                               int tid) {
  int row = w.row0, col = w.col0;
#pragma unroll
  for (int s = 0; s < MAXD / 4; ++s) {
    if (tid + s * kKnnThreads < kKnnRefTile * D) dst[col * kKnnPitch + row] = r.v[s];
    row += w.dq;
    col += w.dr;
    if (col >= D) {
      col -= D;
      ++row;
    }
  }
  if (tid < kKnnRefTile) dst[D * kKnnPitch + tid] = r.norm;
}

// Per wave row state in LDS: threshold, count, |q|^2 and point index (-1
// past the list's end) of each of its 32 queries.
struct alignas(16) WaveRows {
  float thr[kKnnWaves][kKnnWaveQueries];
  int cnt[kKnnWaves][kKnnWaveQueries];
  float nq[kKnnWaves][kKnnWaveQueries];
  int qid[kKnnWaves][kKnnWaveQueries];
};

// Each wave owns 32 queries; lane (c32, h) holds coordinates 2 k2 + h of
// query c32 in registers (the A operand of every MFMA step).  A buffer row
// is compacted to its kp best when it could overflow in the next tile
// (cnt > B - 64); the host picks B >= 2 kp + 64 so that compactions are rare.
// Launch bounds: 2 workgroups per CU (2 waves per SIMD, each with two
// independent MFMA chains).
template <int B, int MAXD>
__global__ __launch_bounds__(kKnnThreads, 2) void k_knn_scan(const float* __restrict__ xc, const float* __restrict__ nrm,
                                                          const int* __restrict__ qlist, int q_offset, int nq, int n,
                                                          int D, int kp, int exclude_self, uint2* __restrict__ buf,
                                                          float* __restrict__ thr_out, int* __restrict__ cnt_out) {
  extern __shared__ float smem[];
  float* const rt0 = smem;  // [D][65], then 64 norms in row D
  float* const rt1 = rt0 + (D + 1) * kKnnPitch;
  __shared__ WaveRows rs;
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid & (kWave - 1);
  const int h = lane >> 5;
  const int c32 = lane & 31;
  const int p0 = static_cast<int>(blockIdx.x) * kKnnQueryBlock;  // first list position of the block

  // this lane's query coordinates
  const int p_lane = p0 + wave * kKnnWaveQueries + c32;
  const int q_lane = p_lane < nq ? query_id(qlist, q_offset, p_lane) : -1;
  float a[MAXD / 2];
  {
    const float* const qrow = xc + static_cast<long long>(q_lane >= 0 ? q_lane : 0) * D;
#pragma unroll
    for (int k2 = 0; k2 < MAXD / 2; ++k2) a[k2] = (q_lane >= 0 && 2 * k2 + h < D) ? qrow[2 * k2 + h] : 0.0f;
  }
  if (lane < kKnnWaveQueries) {
    rs.thr[wave][lane] = INFINITY;
    rs.cnt[wave][lane] = 0;
    rs.qid[wave][lane] = q_lane;
    rs.nq[wave][lane] = q_lane >= 0 ? nrm[q_lane] : 0.0f;
  }

  // references in tiles of 64; the next tile's values are loaded into
  // registers while the current one is used
  const int tiles = (n + kKnnRefTile - 1) / kKnnRefTile;
  const TileWalk walk{tid / D, tid % D, kKnnThreads / D, kKnnThreads % D};
  TileRegs<MAXD> pre;
  knn_load_tile<MAXD>(pre, xc, nrm, 0, D, tid);
  knn_store_tile<MAXD>(pre, rt0, D, walk, tid);
  __syncthreads();
  uint2* const wave_buf = buf + static_cast<long long>(p0 + wave * kKnnWaveQueries) * B;
  for (int t = 0; t < tiles; ++t) {
    const float* const cur = (t & 1) ? rt1 : rt0;
    if (t + 1 < tiles) knn_load_tile<MAXD>(pre, xc, nrm, t + 1, D, tid);
    v16f acc0 = {0}, acc1 = {0};
#pragma unroll
    for (int k2 = 0; k2 < MAXD / 2; ++k2) {
      if (2 * k2 >= D) break;  // D is even
      const int k = 2 * k2 + h;
      const float b0 = cur[k * kKnnPitch + c32];
      const float b1 = cur[k * kKnnPitch + 32 + c32];
      acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[k2], b0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a[k2], b1, acc1, 0, 0, 0);
    }
    // filter: candidates below their query's threshold to the query's
    // buffer.  Output i of this lane is row 8 (i / 4) + 4 h + i % 4 of the
    // wave's 32, column c32 of the 32-column block.  (The block loop stays
    // rolled, which keeps the hoisted LDS reads of one block in registers.)
#pragma unroll 1
    for (int b = 0; b < 2; ++b) {
      const int col = t * kKnnRefTile + b * 32 + c32;
      const float nr = cur[D * kKnnPitch + b * 32 + c32];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int row0 = 8 * g + 4 * h;
        const float4 thr4 = *reinterpret_cast<const float4*>(&rs.thr[wave][row0]);
        const float4 nq4 = *reinterpret_cast<const float4*>(&rs.nq[wave][row0]);
        const int4 qid4 = *reinterpret_cast<const int4*>(&rs.qid[wave][row0]);
        const float thr_a[4] = {thr4.x, thr4.y, thr4.z, thr4.w};
        const float nq_a[4] = {nq4.x, nq4.y, nq4.z, nq4.w};
        const int qid_a[4] = {qid4.x, qid4.y, qid4.z, qid4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = 4 * g + u;
          const float dot = b == 0 ? acc0[i] : acc1[i];
          const float d2 = fmaxf(fmaf(-2.0f, dot, nq_a[u] + nr), 0.0f);
          const bool pass =
              qid_a[u] >= 0 && col < n && d2 < thr_a[u] && !(exclude_self && col == qid_a[u]);
          const unsigned long long m = __ballot(pass);
          if (m != 0ull) {
            const int row = row0 + u;
            const unsigned int half = h ? static_cast<unsigned int>(m >> 32) : static_cast<unsigned int>(m);
            const int base = rs.cnt[wave][row];
            if (pass)
              wave_buf[static_cast<long long>(row) * B + base + __popc(half & ((1u << c32) - 1u))] =
                  make_uint2(__float_as_uint(d2), static_cast<unsigned int>(col));
            if (c32 == 0) rs.cnt[wave][row] = base + __popc(half);
          }
        }
      }
    }
    // rows that could overflow in the next tile: sort, keep kp
    unsigned long long need = __ballot(lane < kKnnWaveQueries && rs.cnt[wave][c32] > B - kKnnRefTile);
    while (need != 0ull) {
      const int r = __ffsll(static_cast<long long>(need)) - 1;
      need &= need - 1ull;
      float thr = rs.thr[wave][r];
      const int c = compact_row<B>(wave_buf + static_cast<long long>(r) * B, rs.cnt[wave][r], kp, lane, &thr);
      if (lane == 0) {
        rs.cnt[wave][r] = c;
        rs.thr[wave][r] = thr;
      }
    }
    __syncthreads();  // every wave is done with the tile it read
    if (t + 1 < tiles) knn_store_tile<MAXD>(pre, (t & 1) ? rt0 : rt1, D, walk, tid);
    __syncthreads();
  }
  // final: keep kp per row; the threshold is what a rejected reference beat
  for (int r = 0; r < kKnnWaveQueries; ++r) {
    const int p = p0 + wave * kKnnWaveQueries + r;
    if (p >= nq) break;  // wave-uniform
    float thr = rs.thr[wave][r];
    int c = rs.cnt[wave][r];
    if (c > kp) c = compact_row<B>(wave_buf + static_cast<long long>(r) * B, c, kp, lane, &thr);
    if (lane == 0) {
      thr_out[p] = thr;
      cnt_out[p] = c;
    }
  }
}

// ---- 3. finalize -------------------------------------------------------------------

// One wave per query: exact squared distances of the candidates from the
// input rows (fp64), sorted by (d2, index); the first k are written as
// 1-based indices and float distances, column-major (neighbour j of point
// q at j * n + q).  Uncertified queries are appended to retry.
template <int B>
__global__ __launch_bounds__(kKnnThreads) void k_knn_finalize(
    const float* __restrict__ x, int n, int d, Strides st, const int* __restrict__ qlist, int q_offset, int nq,
    const uint2* __restrict__ buf, const float* __restrict__ thr_in, const int* __restrict__ cnt_in,
    const float* __restrict__ nrm, const unsigned int* __restrict__ nrm_max_bits, float eps_unit, int k,
    int* __restrict__ idx_out, float* __restrict__ dist_out, int* __restrict__ retry, int* __restrict__ retry_count,
    int* __restrict__ short_rows) {
  constexpr int PER = B / kWave;
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const int p = static_cast<int>(blockIdx.x) * kKnnWaves + static_cast<int>(threadIdx.x) / kWave;
  if (p >= nq) return;  // whole wave
  const int q = query_id(qlist, q_offset, p);
  const int c = cnt_in[p];
  const uint2* cand = buf + static_cast<long long>(p) * B;
  double dd[PER];
  int id[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    dd[j] = INFINITY;
    id[j] = 0x7fffffff;
    if (e < c) {
      const int r = static_cast<int>(cand[e].y);
      double s = 0.0;
      for (int t = 0; t < d; ++t) {
        const double diff = static_cast<double>(x[st.at(q, t)]) - static_cast<double>(x[st.at(r, t)]);
        s = fma(diff, diff, s);
      }
      dd[j] = s;
      id[j] = r;
    }
  }
  wave_sort_pairs<PER>(dd, id, lane);
  double d2k = 0.0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = j * kWave + lane;
    if (e < k && e < c) {
      idx_out[static_cast<long long>(e) * n + q] = id[j] + 1;
      dist_out[static_cast<long long>(e) * n + q] = static_cast<float>(sqrt(dd[j]));
    }
    if (j == (k - 1) / kWave) d2k = dd[j];
  }
  d2k = __shfl(d2k, (k - 1) % kWave);
  if (lane == 0) {
    if (c < k) {
      atomicAdd(short_rows, 1);
    } else {
      const float thr = thr_in[p];
      if (thr < INFINITY) {
        const double eps = static_cast<double>(eps_unit) *
                           (static_cast<double>(nrm[q]) + static_cast<double>(__uint_as_float(*nrm_max_bits)));
        if (!(static_cast<double>(thr) - eps > d2k)) retry[atomicAdd(retry_count, 1)] = q;
      }
    }
  }
}

// Everything one scan + finalize pass over a list of queries needs.
struct KnnPass {
  const float* x;  // input rows (strides st)
  Strides st;
  const float* xc;  // centred, padded rows (n x D)
  const float* nrm;
  const unsigned int* nrm_max_bits;
  int n, d, D, k, exclude_self;
  uint2* buf;  // candidate buffers, nq x B
  float* thr;
  int* cnt;
  int* idx_out;
  float* dist_out;
  int* retry;        // uncertified point indices
  int* retry_count;  // counters[0]
  int* short_rows;   // counters[1]
};

template <int B, int MAXD>
hipError_t launch_scan(const KnnPass& a, int kp, const int* qlist, int q_offset, int nq, hipStream_t stream) {
  const std::size_t lds = 2 * static_cast<std::size_t>(a.D + 1) * kKnnPitch * sizeof(float);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_knn_scan<B, MAXD>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (e != hipSuccess) return e;
  const int blocks = (nq + kKnnQueryBlock - 1) / kKnnQueryBlock;
  k_knn_scan<B, MAXD><<<blocks, kKnnThreads, lds, stream>>>(a.xc, a.nrm, qlist, q_offset, nq, a.n, a.D, kp,
                                                            a.exclude_self, a.buf, a.thr, a.cnt);
  return hipGetLastError();
}

template <int B>
hipError_t launch_scan_finalize(const KnnPass& a, int kp, const int* qlist, int q_offset, int nq,
                                hipStream_t stream) {
  static_assert(kKnnMaxDim <= 128, "a thread prefetches at most 32 values of a 64-row tile");
  hipError_t e = a.D <= 64 ? launch_scan<B, 64>(a, kp, qlist, q_offset, nq, stream)
                           : launch_scan<B, 128>(a, kp, qlist, q_offset, nq, stream);
  if (e != hipSuccess) return e;
  const float eps_unit = static_cast<float>(a.D + 12) * 0x1.0p-23f;
  k_knn_finalize<B><<<(nq + kKnnWaves - 1) / kKnnWaves, kKnnThreads, 0, stream>>>(
      a.x, a.n, a.d, a.st, qlist, q_offset, nq, a.buf, a.thr, a.cnt, a.nrm, a.nrm_max_bits, eps_unit, a.k, a.idx_out,
      a.dist_out, a.retry, a.retry_count, a.short_rows);
  return hipGetLastError();
}

// Candidate count kp of a query: k plus a margin of max(32, k / 2) on the
// first pass, doubled for every rerun, at most kKnnMaxCand.
constexpr int kKnnMaxCand = 1024 - 2 * kKnnRefTile;  // 896

// Smallest buffer with room for kp entries plus at least kp new ones (and a
// tile's 64) between compactions; 1024 for the largest kp.
int buffer_for(int kp) {
  for (int B = 128; B <= 1024; B <<= 1)
    if (B - kKnnRefTile >= 2 * kp) return B;
  return 1024;
}

hipError_t launch_pass(const KnnPass& a, int kp, const int* qlist, int q_offset, int nq, hipStream_t stream) {
#define FEHIP_KNN_PASS(B_) \
  case B_:                 \
    return launch_scan_finalize<B_>(a, kp, qlist, q_offset, nq, stream);
  switch (buffer_for(kp)) {
    FEHIP_KNN_PASS(128)
    FEHIP_KNN_PASS(256)
    FEHIP_KNN_PASS(512)
    FEHIP_KNN_PASS(1024)
    default:
      return hipErrorInvalidValue;
  }
#undef FEHIP_KNN_PASS
}

template <typename T>
struct DevBuf {
  T* p = nullptr;
  hipError_t alloc(std::size_t count) {
    return hipMalloc(reinterpret_cast<void**>(&p), std::max<std::size_t>(count, 1) * sizeof(T));
  }
  ~DevBuf() {
    if (p != nullptr) (void)hipFree(p);
  }
};

}  // namespace

int knn_exact_run(const float* x_in, int n, int d, int x_col_major, int k, int exclude_self, int input_on_device,
                  int* idx_out_in, float* dist_out_in, int output_on_device, long long* stats, std::string& err) {
  auto fail = [&](const std::string& what, hipError_t e) {
    err = what + ": " + hipGetErrorString(e);
    return 1;
  };
  if (x_in == nullptr || idx_out_in == nullptr || dist_out_in == nullptr) {
    err = "null KNN pointer";
    return 1;
  }
  if (n < 2 || d < 1 || k < 1) {
    err = "invalid KNN dimensions (need n >= 2, d >= 1, k >= 1)";
    return 1;
  }
  if (d > kKnnMaxDim) {
    err = "exact KNN supports up to " + std::to_string(kKnnMaxDim) + " dimensions";
    return 1;
  }
  if (k > kKnnMaxK) {
    err = "exact KNN supports k up to " + std::to_string(kKnnMaxK);
    return 1;
  }
  if (k > n - (exclude_self ? 1 : 0)) {
    err = "k exceeds the number of " + std::string(exclude_self ? "non-self " : "") + "neighbors";
    return 1;
  }
  if (n > INT_MAX - kKnnRefTile) {
    err = "exact KNN supports fewer than 2^31 - 64 rows";
    return 1;
  }
  const int D = (d + 1) / 2 * 2;
  const int n_pad = (n + kKnnRefTile - 1) / kKnnRefTile * kKnnRefTile;  // whole reference tiles
  hipStream_t stream = nullptr;
  hipError_t e;
  DevBuf<float> x_dev, xc, nrm, dist_dev;
  DevBuf<double> partial, mean;
  DevBuf<unsigned int> nrm_max;
  DevBuf<int> idx_dev, retry, counters;
  const float* x = x_in;
  if (!input_on_device) {
    if ((e = x_dev.alloc(static_cast<std::size_t>(n) * d)) != hipSuccess) return fail("hipMalloc(KNN input)", e);
    if ((e = hipMemcpy(x_dev.p, x_in, static_cast<std::size_t>(n) * d * sizeof(float), hipMemcpyHostToDevice)) !=
        hipSuccess)
      return fail("hipMemcpy(KNN input)", e);
    x = x_dev.p;
  }
  int* idx_out = idx_out_in;
  float* dist_out = dist_out_in;
  if (!output_on_device) {
    if ((e = idx_dev.alloc(static_cast<std::size_t>(n) * k)) != hipSuccess) return fail("hipMalloc(KNN indices)", e);
    if ((e = dist_dev.alloc(static_cast<std::size_t>(n) * k)) != hipSuccess)
      return fail("hipMalloc(KNN distances)", e);
    idx_out = idx_dev.p;
    dist_out = dist_dev.p;
  }
  const int rows_per = 4096;
  const int pblocks = (n + rows_per - 1) / rows_per;
  if ((e = xc.alloc(static_cast<std::size_t>(n_pad) * D)) != hipSuccess || (e = nrm.alloc(n_pad)) != hipSuccess ||
      (e = partial.alloc(static_cast<std::size_t>(pblocks) * d)) != hipSuccess || (e = mean.alloc(d)) != hipSuccess ||
      (e = nrm_max.alloc(1)) != hipSuccess || (e = retry.alloc(n)) != hipSuccess ||
      (e = counters.alloc(3)) != hipSuccess)
    return fail("hipMalloc(KNN scratch)", e);
  // counters: [0] uncertified rows, [1] rows with fewer than k candidates,
  // [2] rows with non-finite values
  if ((e = hipMemsetAsync(counters.p, 0, 3 * sizeof(int), stream)) != hipSuccess ||
      (e = hipMemsetAsync(nrm_max.p, 0, sizeof(unsigned int), stream)) != hipSuccess)
    return fail("hipMemset", e);
  const Strides st = x_col_major ? Strides{1, n} : Strides{d, 1};
  k_knn_col_partials<<<pblocks, kPrepThreads, 0, stream>>>(x, n, d, st, rows_per, partial.p);
  k_knn_col_means<<<1, kPrepThreads, 0, stream>>>(partial.p, pblocks, d, n, mean.p);
  k_knn_center<<<(n_pad + kPrepThreads - 1) / kPrepThreads, kPrepThreads, 0, stream>>>(
      x, n, n_pad, d, st, D, mean.p, xc.p, nrm.p, nrm_max.p, counters.p + 2);
  if ((e = hipGetLastError()) != hipSuccess) return fail("KNN prep launch", e);
  {
    int bad = 0;
    if ((e = hipMemcpyAsync(&bad, counters.p + 2, sizeof(int), hipMemcpyDeviceToHost, stream)) != hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
      return fail("KNN prep", e);
    if (bad != 0) {
      err = "exact KNN input has " + std::to_string(bad) +
            " rows with non-finite values (or a centred squared norm beyond the fp32 range)";
      return 1;
    }
  }

  // queries in batches (the candidate buffers are batch x B entries)
  int kp = std::min(kKnnMaxCand, k + std::max(32, k / 2));
  const int batch = std::min(n, kKnnBatch);
  DevBuf<uint2> buf;
  DevBuf<float> thr;
  DevBuf<int> cnt;
  if ((e = buf.alloc(static_cast<std::size_t>(batch) * 1024)) != hipSuccess || (e = thr.alloc(batch)) != hipSuccess ||
      (e = cnt.alloc(batch)) != hipSuccess)
    return fail("hipMalloc(KNN candidates)", e);
  KnnPass pass{x,      st,     xc.p,    nrm.p,    nrm_max.p, n,       d,           D,
               k,      exclude_self, buf.p, thr.p, cnt.p, idx_out, dist_out, retry.p,
               counters.p, counters.p + 1};
  for (int q0 = 0; q0 < n; q0 += batch) {
    const int nq = std::min(batch, n - q0);
    if ((e = launch_pass(pass, kp, nullptr, q0, nq, stream)) != hipSuccess) return fail("KNN scan launch", e);
  }
  int host_counts[2] = {0, 0};
  long long retried = 0;
  int passes = 1;
  for (;;) {
    if ((e = hipMemcpyAsync(host_counts, counters.p, sizeof(host_counts), hipMemcpyDeviceToHost, stream)) !=
            hipSuccess ||
        (e = hipStreamSynchronize(stream)) != hipSuccess)
      return fail("KNN pass", e);
    if (host_counts[1] != 0) {
      err = "exact KNN found fewer candidates than k for " + std::to_string(host_counts[1]) + " rows";
      return 1;
    }
    if (host_counts[0] == 0) break;
    if (kp == kKnnMaxCand) {
      err = "exact KNN could not certify " + std::to_string(host_counts[0]) + " rows: more than " +
            std::to_string(kKnnMaxCand) + " points lie within fp32 resolution of their k-th neighbour distance";
      return 1;
    }
    // rerun the uncertified rows with twice the candidates
    retried += host_counts[0];
    ++passes;
    kp = std::min(kKnnMaxCand, 2 * kp);
    DevBuf<int> list;
    const int nr = host_counts[0];
    if ((e = list.alloc(nr)) != hipSuccess) return fail("hipMalloc(KNN retry)", e);
    if ((e = hipMemcpyAsync(list.p, retry.p, nr * sizeof(int), hipMemcpyDeviceToDevice, stream)) != hipSuccess ||
        (e = hipMemsetAsync(counters.p, 0, 2 * sizeof(int), stream)) != hipSuccess)
      return fail("KNN retry setup", e);
    for (int q0 = 0; q0 < nr; q0 += batch) {
      const int nq = std::min(batch, nr - q0);
      if ((e = launch_pass(pass, kp, list.p + q0, 0, nq, stream)) != hipSuccess) return fail("KNN retry launch", e);
    }
    if ((e = hipStreamSynchronize(stream)) != hipSuccess) return fail("KNN retry", e);
  }
  if (!output_on_device) {
    if ((e = hipMemcpy(idx_out_in, idx_out, static_cast<std::size_t>(n) * k * sizeof(int),
                       hipMemcpyDeviceToHost)) != hipSuccess ||
        (e = hipMemcpy(dist_out_in, dist_out, static_cast<std::size_t>(n) * k * sizeof(float),
                       hipMemcpyDeviceToHost)) != hipSuccess)
      return fail("hipMemcpy(KNN output)", e);
  } else if ((e = hipStreamSynchronize(stream)) != hipSuccess) {
    return fail("KNN sync", e);
  }
  if (stats != nullptr) {
    stats[0] = retried;
    stats[1] = passes;
    stats[2] = kp;
  }
  return 0;
}

}  // namespace fehip
