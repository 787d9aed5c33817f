// Small per-theta kernels around the integrator:
//   affine   A = B theta          (replaces torch.sparse.mm, cpab/pytorch/transformer.py:84)
//   expm     Trels = expm(dT A)   (cpab_ops_1d.cu:404-429, 2d.cu:537-653, 3d.cu:538-674)
//   affine + expm in one pass (the forward's table setup)
//   project  dtheta = B^T vec(M)  (replaces torch.sparse.mm, transformer.py:165-166)
//   adjoint table   G = h A + (h^2/2) A^2 per cell (the factored reverse step);
//            also clears the HBM sums and dense-part masks the backward fills
//   finish   moments from the per-cell sums S of the reverse sweep: the HBM
//            sums plus the dense per-workgroup partial tables
//   sum      grad_points.sum(0)   (transformer.py:151-152)
// These are latency-sized (µs) next to the integrator; they exist so the
// whole path stays on HIP with fixed, reproducible summation orders.
#include <hip/hip_runtime.h>
#include <math.h>
#include <algorithm>
#include "cpab_device.hpp"
#include "cpab_launch.hpp"

namespace cpab {

namespace {

__global__ void fill_kernel(float* __restrict__ dst, int64_t n, float value) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = value;
}

// One thread per (theta, row of B): As[b, r] = sum_k B[r, col_k] * theta[b, col_k],
// summed in ascending column order (the order of a coalesced CSR row).
__global__ void affine_kernel(int64_t n_theta, int rows, int d, const float* __restrict__ theta,
                              const int32_t* __restrict__ row_ptr,
                              const int32_t* __restrict__ col_idx,
                              const float* __restrict__ vals, float* __restrict__ As) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n_theta * rows) return;
  const int64_t b = i / rows;
  const int r = (int)(i - b * rows);
  const float* th = theta + b * d;
  float acc = 0.0f;
  for (int k = row_ptr[r]; k < row_ptr[r + 1]; ++k) acc = fmaf(vals[k], th[col_idx[k]], acc);
  As[i] = acc;
}

// grad[b, j] = sum_k B[row_k, j] * M[b, row_k] over the CSC column j of B,
// added in ascending k with one fma per entry (a fixed order).  Each column is
// served by kProjSeg lanes: they load its entries and gather the moments
// together (a column of the 3D basis has up to 80 entries, and walking it
// entry by entry from one lane made the projection a chain of dependent
// memory round trips), stage the (value, moment) pairs in LDS, and the
// segment's first lane adds them in order.  Columns longer than kProjCap
// entries take several rounds.
constexpr int kProjSeg = 16;                        // lanes per column
constexpr int kProjThreads = 256;
constexpr int kProjCols = kProjThreads / kProjSeg;  // columns per workgroup
constexpr int kProjCap = 128;                       // entries staged per round

__global__ __launch_bounds__(kProjThreads) void project_kernel(
    int64_t n_theta, int D, int d, const float* __restrict__ M, const int32_t* __restrict__ col_ptr,
    const int32_t* __restrict__ row_idx, const float* __restrict__ vals, float* __restrict__ grad) {
  constexpr int PER = kProjCap / kProjSeg;  // entries per lane per round
  __shared__ float2 stage[kProjCols][kProjCap];
  const int seg = threadIdx.x / kProjSeg, lane = threadIdx.x % kProjSeg;
  const int64_t i = blockIdx.x * (int64_t)kProjCols + seg;
  const bool live = i < n_theta * d;
  const int64_t b = live ? i / d : 0;
  const int j = live ? (int)(i - b * d) : 0;
  const float* m = M + b * D;
  const int k0 = live ? col_ptr[j] : 0, k1 = live ? col_ptr[j + 1] : 0;
  // rounds: uniform over the workgroup (its longest column decides)
  int rounds = (k1 - k0 + kProjCap - 1) / kProjCap;
  __shared__ int max_rounds;
  if (threadIdx.x == 0) max_rounds = 0;
  __syncthreads();
  if (lane == 0 && rounds > 0) atomicMax(&max_rounds, rounds);
  __syncthreads();
  rounds = max_rounds;
  float acc = 0.0f;
  for (int r = 0; r < rounds; ++r) {
    const int base = k0 + r * kProjCap;
    if (base < k1) {
      // Every load is issued from an in-range index (entries past the column
      // end re-read its last entry) and masked afterwards, so a lane's loads
      // are independent of each other.
      int idx[PER];
      float v[PER], mv[PER];
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int k = min(base + lane + u * kProjSeg, k1 - 1);
        idx[u] = row_idx[k];
        v[u] = vals[k];
      }
#pragma unroll
      for (int u = 0; u < PER; ++u) mv[u] = m[idx[u]];
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const bool ok = base + lane + u * kProjSeg < k1;
        stage[seg][lane + u * kProjSeg] = make_float2(ok ? v[u] : 0.0f, ok ? mv[u] : 0.0f);
      }
    }
    __syncthreads();
    if (lane == 0 && base < k1) {
      const int n = min(kProjCap, k1 - base);
      int k = 0;
      for (; k + 4 <= n; k += 4) {
        const float2 e0 = stage[seg][k], e1 = stage[seg][k + 1];
        const float2 e2 = stage[seg][k + 2], e3 = stage[seg][k + 3];
        acc = fmaf(e0.x, e0.y, acc);
        acc = fmaf(e1.x, e1.y, acc);
        acc = fmaf(e2.x, e2.y, acc);
        acc = fmaf(e3.x, e3.y, acc);
      }
      for (; k < n; ++k) acc = fmaf(stage[seg][k].x, stage[seg][k].y, acc);
    }
    __syncthreads();
  }
  if (live && lane == 0) grad[i] = acc;
}

// Reverse-sweep table.  Each workgroup of kTableThreads covers one block of
// one row's cells (row = blockIdx.x / nblk, block = blockIdx.x % nblk), one
// thread per cell: the entry of the cell (cpab_device.hpp, RevStride):
// G = h A_lin + (h^2/2) A_lin^2 (adjoint_increment) and the inverse one-step
// map (inverse_step_map); the cell's sums zeroed.  The workgroup's largest
// ||M_c||_2 of the inverse maps (inverse_map_norm) goes to amp[blockIdx.x]:
// the backward reads a row's nblk entries to bound how much the recovered
// positions' rounding can grow.  Thread i of the grid also clears
// dense_parts[i] for i < n_words.  2D, ebound not null: the block's part of
// the domain-edge bound of the replay's explicit-midpoint maps
// (cpab_device.hpp, edge_bound_cell_2d) goes to ebound[blockIdx.x] (alpha,
// beta, reach, err); the backward merges a row's nblk parts into its delta_T.
constexpr int kTableThreads = 256;

template <int D>
__global__ __launch_bounds__(kTableThreads) void adjoint_table_kernel(
    int64_t rows, int nC, int nblk, float h, int nx, int ny, const float* __restrict__ As,
    float* __restrict__ G, float* __restrict__ moments, float* __restrict__ amp,
    EdgeAcc* __restrict__ ebound, uint64_t* __restrict__ dense_parts, int64_t n_words) {
  constexpr int P = D * (D + 1);
  constexpr int S = RevStride<D>::S;
  // Entry layout (cpab_device.hpp, RevStride): G at G0, the inverse map's
  // rows (D + 1 floats each) from I0.
  constexpr int G0 = D == 3 ? 12 : 0;
  constexpr int I0 = D == 3 ? 0 : D * D;
  __shared__ float wave_max[kTableThreads / 64];
  __shared__ EdgeAcc wave_edge[kTableThreads / 64];
  const bool edges = D == 2 && ebound != nullptr;
  EdgeAcc edge;
  edge.init();
  const int64_t lin = blockIdx.x * (int64_t)kTableThreads + threadIdx.x;
  if (lin < n_words) dense_parts[lin] = 0;
  const int64_t row = blockIdx.x / nblk;
  const int c = (int)(blockIdx.x - row * nblk) * kTableThreads + (int)threadIdx.x;
  float norm = 0.0f;
  if (row < rows && c < nC) {
    const int64_t i = row * nC + c;
    float a[P], e[S], inv[P];
#pragma unroll
    for (int k = 0; k < S; ++k) e[k] = 0.0f;
#pragma unroll
    for (int k = 0; k < P; ++k) a[k] = As[i * P + k];
    adjoint_increment<D>(a, h, (h * 0.5f) * h, e + G0);
    if (D == 2 && edges) {
      double mm[2][3];
      midpoint_map_2d(a, h, mm);
      edge_bound_cell_2d(mm, c, nx, ny, midpoint_step_err(a, h, h * 0.5f), edge);
    }
    inverse_step_map<D>(a, h, inv);
    norm = inverse_map_norm<D>(inv);
#pragma unroll
    for (int k = 0; k < P; ++k) e[I0 + k] = inv[k];
#pragma unroll
    for (int k = 0; k < S; ++k) G[i * S + k] = e[k];
#pragma unroll
    for (int k = 0; k < P; ++k) moments[i * P + k] = 0.0f;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) norm = fmaxf(norm, __shfl_xor(norm, off));
  if (edges) edge.wave_merge();
  if ((threadIdx.x & 63) == 0) {
    wave_max[threadIdx.x >> 6] = norm;
    if (edges) wave_edge[threadIdx.x >> 6] = edge;
  }
  __syncthreads();
  if (threadIdx.x == 0 && row < rows) {
    float m = wave_max[0];
#pragma unroll
    for (int w = 1; w < kTableThreads / 64; ++w) m = fmaxf(m, wave_max[w]);
    amp[blockIdx.x] = m;
    if (edges) {
      EdgeAcc acc = wave_edge[0];
#pragma unroll
      for (int w = 1; w < kTableThreads / 64; ++w) acc.merge(wave_edge[w]);
      ebound[blockIdx.x] = acc;
    }
  }
}

// Moments of every (row, cell) from the sums of the reverse sweep.  One
// workgroup covers kFinCells<D> cells of one row (blockIdx.x = row * nblk +
// block), one thread per (cell, component): S = the HBM sum in `moments` plus
// partials[row, w, cell] for every part w set in the row's dense-part mask,
// added in ascending w (a fixed order), the parts' loads issued in batches;
// then S and the cell's A go through LDS and each thread forms its component
// of the moments (cpab_device.hpp, moments_from_s), in place.  Consecutive
// threads read consecutive floats of each partial table.
template <int D> constexpr int kFinCells = 256 / (D * (D + 1));

// DET: S from the deterministic reduction's integer sums, divided by the row's
// scale 2^det_shift, or +inf / -inf / NaN where the component's flags record
// non-finite values, in place of the HBM float sums and partials.
template <int D, bool DET = false>
__global__ __launch_bounds__(256) void finish_moments_kernel(
    int64_t rows, int nC, int nblk, int nparts, float h, const float* __restrict__ partials,
    const uint64_t* __restrict__ dense_parts, const float* __restrict__ As,
    float* __restrict__ moments, const unsigned* __restrict__ det_stat,
    const unsigned long long* __restrict__ det_sums, const unsigned* __restrict__ det_flags,
    int64_t det_nP, int det_T) {
  constexpr int P = D * (D + 1);
  constexpr int W = D + 1;
  constexpr int CB = kFinCells<D>;
  __shared__ float s_lds[CB * P], a_lds[CB * P];
  const int64_t row = blockIdx.x / nblk;
  const int c0 = (int)(blockIdx.x - row * nblk) * CB;
  const int t = threadIdx.x;
  const int cl = t / P, comp = t - cl * P;
  const bool live = t < CB * P && c0 + cl < nC;
  const int64_t idx = (row * nC + c0 + cl) * P + comp;   // this thread's float of the row's table
  if (live && DET) {
    const int shift = det_shift(det_stat[row], det_nP, det_T);
    const unsigned f = det_flags[idx];
    s_lds[t] = f == 0u ? (float)ldexp((double)(long long)det_sums[idx], -shift)
                       : (f == 1u ? INFINITY : f == 2u ? -INFINITY : NAN);
    a_lds[t] = As[idx];
  } else if (live) {
    float s = moments[idx];
    if (nparts > 0) {
      const int64_t R = (int64_t)nC * P;
      const int NW = (nparts + 63) / 64;
      const float* src = partials + row * nparts * R + (int64_t)(c0 + cl) * P + comp;
      constexpr int U = 16;
      for (int q = 0; q < NW; ++q) {
        uint64_t bits = dense_parts[row * NW + q];
        while (bits) {
          float x[U];
          bool on[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            on[u] = bits != 0;
            const int w = on[u] ? q * 64 + __builtin_ctzll(bits) : 0;
            bits &= bits - 1;
            x[u] = on[u] ? src[w * R] : 0.0f;
          }
#pragma unroll
          for (int u = 0; u < U; ++u)
            if (on[u]) s += x[u];
        }
      }
    }
    s_lds[t] = s;
    a_lds[t] = As[idx];
  }
  __syncthreads();
  if (!live) return;
  const float* s_ = s_lds + cl * P;
  const float* a_ = a_lds + cl * P;
  const int k = comp / W, q = comp - k * W;
  const float hhh = (h * 0.5f) * h;
  float tt = 0.0f;
  if (q < D) {
#pragma unroll
    for (int r = 0; r < W; ++r) tt = fmaf(s_[k * W + r], a_[q * W + r], tt);
  }
#pragma unroll
  for (int j = 0; j < D; ++j) tt = fmaf(a_[j * W + k], s_[j * W + q], tt);
  moments[idx] = fmaf(h, s_[comp], hhh * tt);
}

// dst[i] = sum_b src[b, i], b ascending.
__global__ void sum_batch_kernel(int64_t n_theta, int64_t n, const float* __restrict__ src,
                                 float* __restrict__ dst) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float acc = 0.0f;
    for (int64_t b = 0; b < n_theta; ++b) acc += src[b * n + i];
    dst[i] = acc;
  }
}

// ---- matrix exponentials of dT*[A; 0] (affine, last row zero) -------------

// One cell's exponential: A is the row-major [D, D+1] block, out the same
// shape.  1D: [exp(m), m01 * (exp(m) - 1) / m].
__device__ __forceinline__ void expm_cell2(const float* A, float dT, float* out) {
  const float m00 = dT * A[0], m01 = dT * A[1];
  float exprel;
  if (fabsf(m00) > 1e-6f) {
    exprel = expm1_cr(m00) / m00;
  } else {
    const float m2 = m00 * m00;
    exprel = fmaf((1.0f / 24.0f) * m2, m00, fmaf(1.0f / 6.0f, m2, fmaf(0.5f, m00, 1.0f)));
  }
  out[0] = exp_cr(m00);
  out[1] = m01 * exprel;
}

__device__ __forceinline__ int n_squarings(float norm) {
  return (norm > 0.5f) ? (int)ceilf(log2f(norm * 2.0f)) : 0;
}

// Pade(3,3) with scaling and squaring: R = Q^{-1} P, P/Q = I +- M/2 + M^2/12.
__device__ __forceinline__ void expm_cell3(const float* A, float dT, float* o) {
  const float a00 = dT * A[0], a01 = dT * A[1], a02 = dT * A[2];
  const float a10 = dT * A[3], a11 = dT * A[4], a12 = dT * A[5];
  float nsq = fmaf(a00, a00, a01 * a01);
  nsq = fmaf(a02, a02, nsq);
  nsq = fmaf(a10, a10, nsq);
  nsq = fmaf(a11, a11, nsq);
  nsq = fmaf(a12, a12, nsq);
  const int ns = n_squarings(sqrtf(nsq));
  float sc = 1.0f;
  for (int k = 0; k < ns; ++k) sc *= 0.5f;
  const float m00 = a00 * sc, m01 = a01 * sc, m02 = a02 * sc;
  const float m10 = a10 * sc, m11 = a11 * sc, m12 = a12 * sc;
  const float s00 = fmaf(m00, m00, m01 * m10), s01 = fmaf(m00, m01, m01 * m11);
  const float s02 = fmaf(m00, m02, m01 * m12), s10 = fmaf(m10, m00, m11 * m10);
  const float s11 = fmaf(m10, m01, m11 * m11), s12 = fmaf(m10, m02, m11 * m12);
  const float c12 = 1.0f / 12.0f;
  const float p00 = fmaf(c12, s00, fmaf(0.5f, m00, 1.0f)), p01 = fmaf(0.5f, m01, c12 * s01);
  const float p02 = fmaf(0.5f, m02, c12 * s02), p10 = fmaf(0.5f, m10, c12 * s10);
  const float p11 = fmaf(c12, s11, fmaf(0.5f, m11, 1.0f)), p12 = fmaf(0.5f, m12, c12 * s12);
  const float q00 = fmaf(c12, s00, fmaf(-0.5f, m00, 1.0f)), q01 = fmaf(-0.5f, m01, c12 * s01);
  const float q02 = fmaf(-0.5f, m02, c12 * s02), q10 = fmaf(-0.5f, m10, c12 * s10);
  const float q11 = fmaf(c12, s11, fmaf(-0.5f, m11, 1.0f)), q12 = fmaf(-0.5f, m12, c12 * s12);
  const float det = fmaf(q00, q11, -(q01 * q10));
  const float id = 1.0f / det;
  const float i00 = q11 * id, i01 = (-q01) * id, i10 = (-q10) * id, i11 = q00 * id;
  const float i02 = -fmaf(i00, q02, i01 * q12);
  const float i12 = -fmaf(i10, q02, i11 * q12);
  float r00 = fmaf(i00, p00, i01 * p10), r01 = fmaf(i00, p01, i01 * p11);
  float r02 = fmaf(i00, p02, i01 * p12) + i02;
  float r10 = fmaf(i10, p00, i11 * p10), r11 = fmaf(i10, p01, i11 * p11);
  float r12 = fmaf(i10, p02, i11 * p12) + i12;
  for (int k = 0; k < ns; ++k) {
    const float n00 = fmaf(r00, r00, r01 * r10), n01 = fmaf(r00, r01, r01 * r11);
    const float n02 = fmaf(r00, r02, r01 * r12) + r02;
    const float n10 = fmaf(r10, r00, r11 * r10), n11 = fmaf(r10, r01, r11 * r11);
    const float n12 = fmaf(r10, r02, r11 * r12) + r12;
    r00 = n00; r01 = n01; r02 = n02; r10 = n10; r11 = n11; r12 = n12;
  }
  o[0] = r00; o[1] = r01; o[2] = r02; o[3] = r10; o[4] = r11; o[5] = r12;
}

// (x1*y1 + x2*y2) + x3*y3 with the first product of the pair fused, then the third.
__device__ __forceinline__ float dot3(float x1, float y1, float x2, float y2, float x3, float y3) {
  return fmaf(x3, y3, fmaf(x1, y1, x2 * y2));
}
// x1*y1 - x2*y2 with the left product fused.
__device__ __forceinline__ float cross2(float x1, float y1, float x2, float y2) {
  return fmaf(x1, y1, -(x2 * y2));
}

__device__ __forceinline__ void expm_cell4(const float* A, float dT, float* o) {
  float a[12];
#pragma unroll
  for (int k = 0; k < 12; ++k) a[k] = dT * A[k];
  float nsq = fmaf(a[0], a[0], a[1] * a[1]);
#pragma unroll
  for (int k = 2; k < 12; ++k) nsq = fmaf(a[k], a[k], nsq);
  const int ns = n_squarings(sqrtf(nsq));
  float sc = 1.0f;
  for (int k = 0; k < ns; ++k) sc *= 0.5f;
  float m[3][4];
#pragma unroll
  for (int r = 0; r < 3; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) m[r][c] = a[4 * r + c] * sc;
  // M^2: linear block and translation column.
  float s[3][3], t[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      s[r][c] = dot3(m[r][0], m[0][c], m[r][1], m[1][c], m[r][2], m[2][c]);
    t[r] = dot3(m[r][0], m[0][3], m[r][1], m[1][3], m[r][2], m[2][3]);
  }
  const float c12 = 1.0f / 12.0f;
  float p[3][3], q[3][3], pt[3], qt[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      if (r == c) {
        p[r][c] = fmaf(c12, s[r][c], fmaf(0.5f, m[r][c], 1.0f));
        q[r][c] = fmaf(c12, s[r][c], fmaf(-0.5f, m[r][c], 1.0f));
      } else {
        p[r][c] = fmaf(0.5f, m[r][c], c12 * s[r][c]);
        q[r][c] = fmaf(-0.5f, m[r][c], c12 * s[r][c]);
      }
    }
    pt[r] = fmaf(0.5f, m[r][3], c12 * t[r]);
    qt[r] = fmaf(-0.5f, m[r][3], c12 * t[r]);
  }
  // Adjugate / determinant of the 3x3 block of Q.
  const float c00 = cross2(q[1][1], q[2][2], q[1][2], q[2][1]);
  const float c10 = cross2(q[1][0], q[2][2], q[1][2], q[2][0]);
  const float c20 = cross2(q[1][0], q[2][1], q[1][1], q[2][0]);
  const float det = fmaf(q[0][2], c20, fmaf(q[0][0], c00, -(q[0][1] * c10)));
  const float id = 1.0f / det;
  float qi[3][3];
  qi[0][0] = c00 * id;
  qi[0][1] = cross2(q[0][2], q[2][1], q[0][1], q[2][2]) * id;
  qi[0][2] = cross2(q[0][1], q[1][2], q[0][2], q[1][1]) * id;
  qi[1][0] = cross2(q[1][2], q[2][0], q[1][0], q[2][2]) * id;
  qi[1][1] = cross2(q[0][0], q[2][2], q[0][2], q[2][0]) * id;
  qi[1][2] = cross2(q[0][2], q[1][0], q[0][0], q[1][2]) * id;
  qi[2][0] = c20 * id;
  qi[2][1] = cross2(q[0][1], q[2][0], q[0][0], q[2][1]) * id;
  qi[2][2] = cross2(q[0][0], q[1][1], q[0][1], q[1][0]) * id;
  float qit[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) qit[r] = -dot3(qi[r][0], qt[0], qi[r][1], qt[1], qi[r][2], qt[2]);
  float R[3][4];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
#pragma unroll
    for (int c = 0; c < 3; ++c)
      R[r][c] = dot3(qi[r][0], p[0][c], qi[r][1], p[1][c], qi[r][2], p[2][c]);
    R[r][3] = dot3(qi[r][0], pt[0], qi[r][1], pt[1], qi[r][2], pt[2]) + qit[r];
  }
  for (int k = 0; k < ns; ++k) {
    float N[3][4];
#pragma unroll
    for (int r = 0; r < 3; ++r) {
#pragma unroll
      for (int c = 0; c < 3; ++c)
        N[r][c] = dot3(R[r][0], R[0][c], R[r][1], R[1][c], R[r][2], R[2][c]);
      N[r][3] = dot3(R[r][0], R[0][3], R[r][1], R[1][3], R[r][2], R[2][3]) + R[r][3];
    }
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) R[r][c] = N[r][c];
  }
#pragma unroll
  for (int r = 0; r < 3; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) o[4 * r + c] = R[r][c];
}

template <int D> __device__ __forceinline__ void expm_cell(const float* A, float dT, float* o);
template <> __device__ __forceinline__ void expm_cell<1>(const float* A, float dT, float* o) { expm_cell2(A, dT, o); }
template <> __device__ __forceinline__ void expm_cell<2>(const float* A, float dT, float* o) { expm_cell3(A, dT, o); }
template <> __device__ __forceinline__ void expm_cell<3>(const float* A, float dT, float* o) { expm_cell4(A, dT, o); }

// One thread per cell matrix: Trels[i] = expm(dT * As[i]).
template <int D>
__global__ void expm_kernel(int64_t n, float dT, const float* __restrict__ As,
                            float* __restrict__ out) {
  constexpr int P = D * (D + 1);
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  float a[P], r[P];
#pragma unroll
  for (int k = 0; k < P; ++k) a[k] = As[i * P + k];
  expm_cell<D>(a, dT, r);
#pragma unroll
  for (int k = 0; k < P; ++k) out[i * P + k] = r[k];
}

// A = B theta and Trels = expm(dT A) in one launch.  A workgroup covers
// kAffCells<D> consecutive (theta, cell) matrices: first one thread per row of
// A forms it exactly as affine_kernel does (summed in ascending column order)
// and stores it (coalesced) and into LDS; then one thread per cell
// exponentiates its block as expm_kernel does and the results leave through
// LDS, coalesced.  Both outputs equal the two-kernel sequence bit for bit.
template <int D> constexpr int kAffCells = D == 1 ? 128 : (D == 2 ? 64 : 32);

template <int D>
__global__ __launch_bounds__(kAffCells<D> * D * (D + 1)) void affine_expm_kernel(
    int64_t n_theta, int nC, int d, const float* __restrict__ theta,
    const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ col_idx,
    const float* __restrict__ vals, float dT, float* __restrict__ As, float* __restrict__ Trels) {
  constexpr int P = D * (D + 1);
  constexpr int CB = kAffCells<D>;
  __shared__ float tile[CB * P];
  const int64_t n = n_theta * nC * P;                  // rows of A in all
  const int64_t base = (int64_t)blockIdx.x * CB * P;   // first row of this block
  const int t = threadIdx.x;
  const int64_t g = base + t;
  if (g < n) {
    const int64_t b = g / ((int64_t)nC * P);
    const int row = (int)(g - b * nC * P);
    const float* th = theta + b * d;
    float acc = 0.0f;
    for (int k = row_ptr[row]; k < row_ptr[row + 1]; ++k) acc = fmaf(vals[k], th[col_idx[k]], acc);
    As[g] = acc;
    tile[t] = acc;
  }
  __syncthreads();
  if (t < CB && base + (int64_t)t * P < n) {
    float a[P], r[P];
#pragma unroll
    for (int k = 0; k < P; ++k) a[k] = tile[t * P + k];
    expm_cell<D>(a, dT, r);
#pragma unroll
    for (int k = 0; k < P; ++k) tile[t * P + k] = r[k];  // only this thread uses these slots
  }
  __syncthreads();
  if (g < n) Trels[g] = tile[t];
}

inline unsigned grid_for(int64_t n, int block) {
  int64_t g = (n + block - 1) / block;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace

hipError_t launch_fill(float* dst, int64_t n, float value, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(fill_kernel, dim3((unsigned)g), dim3(256), 0, s, dst, n, value);
  return hipGetLastError();
}

hipError_t launch_affine(int64_t n_theta, int rows, int d, const float* theta,
                         const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                         float* As, hipStream_t s) {
  const int64_t n = n_theta * rows;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(affine_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, n_theta, rows, d,
                     theta, row_ptr, col_idx, vals, As);
  return hipGetLastError();
}

hipError_t launch_expm(int ndim, int64_t n, float dT, const float* As, float* Trels,
                       hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const dim3 g(grid_for(n, 256)), b(256);
  if (ndim == 1) hipLaunchKernelGGL(expm_kernel<1>, g, b, 0, s, n, dT, As, Trels);
  else if (ndim == 2) hipLaunchKernelGGL(expm_kernel<2>, g, b, 0, s, n, dT, As, Trels);
  else hipLaunchKernelGGL(expm_kernel<3>, g, b, 0, s, n, dT, As, Trels);
  return hipGetLastError();
}

hipError_t launch_affine_expm(int ndim, int64_t n_theta, int nC, int d, const float* theta,
                              const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                              float dT, float* As, float* Trels, hipStream_t s) {
  const int64_t n = n_theta * nC;
  if (n <= 0) return hipSuccess;
  auto go = [&](auto kernel, int cells, int P) {
    const dim3 g((unsigned)((n + cells - 1) / cells)), b((unsigned)(cells * P));
    hipLaunchKernelGGL(kernel, g, b, 0, s, n_theta, nC, d, theta, row_ptr, col_idx, vals, dT, As,
                       Trels);
  };
  if (ndim == 1) go(affine_expm_kernel<1>, kAffCells<1>, 2);
  else if (ndim == 2) go(affine_expm_kernel<2>, kAffCells<2>, 6);
  else go(affine_expm_kernel<3>, kAffCells<3>, 12);
  return hipGetLastError();
}

hipError_t launch_project(int64_t n_theta, int D, int d, const float* moments,
                          const int32_t* col_ptr, const int32_t* row_idx, const float* vals,
                          float* grad_theta, hipStream_t s) {
  const int64_t n = n_theta * d;
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(project_kernel, dim3(grid_for(n, kProjCols)), dim3(kProjThreads), 0, s,
                     n_theta, D, d, moments, col_ptr, row_idx, vals, grad_theta);
  return hipGetLastError();
}

int adjoint_table_blocks(int nC) { return (nC + kTableThreads - 1) / kTableThreads; }

hipError_t launch_adjoint_table(int ndim, int64_t rows, int nx, int ny, int nC, int T,
                                const float* As, float* G, float* moments, float* amp,
                                EdgeAcc* ebound, uint64_t* dense_parts, int64_t n_words,
                                hipStream_t s) {
  if (rows <= 0 || nC <= 0) return hipSuccess;
  const float h = 1.0f / (float)T;
  const int nblk = adjoint_table_blocks(nC);
  // Enough workgroups for one per (row, cell block) and one thread per mask word.
  const int64_t blocks = std::max<int64_t>(rows * nblk, (n_words + kTableThreads - 1) / kTableThreads);
  const dim3 g((unsigned)blocks), b(kTableThreads);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, g, b, 0, s, rows, nC, nblk, h, nx, ny, As, G, moments, amp,
                       ndim == 2 ? ebound : nullptr, dense_parts, n_words);
  };
  if (ndim == 1) go(adjoint_table_kernel<1>);
  else if (ndim == 2) go(adjoint_table_kernel<2>);
  else go(adjoint_table_kernel<3>);
  return hipGetLastError();
}

hipError_t launch_finish_moments(int ndim, int64_t rows, int nC, int nparts, int T,
                                 const float* partials, const uint64_t* dense_parts,
                                 const float* As, float* moments, hipStream_t s) {
  if (rows <= 0 || nC <= 0) return hipSuccess;
  const float h = 1.0f / (float)T;
  auto go = [&](auto kernel, int cb) {
    const int nblk = (nC + cb - 1) / cb;
    hipLaunchKernelGGL(kernel, dim3((unsigned)(rows * nblk)), dim3(256), 0, s, rows, nC, nblk,
                       nparts, h, partials, dense_parts, As, moments, nullptr, nullptr, nullptr,
                       (int64_t)0, 0);
  };
  if (ndim == 1) go(finish_moments_kernel<1>, kFinCells<1>);
  else if (ndim == 2) go(finish_moments_kernel<2>, kFinCells<2>);
  else go(finish_moments_kernel<3>, kFinCells<3>);
  return hipGetLastError();
}

hipError_t launch_finish_moments_det(int ndim, int64_t rows, int nC, int64_t nP, int T,
                                     const unsigned* det_stat, const unsigned long long* det_sums,
                                     const unsigned* det_flags, const float* As, float* moments,
                                     hipStream_t s) {
  if (rows <= 0 || nC <= 0) return hipSuccess;
  const float h = 1.0f / (float)T;
  auto go = [&](auto kernel, int cb) {
    const int nblk = (nC + cb - 1) / cb;
    hipLaunchKernelGGL(kernel, dim3((unsigned)(rows * nblk)), dim3(256), 0, s, rows, nC, nblk, 0,
                       h, nullptr, nullptr, As, moments, det_stat, det_sums, det_flags, nP, T);
  };
  if (ndim == 1) go(finish_moments_kernel<1, true>, kFinCells<1>);
  else if (ndim == 2) go(finish_moments_kernel<2, true>, kFinCells<2>);
  else go(finish_moments_kernel<3, true>, kFinCells<3>);
  return hipGetLastError();
}

hipError_t launch_sum_batch(int64_t n_theta, int64_t n, const float* src, float* dst,
                            hipStream_t s) {
  if (n <= 0) return hipSuccess;
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(sum_batch_kernel, dim3((unsigned)g), dim3(256), 0, s, n_theta, n, src, dst);
  return hipGetLastError();
}

}  // namespace cpab
