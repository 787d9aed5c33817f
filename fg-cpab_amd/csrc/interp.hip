// transform_data gather: border-clamped linear / bilinear / trilinear sampling
// and its backward (cpab/pytorch/interpolation.py:3-159 plus the torch
// autograd backward of those ops).
//
// Index conventions of the reference: grid coordinate k scales by
// (data.shape[2+k] - 1) and indexes data axis 2+k; the warped grid lists points
// with coordinate 0 fastest, p = i0 + o0*(i1 + o1*i2); the output is
// [B, C, o0, o1(, o2)] with the LAST axis fastest.  So the point order and the
// output order are transposes of each other.  HBM-bound, so each workgroup
// takes a kT0 x kTL tile over (i0, i_last) at fixed i_mid, reads the grid rows
// coalesced along i0 into LDS, and computes/writes with i_last across the
// lanes (whole 128-byte output lines and, for smooth warps, near-contiguous
// data rows).
// The backward does the same transpose in the other direction for grad_grid.
// The per-sample arithmetic lives in cpab_sample.hpp.
#include <hip/hip_runtime.h>
#include <math.h>
#include "cpab_launch.hpp"
#include "cpab_sample.hpp"

namespace cpab {
namespace {

constexpr int kT0 = kInterpTile0;      // tile extent along i0 (grid rows are contiguous in i0)
constexpr int kTL = kInterpTileLast;   // tile extent along i_last (output rows are contiguous in i_last)
constexpr int kThreads = kInterpThreads;
static_assert(kThreads % kTL == 0 && kT0 % 4 == 0 && 64 % kTL == 0 && kT0 % (kThreads / kTL) == 0,
              "tile shape");
constexpr int kRows = kThreads / kTL;   // tile rows (along i0) a workgroup covers per pass
constexpr int kPerLane = kT0 / kRows;   // outputs per lane in a whole tile
// Outputs per lane whose gathers the backward issues together (4 corner-pair
// loads in flight per lane).  Larger batches cost occupancy: with the pairs,
// batches of 4 (2D) and 2 (3D) ran the C3 backward 14% and the C4 backward 8%
// slower.
constexpr int gather_batch(int nd) { return nd == 3 ? 1 : 2; }
static_assert(kPerLane % gather_batch(2) == 0 && kPerLane % gather_batch(3) == 0, "batches");
constexpr int kXcds = 8;     // MI355X: accelerator complex dies, each with its own L2

struct Shape {
  int ndim;
  int B, C;
  int in[3];     // data spatial sizes
  int o0, omid, olast;
  int64_t nP;
  int vec4;      // grid rows are 16-byte aligned along i0 (o0 % 4 == 0)
  int tiles0, tilesl;  // tiles along i0 and i_last
};

// Tile of this workgroup, XCD-aware.  The hardware hands consecutive
// workgroup ids to the 8 XCDs in turn, and each XCD has its own L2; the
// remap gives XCD x the x-th eighth of the tile list, so an XCD works through
// whole images (tiles ordered i0 tile, then i_last tile, then b * omid + i_mid)
// and the gathers of one image share that XCD's L2.  Returns false for the
// padding workgroups past the last tile.
__device__ __forceinline__ bool tile_origin(const Shape& s, int& b, int& im, int& t0, int& tl) {
  const int64_t total = (int64_t)s.tiles0 * s.tilesl * s.B * s.omid;
  const int64_t per = (total + kXcds - 1) / kXcds;
  const int64_t n = (int64_t)(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  if (n >= total) return false;
  const int64_t plane = (int64_t)s.tiles0 * s.tilesl;
  const int z = (int)(n / plane);
  const int r = (int)(n - (int64_t)z * plane);
  const int ty = r / s.tiles0;
  b = z / s.omid;
  im = z - b * s.omid;
  t0 = (r - ty * s.tiles0) * kT0;
  tl = ty * kTL;
  return true;
}

// Grid rows of this tile -> LDS crd[k][al][a0] (lanes along i0, float4 when aligned).
template <int ND>
__device__ __forceinline__ void load_tile(const Shape& s, const float* __restrict__ grid, int b,
                                          int im, int t0, int tl, int n0, int nl,
                                          float (*crd)[kTL][kT0 + 1]) {
  const int64_t row0 = (int64_t)s.o0 * (im + (int64_t)s.omid * tl) + t0;  // point of (t0, tl)
  const int64_t rstride = (int64_t)s.o0 * s.omid;                        // next i_last
  if (s.vec4 && n0 == kT0) {
    constexpr int Q = kT0 / 4;
    for (int e = threadIdx.x; e < Q * kTL; e += kThreads) {
      const int q = e % Q, al = e / Q;
      if (al < nl) {
#pragma unroll
        for (int k = 0; k < ND; ++k) {
          const float4 v = *reinterpret_cast<const float4*>(
              grid + ((int64_t)b * ND + k) * s.nP + row0 + al * rstride + 4 * q);
          crd[k][al][4 * q] = v.x;
          crd[k][al][4 * q + 1] = v.y;
          crd[k][al][4 * q + 2] = v.z;
          crd[k][al][4 * q + 3] = v.w;
        }
      }
    }
  } else {
    for (int e = threadIdx.x; e < kT0 * kTL; e += kThreads) {
      const int a0 = e % kT0, al = e / kT0;
      if (a0 < n0 && al < nl) {
#pragma unroll
        for (int k = 0; k < ND; ++k)
          crd[k][al][a0] = grid[((int64_t)b * ND + k) * s.nP + row0 + al * rstride + a0];
      }
    }
  }
}

template <int ND>
__global__ __launch_bounds__(kThreads) void interp_fwd_kernel(Shape s,
                                                              const float* __restrict__ data,
                                                              const float* __restrict__ grid,
                                                              float* __restrict__ out) {
  __shared__ float crd[ND][kTL][kT0 + 1];
  int b, im, t0, tl;
  if (!tile_origin(s, b, im, t0, tl)) return;
  const int n0 = min(kT0, s.o0 - t0), nl = min(kTL, s.olast - tl);
  load_tile<ND>(s, grid, b, im, t0, tl, n0, nl, crd);
  __syncthreads();
  const int al = threadIdx.x % kTL;   // lanes along i_last
  const int w = threadIdx.x / kTL;    // kRows rows at a time
  const int64_t plane_in = (int64_t)s.in[0] * s.in[1] * (ND == 3 ? s.in[2] : 1);
  const int64_t plane_out = (int64_t)s.o0 * s.omid * s.olast;
  const int64_t ostride = (int64_t)s.omid * s.olast;   // next i0 in the output
  const bool pairs = s.in[ND - 1] >= 2;                // corners read in pairs
  if (al >= nl) return;
  if (n0 == kT0) {
    // Whole tile along i0, software-pipelined: the corner loads of a lane's
    // next output are issued before the current output is blended and stored.
    for (int ch = 0; ch < s.C; ++ch) {
      const int64_t bc = (int64_t)b * s.C + ch;
      const ChannelBuf d(data + bc * plane_in, plane_in);
      float* __restrict__ o = out + bc * plane_out + (int64_t)(t0 + w) * ostride +
                              (int64_t)im * s.olast + tl + al;
      Axis ax[2], ay[2], az[2];
      float c[2][1 << ND];
#pragma unroll
      for (int j = -1; j < kPerLane; ++j) {
        if (j + 1 < kPerLane) {
          const int n = (j + 1) & 1;
          const int a0 = w + (j + 1) * kRows;
          ax[n] = axis_of(crd[0][al][a0], s.in[0]);
          ay[n] = axis_of(crd[1][al][a0], s.in[1]);
          az[n] = ND == 3 ? axis_of(crd[ND - 1][al][a0], s.in[2]) : Axis{0, 0, 0.0f};
          if (pairs) gather_pairs<ND>(s.in, d, ax[n], ay[n], az[n], c[n]);
          else gather<ND>(s.in, d, ax[n], ay[n], az[n], c[n]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (j >= 0) {
          const int k = j & 1;
          o[j * kRows * ostride] = blend<ND>(c[k], ax[k], ay[k], az[k]);
        }
      }
    }
    return;
  }
  for (int ch = 0; ch < s.C; ++ch) {
    const int64_t bc = (int64_t)b * s.C + ch;
    const float* __restrict__ d = data + bc * plane_in;
    float* __restrict__ o = out + bc * plane_out + (int64_t)im * s.olast + tl + al;
    for (int a0 = w; a0 < n0; a0 += kRows) {
      const Axis ax = axis_of(crd[0][al][a0], s.in[0]);
      const Axis ay = axis_of(crd[1][al][a0], s.in[1]);
      const Axis az = ND == 3 ? axis_of(crd[ND - 1][al][a0], s.in[2]) : Axis{0, 0, 0.0f};
      o[(int64_t)(t0 + a0) * ostride] = sample<ND>(s.in, d, ax, ay, az);
    }
  }
}

// GD: grad_data is requested (its scatter's state would otherwise cost every
// launch registers).
template <int ND, bool GD>
__global__ __launch_bounds__(kThreads) void interp_bwd_kernel(Shape s,
                                                              const float* __restrict__ data,
                                                              const float* __restrict__ grid,
                                                              const float* __restrict__ grad_out,
                                                              float* __restrict__ grad_grid,
                                                              float* __restrict__ grad_data) {
  __shared__ float crd[ND][kTL][kT0 + 1];
  int b, im, t0, tl;
  if (!tile_origin(s, b, im, t0, tl)) return;
  const int n0 = min(kT0, s.o0 - t0), nl = min(kTL, s.olast - tl);
  load_tile<ND>(s, grid, b, im, t0, tl, n0, nl, crd);
  __syncthreads();
  const int al = threadIdx.x % kTL;
  const int w = threadIdx.x / kTL;
  const int64_t plane_in = (int64_t)s.in[0] * s.in[1] * (ND == 3 ? s.in[2] : 1);
  const int64_t plane_out = (int64_t)s.o0 * s.omid * s.olast;
  const bool pairs = s.in[ND - 1] >= 2;   // corners read in pairs
  if (al < nl && n0 == kT0) {
    // Whole tile along i0: the gathers of gather_batch outputs of a lane
    // overlap.
    constexpr int NB = gather_batch(ND);
#pragma unroll
    for (int j0 = 0; j0 < kPerLane; j0 += NB) {
      Axis ax[NB], ay[NB], az[NB];
      float dd[NB][3];
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int a0 = w + (j0 + j) * kRows;
        ax[j] = axis_of(crd[0][al][a0], s.in[0]);
        ay[j] = axis_of(crd[1][al][a0], s.in[1]);
        az[j] = ND == 3 ? axis_of(crd[ND - 1][al][a0], s.in[2]) : Axis{0, 0, 0.0f};
        dd[j][0] = dd[j][1] = dd[j][2] = 0.0f;
      }
      const int64_t o = ((int64_t)(t0 + w + j0 * kRows) * s.omid + im) * s.olast + tl + al;
      for (int ch = 0; ch < s.C; ++ch) {
        const int64_t bc = (int64_t)b * s.C + ch;
        const ChannelBuf d(data + bc * plane_in, plane_in);
        const float* __restrict__ go = grad_out + bc * plane_out + o;
        float g[NB], c[NB][1 << ND];
        if (grad_grid) {
#pragma unroll
          for (int j = 0; j < NB; ++j) {
            if (pairs) gather_pairs<ND>(s.in, d, ax[j], ay[j], az[j], c[j]);
            else gather<ND>(s.in, d, ax[j], ay[j], az[j], c[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) g[j] = go[(int64_t)j * kRows * s.omid * s.olast];
        // keeps the batch's loads issued before the first use of one
        __builtin_amdgcn_sched_barrier(0);
        if (grad_grid) {
#pragma unroll
          for (int j = 0; j < NB; ++j) blend_grad<ND>(c[j], ax[j], ay[j], az[j], g[j], dd[j]);
        }
        if (GD) {
          float* __restrict__ gd = grad_data + bc * plane_in;
#pragma unroll
          for (int j = 0; j < NB; ++j) scatter<ND>(s.in, gd, ax[j], ay[j], az[j], g[j]);
        }
      }
      if (grad_grid) {
        // (size-1) chain factor of x = g*(size-1); each thread rewrites only
        // the LDS slots it read.
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int k = 0; k < ND; ++k)
            crd[k][al][w + (j0 + j) * kRows] = dd[j][k] * (float)(s.in[k] - 1);
      }
    }
  } else if (al < nl) {
    for (int a0 = w; a0 < n0; a0 += kRows) {
      const Axis ax = axis_of(crd[0][al][a0], s.in[0]);
      const Axis ay = axis_of(crd[1][al][a0], s.in[1]);
      const Axis az = ND == 3 ? axis_of(crd[ND - 1][al][a0], s.in[2]) : Axis{0, 0, 0.0f};
      const int64_t o = ((int64_t)(t0 + a0) * s.omid + im) * s.olast + tl + al;
      float dd[3] = {0.0f, 0.0f, 0.0f};
      for (int ch = 0; ch < s.C; ++ch) {
        const int64_t bc = (int64_t)b * s.C + ch;
        sample_grad<ND>(s.in, data + bc * plane_in, ax, ay, az, grad_out[bc * plane_out + o],
                        grad_grid ? dd : nullptr, GD ? grad_data + bc * plane_in : nullptr);
      }
      if (grad_grid) {
#pragma unroll
        for (int k = 0; k < ND; ++k) crd[k][al][a0] = dd[k] * (float)(s.in[k] - 1);
      }
    }
  }
  if (!grad_grid) return;
  __syncthreads();
  const int64_t row0 = (int64_t)s.o0 * (im + (int64_t)s.omid * tl) + t0;
  const int64_t rstride = (int64_t)s.o0 * s.omid;
  if (s.vec4 && n0 == kT0) {
    constexpr int Q = kT0 / 4;
    for (int e = threadIdx.x; e < Q * kTL; e += kThreads) {
      const int q = e % Q, l = e / Q;
      if (l < nl) {
#pragma unroll
        for (int k = 0; k < ND; ++k) {
          float4 v;
          v.x = crd[k][l][4 * q];
          v.y = crd[k][l][4 * q + 1];
          v.z = crd[k][l][4 * q + 2];
          v.w = crd[k][l][4 * q + 3];
          *reinterpret_cast<float4*>(grad_grid + ((int64_t)b * ND + k) * s.nP + row0 + l * rstride + 4 * q) = v;
        }
      }
    }
  } else {
    for (int e = threadIdx.x; e < kT0 * kTL; e += kThreads) {
      const int a0 = e % kT0, l = e / kT0;
      if (a0 < n0 && l < nl) {
#pragma unroll
        for (int k = 0; k < ND; ++k)
          grad_grid[((int64_t)b * ND + k) * s.nP + row0 + l * rstride + a0] = crd[k][l][a0];
      }
    }
  }
}

// 1D: point order equals output order, one thread per (b, point).
__global__ __launch_bounds__(kThreads) void interp1d_fwd_kernel(int B, int C, int W, int64_t nP,
                                                                const float* __restrict__ data,
                                                                const float* __restrict__ grid,
                                                                float* __restrict__ out) {
  for (int64_t e = blockIdx.x * (int64_t)kThreads + threadIdx.x; e < (int64_t)B * nP;
       e += (int64_t)gridDim.x * kThreads) {
    const int64_t b = e / nP, p = e - b * nP;
    const Axis ax = axis_of(grid[e], W);
    for (int ch = 0; ch < C; ++ch) {
      const float* d = data + (b * C + ch) * W;
      out[(b * C + ch) * nP + p] = lerp_ref(load_at(d, ax.i0), load_at(d, ax.i1), ax.t);
    }
  }
}

__global__ __launch_bounds__(kThreads) void interp1d_bwd_kernel(int B, int C, int W, int64_t nP,
                                                                const float* __restrict__ data,
                                                                const float* __restrict__ grid,
                                                                const float* __restrict__ grad_out,
                                                                float* __restrict__ grad_grid,
                                                                float* __restrict__ grad_data) {
  for (int64_t e = blockIdx.x * (int64_t)kThreads + threadIdx.x; e < (int64_t)B * nP;
       e += (int64_t)gridDim.x * kThreads) {
    const int64_t b = e / nP, p = e - b * nP;
    const Axis ax = axis_of(grid[e], W);
    float gx = 0.0f;
    for (int ch = 0; ch < C; ++ch) {
      const int64_t bc = b * C + ch;
      const float g = grad_out[bc * nP + p];
      const float* d = data + bc * W;
      gx += g * (load_at(d, ax.i1) - load_at(d, ax.i0));
      if (grad_data) {
        add_at(grad_data + bc * W, ax.i0, g * (1.0f - ax.t));
        add_at(grad_data + bc * W, ax.i1, g * ax.t);
      }
    }
    if (grad_grid) grad_grid[e] = gx * (float)(W - 1);
  }
}

Shape make_shape(int ndim, int64_t B, int64_t C, const int64_t* in_size, const int64_t* out_size) {
  Shape s{};
  s.vec4 = 0;
  s.ndim = ndim;
  s.B = (int)B;
  s.C = (int)C;
  for (int k = 0; k < 3; ++k) s.in[k] = k < ndim ? (int)in_size[k] : 1;
  s.o0 = (int)out_size[0];
  s.omid = ndim == 3 ? (int)out_size[1] : 1;
  s.olast = (int)out_size[ndim - 1];
  s.nP = 1;
  for (int k = 0; k < ndim; ++k) s.nP *= out_size[k];
  s.vec4 = (s.o0 % 4) == 0;
  s.tiles0 = (s.o0 + kT0 - 1) / kT0;
  s.tilesl = (s.olast + kTL - 1) / kTL;
  return s;
}

int aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

dim3 tile_grid(const Shape& s) {
  const int64_t total = (int64_t)s.tiles0 * s.tilesl * s.B * s.omid;
  return dim3((unsigned)((total + kXcds - 1) / kXcds * kXcds));
}

}  // namespace

hipError_t launch_interp_forward(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                                 const int64_t* out_size, const float* data, const float* grid,
                                 float* out, hipStream_t st) {
  Shape s = make_shape(ndim, B, C, in_size, out_size);
  s.vec4 &= aligned16(grid);
  if (s.nP <= 0 || B <= 0) return hipSuccess;
  if (ndim == 1) {
    int64_t g = (B * s.nP + kThreads - 1) / kThreads;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(interp1d_fwd_kernel, dim3((unsigned)g), dim3(kThreads), 0, st, s.B, s.C,
                       s.in[0], s.nP, data, grid, out);
  } else {
    if (ndim == 2)
      hipLaunchKernelGGL(interp_fwd_kernel<2>, tile_grid(s), dim3(kThreads), 0, st, s, data, grid, out);
    else
      hipLaunchKernelGGL(interp_fwd_kernel<3>, tile_grid(s), dim3(kThreads), 0, st, s, data, grid, out);
  }
  return hipGetLastError();
}

hipError_t launch_interp_backward(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                                  const int64_t* out_size, const float* data, const float* grid,
                                  const float* grad_out, float* grad_grid, float* grad_data,
                                  hipStream_t st) {
  Shape s = make_shape(ndim, B, C, in_size, out_size);
  s.vec4 &= aligned16(grid) & (grad_grid == nullptr || aligned16(grad_grid));
  if (grad_data) {
    int64_t n = B * C;
    for (int k = 0; k < ndim; ++k) n *= in_size[k];
    hipError_t e = launch_fill(grad_data, n, 0.0f, st);
    if (e != hipSuccess) return e;
  }
  if (s.nP <= 0 || B <= 0) return hipSuccess;
  if (ndim == 1) {
    int64_t g = (B * s.nP + kThreads - 1) / kThreads;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(interp1d_bwd_kernel, dim3((unsigned)g), dim3(kThreads), 0, st, s.B, s.C,
                       s.in[0], s.nP, data, grid, grad_out, grad_grid, grad_data);
  } else {
    auto kernel = ndim == 2 ? (grad_data ? interp_bwd_kernel<2, true> : interp_bwd_kernel<2, false>)
                            : (grad_data ? interp_bwd_kernel<3, true> : interp_bwd_kernel<3, false>);
    hipLaunchKernelGGL(kernel, tile_grid(s), dim3(kThreads), 0, st, s, data, grid, grad_out,
                       grad_grid, grad_data);
  }
  return hipGetLastError();
}

}  // namespace cpab
