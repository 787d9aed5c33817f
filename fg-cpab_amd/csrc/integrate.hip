// Forward integrators (transform_grid forward pass).
//
//   1D: exact closed-form flow with boundary-hit times (cpab_ops_1d.cu:103-243).
//   2D/3D: T fixed steps p <- Trels[cell(p)] [p; 1] with Trels = expm(A/T)
//          (cpab_ops_2d.cu:164-230, cpab_ops_3d.cu:169-241), optional Heun
//          correction on a cell crossing (adaptive_substeps).
//
// MI355X layout: the workgroups of one grid row (blockIdx.y) integrate the
// points of ONE theta, so the L1/L2 serve that theta's per-cell table (nC x 6
// floats in 2D); each lane keeps its current cell's one-step map in registers
// and re-reads it only when some lane of its wave changes cell.  Points are
// SoA ([ndim, nP] rows) and each lane owns whole trajectories, so global reads
// and writes are fully coalesced.  The integrator is fp32 VALU-bound; no MFMA
// is involved.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <math.h>
#include "cpab_device.hpp"
#include "cpab_launch.hpp"
#include "cpab_sample.hpp"

namespace cpab {
namespace {

// ---------------------------------------------------------------------------
// 1D closed form
// ---------------------------------------------------------------------------

__device__ __forceinline__ int sgn(float x) { return (x > 0.0f) - (x < 0.0f); }
__device__ __forceinline__ bool near0(float x) { return fabsf(x) < 1e-7f; }

// Time to leave cell c from x moving for time t, with the exit point and the
// next cell (cpab_ops_1d.cu:133-167).
__device__ float hit_time_1d(float x, float t, int c, float a, float b, int nx, float& xc,
                             int& cc) {
  const int s = sgn(t);
  const float inf_t = INFINITY * (float)s;
  const float v = fmaf(a, x, b);
  if (near0(v)) return inf_t;
  cc = c + sgn(v) * s;
  if (cc < 0 || cc >= nx) return inf_t;
  const float right = (float)(c + 1) / (float)nx + 1e-7f;
  const float left = (float)c / (float)nx - 1e-7f;
  xc = (t > 0.0f) ? ((v > 0.0f) ? right : left) : ((v > 0.0f) ? left : right);
  const float vc = fmaf(a, xc, b);
  if (near0(vc)) return inf_t;
  if (sgn(v) != sgn(vc)) return inf_t;
  if (xc <= 0.0f || xc >= 1.0f) return inf_t;
  if (near0(a)) return (xc - x) / b;
  return log_cr(vc / v) / a;
}

__device__ float closed_form_1d(float x, float t, const float* __restrict__ A, int nx) {
  int c = cell_1d(x, nx);
  const int contmax = max(c, nx - 1 - c) + 1;
  const int s = sgn(t);
  for (int cont = 0;;) {
    const float a = A[2 * c], b = A[2 * c + 1];
    float xc = x;
    int cc = c;
    const float thit = hit_time_1d(x, t, c, a, b, nx, xc, cc);
    if ((float)s * thit > (float)s * t) {
      if (near0(a)) return fmaf(t, b, x);
      const float boa = b / a;
      return fmaf(exp_cr(t * a), x + boa, -boa);
    }
    x = xc;
    c = cc;
    t -= thit;
    if (++cont > contmax) break;
  }
  return x;
}

// K > 1: chain of stages, row (s * n_batch + b) of As for stage s; inputs of
// stages s >= 1 saved to stage_points[s-1] when it is not null.
__global__ __launch_bounds__(256) void fwd1d_closed_kernel(int nP, int batched, int nx, int K,
                                                          const float* __restrict__ points,
                                                          const float* __restrict__ As,
                                                          float* __restrict__ out,
                                                          float* __restrict__ stage_points) {
  const int b = blockIdx.y;
  const int n_batch = gridDim.y;
  const float* pts = points + (batched ? (size_t)b * nP : 0);
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < nP; p += gridDim.x * blockDim.x) {
    float x = pts[p];
    for (int st = 0; st < K; ++st) {
      const size_t row = (size_t)st * n_batch + b;
      if (st > 0 && stage_points) stage_points[((size_t)(st - 1) * n_batch + b) * nP + p] = x;
      x = closed_form_1d(x, 1.0f, As + row * 2 * nx, nx);
    }
    out[(size_t)b * nP + p] = x;
  }
}

// ---------------------------------------------------------------------------
// 2D / 3D fixed-step forward
// ---------------------------------------------------------------------------

// T fixed steps of one transform for PPT points per lane (2D).  The one-step
// map of the current cell stays in registers; it is re-read (through L1) only
// at steps where some lane of the wave changed cell, which keeps table traffic
// off most steps.  With adaptive_substeps a step that leaves its cell is
// redone with Heun's rule (cpab_ops_2d.cu:202-219).
template <bool ADAPTIVE, int PPT>
__device__ __forceinline__ void steps_2d(float (&px)[PPT], float (&py)[PPT],
                                         const float* __restrict__ Tg,
                                         const float* __restrict__ Ag, int T, int nx, int ny,
                                         float hh) {
  CellKey cur[PPT];
  Aff<2> M[PPT];
#pragma unroll
  for (int k = 0; k < PPT; ++k) {
    cur[k] = cell_key_2d(px[k], py[k], nx, ny);
    M[k] = load_aff2(Tg, key_cell(cur[k]));
  }
  // One step of point k from its cell c (M[k] already holds c's map).
  auto advance = [&](int k, const CellKey& ck) {
    float sx, sy;
    apply2(M[k], px[k], py[k], sx, sy);
    if (ADAPTIVE) {
      const int c = key_cell(ck);
      const int ce = cell_2d(sx, sy, nx, ny);
      if (ce != c) {
        float v0x, v0y, v1x, v1y;
        apply2(load_aff2(Ag, c), px[k], py[k], v0x, v0y);
        apply2(load_aff2(Ag, ce), sx, sy, v1x, v1y);
        sx = fmaf(hh, v0x + v1x, px[k]);
        sy = fmaf(hh, v0y + v1y, py[k]);
      }
    }
    px[k] = sx;
    py[k] = sy;
  };
#pragma unroll
  for (int k = 0; k < PPT; ++k) advance(k, cur[k]);
  auto step = [&]() {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const CellKey ck = cell_key_2d(px[k], py[k], nx, ny);
      // Divergent branch on the changed lanes' mask, skipped (exec = 0) when
      // no lane changed cell; marked unlikely so that this case falls through.
      if (__builtin_expect(__builtin_amdgcn_inverse_ballot_w64(key_changed(ck, cur[k])), 0))
        M[k] = load_aff2(Tg, key_cell(ck));
      cur[k] = ck;
      advance(k, ck);
    }
  };
  // Steps 1 .. T-1, two per iteration (written out: the lookup's ballots keep
  // the compiler from unrolling a loop of unknown trip count), so that the
  // loop-carried positions and cells alternate between two register sets
  // instead of being copied back at every step.
  int t = 1;
  for (; t + 1 < T; t += 2) {
    step();
    step();
  }
  if (t < T) step();
}

// T fixed steps of one transform for one point (3D, cpab_ops_3d.cu:169-241),
// with the same cell-change caching of the one-step map as steps_2d.
template <bool ADAPTIVE>
__device__ __forceinline__ void steps_3d(float& px, float& py, float& pz,
                                         const float* __restrict__ Tg,
                                         const float* __restrict__ Ag, int T, int nx, int ny,
                                         int nz, float hh) {
  int cur = cell_3d(px, py, pz, nx, ny, nz);
  Aff<3> M = load_aff3(Tg, cur);
  for (int t = 0; t < T; ++t) {
    const int c = (t == 0) ? cur : cell_3d(px, py, pz, nx, ny, nz);
    // Divergent branch, skipped (exec = 0) when no lane changed cell; marked
    // unlikely so that the no-change case falls through.
    if (__builtin_expect(c != cur, 0)) M = load_aff3(Tg, c);
    cur = c;
    float sx, sy, sz;
    apply3(M, px, py, pz, sx, sy, sz);
    if (ADAPTIVE) {
      const int ce = cell_3d(sx, sy, sz, nx, ny, nz);
      if (ce != c) {
        float v0x, v0y, v0z, v1x, v1y, v1z;
        apply3(load_aff3(Ag, c), px, py, pz, v0x, v0y, v0z);
        apply3(load_aff3(Ag, ce), sx, sy, sz, v1x, v1y, v1z);
        sx = fmaf(hh, v0x + v1x, px);
        sy = fmaf(hh, v0y + v1y, py);
        sz = fmaf(hh, v0z + v1z, pz);
      }
    }
    px = sx;
    py = sy;
    pz = sz;
  }
}

// PPT independent trajectories per lane give the scheduler two dependency
// chains (lookup -> table read -> affine apply) to interleave.  The per-cell
// tables are read through L1/L2: a lane re-reads its cell's map only when some
// lane of its wave changed cell, so staging the table in LDS bought nothing and
// capped occupancy.
//
// K > 1 runs a chain (Cpab.transform_grid_chain): stage s integrates with the
// tables of row (s * n_batch + b) of Trels / As, starting from the previous
// stage's result; the input of every stage s >= 1 is saved to
// stage_points[s-1] (if not null) for the backward.
template <bool ADAPTIVE, int PPT>
__global__ __launch_bounds__(1024) void fwd2d_kernel(int nP, int batched, int T, int nx, int ny,
                                                    int K, const float* __restrict__ points,
                                                    const float* __restrict__ Trels,
                                                    const float* __restrict__ As,
                                                    float* __restrict__ out,
                                                    float* __restrict__ stage_points) {
  const int b = blockIdx.y;
  const int n_batch = gridDim.y;
  const int nC = 4 * nx * ny;
  const float h = 1.0f / (float)T;
  const float hh = 0.5f * h;
  const float* __restrict__ pts = points + (batched ? (size_t)b * 2 * nP : 0);
  float* __restrict__ o = out + (size_t)b * 2 * nP;
  const int stride = gridDim.x * blockDim.x;
  for (int p0 = blockIdx.x * blockDim.x + threadIdx.x; p0 < nP; p0 += PPT * stride) {
    float px[PPT], py[PPT];
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = min(p0 + k * stride, nP - 1);
      px[k] = pts[p];
      py[k] = pts[p + nP];
    }
    edge_priority(px, py);
    for (int st = 0; st < K; ++st) {
      const size_t row = (size_t)st * n_batch + b;
      const float* __restrict__ Tg = Trels + row * nC * 6;
      const float* __restrict__ Ag = As + row * nC * 6;
      if (st > 0 && stage_points) {
        float* sp = stage_points + ((size_t)(st - 1) * n_batch + b) * 2 * nP;
#pragma unroll
        for (int k = 0; k < PPT; ++k) {
          const int p = p0 + k * stride;
          if (p < nP) {
            sp[p] = px[k];
            sp[p + nP] = py[k];
          }
        }
      }
      steps_2d<ADAPTIVE, PPT>(px, py, Tg, Ag, T, nx, ny, hh);
    }  // stages
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int p = p0 + k * stride;
      if (p < nP) {
        o[p] = px[k];
        o[p + nP] = py[k];
      }
    }
  }
}

template <bool ADAPTIVE>
__global__ __launch_bounds__(1024) void fwd3d_kernel(int nP, int batched, int T, int nx, int ny,
                                                    int nz, int K, const float* __restrict__ points,
                                                    const float* __restrict__ Trels,
                                                    const float* __restrict__ As,
                                                    float* __restrict__ out,
                                                    float* __restrict__ stage_points) {
  const int b = blockIdx.y;
  const int n_batch = gridDim.y;
  const int nC = 5 * nx * ny * nz;
  const float h = 1.0f / (float)T;
  const float hh = 0.5f * h;
  const float* __restrict__ pts = points + (batched ? (size_t)b * 3 * nP : 0);
  float* __restrict__ o = out + (size_t)b * 3 * nP;
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < nP; p += gridDim.x * blockDim.x) {
    float px = pts[p], py = pts[p + nP], pz = pts[p + 2 * (size_t)nP];
    for (int st = 0; st < K; ++st) {
      const size_t row = (size_t)st * n_batch + b;
      const float* __restrict__ Tg = Trels + row * nC * 12;
      const float* __restrict__ Ag = As + row * nC * 12;
      if (st > 0 && stage_points) {
        float* sp = stage_points + ((size_t)(st - 1) * n_batch + b) * 3 * nP;
        sp[p] = px;
        sp[p + nP] = py;
        sp[p + 2 * (size_t)nP] = pz;
      }
      steps_3d<ADAPTIVE>(px, py, pz, Tg, Ag, T, nx, ny, nz, hh);
    }  // stages
    o[p] = px;
    o[p + nP] = py;
    o[p + 2 * (size_t)nP] = pz;
  }
}


// Fused transform_data forward (cpab/cpab.py:295-309): output position q
// (image order, last axis fastest) integrates its meshgrid point under theta b
// exactly as cpab_forward / the 1D closed form does, then samples every
// channel of data there exactly as cpab_interp_forward does.  Each wave takes
// one 16 x 4 pixel tile (tile_index) when the size tiles, else a run of 64
// pixels in image order; the image stores and final_points (image order, for
// the backward) go out in 64-byte runs or better.  The start points come from
// the grid's per-axis coordinate vectors.
template <int ND, bool ADAPTIVE>
__global__ __launch_bounds__(1024) void image_forward_kernel(
    ImageShape s, int T, int nx, int ny, int nz, const float* __restrict__ axes,
    const float* __restrict__ Trels, const float* __restrict__ As,
    const float* __restrict__ data, float* __restrict__ out, float* __restrict__ final_points,
    float* __restrict__ seed_grad) {
  const int b = blockIdx.y;
  constexpr int P = ND * (ND + 1);
  const int nC = ND == 1 ? nx : (ND == 2 ? 4 * nx * ny : 5 * nx * ny * nz);
  const float* __restrict__ Tg = Trels + (size_t)b * nC * P;
  const float* __restrict__ Ag = As + (size_t)b * nC * P;
  const float hh = 0.5f / (float)T;
  const float* __restrict__ dat = data + (size_t)b * s.C * s.plane_in;
  float* __restrict__ o = out + (size_t)b * s.C * s.nP;
  float* __restrict__ fin = final_points ? final_points + (size_t)b * ND * s.nP : nullptr;
  // One channel: the sample's spatial gradient too, for the backward's seed.
  float* __restrict__ sg = seed_grad ? seed_grad + (size_t)b * ND * s.nP : nullptr;
  auto emit = [&](int q, const Axis& ax, const Axis& ay, const Axis& az) {
    if (sg) {
      float gr[3];
      o[q] = sample_spatial_grad<ND>(s.in, dat, ax, ay, az, gr);
#pragma unroll
      for (int k = 0; k < ND; ++k) sg[q + (size_t)k * s.nP] = gr[k];
      return;
    }
    for (int c = 0; c < s.C; ++c)
      o[(size_t)c * s.nP + q] = sample<ND>(s.in, dat + c * s.plane_in, ax, ay, az);
  };
  if constexpr (ND == 2 && !ADAPTIVE) {
    // Two output positions per lane, m and m + stride (the second clamped to
    // the last position and not written when past it).
    const int stride = gridDim.x * blockDim.x;
    for (int m0 = blockIdx.x * blockDim.x + threadIdx.x; m0 < s.nP; m0 += 2 * stride) {
      int qs[2];
      float px[2], py[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int m = min(m0 + k * stride, s.nP - 1);
        int ix[3], q = m;
        if (s.walk_tiles) {
          tile_index<2>(s, m, ix);
          q = image_pos<2>(s, ix);
        } else {
          image_index<2>(s, m, ix);
        }
        float x[3];
        grid_point<2>(s, axes, ix, x);
        qs[k] = q;
        px[k] = x[0];
        py[k] = x[1];
      }
      steps_2d<false, 2>(px, py, Tg, Ag, T, nx, ny, hh);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        if (m0 + k * stride >= s.nP) continue;
        const int q = qs[k];
        if (fin) {
          fin[q] = px[k];
          fin[q + (size_t)s.nP] = py[k];
        }
        emit(q, axis_of(px[k], s.in[0]), axis_of(py[k], s.in[1]), Axis{0, 0, 0.0f});
      }
    }
    return;
  }
  for (int m = blockIdx.x * blockDim.x + threadIdx.x; m < s.nP; m += gridDim.x * blockDim.x) {
    int ix[3], q = m;
    if (ND >= 2 && s.walk_tiles) {
      tile_index<ND>(s, m, ix);
      q = image_pos<ND>(s, ix);
    } else {
      image_index<ND>(s, m, ix);
    }
    float x[3];
    grid_point<ND>(s, axes, ix, x);
    if (ND == 1) {
      x[0] = closed_form_1d(x[0], 1.0f, Ag, nx);
    } else if (ND == 2) {
      float px[1] = {x[0]}, py[1] = {x[1]};
      steps_2d<ADAPTIVE, 1>(px, py, Tg, Ag, T, nx, ny, hh);
      x[0] = px[0];
      x[1] = py[0];
    } else {
      steps_3d<ADAPTIVE>(x[0], x[1], x[2], Tg, Ag, T, nx, ny, nz, hh);
    }
    if (fin) {
#pragma unroll
      for (int k = 0; k < ND; ++k) fin[q + (size_t)k * s.nP] = x[k];
    }
    const Axis ax = axis_of(x[0], s.in[0]);
    const Axis ay = ND >= 2 ? axis_of(x[1], s.in[1]) : Axis{0, 0, 0.0f};
    const Axis az = ND == 3 ? axis_of(x[2], s.in[2]) : Axis{0, 0, 0.0f};
    emit(q, ax, ay, az);
  }
}

// Cell index visited at every step of the fixed-step forward, for parity tests
// of the visited-cell sequence (same stepping as fwd2d/fwd3d, table read from
// global memory).  cells: [n_theta, nP, T] int32.
__global__ __launch_bounds__(256) void trace_cells_kernel(int ndim, int nP, int batched, int T,
                                                          int nx, int ny, int nz,
                                                          const float* __restrict__ points,
                                                          const float* __restrict__ Trels,
                                                          const float* __restrict__ As,
                                                          int adaptive, int32_t* __restrict__ cells) {
  const int b = blockIdx.y;
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= nP) return;
  const int P = ndim * (ndim + 1);
  const int nC = ndim == 2 ? 4 * nx * ny : 5 * nx * ny * nz;
  const float* Tg = Trels + (size_t)b * nC * P;
  const float* Ag = As + (size_t)b * nC * P;
  const float* pts = points + (batched ? (size_t)b * ndim * nP : 0);
  const float h = 1.0f / (float)T, hh = 0.5f * h;
  int32_t* cl = cells + ((size_t)b * nP + p) * T;
  if (ndim == 2) {
    float px = pts[p], py = pts[p + nP];
    for (int t = 0; t < T; ++t) {
      const int c = cell_2d(px, py, nx, ny);
      cl[t] = c;
      float sx, sy;
      apply2(load_aff2(Tg, c), px, py, sx, sy);
      if (adaptive) {
        const int ce = cell_2d(sx, sy, nx, ny);
        if (ce != c) {
          float v0x, v0y, v1x, v1y;
          apply2(load_aff2(Ag, c), px, py, v0x, v0y);
          apply2(load_aff2(Ag, ce), sx, sy, v1x, v1y);
          sx = fmaf(hh, v0x + v1x, px);
          sy = fmaf(hh, v0y + v1y, py);
        }
      }
      px = sx;
      py = sy;
    }
  } else {
    float px = pts[p], py = pts[p + nP], pz = pts[p + 2 * (size_t)nP];
    for (int t = 0; t < T; ++t) {
      const int c = cell_3d(px, py, pz, nx, ny, nz);
      cl[t] = c;
      float sx, sy, sz;
      apply3(load_aff3(Tg, c), px, py, pz, sx, sy, sz);
      if (adaptive) {
        const int ce = cell_3d(sx, sy, sz, nx, ny, nz);
        if (ce != c) {
          float v0x, v0y, v0z, v1x, v1y, v1z;
          apply3(load_aff3(Ag, c), px, py, pz, v0x, v0y, v0z);
          apply3(load_aff3(Ag, ce), sx, sy, sz, v1x, v1y, v1z);
          sx = fmaf(hh, v0x + v1x, px);
          sy = fmaf(hh, v0y + v1y, py);
          sz = fmaf(hh, v0z + v1z, pz);
        }
      }
      px = sx;
      py = sy;
      pz = sz;
    }
  }
}

template <typename Kern>
hipError_t launch2d(Kern kernel, dim3 grid, dim3 block, hipStream_t s, int nP, int batched, int T,
                    int nx, int ny, int K, const float* points, const float* Trels,
                    const float* As, float* out, float* stage_points) {
  hipLaunchKernelGGL(kernel, grid, block, 0, s, nP, batched, T, nx, ny, K, points, Trels, As, out,
                     stage_points);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_forward_1d(const Geometry& g, int64_t nP, int64_t n_batch, int batched, int K,
                             const float* points, const float* As, float* out,
                             float* stage_points, hipStream_t s) {
  if (nP <= 0 || n_batch <= 0 || K <= 0) return hipSuccess;
  int64_t gx = (nP + 255) / 256;
  if (gx > 4096) gx = 4096;
  hipLaunchKernelGGL(fwd1d_closed_kernel, dim3((unsigned)gx, (unsigned)n_batch), dim3(256), 0, s,
                     (int)nP, batched, g.nx, K, points, As, out, stage_points);
  return hipGetLastError();
}

hipError_t launch_forward(const Geometry& g, int64_t nP, int64_t n_batch, int batched, int T,
                          int K, int adaptive, const float* points, const float* Trels,
                          const float* As, float* out, float* stage_points, const LaunchCfg& cfg,
                          hipStream_t s) {
  if (nP <= 0 || n_batch <= 0 || K <= 0) return hipSuccess;
  const dim3 grid((unsigned)cfg.chunks, (unsigned)n_batch), block((unsigned)cfg.block);
  if (g.ndim == 2) {
    if (adaptive)
      return launch2d(fwd2d_kernel<true, 1>, grid, block, s, (int)nP, batched, T, g.nx,
                             g.ny, K, points, Trels, As, out, stage_points);
    if (K > 1) {
      // A chain runs every stage of a trajectory in one lane, so few points
      // (C5: 262,144, 4 waves per SIMD) leave the kernel latency-bound: one
      // point per lane, one pass over the points, and no barrier between
      // stages (each wave reads the stage tables through L1/L2 at its own
      // pace; staging them in LDS held every workgroup to its slowest wave at
      // each stage: C5 forward 123 -> 116 us).
      const int64_t need1 = (nP + (int64_t)cfg.block - 1) / (int64_t)cfg.block;
      const dim3 grid1((unsigned)need1, (unsigned)n_batch);
      return launch2d(fwd2d_kernel<false, 1>, grid1, block, s, (int)nP, batched, T, g.nx,
                             g.ny, K, points, Trels, As, out, stage_points);
    }
    // Two points per lane: no more workgroups than it takes to cover nP once
    // (a lane's second point would otherwise duplicate work on a clamped index).
    const int64_t need = (nP + 2 * (int64_t)cfg.block - 1) / (2 * (int64_t)cfg.block);
    const dim3 grid2((unsigned)std::max<int64_t>(1, std::min<int64_t>(cfg.chunks, need)),
                     (unsigned)n_batch);
    return launch2d(fwd2d_kernel<false, 2>, grid2, block, s, (int)nP, batched, T, g.nx,
                           g.ny, K, points, Trels, As, out, stage_points);
  }
  // 3D: the kernel takes nz as an extra argument.
  auto go = [&](auto kernel) -> hipError_t {
    hipLaunchKernelGGL(kernel, grid, block, 0, s, (int)nP, batched, T, g.nx, g.ny, g.nz, K,
                       points, Trels, As, out, stage_points);
    return hipGetLastError();
  };
  return adaptive ? go(fwd3d_kernel<true>) : go(fwd3d_kernel<false>);
}

hipError_t launch_image_forward(const Geometry& g, const ImageShape& img, int64_t n_batch, int T,
                                int adaptive, const float* axes, const float* Trels,
                                const float* As, const float* data, float* out,
                                float* final_points, float* seed_grad, const LaunchCfg& cfg,
                                hipStream_t s) {
  if (img.nP <= 0 || n_batch <= 0) return hipSuccess;
  const int per_lane = (g.ndim == 2 && !adaptive) ? 2 : 1;
  const int64_t need = (img.nP + (int64_t)per_lane * cfg.block - 1) / ((int64_t)per_lane * cfg.block);
  const dim3 blocks((unsigned)std::max<int64_t>(1, std::min<int64_t>(cfg.chunks, need)),
                    (unsigned)n_batch);
  const dim3 threads((unsigned)cfg.block);
  auto go = [&](auto kernel) -> hipError_t {
    hipLaunchKernelGGL(kernel, blocks, threads, 0, s, img, T, g.nx, g.ny, g.nz, axes, Trels, As,
                       data, out, final_points, seed_grad);
    return hipGetLastError();
  };
  switch (g.ndim * 2 + (adaptive ? 1 : 0)) {
    case 2: return go(image_forward_kernel<1, false>);
    case 3: return go(image_forward_kernel<1, true>);
    case 4: return go(image_forward_kernel<2, false>);
    case 5: return go(image_forward_kernel<2, true>);
    case 6: return go(image_forward_kernel<3, false>);
    default: return go(image_forward_kernel<3, true>);
  }
}

hipError_t launch_trace_cells(const Geometry& g, int64_t nP, int64_t n_theta, int batched, int T,
                              int adaptive, const float* points, const float* Trels,
                              const float* As, int32_t* cells, hipStream_t s) {
  if (nP <= 0 || n_theta <= 0) return hipSuccess;
  hipLaunchKernelGGL(trace_cells_kernel, dim3((unsigned)((nP + 255) / 256), (unsigned)n_theta),
                     dim3(256), 0, s, g.ndim, (int)nP, batched, T, g.nx, g.ny, g.nz, points, Trels,
                     As, adaptive, cells);
  return hipGetLastError();
}

}  // namespace cpab
