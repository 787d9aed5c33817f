// Fused backward: midpoint-trajectory replay + discrete adjoint + cell moments
// (cpab_ops_1d.cu:331-422, cpab_ops_2d.cu:384-513, cpab_ops_3d.cu:405-532).
//
// Per trajectory (one lane), two variants:
//   register  (T == kRegSteps) phase 1 runs the T explicit-midpoint steps
//             fully unrolled and keeps every cell in VGPRs (two per
//             register); phase 2 walks them backwards, recovering each
//             position from the next through the cell's inverse one-step map
//             (with adaptive substeps, whose steps are not fixed affine maps,
//             the positions are kept in VGPRs too).  One midpoint pass per
//             trajectory.
//   segmented (any T <= 100) phase 1 keeps a checkpoint every kSeg steps in a
//             VGPR shift register; phase 2 replays each segment from its
//             checkpoint into registers and walks it backwards (the
//             reference's scheme, cpab_ops_2d.cu:236-263).
// Both visit the reference's cells; the positions fed to the sums may differ
// from the replayed ones by a few ulps in the register variant.
// In both, phase 2 propagates lambda and accumulates the 2x3 (1x2, 3x4) sum
// S = sum lam (x) [p; 1] of the current cell, flushing it whenever the cell
// changes, as the reference groups its moment flushes.  The reverse step is the
// factored form of cpab_ops_2d.cu:334-382 (cpab_device.hpp, adjoint_s*): lam is
// advanced with the per-cell increment G = h A + (h^2/2) A^2 and the moments
// are formed from S once per cell after the partial tables are summed
// (basis.hip, finish_moments_kernel).
//
// Moment accumulation on MI355X: each workgroup serves ONE theta and one
// contiguous range of points (spatially coherent for meshgrid inputs).
//   full bins  the nC x ppc table fits in LDS: the workgroup keeps a private
//              copy of that theta's sums there (ds_add_f32, no HBM atomics
//              while integrating).  At the end a workgroup that touched at
//              least a quarter of the cells (random points: every workgroup
//              touches nearly every cell) stores its whole table as its
//              partial (plain coalesced stores) and sets its bit in the row's
//              dense-part mask; one that touched fewer (meshgrids, chains:
//              few workgroups share a cell) adds its cells' sums to the HBM
//              table with global atomics instead.  A separate pass adds the
//              dense partials, in ascending order, to the HBM sums and forms
//              the moments.  Cross-XCD atomics on shared addresses are what
//              the dense case avoids.
//   cache      the table does not fit (3D at 10x10x10: 234 KiB): a
//              direct-mapped LDS cache of kCacheSlots cells (linear probing,
//              kCacheProbes slots) collects the flushes of the cells the
//              workgroup touches; at the end each occupied slot is added to
//              HBM with global atomics.  Flushes that find no slot go
//              straight to HBM.  The HBM table holds sums S; a separate pass
//              forms the moments in place.
// The cache takes at most 104 KiB of LDS (3D), within the 160 KiB a gfx950
// workgroup may use, so every tessellation runs one of the two.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include "cpab_device.hpp"
#include "cpab_launch.hpp"
#include "cpab_sample.hpp"
#include "backward_body.hpp"

namespace cpab {
namespace {

// TS == 0: segmented variant; TS > 0: register variant.  Both accumulate in
// full LDS bins or the LDS cell cache.
// One workgroup = one theta x one contiguous point range (wg_slot).  A chain
// of K stages (Cpab.transform_grid_chain) runs its stages last to first
// inside the kernel: stage k reads its input points from
// `points` (k = 0) or stage_points[k-1], its seed from grad_out (k = K-1) or
// the lam buffer the stage above wrote for the same points, and writes the
// adjoint of its input to lam (k > 0) or grad_points (k = 0).  The per-cell
// sums of stage k go to row (k * n_batch + b): added to that moments row (zero
// on entry), or, from a dense full-bin workgroup, to its partial table with
// its dense-part bit set; the reverse-sweep table G holds the same rows
// (RevStride<D>::S floats per cell).
// Launch bound: 1024 threads (4 waves per SIMD, up to 128 VGPRs) for the
// register variant without adaptive substeps (cells only in registers: ~90
// VGPRs in 2D, ~120 in 3D); 768 (3 waves per SIMD, up to 168 VGPRs) for the
// segmented variant and the adaptive register variant, whose trajectory takes
// D x 50 VGPRs.
template <int D, bool ADAPTIVE, int TS>
constexpr int kBwdThreads = (TS > 0 && !ADAPTIVE) ? 1024 : 768;

template <int D, bool ADAPTIVE, bool LDS_A, int BINS, int TS>
__global__ __launch_bounds__((kBwdThreads<D, ADAPTIVE, TS>)) void backward_kernel(
    int nP, int batched, int T, Cells g, int nC, int K, const float* __restrict__ points,
    const float* __restrict__ stage_points, const float* __restrict__ As,
    const float* __restrict__ Gs, Recover rec, const float* __restrict__ grad_out,
    float* __restrict__ moments, float* __restrict__ partials, uint64_t* __restrict__ dense_parts,
    float* __restrict__ lam, float* __restrict__ grad_points) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int touched_cnt;
  const WgSlot w = wg_slot();
  const int b = w.row;
  const int n_batch = gridDim.y;
  const int R = nC * Dim<D>::P;
  const size_t plane = (size_t)D * nP;  // one theta's [D, nP] block
  const StageLds<D, LDS_A, BINS> L(lds, R);
  for (int k = K - 1; k >= 0; --k) {
    const size_t row = (size_t)k * n_batch + b;
    const float* __restrict__ Ag = As + row * R;
    const float* __restrict__ Gg = Gs + row * nC * RevStride<D>::S;
    PlainIO<D> io;
    io.nP = nP;
    io.pts = k == 0 ? points + (batched ? (size_t)b * plane : 0)
                    : stage_points + ((size_t)(k - 1) * n_batch + b) * plane;
    io.gout = k == K - 1 ? grad_out + (size_t)b * plane : lam + (size_t)b * plane;
    io.lam_out = k == 0 ? (grad_points ? grad_points + (size_t)b * plane : nullptr)
                        : lam + (size_t)b * plane;
    const float delta = stage_delta<D, ADAPTIVE, TS>(rec, row, g);
    L.begin(Ag, Gg, R, nC * RevStride<D>::S, &touched_cnt);
    run_stage<D, ADAPTIVE, LDS_A, BINS, TS>(L, Ag, Gg, nP, T, g, io, moments + row * R, rec, row,
                                            delta);
    // Every lane is done with this stage's tables before they are written out
    // (and, for the next stage, overwritten).
    const size_t part = row * gridDim.x + w.part;
    L.end(partials + part * R, dense_parts + row * ((gridDim.x + 63) / 64), w.part,
          moments + row * R, nC, &touched_cnt);
    if (k > 0) __syncthreads();
  }
}

// Fused transform_data backward: one workgroup = one theta x one contiguous
// range of output positions.
template <int D, bool ADAPTIVE, bool LDS_A, int BINS, int TS>
__global__ __launch_bounds__((kBwdThreads<D, ADAPTIVE, TS>)) void image_backward_kernel(
    ImageShape s, int T, Cells g, int nC, const float* __restrict__ axes,
    const float* __restrict__ final_points, const float* __restrict__ seed_grad,
    const float* __restrict__ As,
    const float* __restrict__ Gs, Recover rec, const float* __restrict__ data,
    const float* __restrict__ grad_out,
    float* __restrict__ moments, float* __restrict__ partials, uint64_t* __restrict__ dense_parts,
    float* __restrict__ grad_data) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int touched_cnt;
  const WgSlot w = wg_slot();
  const int b = w.row;
  const int R = nC * Dim<D>::P;
  const StageLds<D, LDS_A, BINS> L(lds, R);
  const float* __restrict__ Ag = As + (size_t)b * R;
  const float* __restrict__ Gg = Gs + (size_t)b * nC * RevStride<D>::S;
  ImageIO<D> io;
  io.s = s;
  io.axes = axes;
  io.fin = final_points ? final_points + (size_t)b * D * s.nP : nullptr;
  io.sgrad = seed_grad ? seed_grad + (size_t)b * D * s.nP : nullptr;
  io.gout = grad_out + (size_t)b * s.C * s.nP;
  io.data = data + (size_t)b * s.C * s.plane_in;
  io.gdata = FloatScatter{grad_data ? grad_data + (size_t)b * s.C * s.plane_in : nullptr};
  const float delta = stage_delta<D, ADAPTIVE, TS>(rec, (size_t)b, g);
  L.begin(Ag, Gg, R, nC * RevStride<D>::S, &touched_cnt);
  run_stage<D, ADAPTIVE, LDS_A, BINS, TS>(L, Ag, Gg, s.nP, T, g, io, moments + (size_t)b * R, rec,
                                          (size_t)b, delta);
  const size_t part = (size_t)b * gridDim.x + w.part;
  L.end(partials + part * R, dense_parts + (size_t)b * ((gridDim.x + 63) / 64), w.part,
        moments + (size_t)b * R, nC, &touched_cnt);
}

template <int D, bool LDS_A, int BINS>
size_t stage_lds_bytes(int nC) {
  const size_t R = (size_t)nC * Dim<D>::P;
  size_t lds = LDS_A ? R * sizeof(float) : 0;
  if (full_bins(BINS)) lds += R * sizeof(float);
  if (BINS == kBinsFullRev) lds += (((R + 3) & ~(size_t)3) - R + (size_t)nC * RevStride<D>::S) * sizeof(float);
  if (BINS == kBinsCache) lds += (size_t)kCacheSlots * (Dim<D>::P + 1) * sizeof(float);
  return lds;
}

template <int D, bool ADAPTIVE, bool LDS_A, int BINS, int TS>
hipError_t go(const BackwardJob& j, const LaunchCfg& cfg, hipStream_t s) {
  const size_t lds = stage_lds_bytes<D, LDS_A, BINS>(j.geo.nC);
  const Cells g{j.geo.nx, j.geo.ny, j.geo.nz};
  const Recover rec{j.amp, adjoint_table_blocks(j.geo.nC),
                    (float)std::pow((double)kRecoverGrowth, 1.0 / (double)j.T), j.edge};
  const dim3 grid((unsigned)cfg.chunks, (unsigned)j.n_batch), block((unsigned)cfg.block);
  if (j.image) {
    auto kernel = image_backward_kernel<D, ADAPTIVE, LDS_A, BINS, TS>;
    hipError_t e = allow_lds(kernel, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, grid, block, lds, s, *j.image, j.T, g, j.geo.nC, j.axes,
                       j.final_points, j.seed_grad, j.As, j.G, rec, j.data, j.grad_out, j.moments,
                       j.partials, j.dense_parts, j.grad_data);
  } else {
    auto kernel = backward_kernel<D, ADAPTIVE, LDS_A, BINS, TS>;
    hipError_t e = allow_lds(kernel, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, grid, block, lds, s, (int)j.nP, j.batched, j.T, g, j.geo.nC, j.K,
                       j.points, j.stage_points, j.As, j.G, rec, j.grad_out, j.moments, j.partials,
                       j.dense_parts, j.lam, j.grad_points);
  }
  return hipGetLastError();
}

template <int D>
hipError_t dispatch(const BackwardJob& j, int adaptive, const LaunchCfg& cfg, hipStream_t s) {
#define CPAB_GO(AD, LA, LB, TS) return go<D, AD, LA, LB, TS>(j, cfg, s)
  // Register variant (the launch policy asks for it with full bins in 1D/2D,
  // and without adaptive substeps in 3D, whose 150 VGPRs of trajectory leave
  // no room for the adaptive step).
  if (cfg.reg_steps == kRegSteps && j.T == kRegSteps) {
    if constexpr (D <= 2) {
      if (cfg.lds_bins) {
        if (cfg.lds_rev) {
          if (adaptive) CPAB_GO(true, false, kBinsFullRev, kRegSteps);
          CPAB_GO(false, false, kBinsFullRev, kRegSteps);
        }
        if (adaptive) CPAB_GO(true, false, kBinsFull, kRegSteps);
        CPAB_GO(false, false, kBinsFull, kRegSteps);
      }
    } else {
      if (!adaptive) {
        if (cfg.lds_bins) CPAB_GO(false, false, kBinsFull, kRegSteps);
        CPAB_GO(false, false, kBinsCache, kRegSteps);
      }
    }
  }
  const int key = (adaptive ? 4 : 0) + (cfg.lds_table ? 2 : 0) + (cfg.lds_bins ? 1 : 0);
  switch (key) {
    case 0: CPAB_GO(false, false, kBinsCache, 0);
    case 1: CPAB_GO(false, false, kBinsFull, 0);
    case 2: CPAB_GO(false, true, kBinsCache, 0);
    case 3: CPAB_GO(false, true, kBinsFull, 0);
    case 4: CPAB_GO(true, false, kBinsCache, 0);
    case 5: CPAB_GO(true, false, kBinsFull, 0);
    case 6: CPAB_GO(true, true, kBinsCache, 0);
    default: CPAB_GO(true, true, kBinsFull, 0);
  }
#undef CPAB_GO
}

hipError_t dispatch_any(const BackwardJob& j, int adaptive, const LaunchCfg& cfg, hipStream_t s) {
  if (j.nP <= 0 || j.n_batch <= 0 || j.K <= 0) return hipSuccess;
  if (j.det_pass) return dispatch_det_any(j, adaptive, cfg, s);
  switch (j.geo.ndim) {
    case 1: return dispatch<1>(j, adaptive, cfg, s);
    case 2: return dispatch<2>(j, adaptive, cfg, s);
    default: return dispatch<3>(j, adaptive, cfg, s);
  }
}

}  // namespace

hipError_t launch_backward(const Geometry& g, int64_t nP, int64_t n_batch, int batched, int T,
                           int K, int adaptive, const float* points, const float* stage_points,
                           const float* As, const float* G, const float* amp,
                           const EdgeAcc* edge, const float* grad_out, float* moments,
                           float* partials, uint64_t* dense_parts, float* lam, float* grad_points,
                           const LaunchCfg& cfg, hipStream_t s, int det_pass, unsigned* det_stat,
                           unsigned long long* det_sums, unsigned* det_flags) {
  BackwardJob j{};
  j.det_pass = det_pass;
  j.det_stat = det_stat;
  j.det_sums = det_sums;
  j.det_flags = det_flags;
  j.edge = edge;
  j.geo = g;
  j.nP = nP;
  j.n_batch = n_batch;
  j.batched = batched;
  j.T = T;
  j.K = K;
  j.points = points;
  j.stage_points = stage_points;
  j.As = As;
  j.G = G;
  j.amp = amp;
  j.grad_out = grad_out;
  j.moments = moments;
  j.partials = partials;
  j.dense_parts = dense_parts;
  j.lam = lam;
  j.grad_points = grad_points;
  return dispatch_any(j, adaptive, cfg, s);
}

hipError_t launch_image_backward(const Geometry& g, const ImageShape& img, int64_t n_batch, int T,
                                 int adaptive, const float* axes, const float* final_points,
                                 const float* seed_grad,
                                 const float* As, const float* G, const float* amp,
                                 const EdgeAcc* edge, const float* data,
                                 const float* grad_out, float* moments, float* partials,
                                 uint64_t* dense_parts, float* grad_data, const LaunchCfg& cfg,
                                 hipStream_t s, int det_pass, unsigned* det_stat,
                                 unsigned long long* det_sums, unsigned* det_flags,
                                 const unsigned* det_gstat, unsigned long long* det_gsums) {
  BackwardJob j{};
  j.det_pass = det_pass;
  j.det_stat = det_stat;
  j.det_sums = det_sums;
  j.det_flags = det_flags;
  j.det_gstat = det_gstat;
  j.det_gsums = det_gsums;
  j.edge = edge;
  j.geo = g;
  j.nP = img.nP;
  j.n_batch = n_batch;
  j.T = T;
  j.K = 1;
  j.As = As;
  j.G = G;
  j.amp = amp;
  j.grad_out = grad_out;
  j.moments = moments;
  j.partials = partials;
  j.dense_parts = dense_parts;
  j.image = &img;
  j.axes = axes;
  j.final_points = final_points;
  j.seed_grad = seed_grad;
  j.data = data;
  j.grad_data = grad_data;
  return dispatch_any(j, adaptive, cfg, s);
}

}  // namespace cpab
