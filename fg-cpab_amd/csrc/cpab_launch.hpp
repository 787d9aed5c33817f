// Internal (C++) launch interface between the C-ABI layer (capi.cpp) and the
// kernel translation units.  Every launcher assumes its arguments were
// validated by the caller and only enqueues work on `stream`.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "cpab_sample.hpp"

namespace cpab {

struct EdgeAcc;  // cpab_device.hpp: one part of a row's domain-edge bound (4 doubles)
constexpr int kEdgeAccBytes = 32;
// Workgroup size and workgroups per CU of the deterministic backward passes,
// and the LDS of their second pass (adjoint_det.hip): a row's full table of 64-bit
// sums when it takes at most kDetFullBytes (an equal share of a CU's 160 KiB),
// else a hashed cache of kDetCacheSlots cells.  Per ndim: 1D/2D 512 threads,
// two per CU (16 waves at ~100 VGPRs); 3D 256 threads, four per CU (its
// ~150 VGPRs leave room for 3 waves per SIMD, which 512-thread groups waste).
constexpr int kDetBlock[4] = {0, 512, 512, 256};
constexpr int kDetPerCU[4] = {0, 2, 2, 4};
constexpr int64_t kDetFullBytes[4] = {0, (80 << 10) - 256, (80 << 10) - 256, (40 << 10) - 256};
constexpr int kDetCacheSlots[4] = {0, 1024, 1024, 256};
constexpr int64_t det_full_bytes_for(int ndim, int nC) {
  return (int64_t)nC * ndim * (ndim + 1) * 8;
}
constexpr int64_t det_cache_bytes_for(int ndim) {
  return (int64_t)kDetCacheSlots[ndim] * (ndim * (ndim + 1) * 8 + 4);
}

struct Geometry {
  int ndim;
  int nx, ny, nz;   // cells per axis (unused axes = 1)
  int nC;           // number of cells (nx | 4*nx*ny | 5*nx*ny*nz)
  int ppc() const { return ndim * (ndim + 1); }
};

// Resampling tiles: one workgroup of kInterpThreads per kInterpTile0 x
// kInterpTileLast block of (i0, i_last) outputs.  Swept at C3 (16 x 512^2) and
// C4 (128^3) against 64 x 32, 32 x 64, 16 x 64 (256 threads), 32 x 32 with 512
// threads and 16 x 32 with 128: 32 x 32 with 256 was fastest or within noise
// in both.
constexpr int kInterpTile0 = 32;
constexpr int kInterpTileLast = 32;
constexpr int kInterpThreads = 256;

// Launch shape, chosen per problem by the C-ABI layer (capi.cpp).
struct LaunchCfg {
  int block;        // threads per workgroup
  int chunks;       // workgroups per theta (gridDim.x)
  int lds_table;    // backward, segmented variant: stage the per-theta affine table in LDS
  int lds_bins;     // backward: accumulate moments in full LDS bins (per-workgroup partials)
  int lds_cache;    // backward: else accumulate in the hashed LDS cell cache
  int reg_steps;    // backward: compile-time step count of the register variant (0 = segmented)
  int lds_rev;      // backward, register variant with full bins: the reverse-sweep table in LDS too
};

hipError_t launch_fill(float* dst, int64_t n, float value, hipStream_t s);
hipError_t launch_affine(int64_t n_theta, int rows, int d, const float* theta,
                         const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                         float* As, hipStream_t s);
hipError_t launch_expm(int ndim, int64_t n, float dT, const float* As, float* Trels, hipStream_t s);
// launch_affine then launch_expm as one kernel (one thread per theta and cell).
hipError_t launch_affine_expm(int ndim, int64_t n_theta, int nC, int d, const float* theta,
                              const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                              float dT, float* As, float* Trels, hipStream_t s);
hipError_t launch_project(int64_t n_theta, int D, int d, const float* moments,
                          const int32_t* col_ptr, const int32_t* row_idx, const float* vals,
                          float* grad_theta, hipStream_t s);
// G [rows, nC, RevStride]: per cell h A + (h^2/2) A^2 and the inverse one-step
// map (cpab_device.hpp), h = 1/T; amp [rows, adjoint_table_blocks(nC)]: the
// largest ||M_c||_2 of the inverse maps over each block of a row's cells;
// ebound (2D, may be null) [rows, adjoint_table_blocks(nC)]: each block's part
// of the row's domain-edge bound of the replay maps (nx, ny: the 2D grid);
// zeroes moments [rows, nC, ppc] (the HBM sums) and dense_parts [n_words].
int adjoint_table_blocks(int nC);
hipError_t launch_adjoint_table(int ndim, int64_t rows, int nx, int ny, int nC, int T,
                                const float* As, float* G, float* moments, float* amp,
                                EdgeAcc* ebound, uint64_t* dense_parts, int64_t n_words,
                                hipStream_t s);
// moments [rows, nC, ppc] from the reverse sweep's per-cell sums S, in place:
// the HBM sums in `moments` plus the partial tables [rows, nparts, nC, ppc] of
// the parts set in dense_parts [rows, ceil(nparts/64)], in ascending order.
hipError_t launch_finish_moments(int ndim, int64_t rows, int nC, int nparts, int T,
                                 const float* partials, const uint64_t* dense_parts,
                                 const float* As, float* moments, hipStream_t s);
// The same from the deterministic reduction's integer sums and non-finite
// flags [rows, nC, ppc] and row stats (launch_backward with det_pass 1 then 2,
// nP trajectories per row).
hipError_t launch_finish_moments_det(int ndim, int64_t rows, int nC, int64_t nP, int T,
                                     const unsigned* det_stat, const unsigned long long* det_sums,
                                     const unsigned* det_flags, const float* As, float* moments,
                                     hipStream_t s);
hipError_t launch_sum_batch(int64_t n_theta, int64_t n, const float* src, float* dst, hipStream_t s);

hipError_t launch_forward_1d(const Geometry& g, int64_t nP, int64_t n_batch, int batched, int K,
                             const float* points, const float* As, float* out,
                             float* stage_points, hipStream_t s);
// K = number of chained stages (1 = one transform); tables hold K * n_batch rows,
// row = stage * n_batch + batch.  stage_points [K-1, n_batch, ndim, nP] may be null.
hipError_t launch_forward(const Geometry& g, int64_t nP, int64_t n_batch, int batched, int T,
                          int K, int adaptive, const float* points, const float* Trels,
                          const float* As, float* out, float* stage_points, const LaunchCfg& cfg,
                          hipStream_t s);
hipError_t launch_trace_cells(const Geometry& g, int64_t nP, int64_t n_theta, int batched, int T,
                              int adaptive, const float* points, const float* Trels,
                              const float* As, int32_t* cells, hipStream_t s);
// lam: [n_batch, ndim, nP] scratch carrying the adjoint between stages (K > 1).
// G, amp, edge: the reverse-sweep table, its per-block norms and (2D, may be
// null) the domain-edge bound parts from launch_adjoint_table, same rows as
// As; with edge, waves whose trajectories provably stay inside the domain
// replay them without the lookup's per-step edge test.  The register variant recovers
// positions through the inverse maps only for rows whose amplification bound
// (max ||M_c||_2)^T stays within kRecoverGrowth; other rows replay from
// checkpoints.
// The per-cell sums S go to moments (HBM sums, zero on entry) or, for a
// full-bin workgroup that touched a quarter of the cells or more, to its
// partial table [rows, chunks, nC, ppc] with its bit set in dense_parts
// [rows, ceil(chunks/64)] (zero on entry).  launch_finish_moments follows.
// det_pass 1, 2: the two passes of the deterministic reduction (segmented
// body, LDS cell cache of 64-bit integers; det_stat [rows], det_sums
// [rows, nC, ppc] and det_flags [rows, nC, ppc] zero before pass 1; partials
// and dense_parts unused), then launch_finish_moments_det.
hipError_t launch_backward(const Geometry& g, int64_t nP, int64_t n_batch, int batched, int T,
                           int K, int adaptive, const float* points, const float* stage_points,
                           const float* As, const float* G, const float* amp,
                           const EdgeAcc* edge, const float* grad_out, float* moments,
                           float* partials, uint64_t* dense_parts, float* lam, float* grad_points,
                           const LaunchCfg& cfg, hipStream_t s, int det_pass = 0,
                           unsigned* det_stat = nullptr, unsigned long long* det_sums = nullptr,
                           unsigned* det_flags = nullptr);

// Fused transform_data (image-ordered outputs; see cpab_sample.hpp ImageShape).
hipError_t launch_image_forward(const Geometry& g, const ImageShape& img, int64_t n_batch, int T,
                                int adaptive, const float* axes, const float* Trels,
                                const float* As, const float* data, float* out,
                                float* final_points, float* seed_grad, const LaunchCfg& cfg,
                                hipStream_t s);
hipError_t launch_image_backward(const Geometry& g, const ImageShape& img, int64_t n_batch, int T,
                                 int adaptive, const float* axes, const float* final_points,
                                 const float* seed_grad,
                                 const float* As, const float* G, const float* amp,
                                 const EdgeAcc* edge, const float* data,
                                 const float* grad_out, float* moments, float* partials,
                                 uint64_t* dense_parts, float* grad_data, const LaunchCfg& cfg,
                                 hipStream_t s, int det_pass = 0, unsigned* det_stat = nullptr,
                                 unsigned long long* det_sums = nullptr,
                                 unsigned* det_flags = nullptr, const unsigned* det_gstat = nullptr,
                                 unsigned long long* det_gsums = nullptr);
// Deterministic grad_data of the image backward: det_gstat [n_batch] (zero
// before) gets each batch row's largest finite |scatter contribution| from the
// final points and grad_out; det pass 2 of launch_image_backward then adds the
// contributions as 64-bit integers into det_gsums [n_batch, C, plane_in] (zero
// before), and launch_det_data_finish adds their float value into grad_data.
hipError_t launch_det_data_stat(int ndim, const ImageShape& img, int64_t n_batch,
                                const float* final_points, const float* grad_out,
                                unsigned* det_gstat, hipStream_t s);
hipError_t launch_det_data_finish(int ndim, const ImageShape& img, int64_t n_batch,
                                  const unsigned* det_gstat, const unsigned long long* det_gsums,
                                  float* grad_data, hipStream_t s);
// grad_data [B, per_row] += gsums / 2^shift_b (det_shift of gstat[b] for nP
// output positions of 2^ndim contributions each).
hipError_t launch_det_finish_rows(int ndim, int64_t n_batch, int64_t per_row, int64_t nP,
                                  const unsigned* gstat, const unsigned long long* gsums,
                                  float* grad_data, hipStream_t s);
// Cpab.interpolate's grad_data [B, C, *in_size] in the deterministic mode,
// from the grid [B, ndim, prod(out_size)] and grad_out [B, C, *out_size]:
// gstat [B] and gsums [B, C, prod(in_size)] zero, grad_data zero before.
hipError_t launch_det_interp_data(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                                  const int64_t* out_size, const float* grid,
                                  const float* grad_out, unsigned* gstat,
                                  unsigned long long* gsums, float* grad_data, hipStream_t s);

hipError_t launch_interp_forward(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                                 const int64_t* out_size, const float* data, const float* grid,
                                 float* out, hipStream_t s);
hipError_t launch_interp_backward(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                                  const int64_t* out_size, const float* data, const float* grid,
                                  const float* grad_out, float* grad_grid, float* grad_data,
                                  hipStream_t s);

}  // namespace cpab
