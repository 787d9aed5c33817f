/*
 * cpab_hip.h -- C ABI of the MI355X CPAB transform library (libcpab_hip.so).
 *
 * Drop-in replacement for the reference's pybind11 module `cpab_gpu`
 * (cpab/pytorch/transformer_cuda.cpp:172-179) and for the two torch.sparse.mm
 * calls and the torch interpolation ops around it.  Conventions:
 *
 *   - every pointer is a device pointer to contiguous float32 (or int32 index)
 *     memory owned by the caller; nothing is allocated by the library; the
 *     per-cell tables (As, Trels) and workspaces must be 16-byte aligned (they
 *     are read as vectors; misaligned ones are rejected with CPAB_ERR_INVALID);
 *   - `stream` is a hipStream_t (pass 0 for the null stream); all work is
 *     enqueued asynchronously on it;
 *   - the return value is CPAB_OK or an error code; argument checking happens
 *     before any HIP call, and cpab_last_error_string() gives the message of
 *     the calling thread's last failure (the reference raised RuntimeError via
 *     TORCH_CHECK, or exit()ed on a launch error, transformer_cuda.cu:12-18);
 *   - `batched` = 1 when points are [n_theta, ndim, nP], 0 when one [ndim, nP]
 *     set is shared by all thetas (the reference's `broadcast` flag,
 *     transformer_cuda.cpp:43);
 *   - size limits (CPAB_ERR_INVALID beyond them): fewer than 2^24 cells
 *     (cell ids and table offsets are 24/32-bit in the kernels), nP below
 *     2^31 / 3, n_theta (n_batch, n_stages * n_batch) below 65536, and at
 *     most 2^30 values per data channel of the image entry points (the
 *     gathers address a channel with 32-bit byte offsets).
 *
 * Layouts: theta [n_theta, d]; As/Trels [n_theta, nC, ndim, ndim+1] row-major;
 * moments [n_theta, nC, ndim*(ndim+1)]; points/outputs SoA rows [.., ndim, nP].
 */
#ifndef CPAB_HIP_H
#define CPAB_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CPAB_OK 0
#define CPAB_ERR_INVALID 1 /* bad argument: nothing was enqueued */
#define CPAB_ERR_DEVICE 2  /* HIP runtime / launch failure */

#define CPAB_MAX_STEPS 100 /* same cap as cpab/core/cpab_ops_2d.cuh:8 */

/* Message for the calling thread's last failed call ("" if none). */
const char* cpab_last_error_string(void);

/* ABI version (major*100 + minor).  400: the transform_data entry points take
 * seed_grad.  401: the deterministic mode (cpab_set_deterministic and the
 * workspace sizes and cpab_interp_backward_ws that go with it). */
int cpab_abi_version(void);

/* A = B theta per theta: As[b, r] = sum_k vals[k] * theta[b, col_idx[k]] over
 * the CSR row r of B (rows = nC*ndim*(ndim+1)).
 * Replaces torch.sparse.mm(B, theta^T) in cpab/pytorch/transformer.py:84. */
int cpab_affine(int ndim, int64_t n_theta, int nC, int d, const float* theta,
                const int32_t* row_ptr, const int32_t* col_idx, const float* vals,
                float* As, void* stream);

/* Trels = expm(dT * [A; 0]) for n_matrices affine blocks of shape [ndim, ndim+1].
 * Replaces cpab_gpu.expm, transformer_cuda.cpp:159-170. */
int cpab_expm(int ndim, int64_t n_matrices, float dT, const float* As, float* Trels,
              void* stream);

/* cpab_affine followed by cpab_expm(ndim, n_theta * nC, dT, As, Trels) in one
 * launch; both outputs equal the two-call sequence bit for bit.  Replaces the
 * reference forward's first two steps, sparse.mm(B, theta^T)
 * (cpab/pytorch/transformer.py:84) and cpab_gpu.expm (transformer_cuda.cpp:159-170). */
int cpab_affine_expm(int ndim, int64_t n_theta, int nC, int d, const float* theta,
                     const int32_t* row_ptr, const int32_t* col_idx, const float* vals, float dT,
                     float* As, float* Trels, void* stream);

/* Forward integration: out[b] = phi(points[b or shared]; theta_b), [n_theta, ndim, nP].
 * ndim 2/3: nstepsolver steps of Trels (+ Heun on crossings if adaptive);
 * ndim 1: the closed form (Trels unused), as the reference does.
 * Replaces cpab_gpu.forward, transformer_cuda.cpp:32-61. */
int cpab_forward(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                 int ncx, int ncy, int ncz, int adaptive, const float* points,
                 const float* Trels, const float* As, float* out, void* stream);

/* 1D closed-form forward.  Replaces cpab_gpu.forward_1d_closed_form,
 * transformer_cuda.cpp:66-85. */
int cpab_forward_1d_closed_form(int64_t nP, int64_t n_theta, int batched, int ncx,
                                const float* points, const float* As, float* out,
                                void* stream);

/* Debug / parity aid: the cell index visited at each of the nstepsolver steps
 * of cpab_forward (ndim 2/3) into cells [n_theta, nP, nstepsolver] int32.  No
 * reference counterpart (the reference exposes no trajectory); it makes the
 * visited-cell sequence of the fixed-step forward observable for tests. */
int cpab_trace_cells(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                     int ncx, int ncy, int ncz, int adaptive, const float* points,
                     const float* Trels, const float* As, int32_t* cells, void* stream);

/* Bytes of device workspace cpab_backward needs for this problem: per-cell
 * reverse-sweep tables (per cell and theta: the adjoint increment h*A + (h^2/2)*A^2 and the
 * inverse of the one-step map; 4, 12 or 24 floats)
 * and, where the sums are privatised per workgroup, the partial tables with
 * their touched-cell masks. */
int64_t cpab_backward_workspace_size(int ndim, int64_t nP, int64_t n_theta, int nC);

/* Fused backward: cell moments [n_theta, nC, ndim*(ndim+1)] (overwritten, no
 * need to zero them) and, if grad_points != NULL, the point adjoints
 * [n_theta, ndim, nP].  `workspace` must hold
 * cpab_backward_workspace_size(...) bytes.  The reverse sweep is the
 * reference's discrete adjoint (cpab_ops_2d.cu:334-382) in factored form, so
 * moments and point adjoints agree with it to rounding (a few ulp per step),
 * not bit for bit; the replayed trajectory and its cells are bit-exact.
 * Replaces cpab_gpu.backward_moments (transformer_cuda.cpp:92-116) and
 * cpab_gpu.backward_moments_and_points (transformer_cuda.cpp:122-153). */
int cpab_backward(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                  int ncx, int ncy, int ncz, int adaptive, const float* points,
                  const float* As, const float* grad_out, float* moments,
                  float* grad_points, void* workspace, int64_t workspace_bytes,
                  void* stream);

/* cpab_backward followed by cpab_project of its moments, in one call: moments
 * as cpab_backward writes them, grad_theta [n_theta, d] as
 * cpab_project(n_theta, nC*ndim*(ndim+1), d, moments, col_ptr, row_idx, vals,
 * ...) writes it, bit for bit.  Replaces the
 * reference backward's cpab_gpu.backward_moments[_and_points] call and the
 * torch.sparse.mm projection after it (cpab/pytorch/transformer.py:141-166). */
int cpab_backward_project(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                          int ncx, int ncy, int ncz, int adaptive, const float* points,
                          const float* As, const float* grad_out, int d, const int32_t* col_ptr,
                          const int32_t* row_idx, const float* vals, float* moments,
                          float* grad_theta, float* grad_points, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* Deterministic backward, for debugging (no counterpart in the reference,
 * whose float atomics make the theta gradients vary in their last bits from
 * run to run: stn/demos/demo_classify_2d.py:7-10).  With on != 0, the backward
 * entry points called afterwards from the calling thread (cpab_backward,
 * cpab_backward_project, cpab_backward_noalloc, cpab_chain_backward,
 * cpab_transform_data_backward) reduce the per-cell sums in two passes over
 * the trajectories: the first finds each theta row's largest flushed value,
 * the second adds every value as a 64-bit integer at a per-row power-of-two
 * scale (integer sums do not depend on their order), so moments, theta
 * gradients and point adjoints are the same bit for bit on every run on the
 * same device.  They equal the default mode's to its tolerance (the integer
 * quantum is 2^-(62 - ceil(log2(nP * nstepsolver))) of the row's largest
 * value); a component that sums non-finite values is +inf, -inf or NaN as
 * the float sum would be.  grad_data of cpab_transform_data_backward is
 * summed the same way (64-bit integers at each batch row's scale, from its
 * largest scatter contribution; non-finite terms as floats), which takes
 * cpab_transform_data_backward_data_workspace_size(...) more bytes of
 * workspace (CPAB_ERR_INVALID without them); cpab_interp_backward_ws does
 * the same for the resampling's grad_data.  Both passes take the default's
 * bodies; the benchmark steps take 1.8-2.2x their default time.  The
 * *_workspace_size functions size the workspace of the calling thread's
 * current mode. */
void cpab_set_deterministic(int on);
int cpab_deterministic(void);

/* Device memory the library keeps per GPU for cpab_backward_noalloc. */
#define CPAB_NOALLOC_SCRATCH_BYTES (32LL << 20)

/* Allocation-free cpab_backward.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * results and kernels as cpab_backward without the workspace: the workspace
 * is a library-owned device array of CPAB_NOALLOC_SCRATCH_BYTES on each GPU
 * (held until the process ends), and the call allocates nothing.  A problem
 * is rejected with CPAB_ERR_INVALID, before anything is enqueued, when the
 * workspace of the backward variant that will run for it exceeds that size;
 * that workspace is at most cpab_backward_workspace_size(...), which also
 * covers the other variant, so a problem within the limit by that size is
 * always accepted and some above it are too.  Every call on one GPU uses
 * that GPU's one array: calls that overlap on a GPU (other streams, other
 * host threads) race and must be serialised by the caller.  Kernel timing
 * (cpab_profile_enable) does not cover these calls. */
int cpab_backward_noalloc(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                          int ncx, int ncy, int ncz, int adaptive, const float* points,
                          const float* As, const float* grad_out, float* moments,
                          float* grad_points, void* stream);

/* Chain of n_stages transforms (cpab/cpab.py:237-280, Cpab.transform_grid_chain:
 * stage s maps the output of stage s-1 with theta_chain[s]; the reference runs
 * one cpab_gpu.forward per stage from a Python loop).  Tables hold
 * n_stages * n_batch rows, row = s * n_batch + b ([n_stages, n_batch, nC,
 * ndim, ndim+1]); points as in cpab_forward (shared or batched) feed stage 0.
 * out [n_batch, ndim, nP].  If stage_points is not NULL it receives the input
 * of every stage s >= 1, [n_stages-1, n_batch, ndim, nP], which
 * cpab_chain_backward needs.  Each stage's arithmetic is that of cpab_forward,
 * so the result equals n_stages chained cpab_forward calls bit for bit.
 * ndim 1 uses the closed form per stage (Trels unused, may be NULL). */
int cpab_chain_forward(int ndim, int64_t nP, int64_t n_batch, int batched, int n_stages,
                       int nstepsolver, int ncx, int ncy, int ncz, int adaptive,
                       const float* points, const float* Trels, const float* As, float* out,
                       float* stage_points, void* stream);

/* Bytes of device workspace cpab_chain_backward needs (adjoint increments,
 * partial tables and the adjoint carried between stages). */
int64_t cpab_chain_backward_workspace_size(int ndim, int64_t nP, int64_t n_batch, int n_stages,
                                           int nC);

/* Backward of cpab_chain_forward in one launch: replaces the n_stages
 * autograd nodes of the reference's chain, each a
 * cpab_gpu.backward_moments_and_points call (transformer_cuda.cpp:122-153)
 * whose grad_points seeds the stage below, and their projections
 * (transformer.py:165-166).  moments [n_stages, n_batch, nC, ndim*(ndim+1)]
 * (overwritten); grad_theta (may be NULL) [n_stages, n_batch, d]: each row's
 * moments projected through B's CSC tables (col_ptr, row_idx, vals, as
 * cpab_project takes them; ignored when grad_theta is NULL); grad_points (may
 * be NULL) = adjoint of the stage-0 input points, [n_batch, ndim, nP] (sum
 * over n_batch for shared points, as cpab_sum_batch does).  stage_points as
 * written by cpab_chain_forward (may be NULL when n_stages == 1). */
int cpab_chain_backward(int ndim, int64_t nP, int64_t n_batch, int batched, int n_stages,
                        int nstepsolver, int ncx, int ncy, int ncz, int adaptive,
                        const float* points, const float* stage_points, const float* As,
                        const float* grad_out, int d, const int32_t* col_ptr,
                        const int32_t* row_idx, const float* vals, float* moments,
                        float* grad_theta, float* grad_points, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* grad_theta[b, j] = sum_k vals[k] * moments[b, row_idx[k]] over the CSC column
 * j of B (D = rows of B).  Replaces torch.sparse.mm(B^T, M^T) in
 * cpab/pytorch/transformer.py:165-166. */
int cpab_project(int64_t n_theta, int D, int d, const float* moments,
                 const int32_t* col_ptr, const int32_t* row_idx, const float* vals,
                 float* grad_theta, void* stream);

/* dst[i] = sum_b src[b, i] (b ascending).  Replaces grad_points.sum(0) for
 * shared points, cpab/pytorch/transformer.py:151-152. */
int cpab_sum_batch(int64_t n_theta, int64_t n, const float* src, float* dst, void* stream);

/* Fused Cpab.transform_data forward (cpab/cpab.py:295-309: uniform_meshgrid ->
 * transform_grid -> interpolate, i.e. cpab_forward followed by
 * cpab_interp_forward).  axes: the uniform grid's coordinates per axis,
 * concatenated (out_size[0] values of coordinate 0, then out_size[1] of
 * coordinate 1, ...), whose Cartesian product is uniform_meshgrid(out_size),
 * shared by all n_batch thetas; Trels / As
 * [n_batch, nC, ndim, ndim+1] (Trels unused in 1D, may be NULL); data
 * [n_batch, C, *in_size]; out [n_batch, C, *out_size].  Each output pixel
 * integrates its meshgrid point with cpab_forward's arithmetic and samples
 * data there with cpab_interp_forward's, so out equals the unfused pair bit
 * for bit.  final_points (may be NULL): the integrated points
 * [n_batch, ndim, prod(out_size)] in IMAGE order (last output axis fastest),
 * which cpab_transform_data_backward takes.  seed_grad (may be NULL; only
 * with n_channels == 1): the sample's spatial gradient d out / d x_k at each
 * integrated point, before the (in_size[k] - 1) chain factor, same layout,
 * from which the backward seeds each pixel's adjoint without re-reading data.
 * No counterpart entry point in the reference, whose transform_data is three
 * separate steps. */
int cpab_transform_data_forward(int ndim, int64_t n_batch, int64_t n_channels,
                                const int64_t* in_size, const int64_t* out_size, int nstepsolver,
                                int ncx, int ncy, int ncz, int adaptive, const float* axes,
                                const float* Trels, const float* As, const float* data,
                                float* out, float* final_points, float* seed_grad, void* stream);

/* Bytes of device workspace cpab_transform_data_backward needs. */
int64_t cpab_transform_data_backward_workspace_size(int ndim, int64_t n_batch,
                                                    const int64_t* out_size, int nC);

/* Additional workspace bytes cpab_transform_data_backward needs for
 * grad_data in the deterministic mode (no counterpart in the reference; for
 * the callers of cpab_set_deterministic): 0 in the default mode; in the
 * calling thread's deterministic mode, a 64-bit integer sum per grad_data
 * element (n_batch * n_channels * prod(in_size) * 8 bytes and a few hundred
 * more).  A deterministic backward that is given grad_data needs this and
 * cpab_transform_data_backward_workspace_size(...) added together. */
int64_t cpab_transform_data_backward_data_workspace_size(int ndim, int64_t n_batch,
                                                         int64_t n_channels,
                                                         const int64_t* in_size);

/* Backward of cpab_transform_data_forward in one launch: the resampling
 * gradient at each final point (the interp backward, summed over channels)
 * seeds the adjoint of that pixel's trajectory, as the reference's autograd
 * does through interpolate's backward and cpab_gpu.backward_moments_and_points
 * (transformer_cuda.cpp:122-153), then the projection
 * (transformer.py:165-166).  moments [n_batch, nC, ndim*(ndim+1)]
 * (overwritten); grad_theta (may be NULL) [n_batch, d] through B's CSC tables
 * as in cpab_chain_backward; grad_data [n_batch, C, *in_size] (may be NULL;
 * overwritten).  grad_out is the image gradient [n_batch, C, *out_size]; axes
 * as for the forward.  The seed comes from seed_grad when it is given (as the
 * forward wrote it; n_channels == 1), else from final_points and data;
 * final_points is required unless seed_grad is given and grad_data is NULL.
 * With seed_grad the seed's x term (2D) rounds differently from the
 * resampling backward's, within the backward's tolerance. */
int cpab_transform_data_backward(int ndim, int64_t n_batch, int64_t n_channels,
                                 const int64_t* in_size, const int64_t* out_size, int nstepsolver,
                                 int ncx, int ncy, int ncz, int adaptive, const float* axes,
                                 const float* final_points, const float* seed_grad,
                                 const float* As, const float* data,
                                 const float* grad_out, int d, const int32_t* col_ptr,
                                 const int32_t* row_idx, const float* vals, float* moments,
                                 float* grad_theta, float* grad_data, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/* Border-clamped linear/bilinear/trilinear resampling of data
 * [n_batch, C, *in_size] at grid [n_batch, ndim, prod(out_size)] (coordinate 0
 * fastest) into out [n_batch, C, *out_size].
 * Replaces cpab/pytorch/interpolation.py:3-159 (forward). */
int cpab_interp_forward(int ndim, int64_t n_batch, int64_t n_channels, const int64_t* in_size,
                        const int64_t* out_size, const float* data, const float* grid,
                        float* out, void* stream);

/* Backward of cpab_interp_forward: grad_grid [n_batch, ndim, nP] (may be NULL)
 * and grad_data [n_batch, C, *in_size] (may be NULL; overwritten).
 * Replaces the torch autograd backward of interpolation.py:3-159. */
int cpab_interp_backward(int ndim, int64_t n_batch, int64_t n_channels, const int64_t* in_size,
                         const int64_t* out_size, const float* data, const float* grid,
                         const float* grad_out, float* grad_grid, float* grad_data,
                         void* stream);

/* Workspace bytes cpab_interp_backward_ws needs for grad_data: 0 in the
 * default mode; in the calling thread's deterministic mode
 * (cpab_set_deterministic) a 64-bit integer sum per grad_data element
 * (B * C * prod(in_size) * 8 bytes and a few hundred more).  No counterpart
 * in the reference; for the callers of cpab_set_deterministic. */
int64_t cpab_interp_backward_workspace_size(int ndim, int64_t B, int64_t C,
                                            const int64_t* in_size);

/* cpab_interp_backward with a workspace (no counterpart in the reference).
 * In the calling thread's deterministic mode, grad_data (when requested) is
 * summed as 64-bit integers at each batch row's scale, from its largest
 * scatter contribution (non-finite terms as floats), so it is the same on
 * every run; the workspace must hold cpab_interp_backward_workspace_size(...)
 * bytes.  Otherwise it is cpab_interp_backward (the workspace unused). */
int cpab_interp_backward_ws(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                            const int64_t* out_size, const float* data, const float* grid,
                            const float* grad_out, float* grad_grid, float* grad_data,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* Kernel timing for benchmarks (no reference counterpart; the reference timed
 * with torch.cuda.synchronize + perf_counter, benchmarks/benchmark_transformer.py:76-84).
 * While enabled, HIP events are recorded on the launch stream around the
 * hot kernels ("forward": the forward integrator, fixed-step or 1D closed form;
 * "backward": the fused replay/adjoint kernel; "interp_forward" /
 * "interp_backward": the resampling kernels; "image_forward" /
 * "image_backward": the fused transform_data kernels).  cpab_profile_read waits for and sums the
 * recorded launches of one kernel and forgets them. */
void cpab_profile_enable(int on);
int cpab_profile_read(const char* kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* CPAB_HIP_H */
