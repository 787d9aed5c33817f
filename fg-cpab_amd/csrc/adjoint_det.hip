// Deterministic backward (cpab_set_deterministic): the default backward's
// trajectory bodies (backward_body.hpp) run twice with integer sinks; see
// the comment below.
//
// In the integer pass the register variant's reverse sweep is too large to
// unroll fully (a 64-bit conversion and probe at each of its 50 possible
// flushes); the compiler unrolls it in part and reads the cells through
// indexed register moves.  A build with the unroll limit raised ran the same
// (C2 to C5) at twice the code size, so the remark is silenced here.
#pragma clang diagnostic ignored "-Wpass-failed"
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include "cpab_device.hpp"
#include "cpab_launch.hpp"
#include "cpab_sample.hpp"
#include "backward_body.hpp"

namespace cpab {
namespace {

// ---------------------------------------------------------------------------
// Deterministic reduction (opt in: cpab_set_deterministic).  Float atomics add
// the runs' sums in whatever order the lanes, waves and workgroups reach them,
// so the last bits of the moments vary from run to run.  Here the backward
// runs twice over the same trajectories, with the same bodies and launch
// shape, so both passes flush the same values.  Pass 0 records each row's
// largest finite |flushed value| (an atomic max: the same result in any
// order).  Pass 1 adds every finite flushed value as a 64-bit integer,
// rint(value * 2^s) with the row's scale 2^s, into LDS (the row's full table
// or a cell cache) and HBM: integer adds give the same sums in any order.
// The scale leaves the sums of all of a row's flushes below 2^62 in magnitude
// (det_shift), so none overflows; the quantum is 2^-(62 - lg) of the row's
// largest value, lg = ceil(log2(nP T)).  A non-finite value sets its component's flag instead
// (bit 0 +inf, bit 1 -inf, bit 2 NaN, an atomic or), and the finish gives
// that component the float sum's result: +inf, -inf or NaN.  The finish
// divides the integer sums by the scale.
// ---------------------------------------------------------------------------
template <int D> constexpr int kDetSlots = kDetCacheSlots[D];
template <int D> constexpr int kDetThreads = kDetBlock[D];

// Dynamic LDS of a pass: none for pass 0; for pass 1 the row's full table
// (FULL, direct-indexed by cell) or the hashed cache of kDetSlots cells.
template <int D, int PASS, bool FULL>
size_t det_lds_bytes(int nC) {
  constexpr int P = Dim<D>::P;
  if (PASS == 0) return 0;
  if (FULL) return (size_t)nC * P * sizeof(unsigned long long);
  return (size_t)kDetSlots<D> * (P * sizeof(unsigned long long) + sizeof(int));
}
static_assert(det_cache_bytes_for(1) == (int64_t)kDetSlots<1> * (2 * 8 + 4) &&
                  det_cache_bytes_for(2) == (int64_t)kDetSlots<2> * (6 * 8 + 4) &&
                  det_cache_bytes_for(3) == (int64_t)kDetSlots<3> * (12 * 8 + 4),
              "the host's LDS size is the kernel's");

template <int D, int PASS, bool FULL>
struct DetSink {
  static constexpr bool kSpread = false;
  int* keys;                               // LDS [kDetSlots] (cache)
  unsigned long long* vals;                // LDS [nC * P] (FULL) or [kDetSlots * P] (cache)
  unsigned long long* __restrict__ mom;    // HBM sums of this row [nC * P]
  unsigned* wg_max;                        // LDS
  unsigned* __restrict__ flags;            // HBM non-finite flags of this row [nC * P]
  int shift;                               // the row's scale exponent (det_shift)
  __device__ __forceinline__ void operator()(int c, const float (&m)[Dim<D>::P]) const {
    constexpr int P = Dim<D>::P;
    if constexpr (PASS == 0) {
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < P; ++k)
        if (__builtin_isfinite(m[k])) a = fmaxf(a, fabsf(m[k]));
      __hip_atomic_fetch_max(wg_max, __float_as_uint(a), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
      unsigned long long q[P];
      bool fin = true;
#pragma unroll
      for (int k = 0; k < P; ++k) fin = fin && __builtin_isfinite(m[k]);
      if (__builtin_expect(fin, 1)) {
#pragma unroll
        for (int k = 0; k < P; ++k) q[k] = det_fixed(m[k], shift);
      } else {
#pragma unroll
        for (int k = 0; k < P; ++k) {
          const bool f = __builtin_isfinite(m[k]);
          q[k] = f ? det_fixed(m[k], shift) : 0ull;
          if (!f)
            __hip_atomic_fetch_or(flags + (size_t)c * P + k,
                                  m[k] != m[k] ? 4u : (m[k] > 0.0f ? 1u : 2u), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if constexpr (FULL) {
#pragma unroll
        for (int j = 0; j < P; ++j)
          __hip_atomic_fetch_add(vals + (size_t)c * P + j, q[j], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
        return;
      }
      int slot = c & (kDetSlots<D> - 1);
      for (int probe = 0; probe < kCacheProbes; ++probe) {
        int k = __hip_atomic_load(keys + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (k == -1) {
          int expected = -1;
          __hip_atomic_compare_exchange_strong(keys + slot, &expected, c, __ATOMIC_RELAXED,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          k = expected == -1 ? c : expected;
        }
        if (k == c) {
#pragma unroll
          for (int j = 0; j < P; ++j)
            __hip_atomic_fetch_add(vals + (size_t)slot * P + j, q[j], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
          return;
        }
        slot = (slot + 1) & (kDetSlots<D> - 1);
      }
#pragma unroll
      for (int j = 0; j < P; ++j)
        __hip_atomic_fetch_add(mom + (size_t)c * P + j, q[j], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
  }
};

// Clears the workgroup maximum (pass 0) or the LDS sums (pass 1) before a
// stage, then, after it, publishes them: pass 0 the maximum into the row's
// stat, pass 1 the nonzero sums into the row's HBM sums.
template <int D, int PASS, bool FULL>
struct DetLds {
  int* keys;
  unsigned long long* vals;
  unsigned* wg_max;
  int nC;
  __device__ __forceinline__ int n_vals() const {
    return FULL ? nC * Dim<D>::P : kDetSlots<D> * Dim<D>::P;
  }
  __device__ __forceinline__ void begin() const {
    if constexpr (PASS == 0) {
      if (threadIdx.x == 0) *wg_max = 0u;
    } else {
      if constexpr (!FULL)
        for (int i = threadIdx.x; i < kDetSlots<D>; i += blockDim.x) keys[i] = -1;
      for (int i = threadIdx.x; i < n_vals(); i += blockDim.x) vals[i] = 0ull;
    }
    __syncthreads();
  }
  __device__ __forceinline__ void end(unsigned* __restrict__ stat,
                                      unsigned long long* __restrict__ mom) const {
    constexpr int P = Dim<D>::P;
    __syncthreads();
    if constexpr (PASS == 0) {
      if (threadIdx.x == 0 && *wg_max != 0u)
        __hip_atomic_fetch_max(stat, *wg_max, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      for (int i = threadIdx.x; i < n_vals(); i += blockDim.x) {
        const int c = FULL ? i / P : keys[i / P];
        if (c >= 0 && vals[i] != 0ull)
          __hip_atomic_fetch_add(mom + (size_t)c * P + (i % P), vals[i], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
};

// grad_data of the deterministic image backward (pass 1): every finite
// contribution added as a 64-bit integer rint(v * 2^shift) into `q`, the
// batch row's integer sums, at the row's scale; a non-finite one as a float
// atomic into grad_data itself (`f`, zero before), whose sum of +inf, -inf and
// NaN terms is the same in any order.  det_data_finish adds the two.
struct FixedScatter {
  unsigned long long* __restrict__ q;
  float* __restrict__ f;
  int shift;
  __device__ __forceinline__ bool on() const { return q != nullptr; }
  __device__ __forceinline__ FixedScatter channel(int64_t off) const {
    return {q + off, f + off, shift};
  }
  __device__ __forceinline__ void add(int i, float v) const {
    if (__builtin_isfinite(v))
      __hip_atomic_fetch_add(q + i, det_fixed(v, shift), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    else
      add_at(f, i, v);
  }
};

// The largest finite |contribution| of a scatter, through the same arithmetic.
struct AbsMaxSink {
  float* m;
  __device__ __forceinline__ void add(int, float v) const {
    if (__builtin_isfinite(v)) *m = fmaxf(*m, fabsf(v));
  }
};

// A deterministic pass's body: the register variant where the default
// backward takes it (T == TS > 0; without adaptive substeps only for rows whose
// positions may be recovered), else the segmented one.
template <int D, bool ADAPTIVE, int TS, typename P, typename IO, typename Sink>
__device__ __forceinline__ void det_body(P tab, const float* __restrict__ gtab, int nP, int T,
                                         const Cells& g, const IO& io, const Sink& sink,
                                         const Recover& rec, size_t row) {
  if constexpr (TS > 0) {
    if (ADAPTIVE || recover_ok(rec.amp + row * rec.namp, rec.namp, rec.amp_max))
      register_body<D, ADAPTIVE, TS>(tab, gtab, nP, g, io, sink, INFINITY);
    else
      segmented_run<D, ADAPTIVE, (TS + kSeg - 1) / kSeg>(tab, gtab, nP, TS, g, io, sink);
  } else {
    segmented_run<D, ADAPTIVE, kMaxSeg>(tab, gtab, nP, T, g, io, sink);
  }
}

template <int D, bool ADAPTIVE, int PASS, bool FULL, int TS>
__global__ __launch_bounds__(kDetThreads<D>) void det_backward_kernel(
    int nP, int batched, int T, Cells g, int nC, int K, const float* __restrict__ points,
    const float* __restrict__ stage_points, const float* __restrict__ As,
    const float* __restrict__ Gs, Recover rec, const float* __restrict__ grad_out,
    unsigned* __restrict__ stat, unsigned long long* __restrict__ sums,
    unsigned* __restrict__ flags, float* __restrict__ lam, float* __restrict__ grad_points) {
  extern __shared__ __align__(16) unsigned long long det_lds[];
  __shared__ unsigned wg_max;
  constexpr int P = Dim<D>::P;
  const DetLds<D, PASS, FULL> L{reinterpret_cast<int*>(det_lds + (size_t)kDetSlots<D> * P),
                                det_lds, &wg_max, nC};
  const WgSlot w = wg_slot();
  const int b = w.row;
  const int n_batch = gridDim.y;
  const int R = nC * P;
  const size_t plane = (size_t)D * nP;
  for (int k = K - 1; k >= 0; --k) {
    const size_t row = (size_t)k * n_batch + b;
    PlainIO<D> io;
    io.nP = nP;
    io.pts = k == 0 ? points + (batched ? (size_t)b * plane : 0)
                    : stage_points + ((size_t)(k - 1) * n_batch + b) * plane;
    io.gout = k == K - 1 ? grad_out + (size_t)b * plane : lam + (size_t)b * plane;
    io.lam_out = k == 0 ? (grad_points ? grad_points + (size_t)b * plane : nullptr)
                        : lam + (size_t)b * plane;
    const int shift = PASS == 0 ? 0 : det_shift(stat[row], nP, T);
    L.begin();
    det_body<D, ADAPTIVE, TS>(
        As + row * R, Gs + row * nC * RevStride<D>::S, nP, T, g, io,
        DetSink<D, PASS, FULL>{L.keys, L.vals, sums + row * R, L.wg_max, flags + row * R, shift},
        rec, row);
    L.end(stat + row, sums + row * R);
    if (k > 0) __syncthreads();
  }
}

template <int D, bool ADAPTIVE, int PASS, bool FULL, int TS>
__global__ __launch_bounds__(kDetThreads<D>) void det_image_backward_kernel(
    ImageShape s, int T, Cells g, int nC, const float* __restrict__ axes,
    const float* __restrict__ final_points, const float* __restrict__ seed_grad,
    const float* __restrict__ As, const float* __restrict__ Gs, Recover rec,
    const float* __restrict__ data,
    const float* __restrict__ grad_out, unsigned* __restrict__ stat,
    unsigned long long* __restrict__ sums, unsigned* __restrict__ flags,
    float* __restrict__ grad_data, const unsigned* __restrict__ gstat,
    unsigned long long* __restrict__ gsums) {
  extern __shared__ __align__(16) unsigned long long det_lds[];
  __shared__ unsigned wg_max;
  constexpr int P = Dim<D>::P;
  const DetLds<D, PASS, FULL> L{reinterpret_cast<int*>(det_lds + (size_t)kDetSlots<D> * P),
                                det_lds, &wg_max, nC};
  const WgSlot w = wg_slot();
  const int b = w.row;
  const int R = nC * P;
  ImageIO<D, FixedScatter> io;
  io.s = s;
  io.axes = axes;
  io.fin = final_points ? final_points + (size_t)b * D * s.nP : nullptr;
  io.sgrad = seed_grad ? seed_grad + (size_t)b * D * s.nP : nullptr;
  io.gout = grad_out + (size_t)b * s.C * s.nP;
  io.data = data + (size_t)b * s.C * s.plane_in;
  // grad_data is scattered once, in pass 1, at the batch row's scale for at
  // most 2^D contributions per output position into one element
  const size_t goff = (size_t)b * s.C * s.plane_in;
  io.gdata = (PASS == 1 && grad_data)
                 ? FixedScatter{gsums + goff, grad_data + goff, det_shift(gstat[b], s.nP, 1 << D)}
                 : FixedScatter{nullptr, nullptr, 0};
  const int shift = PASS == 0 ? 0 : det_shift(stat[b], s.nP, T);
  L.begin();
  det_body<D, ADAPTIVE, TS>(As + (size_t)b * R, Gs + (size_t)b * nC * RevStride<D>::S, s.nP, T, g,
                            io,
                            DetSink<D, PASS, FULL>{L.keys, L.vals, sums + (size_t)b * R, L.wg_max,
                                                   flags + (size_t)b * R, shift},
                            rec, (size_t)b);
  L.end(stat + b, sums + (size_t)b * R);
}

template <int D, bool ADAPTIVE, int PASS, bool FULL, int TS>
hipError_t go_det(const BackwardJob& j, const LaunchCfg& cfg, hipStream_t s) {
  const size_t lds = det_lds_bytes<D, PASS, FULL>(j.geo.nC);
  const Cells g{j.geo.nx, j.geo.ny, j.geo.nz};
  const Recover rec{j.amp, adjoint_table_blocks(j.geo.nC),
                    (float)std::pow((double)kRecoverGrowth, 1.0 / (double)j.T), nullptr};
  const dim3 grid((unsigned)cfg.chunks, (unsigned)j.n_batch), block((unsigned)kDetThreads<D>);
  if (j.image) {
    auto kernel = det_image_backward_kernel<D, ADAPTIVE, PASS, FULL, TS>;
    hipError_t e = allow_lds(kernel, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, grid, block, lds, s, *j.image, j.T, g, j.geo.nC, j.axes,
                       j.final_points, j.seed_grad, j.As, j.G, rec, j.data, j.grad_out,
                       j.det_stat, j.det_sums, j.det_flags, j.grad_data, j.det_gstat,
                       j.det_gsums);
  } else {
    auto kernel = det_backward_kernel<D, ADAPTIVE, PASS, FULL, TS>;
    hipError_t e = allow_lds(kernel, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, grid, block, lds, s, (int)j.nP, j.batched, j.T, g, j.geo.nC, j.K,
                       j.points, j.stage_points, j.As, j.G, rec, j.grad_out, j.det_stat,
                       j.det_sums, j.det_flags, j.lam, j.grad_points);
  }
  return hipGetLastError();
}

// Both passes must flush the same values, so they take the same body: the
// register variant for T == kRegSteps, with adaptive substeps only in 1D/2D
// with full tables (as the default backward; with the cache its unrolled
// steps do not fit in registers).
template <int D, bool ADAPTIVE, int PASS, bool FULL>
hipError_t go_det_steps(const BackwardJob& j, const LaunchCfg& cfg, hipStream_t s) {
  if constexpr (D == 3 && ADAPTIVE) {
    return go_det<D, ADAPTIVE, PASS, FULL, 0>(j, cfg, s);
  } else if constexpr (ADAPTIVE && PASS == 1 && !FULL) {
    return go_det<D, ADAPTIVE, PASS, FULL, 0>(j, cfg, s);
  } else {
    if (j.T == kRegSteps && (!ADAPTIVE || cfg.lds_bins))
      return go_det<D, ADAPTIVE, PASS, FULL, kRegSteps>(j, cfg, s);
    return go_det<D, ADAPTIVE, PASS, FULL, 0>(j, cfg, s);
  }
}

// Pass 0 needs no LDS table (FULL false); pass 1 takes cfg.lds_bins: the
// row's full table in LDS, else the cache.
template <int D>
hipError_t dispatch_det(const BackwardJob& j, int adaptive, const LaunchCfg& cfg, hipStream_t s) {
  if (j.det_pass == 1)
    return adaptive ? go_det_steps<D, true, 0, false>(j, cfg, s)
                    : go_det_steps<D, false, 0, false>(j, cfg, s);
  if (cfg.lds_bins)
    return adaptive ? go_det_steps<D, true, 1, true>(j, cfg, s)
                    : go_det_steps<D, false, 1, true>(j, cfg, s);
  return adaptive ? go_det_steps<D, true, 1, false>(j, cfg, s)
                  : go_det_steps<D, false, 1, false>(j, cfg, s);
}

// gstat[b]: the bits of the largest finite |contribution| of batch row b's
// grad_data scatter (the scatter's own arithmetic, AbsMaxSink), over every
// output position and channel; zero before.  One thread per output position.
template <int D>
__global__ __launch_bounds__(256) void det_data_stat_kernel(ImageShape s,
                                                            const float* __restrict__ fin,
                                                            const float* __restrict__ gout,
                                                            unsigned* __restrict__ gstat) {
  const int b = blockIdx.y;
  float m = 0.0f;
  const float* fb = fin + (size_t)b * D * s.nP;
  const float* gb = gout + (size_t)b * s.C * s.nP;
  for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < s.nP; q += gridDim.x * blockDim.x) {
    const Axis ax = axis_of(fb[q], s.in[0]);
    const Axis ay = D >= 2 ? axis_of(fb[q + (size_t)s.nP], s.in[1]) : Axis{0, 0, 0.0f};
    const Axis az = D == 3 ? axis_of(fb[q + 2 * (size_t)s.nP], s.in[2]) : Axis{0, 0, 0.0f};
    for (int c = 0; c < s.C; ++c)
      scatter_to<D>(s.in, AbsMaxSink{&m}, ax, ay, az, gb[(size_t)c * s.nP + q]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (__lane_id() == 0 && m > 0.0f)
    __hip_atomic_fetch_max(gstat + b, __float_as_uint(m), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// grad_data[b, i] = gsums[b, i] / 2^shift_b + grad_data[b, i] (the non-finite
// contributions' float sum, else zero).
__global__ __launch_bounds__(256) void det_data_finish_kernel(int64_t per_row, int nP, int ndim,
                                                              const unsigned* __restrict__ gstat,
                                                              const unsigned long long* __restrict__ gsums,
                                                              float* __restrict__ grad_data) {
  const int b = blockIdx.y;
  const int shift = det_shift(gstat[b], nP, 1 << ndim);
  const size_t base = (size_t)b * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < per_row;
       i += (int64_t)gridDim.x * blockDim.x)
    grad_data[base + i] =
        (float)ldexp((double)(long long)gsums[base + i], -shift) + grad_data[base + i];
}

// Cpab.interpolate's data gradient in the deterministic mode, per grid point
// p = i0 + o0 (i1 + o1 i2) (the reference's point order; the output is
// [B, C, o0(, o1(, o2))] with the last axis fastest): MODE 0 takes each batch
// row's largest finite |contribution| into gstat (zero before), MODE 1 adds
// the contributions through FixedScatter at the row's scale.  The
// contributions are the gather kernels' scatter (scatter_to, the same
// arithmetic).  One thread per grid point.
template <int ND, int MODE>
__global__ __launch_bounds__(256) void interp_det_kernel(int C, int in0, int in1, int in2, int o0,
                                                         int o1, int o2, int nP,
                                                         const float* __restrict__ grid,
                                                         const float* __restrict__ grad_out,
                                                         unsigned* __restrict__ gstat,
                                                         unsigned long long* __restrict__ gsums,
                                                         float* __restrict__ grad_data) {
  const int b = blockIdx.y;
  const int in[3] = {in0, in1, in2};
  const int64_t plane_in = (int64_t)in0 * (ND >= 2 ? in1 : 1) * (ND == 3 ? in2 : 1);
  const int shift = MODE == 1 ? det_shift(gstat[b], nP, 1 << ND) : 0;
  float m = 0.0f;
  for (int p = blockIdx.x * blockDim.x + threadIdx.x; p < nP; p += gridDim.x * blockDim.x) {
    const int i0 = p % o0, r = p / o0;
    const int i1 = ND >= 2 ? r % o1 : 0, i2 = ND == 3 ? r / o1 : 0;
    const int o = ND == 1 ? p : ND == 2 ? i0 * o1 + i1 : (i0 * o1 + i1) * o2 + i2;
    const float* gp = grid + (size_t)b * ND * nP + p;
    const Axis ax = axis_of(gp[0], in0);
    const Axis ay = ND >= 2 ? axis_of(gp[(size_t)nP], in1) : Axis{0, 0, 0.0f};
    const Axis az = ND == 3 ? axis_of(gp[2 * (size_t)nP], in2) : Axis{0, 0, 0.0f};
    for (int c = 0; c < C; ++c) {
      const size_t bc = (size_t)b * C + c;
      const float g = grad_out[bc * nP + o];
      if constexpr (MODE == 0)
        scatter_to<ND>(in, AbsMaxSink{&m}, ax, ay, az, g);
      else
        scatter_to<ND>(in, FixedScatter{gsums + bc * plane_in, grad_data + bc * plane_in, shift},
                       ax, ay, az, g);
    }
  }
  if constexpr (MODE == 0) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (__lane_id() == 0 && m > 0.0f)
      __hip_atomic_fetch_max(gstat + b, __float_as_uint(m), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

hipError_t launch_det_interp_data(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                                  const int64_t* out_size, const float* grid,
                                  const float* grad_out, unsigned* gstat,
                                  unsigned long long* gsums, float* grad_data, hipStream_t s) {
  int64_t nP = 1, plane = 1;
  for (int k = 0; k < ndim; ++k) {
    nP *= out_size[k];
    plane *= in_size[k];
  }
  if (B <= 0 || nP <= 0 || C <= 0) return hipSuccess;
  const int in0 = (int)in_size[0], in1 = ndim >= 2 ? (int)in_size[1] : 1;
  const int in2 = ndim == 3 ? (int)in_size[2] : 1;
  const int o0 = (int)out_size[0], o1 = ndim >= 2 ? (int)out_size[1] : 1;
  const int o2 = ndim == 3 ? (int)out_size[2] : 1;
  const dim3 blocks((unsigned)std::min<int64_t>((nP + 255) / 256, 1024), (unsigned)B);
  auto run = [&](auto stat_kernel, auto add_kernel) {
    hipLaunchKernelGGL(stat_kernel, blocks, dim3(256), 0, s, (int)C, in0, in1, in2, o0, o1, o2,
                       (int)nP, grid, grad_out, gstat, gsums, grad_data);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(add_kernel, blocks, dim3(256), 0, s, (int)C, in0, in1, in2, o0, o1, o2,
                       (int)nP, grid, grad_out, gstat, gsums, grad_data);
    return hipGetLastError();
  };
  hipError_t e;
  if (ndim == 1) e = run(interp_det_kernel<1, 0>, interp_det_kernel<1, 1>);
  else if (ndim == 2) e = run(interp_det_kernel<2, 0>, interp_det_kernel<2, 1>);
  else e = run(interp_det_kernel<3, 0>, interp_det_kernel<3, 1>);
  if (e != hipSuccess) return e;
  return launch_det_finish_rows(ndim, B, C * plane, nP, gstat, gsums, grad_data, s);
}

hipError_t launch_det_data_stat(int ndim, const ImageShape& img, int64_t n_batch,
                                const float* final_points, const float* grad_out,
                                unsigned* gstat, hipStream_t s) {
  if (n_batch <= 0 || img.nP <= 0) return hipSuccess;
  const dim3 grid((unsigned)std::min<int64_t>(((int64_t)img.nP + 255) / 256, 1024),
                  (unsigned)n_batch);
  if (ndim == 1)
    hipLaunchKernelGGL(det_data_stat_kernel<1>, grid, dim3(256), 0, s, img, final_points, grad_out,
                       gstat);
  else if (ndim == 2)
    hipLaunchKernelGGL(det_data_stat_kernel<2>, grid, dim3(256), 0, s, img, final_points, grad_out,
                       gstat);
  else
    hipLaunchKernelGGL(det_data_stat_kernel<3>, grid, dim3(256), 0, s, img, final_points, grad_out,
                       gstat);
  return hipGetLastError();
}

hipError_t launch_det_finish_rows(int ndim, int64_t n_batch, int64_t per_row, int64_t nP,
                                  const unsigned* gstat, const unsigned long long* gsums,
                                  float* grad_data, hipStream_t s) {
  if (n_batch <= 0 || per_row <= 0) return hipSuccess;
  const dim3 grid((unsigned)std::min<int64_t>((per_row + 255) / 256, 4096), (unsigned)n_batch);
  hipLaunchKernelGGL(det_data_finish_kernel, grid, dim3(256), 0, s, per_row, (int)nP, ndim, gstat,
                     gsums, grad_data);
  return hipGetLastError();
}

hipError_t launch_det_data_finish(int ndim, const ImageShape& img, int64_t n_batch,
                                  const unsigned* gstat, const unsigned long long* gsums,
                                  float* grad_data, hipStream_t s) {
  return launch_det_finish_rows(ndim, n_batch, (int64_t)img.C * img.plane_in, img.nP, gstat, gsums,
                                grad_data, s);
}

hipError_t dispatch_det_any(const BackwardJob& j, int adaptive, const LaunchCfg& cfg,
                            hipStream_t s) {
  switch (j.geo.ndim) {
    case 1: return dispatch_det<1>(j, adaptive, cfg, s);
    case 2: return dispatch_det<2>(j, adaptive, cfg, s);
    default: return dispatch_det<3>(j, adaptive, cfg, s);
  }
}

}  // namespace cpab
