// Device code shared by the backward kernels: the default ones (adjoint.hip)
// and the deterministic two-pass ones (adjoint_det.hip).  Cell lookup, the
// midpoint replay step and the adjoint step, the moment sinks, the workgroup
// map, the trajectory bodies (segmented and register variants) and the
// per-stage LDS layout; see adjoint.hip for the scheme.
#pragma once
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include "cpab_device.hpp"
#include "cpab_launch.hpp"
#include "cpab_sample.hpp"

namespace cpab {

// Problem handed to one backward launch (a plain / chain backward, or the fused
// transform_data backward when `image` is set).
struct BackwardJob {
  Geometry geo;
  int64_t nP, n_batch;
  int batched, T, K;
  const float *points, *stage_points, *As, *G, *amp, *grad_out;
  const EdgeAcc* edge;
  float *moments, *partials, *lam, *grad_points;
  uint64_t* dense_parts;
  const ImageShape* image;
  const float *axes, *final_points, *seed_grad, *data;
  float* grad_data;
  // deterministic reduction: pass 1 or 2 (0: float atomics), its row stats and
  // integer sums
  int det_pass;
  unsigned* det_stat;
  unsigned long long* det_sums;
  unsigned* det_flags;
  // and of grad_data (the image backward): batch rows' scales and integer sums
  const unsigned* det_gstat;
  unsigned long long* det_gsums;
};


// The deterministic backward's launches (adjoint_det.hip): job.det_pass 1 or 2.
hipError_t dispatch_det_any(const BackwardJob& j, int adaptive, const LaunchCfg& cfg,
                            hipStream_t s);

namespace {

template <int D> struct Dim;
template <> struct Dim<1> { static constexpr int P = 2; };
template <> struct Dim<2> { static constexpr int P = 6; };
template <> struct Dim<3> { static constexpr int P = 12; };

struct Cells { int nx, ny, nz; };

template <int D> __device__ __forceinline__ int lookup(const float (&p)[D], const Cells& g);
template <> __device__ __forceinline__ int lookup<1>(const float (&p)[1], const Cells& g) {
  return cell_1d(p[0], g.nx);
}
template <> __device__ __forceinline__ int lookup<2>(const float (&p)[2], const Cells& g) {
  return cell_2d(p[0], p[1], g.nx, g.ny);
}
template <> __device__ __forceinline__ int lookup<3>(const float (&p)[3], const Cells& g) {
  return cell_3d(p[0], p[1], p[2], g.nx, g.ny, g.nz);
}
// 2D: the inside rule only, for waves whose trajectories stay in
// (0, kClampHi]^2 (other dimensions: the full lookup).
template <int D>
__device__ __forceinline__ int lookup_inside(const float (&p)[D], const Cells& g) {
  if constexpr (D == 2) return key_cell(cell_key_2d_inside(p[0], p[1], g.nx, g.ny));
  else return lookup<D>(p, g);
}

template <int D> struct Fetch;
template <> struct Fetch<1> {
  template <typename P> static __device__ __forceinline__ Aff<1> at(P tab, int c) { return load_aff1(tab, c); }
};
template <> struct Fetch<2> {
  template <typename P> static __device__ __forceinline__ Aff<2> at(P tab, int c) { return load_aff2(tab, c); }
};
template <> struct Fetch<3> {
  template <typename P> static __device__ __forceinline__ Aff<3> at(P tab, int c) { return load_aff3(tab, c); }
};
template <int D, typename P> __device__ __forceinline__ Aff<D> fetch(P tab, int c) {
  return Fetch<D>::at(tab, c);
}

template <int D> struct FetchRev;
template <> struct FetchRev<1> {
  template <typename P> static __device__ __forceinline__ Adj<1> adj(P tab, int c) { return load_adj1(tab, c); }
  template <typename P> static __device__ __forceinline__ Inv<1> inv(P tab, int c) { return load_inv1(tab, c); }
};
template <> struct FetchRev<2> {
  template <typename P> static __device__ __forceinline__ Adj<2> adj(P tab, int c) { return load_adj2(tab, c); }
  template <typename P> static __device__ __forceinline__ Inv<2> inv(P tab, int c) { return load_inv2(tab, c); }
};
template <> struct FetchRev<3> {
  template <typename P> static __device__ __forceinline__ Adj<3> adj(P tab, int c) { return load_adj3(tab, c); }
  template <typename P> static __device__ __forceinline__ Inv<3> inv(P tab, int c) { return load_inv3(tab, c); }
};
// Reverse-sweep table entries (G, the inverse one-step map) from a global or
// an LDS table.
template <int D, typename P> __device__ __forceinline__ Adj<D> fetch_adj(P tab, int c) {
  return FetchRev<D>::adj(tab, c);
}
template <int D, typename P> __device__ __forceinline__ Inv<D> fetch_inv(P tab, int c) {
  return FetchRev<D>::inv(tab, c);
}

__device__ __forceinline__ void velocity(const Aff<1>& A, const float (&p)[1], float (&v)[1]) {
  v[0] = fmaf(A.a, p[0], A.b);
}
__device__ __forceinline__ void velocity(const Aff<2>& A, const float (&p)[2], float (&v)[2]) {
  apply2(A, p[0], p[1], v[0], v[1]);
}
__device__ __forceinline__ void velocity(const Aff<3>& A, const float (&p)[3], float (&v)[3]) {
  apply3(A, p[0], p[1], p[2], v[0], v[1], v[2]);
}

__device__ __forceinline__ void midpoint(const Aff<1>& A, float (&p)[1], float h, float hh) {
  p[0] = midpoint1(A, p[0], h, hh);
}
__device__ __forceinline__ void midpoint(const Aff<2>& A, float (&p)[2], float h, float hh) {
  midpoint2(A, p[0], p[1], h, hh);
}
__device__ __forceinline__ void midpoint(const Aff<3>& A, float (&p)[3], float h, float hh) {
  midpoint3(A, p[0], p[1], p[2], h, hh);
}

__device__ __forceinline__ void adjoint(const Adj<1>& G, const float (&p)[1], float (&s)[2],
                                        float (&l)[1]) {
  adjoint_s1(G, p[0], s, l[0]);
}
__device__ __forceinline__ void adjoint(const Adj<2>& G, const float (&p)[2], float (&s)[6],
                                        float (&l)[2]) {
  adjoint_s2(G, p[0], p[1], s, l[0], l[1]);
}
__device__ __forceinline__ void adjoint(const Adj<3>& G, const float (&p)[3], float (&s)[12],
                                        float (&l)[3]) {
  adjoint_s3(G, p[0], p[1], p[2], s, l[0], l[1], l[2]);
}

// One replay step from p in cell c (already looked up): explicit midpoint, or
// with adaptive_substeps the Heun correction when the step leaves the cell
// (cpab_ops_2d.cu:294-332).
template <int D, bool ADAPTIVE, typename P>
__device__ __forceinline__ void replay_step_with(P tab, const Aff<D>& A, int c, float (&p)[D],
                                                 float h, float hh, const Cells& g) {
  if (!ADAPTIVE) {
    midpoint(A, p, h, hh);
    return;
  }
  float q[D];
#pragma unroll
  for (int k = 0; k < D; ++k) q[k] = p[k];
  midpoint(A, q, h, hh);
  const int ce = lookup<D>(q, g);
  if (ce == c) {
#pragma unroll
    for (int k = 0; k < D; ++k) p[k] = q[k];
    return;
  }
  float v0[D], v1[D];
  velocity(A, p, v0);
  velocity(fetch<D>(tab, ce), q, v1);
#pragma unroll
  for (int k = 0; k < D; ++k) p[k] = fmaf(hh, v0[k] + v1[k], p[k]);
}

template <int D, bool ADAPTIVE, typename P>
__device__ __forceinline__ void replay_step(P tab, int c, float (&p)[D], float h, float hh,
                                            const Cells& g) {
  replay_step_with<D, ADAPTIVE>(tab, fetch<D>(tab, c), c, p, h, hh, g);
}

// Checkpoint stack in VGPRs.  Phase 2 consumes checkpoints in exactly the
// reverse order phase 1 produces them, so a shift register with static
// indices suffices: push shifts every entry up one slot, pop shifts down.
// (A select chain over a runtime index gets turned into a scratch-memory
// table by the compiler; shifting keeps everything in registers.)
template <int N>
__device__ __forceinline__ void stack_push(float (&a)[N], float v) {
#pragma unroll
  for (int k = N - 1; k > 0; --k) a[k] = a[k - 1];
  a[0] = v;
}
template <int N>
__device__ __forceinline__ float stack_pop(float (&a)[N]) {
  const float v = a[0];
#pragma unroll
  for (int k = 0; k < N - 1; ++k) a[k] = a[k + 1];
  return v;
}

// Where the backward keeps its per-cell sums: full LDS bins, the hashed LDS
// cell cache, or full bins with the reverse-sweep table (G and the inverse
// one-step maps) staged in LDS beside them (register variant, 1D/2D).
enum Bins { kBinsFull = 1, kBinsCache = 2, kBinsFullRev = 3 };
constexpr bool full_bins(int b) { return b == kBinsFull || b == kBinsFullRev; }

template <int P>
__device__ __forceinline__ void flush_lds(float* bins, int c, const float (&m)[P]) {
  float* q = bins + P * c;
#pragma unroll
  for (int k = 0; k < P; ++k)
    __hip_atomic_fetch_add(q + k, m[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Sums of a converged wave's last flush, pre-added per run of lanes with the
// same cell.  Meshgrid inputs start neighbouring trajectories in the same
// cell, so without this up to 64 lanes add into the same few LDS words,
// which serialises on the atomic unit.  When the lanes' cells form at most 16
// runs (counted per row of 16 lanes), each row runs a segmented inclusive scan
// over its runs (DPP row shifts by 1, 2, 4, 8, guarded by the run id) and only
// the last lane of each run keeps a flush (`on`), holding the run's sums in
// `out`; otherwise (scattered cells, e.g. random points) `out` = m and
// `on` = need.  Lanes with need == false take part in no run.
// One step of the segmented scan: add the value CTRL's row shift brings in
// when it comes from the same run (lanes shifted in from outside the row read
// 0, which matches no run id).
template <int CTRL, int P>
__device__ __forceinline__ void run_scan_step(int run, float (&v)[P]) {
  const int rd = __builtin_amdgcn_update_dpp(0, run, CTRL, 0xf, 0xf, true);
  const float f = rd == run ? 1.0f : 0.0f;
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const float t = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[k]), CTRL, 0xf, 0xf, true));
    v[k] = fmaf(t, f, v[k]);
  }
}

template <int P>
__device__ __forceinline__ void wave_run_sums(bool need, int c, const float (&m)[P],
                                              float (&out)[P], bool& on) {
  const int lane = __lane_id();
  const int key = need ? c : -1;
  const int before = __shfl_up(key, 1);
  const bool head = (lane & 15) == 0 || key != before;
  const uint64_t heads = __ballot(head);
#pragma unroll
  for (int k = 0; k < P; ++k) out[k] = need ? m[k] : 0.0f;
  on = need;
  if (__popcll(heads) > 16) return;  // wave-uniform
  // run id: heads at or below this lane (>= 1, since every row starts a run)
  const int run = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(heads >> 32),
                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)heads, 0u)) +
                  (head ? 1 : 0);
  run_scan_step<0x111, P>(run, out);  // row_shr:1
  run_scan_step<0x112, P>(run, out);  // row_shr:2
  run_scan_step<0x114, P>(run, out);  // row_shr:4
  run_scan_step<0x118, P>(run, out);  // row_shr:8
  const bool last = (lane & 15) == 15 || ((heads >> (lane < 63 ? lane + 1 : 63)) & 1);
  on = need && last;
}

// LDS cache flush (divergent lanes allowed).  The slot of cell c is claimed
// with a compare-and-swap on its key; a lane whose probe sequence meets only
// other cells adds to HBM instead.
template <int P>
__device__ __forceinline__ void flush_cache(int* keys, float* vals, float* __restrict__ mom, int c,
                                            const float (&m)[P]) {
  int slot = c & (kCacheSlots - 1);
  for (int probe = 0; probe < kCacheProbes; ++probe) {
    int k = __hip_atomic_load(keys + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (k == -1) {
      int expected = -1;
      __hip_atomic_compare_exchange_strong(keys + slot, &expected, c, __ATOMIC_RELAXED,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      k = expected == -1 ? c : expected;
    }
    if (k == c) {
      flush_lds<P>(vals, slot, m);
      return;
    }
    slot = (slot + 1) & (kCacheSlots - 1);
  }
#pragma unroll
  for (int k = 0; k < P; ++k) unsafeAtomicAdd(mom + (size_t)P * c + k, m[k]);
}

// Logical (part, row) of a backward workgroup: `part` indexes the point
// ranges of one row (gridDim.x of them), `row` the thetas (gridDim.y).  The
// hardware hands workgroups to the 8 XCDs round-robin by linear id, and each
// XCD has its own L2.  The logical grid is listed in blocks of kRowBlock rows
// (parts in order inside a block, rows fastest) and that list is cut into 8
// contiguous ranges, one per XCD: an XCD serves a few rows over a contiguous
// share of their points, so each row's affine and reverse-sweep tables are
// fetched from HBM by few L2s (at C2: by 2 of the 8 instead of all 8), and so
// are shared input points (by 4).  The map is a bijection for any grid.
constexpr int kRowBlock = 4;
struct WgSlot { int part, row; };
__device__ __forceinline__ WgSlot wg_slot() {
  const int nx = gridDim.x, ny = gridDim.y, n = nx * ny;
  const int lin = blockIdx.y * nx + blockIdx.x;
  const int x = lin & 7, k = lin >> 3, q = n >> 3, r = n & 7;
  const int L = x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
  const int rb = ny < kRowBlock ? ny : kRowBlock;
  const int full = (ny / rb) * rb * nx;   // entries in whole row blocks
  if (L < full) {
    const int blk = L / (rb * nx), rem = L - blk * rb * nx;
    return {rem / rb, blk * rb + rem % rb};
  }
  const int rr = ny - (ny / rb) * rb, rem = L - full;   // the last, partial block
  return {rem / rr, (ny / rb) * rb + rem % rr};
}

// Contiguous point range [lo, hi) of this workgroup, a whole number of blocks long.
__device__ __forceinline__ void wg_range(int nP, int& lo, int& hi) {
  const int64_t per = ((int64_t)nP + gridDim.x - 1) / gridDim.x;
  const int64_t span = (per + blockDim.x - 1) / blockDim.x * blockDim.x;
  const int64_t l = (int64_t)wg_slot().part * span;
  lo = (int)std::min<int64_t>(l, nP);
  hi = (int)std::min<int64_t>(l + span, nP);
}

// Where the trajectories of one stage start and where their adjoint seed
// comes from.  PlainIO: point and seed arrays [D, nP] (cpab_backward, chain
// stages).  ImageIO: the fused transform_data backward, where point q is an
// output pixel, the trajectory starts at its meshgrid point and the seed is
// the resampling gradient at the integrated point (the interp backward of
// cpab_sample.hpp, summed over channels, times size-1), as
// interpolation.py:3-159 followed by transformer.py:128-168 computes it.
template <int D>
struct PlainIO {
  const float* __restrict__ pts;
  const float* __restrict__ gout;
  float* __restrict__ lam_out;
  int nP;
  __device__ __forceinline__ void start(int i, float (&p)[D]) const {
#pragma unroll
    for (int k = 0; k < D; ++k) p[k] = pts[i + (size_t)k * nP];
  }
  __device__ __forceinline__ void seed(int i, bool, float (&lam)[D]) const {
#pragma unroll
    for (int k = 0; k < D; ++k) lam[k] = gout[i + (size_t)k * nP];
  }
  __device__ __forceinline__ void finish(int i, bool valid, const float (&lam)[D]) const {
    if (lam_out && valid) {
#pragma unroll
      for (int k = 0; k < D; ++k) lam_out[i + (size_t)k * nP] = lam[k];
    }
  }
};

//
// Trajectory order: the tiled walk (tile_index: one 16 x 4 pixel tile per
// wave) when the output size tiles, which keeps a wave's cells few and its
// seed reads in 64-byte runs.  Otherwise 1D/2D walk the points in image order
// (coalesced seed reads) and 3D in meshgrid order (lanes along coordinate 0:
// fewer cells per wave than image order, strided seed reads).  Start points
// come from the per-axis coordinate vectors either way.  GS: where the seed's
// corner scatter adds grad_data (FloatScatter: float atomics).
template <int D, typename GS = FloatScatter>
struct ImageIO {
  static constexpr bool kMeshOrder = D == 3;
  ImageShape s;
  const float* __restrict__ axes;   // per-axis coordinates of the uniform grid (shared by all thetas)
  const float* __restrict__ fin;    // [D, nP] integrated points of this theta, image order
  const float* __restrict__ sgrad;  // [D, nP] the sample's spatial gradient there (one channel, no
                                    // grad_data), or null
  const float* __restrict__ gout;   // [C, nP] image gradient of this theta
  const float* __restrict__ data;   // [C, plane_in]
  GS gdata;                         // [C, plane_in], off (on() false) without grad_data
  __device__ __forceinline__ void walk_index(int i, int (&ix)[3]) const {
    if (D >= 2 && s.walk_tiles) tile_index<D>(s, i, ix);
    else if (kMeshOrder) mesh_index<D>(s, i, ix);
    else image_index<D>(s, i, ix);
  }
  __device__ __forceinline__ void start(int i, float (&p)[D]) const {
    int ix[3];
    walk_index(i, ix);
    float x[3];
    grid_point<D>(s, axes, ix, x);
#pragma unroll
    for (int k = 0; k < D; ++k) p[k] = x[k];
  }
  __device__ __forceinline__ void seed(int i, bool valid, float (&lam)[D]) const {
    int q = i;  // image position of walk position i
    if (kMeshOrder || (D >= 2 && s.walk_tiles)) {
      int ix[3];
      walk_index(i, ix);
      q = image_pos<D>(s, ix);
    }
    if (sgrad) {
      // The forward's spatial gradient at the final point: three coalesced
      // reads and no corner reads behind them.
      const float g = gout[q];
#pragma unroll
      for (int k = 0; k < D; ++k) lam[k] = (g * sgrad[q + (size_t)k * s.nP]) * (float)(s.in[k] - 1);
      return;
    }
    const Axis ax = axis_of(fin[q], s.in[0]);
    const Axis ay = D >= 2 ? axis_of(fin[q + (size_t)s.nP], s.in[1]) : Axis{0, 0, 0.0f};
    const Axis az = D == 3 ? axis_of(fin[q + 2 * (size_t)s.nP], s.in[2]) : Axis{0, 0, 0.0f};
    float dd[3] = {0.0f, 0.0f, 0.0f};
    const bool scatter = gdata.on() && valid;
    for (int c = 0; c < s.C; ++c) {
      const GS gc = scatter ? gdata.channel(c * s.plane_in) : gdata;
      sample_grad_to<D>(s.in, data + c * s.plane_in, ax, ay, az, gout[(size_t)c * s.nP + q], dd,
                        scatter ? &gc : nullptr);
    }
#pragma unroll
    for (int k = 0; k < D; ++k) lam[k] = dd[k] * (float)(s.in[k] - 1);
  }
  __device__ __forceinline__ void finish(int, bool, const float (&)[D]) const {}
};

// Where a flush adds a run's sums: full LDS bins, or the LDS cell cache with
// HBM for the cells it has no slot for.
// kSpread: full bins, whose components the register variant may add one at a
// time (add1).
template <int BINS, int PP>
struct FloatSink {
  static constexpr bool kSpread = full_bins(BINS);
  float* bins;
  int* keys;
  float* __restrict__ mom;
  __device__ __forceinline__ void operator()(int c, const float (&m)[PP]) const {
    if (full_bins(BINS)) flush_lds<PP>(bins, c, m);
    else flush_cache<PP>(keys, bins, mom, c, m);
  }
  __device__ __forceinline__ void add1(int c, int k, float v) const {
    __hip_atomic_fetch_add(bins + PP * c + k, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
};

// Segmented variant (any T <= kSeg * MAXSEG).
// One stage of one theta over this workgroup's point range; each run's sums go
// to `flush` (a sink above, or the deterministic one below).
template <int D, bool ADAPTIVE, int MAXSEG, typename P, typename IO, typename Sink>
__device__ __forceinline__ void segmented_run(P tab, const float* __restrict__ gtab, int nP, int T,
                                              const Cells& g, const IO& io, const Sink& flush) {
  constexpr int PP = Dim<D>::P;
  const float h = 1.0f / (float)T;
  const float hh = h * 0.5f;
  const int nseg = (T + kSeg - 1) / kSeg;
  // The loop bound is uniform so every wave stays converged (the last flush
  // pre-adds runs of lanes across the wave); lanes past the range replay a
  // clamped point and contribute nothing.
  int lo, hi;
  wg_range(nP, lo, hi);
  for (int base = lo; base < hi; base += blockDim.x) {
    const int pi0 = base + (int)threadIdx.x;
    const bool valid = pi0 < hi;
    const int pi = valid ? pi0 : hi - 1;
    float p[D];
    io.start(pi, p);

    // The adjoint seed first: its reads (for the fused transform_data backward,
    // the resampling gradient over every channel) are done before the
    // checkpoints take their registers.
    float lam[D];
    io.seed(pi, valid, lam);

    // Phase 1: checkpoint (position before step seg*kSeg) pushed per segment.
    float ck[D][MAXSEG];
#pragma unroll
    for (int k = 0; k < D; ++k)
#pragma unroll
      for (int i = 0; i < MAXSEG; ++i) ck[k][i] = 0.0f;
    for (int seg = 0; seg < nseg; ++seg) {
#pragma unroll
      for (int k = 0; k < D; ++k) stack_push(ck[k], p[k]);
      const int len = min(kSeg, T - seg * kSeg);
      // Not unrolled: in 1D the compiler otherwise unrolls this short loop into
      // a register-hungry block that spills beside the register variant.
#pragma unroll 1
      for (int s = 0; s < len; ++s) replay_step<D, ADAPTIVE>(tab, lookup<D>(p, g), p, h, hh, g);
    }

    // Phase 2: reverse sweep.
    float m[PP];
#pragma unroll
    for (int k = 0; k < PP; ++k) m[k] = 0.0f;
    int prev = -1;
    for (int seg = nseg - 1; seg >= 0; --seg) {
      const int len = min(kSeg, T - seg * kSeg);
      float q[D];
#pragma unroll
      for (int k = 0; k < D; ++k) q[k] = stack_pop(ck[k]);
      float sp[kSeg][D];
      int sc[kSeg];
#pragma unroll
      for (int s = 0; s < kSeg; ++s) {
        if (s < len) {
          const int c = lookup<D>(q, g);
          sc[s] = c;
#pragma unroll
          for (int k = 0; k < D; ++k) sp[s][k] = q[k];
          replay_step<D, ADAPTIVE>(tab, c, q, h, hh, g);
        }
      }
#pragma unroll
      for (int s = kSeg - 1; s >= 0; --s) {
        if (s < len) {
          const int c = sc[s];
          const bool need = valid && c != prev && prev >= 0;
          if (need) flush(prev, m);
          if (c != prev) {
#pragma unroll
            for (int k = 0; k < PP; ++k) m[k] = 0.0f;
            prev = c;
          }
          adjoint(fetch_adj<D>(gtab, c), sp[s], m, lam);
        }
      }
    }
    float r[PP];
    bool on;
    wave_run_sums<PP>(valid, prev, m, r, on);
    if (on) flush(prev, r);
    io.finish(pi, valid, lam);
  }
}

template <int D, bool ADAPTIVE, int BINS, int MAXSEG = kMaxSeg, typename P, typename IO>
__device__ __forceinline__ void segmented_body(P tab, const float* __restrict__ gtab, int nP, int T,
                                               const Cells& g, const IO& io, float* bins,
                                               int* keys, float* __restrict__ mom_b) {
  segmented_run<D, ADAPTIVE, MAXSEG>(tab, gtab, nP, T, g, io,
                                     FloatSink<BINS, Dim<D>::P>{bins, keys, mom_b});
}

// Register variant: T == TS known at compile time; each run's sums go to
// `flush` (FloatSink: full LDS bins or, 3D, the LDS cell cache; or the
// deterministic sink).  Without adaptive substeps every replay step is
// p' = E_c [p; 1] with the cell's fixed midpoint map, so phase 1 keeps only
// the cells and phase 2 recovers each position from the next through the
// cell's inverse map (a few ulp per step; the positions only feed the sums
// S, the cells stay exact).  With adaptive substeps (Heun on crossings) the
// positions are kept in registers instead.  delta (2D without adaptive
// substeps, else +inf): the row's domain-edge bound for TS replay steps; a wave
// whose lanes all start at least that far from every edge replays without the
// lookup's per-step edge test (the same cells).
template <int D, bool ADAPTIVE, int TS, typename P, typename PG, typename IO, typename Sink>
__device__ __forceinline__ void register_body(P tab, PG gtab, int nP, const Cells& g,
                                              const IO& io, const Sink& flush, float delta) {
  constexpr int PP = Dim<D>::P;
  // A trajectory's last flush has all 64 lanes of every wave adding to
  // scattered bins at the same moment, a burst the LDS atomic pipe drains at
  // about one lane per clock.  With full bins (1D/2D, no adaptive substeps:
  // registers to spare) it is kept pending instead and issued one component
  // every TS / PP steps during the next range's phase 1, alongside its VALU
  // work; the last range's flush follows the loop.
  constexpr bool kSpread = D <= 2 && !ADAPTIVE && Sink::kSpread;
  const float h = 1.0f / (float)TS;
  const float hh = h * 0.5f;
  float pend[PP];
#pragma unroll
  for (int k = 0; k < PP; ++k) pend[k] = 0.0f;
  int pend_c = 0;
  bool pend_on = false;
  int lo, hi;
  wg_range(nP, lo, hi);
  for (int base = lo; base < hi; base += blockDim.x) {
    const int pi0 = base + (int)threadIdx.x;
    const bool valid = pi0 < hi;
    const int pi = valid ? pi0 : hi - 1;
    float p[D];
    io.start(pi, p);
    float lam[D];
    io.seed(pi, valid, lam);

    // Phase 1: the whole midpoint trajectory, positions and cells in VGPRs.
    // The current cell's affine block stays in registers and is re-read only
    // at steps where some lane of the wave changed cell.
    float traj[TS][D];
    uint32_t cells[(TS + 1) / 2];
    auto phase1 = [&](auto inside) {
      constexpr bool kInside = decltype(inside)::value;
      auto look = [&]() {
        if constexpr (kInside) return lookup_inside<D>(p, g);
        else return lookup<D>(p, g);
      };
      int cur = look();
      Aff<D> A = fetch<D>(tab, cur);
#pragma unroll
      for (int t = 0; t < TS; ++t) {
        if constexpr (kSpread) {
#pragma unroll
          for (int k = 0; k < PP; ++k) {
            if (t == (k * TS) / PP && pend_on) flush.add1(pend_c, k, pend[k]);
          }
        }
        const int c = (t == 0) ? cur : look();
        // Divergent branch, skipped (exec = 0) when no lane changed cell; marked
        // unlikely so that the no-change case falls through.
        if (__builtin_expect(c != cur, 0)) A = fetch<D>(tab, c);
        cur = c;
        if (t & 1) cells[t >> 1] |= (uint32_t)c << 16;
        else cells[t >> 1] = (uint32_t)c;
        if (ADAPTIVE) {
#pragma unroll
          for (int k = 0; k < D; ++k) traj[t][k] = p[k];
        }
        replay_step_with<D, ADAPTIVE>(tab, A, c, p, h, hh, g);
      }
    };
    if constexpr (D == 2 && !ADAPTIVE) {
      const float x0[1] = {p[0]}, y0[1] = {p[1]};
      if (edge_safe(x0, y0, delta)) phase1(std::integral_constant<bool, true>{});
      else phase1(std::integral_constant<bool, false>{});
    } else {
      phase1(std::integral_constant<bool, false>{});
    }

    // Phase 2: reverse sweep.  A cell change is handled at the end of the
    // step before it (flush the finished cell, load the next cell's entry),
    // so each load writes the registers the next step reads.
    auto cell_at = [&](int t) {
      return (int)((t & 1) ? (cells[t >> 1] >> 16) : (cells[t >> 1] & 0xffffu));
    };
    float m[PP];
#pragma unroll
    for (int k = 0; k < PP; ++k) m[k] = 0.0f;
    int c = cell_at(TS - 1);
    Adj<D> G = fetch_adj<D>(gtab, c);
    Inv<D> E;
    if (!ADAPTIVE) E = fetch_inv<D>(gtab, c);
#pragma unroll
    for (int t = TS - 1; t >= 0; --t) {
      if constexpr (ADAPTIVE) {
        adjoint(G, traj[t], m, lam);
      } else {
        step_back<D>(E, p);  // p = position at step t
        adjoint(G, p, m, lam);
      }
      // The lambda update reads G: finish it before the branch that reloads G.
      pin(lam);
      if (t > 0) {
        const int cn = cell_at(t - 1);
        // Divergent branch: skipped by the hardware (exec = 0) at steps where
        // no lane of the wave changes cell; marked unlikely so that this case
        // falls through.
        if (__builtin_expect(cn != c, 0)) {
          // The next cell's entry is read before the finished cell's sums are
          // added: LDS operations retire in order, so a read issued after the
          // adds would wait for them before the next step can use it.
          G = fetch_adj<D>(gtab, cn);
          if (!ADAPTIVE) E = fetch_inv<D>(gtab, cn);
          if (valid) flush(c, m);
#pragma unroll
          for (int k = 0; k < PP; ++k) m[k] = 0.0f;
        }
        c = cn;
      }
    }
    if constexpr (kSpread) {
      wave_run_sums<PP>(valid, c, m, pend, pend_on);
      pend_c = c;
    } else {
      float r[PP];
      bool on;
      wave_run_sums<PP>(valid, c, m, r, on);
      if (on) flush(c, r);
    }
    io.finish(pi, valid, lam);
  }
  if (kSpread && pend_on) flush(pend_c, pend);
}

// LDS layout of a backward workgroup: [A table (LDS_A)] then either the full
// bins (R floats) or the cache (kCacheSlots keys, then kCacheSlots * PP floats).
template <int D, bool LDS_A, int BINS>
struct StageLds {
  float* ldsA;
  int* keys;
  float* bins;
  float* ldsG;   // kBinsFullRev: the reverse-sweep table after the bins
  __device__ __forceinline__ StageLds(float* lds, int R) {
    ldsA = lds;
    float* after_a = lds + (LDS_A ? R : 0);
    keys = reinterpret_cast<int*>(after_a);
    bins = BINS == kBinsCache ? after_a + kCacheSlots : after_a;
    ldsG = bins + ((R + 3) & ~3);   // 16-byte aligned
  }
  // Stage the tables, clear the bins / cache (and the touched-cell counter).
  __device__ __forceinline__ void begin(const float* __restrict__ Ag, const float* __restrict__ Gg,
                                        int R, int nG, int* touched_cnt) const {
    constexpr int PP = Dim<D>::P;
    if (LDS_A) {
      const float2* s2 = reinterpret_cast<const float2*>(Ag);
      float2* d2 = reinterpret_cast<float2*>(ldsA);
      for (int i = threadIdx.x; i < R / 2; i += blockDim.x) d2[i] = s2[i];
    }
    if (BINS == kBinsFullRev) {
      // nG floats, a multiple of 4 (RevStride); the table and the LDS copy are
      // 16-byte aligned.
      const float4* s4 = reinterpret_cast<const float4*>(Gg);
      float4* d4 = reinterpret_cast<float4*>(ldsG);
      for (int i = threadIdx.x; i < nG / 4; i += blockDim.x) d4[i] = s4[i];
    }
    if (full_bins(BINS)) {
      for (int i = threadIdx.x; i < R; i += blockDim.x) bins[i] = 0.0f;
      if (threadIdx.x == 0) *touched_cnt = 0;
    } else {
      for (int i = threadIdx.x; i < kCacheSlots; i += blockDim.x) keys[i] = -1;
      for (int i = threadIdx.x; i < kCacheSlots * PP; i += blockDim.x) bins[i] = 0.0f;
    }
    __syncthreads();
  }
  // After every lane is done: full bins -> a dense workgroup's table into its
  // partial (and its bit `part` into the row's dense-part mask), a sparse
  // one's touched cells added to the HBM sums; cache -> HBM atomics of the
  // occupied slots' sums.  `touched_cnt` is an LDS counter that begin() cleared.
  __device__ __forceinline__ void end(float* __restrict__ partial,
                                      uint64_t* __restrict__ dense_parts, int part,
                                      float* __restrict__ mom_b, int nC, int* touched_cnt) const {
    constexpr int PP = Dim<D>::P;
    __syncthreads();
    if (full_bins(BINS)) {
      auto cell_touched = [&](int i) {
        bool t = false;
#pragma unroll
        for (int k = 0; k < PP; ++k) t |= bins[i * PP + k] != 0.0f;
        return t;
      };
      int cnt = 0;
      for (int i = threadIdx.x; i < nC; i += blockDim.x) cnt += cell_touched(i) ? 1 : 0;
      if (cnt) __hip_atomic_fetch_add(touched_cnt, cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __syncthreads();
      const bool dense = 4 * *touched_cnt >= nC;
      if (dense) {
        for (int i = threadIdx.x; i < nC * PP; i += blockDim.x) partial[i] = bins[i];
        if (threadIdx.x == 0)
          __hip_atomic_fetch_or(dense_parts + part / 64, 1ull << (part & 63), __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
      } else {
        for (int i = threadIdx.x; i < nC; i += blockDim.x) {
          if (!cell_touched(i)) continue;
#pragma unroll
          for (int k = 0; k < PP; ++k) unsafeAtomicAdd(mom_b + (size_t)i * PP + k, bins[i * PP + k]);
        }
      }
    } else {
      for (int i = threadIdx.x; i < kCacheSlots * PP; i += blockDim.x) {
        const int slot = i / PP;
        const int c = keys[slot];
        if (c >= 0) unsafeAtomicAdd(mom_b + (size_t)PP * c + (i - slot * PP), bins[i]);
      }
    }
  }
};

// Whether the positions of this row's trajectories may be recovered through
// the inverse one-step maps: the largest ||M_c||_2 over the row's cells (the
// row's amp_row[0 .. namp) block maxima) at most amp_max = kRecoverGrowth^(1/T).
// Wave-uniform (read into a scalar register).
__device__ __forceinline__ bool recover_ok(const float* __restrict__ amp_row, int namp,
                                          float amp_max) {
  float a = 0.0f;
  for (int i = __lane_id(); i < namp; i += 64) a = fmaxf(a, amp_row[i]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off));
  return __builtin_amdgcn_readfirstlane(a <= amp_max ? 1 : 0) != 0;
}

// Row stability of the register variant: the per-row block maxima of ||M_c||_2
// and the bound they are held to.
struct Recover {
  const float* __restrict__ amp;  // [rows, namp]
  int namp;
  float amp_max;
  // 2D, may be null: [rows, namp] parts of the rows' domain-edge bounds of the
  // replay maps (adjoint_table_kernel).
  const EdgeAcc* __restrict__ edge;
};

// delta_T of a row from its namp bound parts (cpab_device.hpp, edge_delta_2d),
// the same value in every lane of the wave.
__device__ __forceinline__ float row_edge_delta(const EdgeAcc* __restrict__ parts, int namp, int T,
                                                int nx, int ny) {
  EdgeAcc acc;
  acc.init();
  for (int i = __lane_id(); i < namp; i += 64) acc.merge(parts[i]);
  acc.wave_merge();
  const float d = edge_delta_2d(acc, T, nx, ny);
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, d)));
}

// The row's domain-edge bound for the register variant's replay (2D without
// adaptive substeps and with bound parts), else +inf.  Called before the
// stage's tables are staged, so that its loads overlap theirs.
template <int D, bool ADAPTIVE, int TS>
__device__ __forceinline__ float stage_delta(const Recover& rec, size_t row, const Cells& g) {
  if constexpr (D == 2 && !ADAPTIVE && TS > 0) {
    if (rec.edge) return row_edge_delta(rec.edge + row * rec.namp, rec.namp, TS, g.nx, g.ny);
  }
  return INFINITY;
}

template <int D, bool ADAPTIVE, bool LDS_A, int BINS, int TS, typename IO>
__device__ __forceinline__ void run_stage(const StageLds<D, LDS_A, BINS>& L, const float* Ag,
                                          const float* Gg, int nP, int T, const Cells& g,
                                          const IO& io, float* __restrict__ mom_b,
                                          const Recover& rec, size_t row, float delta) {
  if constexpr (TS > 0) {
    if constexpr (!ADAPTIVE) {
      // Rows whose inverse maps could amplify the recovered positions' rounding
      // beyond kRecoverGrowth replay each segment from a checkpoint instead.
      if (!recover_ok(rec.amp + row * rec.namp, rec.namp, rec.amp_max)) {
        constexpr int kSegs = (TS + kSeg - 1) / kSeg;
        if (LDS_A) segmented_body<D, false, BINS, kSegs>(as_lds(L.ldsA), Gg, nP, TS, g, io, L.bins, L.keys, mom_b);
        else segmented_body<D, false, BINS, kSegs>(Ag, Gg, nP, TS, g, io, L.bins, L.keys, mom_b);
        return;
      }
    }
    const FloatSink<BINS, Dim<D>::P> sink{L.bins, L.keys, mom_b};
    if constexpr (BINS == kBinsFullRev)
      register_body<D, ADAPTIVE, TS>(Ag, as_lds(L.ldsG), nP, g, io, sink, delta);
    else if (LDS_A) register_body<D, ADAPTIVE, TS>(as_lds(L.ldsA), Gg, nP, g, io, sink, delta);
    else register_body<D, ADAPTIVE, TS>(Ag, Gg, nP, g, io, sink, delta);
  } else {
    if (LDS_A) segmented_body<D, ADAPTIVE, BINS>(as_lds(L.ldsA), Gg, nP, T, g, io, L.bins, L.keys, mom_b);
    else segmented_body<D, ADAPTIVE, BINS>(Ag, Gg, nP, T, g, io, L.bins, L.keys, mom_b);
  }
}

template <typename Kern>
hipError_t allow_lds(Kern kernel, size_t lds) {
  if (lds <= 65536) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

}  // namespace
}  // namespace cpab
