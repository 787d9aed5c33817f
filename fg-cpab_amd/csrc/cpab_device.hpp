// Device-side building blocks of the CPAB integrator for gfx950 (CDNA4).
//
// Everything here is a __forceinline__ helper used by the kernels in
// integrate.hip / adjoint.hip / adjoint_det.hip.  Floating-point operation order is fixed on
// purpose: the whole library is compiled with -ffp-contract=off, every fused
// multiply-add is written as fmaf(), and the oracle under oracle/ performs the
// same sequence so the two agree bit for bit.
//
// Where the reference (cpab/core/cpab_ops_{1d,2d,3d}.cu) writes __fmaf_rn the
// fma is copied.  Where it writes a plain `a*b + c` nvcc contracts it by
// default (--fmad=true); we contract those the way LLVM's FMA combiner does:
// the left product of a sum is fused, `(a*b + c*d)` -> fmaf(a, b, c*d), and a
// further `+ e*f` is fused around the partial sum.  Which product nvcc fuses is
// not observable without an NVIDIA GPU, so those last bits are a documented
// tolerance, not a parity claim.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cpab {

// Same cap as CPAB_MAX_STEPS in the reference (cpab/core/cpab_ops_2d.cuh:8).
constexpr int kMaxSteps = 100;
// Trajectory checkpoint spacing for the backward replay.  Any value gives
// identical results (the replay is deterministic); 8 keeps the per-segment
// position buffer in 26 VGPRs.
constexpr int kSeg = 8;
constexpr int kMaxSeg = (kMaxSteps + kSeg - 1) / kSeg;
// Step count whose backward keeps the whole trajectory in registers (the
// library default nstepsolver=50); other step counts use the segmented replay.
constexpr int kRegSteps = 50;
// The register backward recovers positions step by step through each cell's
// inverse one-step map M_c, which multiplies the rounding error of a recovered
// position by up to ||M_c||_2 per step.  It does so only for rows (thetas)
// whose bound (max_c ||M_c||_2)^T is at most kRecoverGrowth; other rows replay
// the trajectory from checkpoints, which reproduces the replayed positions
// exactly.  Measured on a CPU emulation of the recovery (1D/2D/3D rows): the
// largest position error is about 4e-6 below a bound of 2 (theta ~ N(0, 0.5^2),
// the benchmark scale), 7e-6 below 8 and 1.5e-5 below 16; rows at 1e2 .. 1e3
// reach 3e-5 .. 2.7e-4.
constexpr float kRecoverGrowth = 16.0f;
// Hashed LDS cell cache of the backward when the full moment table does not
// fit in LDS: slots (a power of two) and linear-probe length.  3D: 2048 x 13
// words = 104 KiB.
constexpr int kCacheSlots = 2048;
constexpr int kCacheProbes = 4;

// Correctly rounded float exp / log / expm1: evaluated in double and rounded
// once.  The reference calls CUDA's expf/logf (a few ulp, implementation
// specific); rounding the double result gives the nearest float, so device
// and host (oracle) agree and both stay within an ulp of the exact value.
__device__ __forceinline__ float exp_cr(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float log_cr(float x) { return (float)log((double)x); }
__device__ __forceinline__ float expm1_cr(float x) { return (float)expm1((double)x); }

// ---------------------------------------------------------------------------
// Cell lookup.  Indexing and tie-breaking follow
//   1D: cpab_ops_1d.cu:52-59   2D: cpab_ops_2d.cu:71-128   3D: cpab_ops_3d.cu:67-131
// ---------------------------------------------------------------------------

// Clamp bound of the 1D/2D lookups: 1 - 1e-7 rounds to 1 - 2^-23.  For any
// n < 2^24, clamp(x) * n rounds to a value strictly below n, so
// floor(clamp(x) * n) <= n - 1 and the reference's min(cell, n-1) never binds;
// the float floor is then the exact cell coordinate.
constexpr float kClampHi = 1.0f - 1e-7f;

__device__ __forceinline__ float clamp_lookup(float x) {
  return __builtin_amdgcn_fmed3f(x, 0.0f, kClampHi);
}

__device__ __forceinline__ int cell_1d(float px, int nx) {
  return (int)__builtin_floorf(clamp_lookup(px) * (float)nx);
}

// 4 * square + triangle in two adds with a carry-in.  The triangle within a
// square comes from its local coordinates (lx, ly): b3 = lx < ly (above the
// main diagonal), b1 = (1 - lx) < ly (above the anti-diagonal), and raw
// 0,1,2,3 -> triangle 0,1,3,2 (cpab_ops_2d.cu:119-127), i.e. tri = 3*b3 ^ b1
// = 2*b3 + (b3 ^ b1).  So the cell is 2 * (2 * square + b3) + (b3 ^ b1): each
// "x + x + bit" is one v_addc_co_u32 whose carry-in is the bit's lane mask
// (a compare's own result; the xor of two masks is a scalar op), where the
// select form takes a shift, two selects and an or.  The masks come in as
// arguments so that the out-of-domain rules can replace lanes' bits first.
__device__ __forceinline__ int cell_from_bits(int square, uint64_t m3, uint64_t m1) {
  const uint64_t m0 = m3 ^ m1;
  int u, c;
  uint64_t co;
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(u), "=s"(co) : "v"(square), "s"(m3));
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(c), "=s"(co) : "v"(u), "s"(m0));
  return c;
}

// Square (cx, cy) holds triangles 4*(cx + cy*nx) + {0 bottom, 1 right, 2 top, 3 left}.
//
// A wave whose lanes all lie in (0, kClampHi]^2, where the lookup clamp is the
// identity, takes the inside rule on the raw coordinates.  Otherwise (a
// wave-uniform branch) the inside rule runs on the clamped coordinates and
// the out-of-domain rules of cpab_ops_2d.cu:97-117 decide the triangle of
// lanes on or beyond a side:
//   px <= 0 -> left (3), else px >= 1 -> right (1), else py <= 0 -> bottom
//   (0), else py >= 1 -> top (2); the square is the clamped point's either way;
//   beyond a corner (an x rule and a y rule both apply) the diagonal through
//   the corner picks the y side's triangle or the x side's, with the
//   reference's products term for term.
// Lanes with no rule (inside, or NaN coordinates, which fail every compare as
// in the reference) keep the inside rule's bits.  Meshgrid inputs put a point
// on the domain's left and right edges in every row, so half the waves or
// more of such a workload take this path at most steps, and in a chain those
// waves run longest.  The side rules enter as substituted local coordinates
// (below), the corner rule behind a scalar branch on the lanes beyond a
// corner.
//
// The lookup yields the cell as a key: the square's index as a float (an
// integer below 2^22, exact) and the lane masks of the two triangle bits.
// key_cell() forms the cell id (a convert and the two carry-in adds).  A
// trajectory tests for a cell change on the key, one float compare and scalar
// mask operations, and forms the id only where the cell changed (C2 forward
// 60.5 -> 58.2 us).
struct CellKey {
  float sq;
  uint64_t m3, m1;
};
__device__ __forceinline__ int key_cell(const CellKey& k) {
  return cell_from_bits((int)k.sq, k.m3, k.m1);
}
// Lane mask of the lanes whose cell differs between two keys.
__device__ __forceinline__ uint64_t key_changed(const CellKey& a, const CellKey& b) {
  return __builtin_amdgcn_ballot_w64(a.sq != b.sq) | (a.m3 ^ b.m3) | (a.m1 ^ b.m1);
}
__device__ __forceinline__ CellKey cell_key_2d(float px, float py, int nx, int ny) {
  const float fx = (float)nx, fy = (float)ny;
  // x lies in (0, kClampHi] iff its bit pattern minus one, as an unsigned
  // integer, lies below kClampHi's: +0 wraps to the top, and negative values,
  // -0, NaN and infinities lie above (checked over all 2^32 patterns).  One
  // compare of the larger of the two feeds the branch directly; four float
  // compares needed three scalar ORs and a scalar compare between the vector
  // compares and the branch, on the critical path of every step (C5 chain
  // forward 115 -> 107 us, C2 forward 62 -> 59 us).
  const uint32_t ux = __builtin_bit_cast(uint32_t, px) - 1u;
  const uint32_t uy = __builtin_bit_cast(uint32_t, py) - 1u;
  const uint64_t edge =
      __builtin_amdgcn_ballot_w64((ux > uy ? ux : uy) >= __builtin_bit_cast(uint32_t, kClampHi));
  if (!edge) {
    const float sx = __builtin_floorf(px * fx), sy = __builtin_floorf(py * fy);
    const float lx = fmaf(px, fx, -sx), ly = fmaf(py, fy, -sy);
    return {fmaf(sy, fx, sx), __builtin_amdgcn_ballot_w64(lx < ly),
            __builtin_amdgcn_ballot_w64((1.0f - lx) < ly)};
  }
  const float xc = clamp_lookup(px), yc = clamp_lookup(py);
  const float sx = __builtin_floorf(xc * fx), sy = __builtin_floorf(yc * fy);
  const float lx = fmaf(xc, fx, -sx), ly = fmaf(yc, fy, -sy);
  const float square = fmaf(sy, fx, sx);  // exact: cx + cy*nx < 2^22
  // The side rules as substituted local coordinates: the inside rule's two
  // compares, b3 = lx < ly and b1 = (1 - lx) < ly, give left (1,0) for
  // lx = -4, right (0,1) for lx = 4, bottom (0,0) for ly = -2 and top (1,1)
  // for ly = 2, against any ly in [0, 1) or lx in [0, 1) respectively; with
  // both substituted the x side wins (lx = -4 or 4 decides both bits against
  // ly = -2 or 2), as the reference tests x first.  Four selects replace the
  // ~13 dependent scalar mask operations of the side rules (C5 chain forward
  // 87.7 -> 79.4 us).
  const bool xl_lane = px <= 0.0f, yl_lane = py <= 0.0f;
  const bool xh_lane = px >= 1.0f, yh_lane = py >= 1.0f;
  const float lxs = xl_lane ? -4.0f : (xh_lane ? 4.0f : lx);
  const float lys = yl_lane ? -2.0f : (yh_lane ? 2.0f : ly);
  uint64_t m3 = __builtin_amdgcn_ballot_w64(lxs < lys);
  uint64_t m1 = __builtin_amdgcn_ballot_w64((1.0f - lxs) < lys);
  const uint64_t corner =
      (__builtin_amdgcn_ballot_w64(xl_lane) | __builtin_amdgcn_ballot_w64(xh_lane)) &
      (__builtin_amdgcn_ballot_w64(yl_lane) | __builtin_amdgcn_ballot_w64(yh_lane));
  if (corner) {
    const uint64_t yh = __builtin_amdgcn_ballot_w64(yh_lane);
    // cpab_ops_2d.cu:98-113: below-left pyfy < pxfx, above-left yhi > -pxfx,
    // below-right -pyfy > xhi (as -xhi > pyfy), above-right yhi > xhi; where
    // it holds the y side's triangle, else the x side's.
    const float pxfx = px * fx, pyfy = py * fy;
    const float xhi = fmaf(px, fx, -fx), yhi = fmaf(py, fy, -fy);
    const float lhs = yl_lane ? (xl_lane ? pxfx : -xhi) : yhi;
    const float rhs = yl_lane ? pyfy : (xl_lane ? -pxfx : xhi);
    const uint64_t y_wins = __builtin_amdgcn_ballot_w64(lhs > rhs) & corner;
    m3 = (m3 & ~y_wins) | (y_wins & yh);
    m1 = (m1 & ~y_wins) | (y_wins & yh);
  }
  return {square, m3, m1};
}
__device__ __forceinline__ int cell_2d(float px, float py, int nx, int ny) {
  return key_cell(cell_key_2d(px, py, nx, ny));
}

// The inside rule alone: the key cell_key_2d returns for a wave whose lanes
// all lie in (0, kClampHi]^2, without the per-step domain-edge test.  Used by
// waves that edge_safe (below) has shown stay there for the whole trajectory.
__device__ __forceinline__ CellKey cell_key_2d_inside(float px, float py, int nx, int ny) {
  const float fx = (float)nx, fy = (float)ny;
  const float sx = __builtin_floorf(px * fx), sy = __builtin_floorf(py * fy);
  const float lx = fmaf(px, fx, -sx), ly = fmaf(py, fy, -sy);
  return {fmaf(sy, fx, sx), __builtin_amdgcn_ballot_w64(lx < ly),
          __builtin_amdgcn_ballot_w64((1.0f - lx) < ly)};
}

// ---------------------------------------------------------------------------
// Domain-edge bound of a theta row's replay maps (2D).
//
// cell_key_2d spends 4 VALU operations and a branch per step on the test
// whether some lane lies outside (0, kClampHi]^2.  The test can be skipped for
// a trajectory that provably stays inside.  For each edge e of the domain
// (left: d = x, right: d = 1 - x, bottom: y, top: 1 - y), with d' the distance
// after one computed step:
//   - over the cells a point at d < r_lo = 1/(2n) can lie in (the triangles
//     with a vertex closer than r_lo), d' >= alpha d - beta;
//   - over all cells, d' >= d - reach;
// both up to the computed step's rounding err.  The exact step map is affine
// in each cell, so both hold on a triangle where they hold at its three
// vertices; they are widened by kEdgeEta times the map's slope for points the
// lookup assigns to a cell from just outside it (the rounded cell coordinates
// misplace a point by a few 2^-24 at most).  With m = min(alpha, 1) > 0,
// b = beta + err and thr = 2^-23, a point with d >= delta_k =
// (thr + (k - 1) b) / m^(k-1) stays at d > thr for k steps: a step takes
// d in [delta_k, r_lo) to alpha d - b >= delta_{k-1}, and d >= r_lo to
// d - reach - err >= delta_{k-1}, provided delta_T < r_lo and
// delta_T + reach + err <= r_lo.  d > thr on all four edges puts the point in
// (0, kClampHi]^2.  So a wave whose lanes all start at distance >= the row's
// delta_T from every edge takes the inside rule at each of its T steps: the
// same cells, bit for bit, without the test.
//
// adjoint_table_kernel evaluates this in double from the fp32 fields for the
// backward replay's explicit-midpoint maps, per block of cells; the backward
// merges a row's blocks and forms delta_T (rounded up); rows whose maps are
// not finite, or push points toward an edge too fast, get +inf (never skip).
// ---------------------------------------------------------------------------

// Largest distance (domain units) between a point and the triangle the lookup
// assigns it to: floor(x n) and the local coordinates are each rounded once
// (about 4 * 2^-24 in all); 2^-20 leaves a wide margin.
constexpr double kEdgeEta = 9.5367431640625e-07;  // 2^-20
constexpr double kUlp = 5.9604644775390625e-08;    // 2^-24, fp32 unit roundoff

// Over a row's cells and the four edges: the smallest alpha, the largest
// beta, reach and rounding bound (delta_T needs no more: it grows as alpha
// falls and as the others grow).
struct EdgeAcc {
  double alpha, beta, reach, err;
  __device__ __forceinline__ void init() {
    alpha = INFINITY;
    beta = reach = err = 0.0;
  }
  __device__ __forceinline__ void merge(const EdgeAcc& o) {
    alpha = fmin(alpha, o.alpha);
    beta = fmax(beta, o.beta);
    reach = fmax(reach, o.reach);
    err = fmax(err, o.err);
  }
  // All 64 lanes of the wave end with the wave's merged value.
  __device__ __forceinline__ void wave_merge() {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      EdgeAcc o;
      o.alpha = __shfl_xor(alpha, off);
      o.beta = __shfl_xor(beta, off);
      o.reach = __shfl_xor(reach, off);
      o.err = __shfl_xor(err, off);
      merge(o);
    }
  }
};

// Rounding bound of one computed explicit-midpoint replay step with the cell's
// velocity field a (row-major 2x3): v = A [p; 1], p_mid = p + hh v,
// v_mid = A [p_mid; 1], p' = p + h v_mid, each rounded, for |x|, |y| <= 1.
__device__ __forceinline__ double midpoint_step_err(const float* a, double h, double hh) {
  double S = 0.0;
#pragma unroll
  for (int r = 0; r < 2; ++r)
    S = fmax(S, fabs((double)a[3 * r]) + fabs((double)a[3 * r + 1]) + fabs((double)a[3 * r + 2]));
  const double dv = 2.02 * kUlp * S;                   // v
  const double pm = 1.0 + hh * S;                      // |p_mid| bound
  const double dpm = hh * dv + 1.01 * kUlp * pm;       // p_mid
  const double dvm = 2.02 * kUlp * S * pm + S * dpm;   // v_mid
  return 1.05 * (h * dvm + 1.01 * kUlp * (1.0 + h * S * pm));  // p'
}

// The replay step of field a as an exact affine map of p:
// [I + h A + h hh A^2 | h b + h hh A b] (float h and hh as the replay uses them).
__device__ __forceinline__ void midpoint_map_2d(const float* a, float h, double (&m)[2][3]) {
  const double hd = h, h2 = (double)h * (double)(h * 0.5f);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const double ab = (double)a[3 * i] * a[2] + (double)a[3 * i + 1] * a[5];
    m[i][2] = hd * a[3 * i + 2] + h2 * ab;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const double sq = (double)a[3 * i] * a[j] + (double)a[3 * i + 1] * a[3 + j];
      m[i][j] = (i == j ? 1.0 : 0.0) + hd * a[3 * i + j] + h2 * sq;
    }
  }
}

// Adds cell c (triangle t of square (cx, cy), c = 4 (cx + cy nx) + t) whose one
// step is p' = m [p; 1] in exact arithmetic, computed with rounding error at
// most err per coordinate, for each of the four edges.  A non-finite map or
// err makes the row unusable (alpha = -inf).
__device__ __forceinline__ void edge_bound_cell_2d(const double (&m)[2][3], int c, int nx, int ny,
                                                   double err, EdgeAcc& acc) {
  const int sq = c >> 2, t = c & 3;
  const int cy = sq / nx, cx = sq - cy * nx;
  const double x0 = (double)cx / nx, x1 = (double)(cx + 1) / nx;
  const double y0 = (double)cy / ny, y1 = (double)(cy + 1) / ny;
  const double xc = 0.5 * (x0 + x1), yc = 0.5 * (y0 + y1);
  // t: 0 bottom, 1 right, 2 top, 3 left (cpab_ops_2d.cu:119-127); the
  // square's centre is every triangle's third vertex.
  const double vx[3] = {t == 1 ? x1 : x0, t == 3 ? x0 : x1, xc};
  const double vy[3] = {t == 2 ? y1 : y0, t == 0 ? y0 : y1, yc};
  bool finite = isfinite(err);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int j = 0; j < 3; ++j) finite = finite && isfinite(m[a][j]);
  if (!finite) {
    acc.alpha = -INFINITY;
    return;
  }
  acc.err = fmax(acc.err, err);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int ax = e >> 1;
    const bool far_side = e & 1;
    const double rlo = 0.5 / (ax ? ny : nx);
    double d[3], dp[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const double pos = ax ? vy[k] : vx[k];
      const double img = m[ax][0] * vx[k] + m[ax][1] * vy[k] + m[ax][2];
      d[k] = far_side ? 1.0 - pos : pos;
      dp[k] = far_side ? 1.0 - img : img;
    }
    const double dmin = fmin(fmin(d[0], d[1]), d[2]);
    const double slope = fabs(m[ax][0]) + fabs(m[ax][1]);
    double approach = 0.0;
#pragma unroll
    for (int k = 0; k < 3; ++k) approach = fmax(approach, d[k] - dp[k]);
    acc.reach = fmax(acc.reach, approach + (slope + 1.0) * kEdgeEta);
    if (dmin < rlo) {
      double bv = 0.0;
#pragma unroll
      for (int k = 0; k < 3; ++k)
        if (d[k] == 0.0) bv = fmax(bv, -dp[k]);
      double al = INFINITY;
#pragma unroll
      for (int k = 0; k < 3; ++k)
        if (d[k] > 0.0) al = fmin(al, (dp[k] + bv) / d[k]);
      acc.alpha = fmin(acc.alpha, al);
      acc.beta = fmax(acc.beta, bv + (slope + fmax(fabs(al), 1.0)) * kEdgeEta);
    }
  }
}

// x^n for n >= 0 by square and multiply (a fixed sequence of double products).
__device__ __forceinline__ double pow_int(double x, int n) {
  double r = 1.0;
  while (n > 0) {
    if (n & 1) r *= x;
    x *= x;
    n >>= 1;
  }
  return r;
}

// delta_T of a row from its merged accumulator, rounded up to float; +inf when
// the row allows no bound.
__device__ __forceinline__ float edge_delta_2d(const EdgeAcc& acc, int T, int nx, int ny) {
  // alpha > 0 fails for NaN and for an unusable row (-inf)
  const double U =
      acc.alpha > 0.0 ? pow_int(1.0 / fmin(acc.alpha, 1.0), T - 1) * (1.0 + 1e-12) : INFINITY;
  const double E = acc.err;
  const double delta = U * (1.1920928955078125e-07 + (double)(T - 1) * (acc.beta + E)) * (1.0 + 1e-12);
  const double rlo = 0.5 / (double)max(nx, ny);
  const bool ok = T >= 1 && delta < rlo && (delta + acc.reach + E) * (1.0 + 1e-12) <= rlo;
  return ok ? __double2float_ru(delta) : INFINITY;
}

// Whether every lane of the wave starts at distance >= delta from each domain
// edge (so that its next T steps stay in (0, kClampHi]^2, delta being the
// row's delta_T); NaN coordinates fail.
template <int N>
__device__ __forceinline__ bool edge_safe(const float (&x)[N], const float (&y)[N], float delta) {
  bool ok = true;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const float d = fminf(fminf(x[k], 1.0f - x[k]), fminf(y[k], 1.0f - y[k]));
    ok = ok && x[k] == x[k] && y[k] == y[k] && d >= delta;
  }
  return __builtin_amdgcn_ballot_w64(!ok) == 0;
}

// Scale exponent s of a row's integer sums in the deterministic reduction:
// `stat` holds the bits of the row's largest finite |flushed value| (0 when
// all were zero).  A row has at most nP * T flushes (a trajectory flushes at
// most once per step), so with every value below 2^e, value * 2^s < 2^(62 - lg)
// and the sum of all of them stays below 2^62 in magnitude.
__device__ __forceinline__ int det_shift(unsigned stat, int64_t nP, int T) {
  if (stat == 0u || stat >= 0x7f800000u) return 0;
  int e;
  frexpf(__uint_as_float(stat), &e);  // value < 2^e
  const int64_t n = nP * (int64_t)T;
  const int lg = n > 1 ? 64 - __builtin_clzll((unsigned long long)(n - 1)) : 0;
  return 62 - e - lg;
}

// rint(v * 2^s) as a two's-complement 64-bit integer, for finite v with
// |v| 2^s < 2^63.  v * 2^s is exact in float (ldexp), and so is its rounding to
// an integer; the magnitude a then splits exactly into 32-bit words: the high
// word floor(a 2^-32) and the low word a - high 2^32, which is below 2^32 and,
// when a >= 2^32, a multiple of a's ulp (>= 2^9), so it needs at most 23 bits.
__device__ __forceinline__ unsigned long long det_fixed(float v, int s) {
  const float x = __builtin_rintf(ldexpf(v, s));
  const float a = fabsf(x);
  const float hi = floorf(a * 0x1p-32f);
  const float lo = fmaf(-hi, 0x1p32f, a);
  const unsigned long long u =
      ((unsigned long long)(unsigned)hi << 32) | (unsigned long long)(unsigned)lo;
  return x < 0.0f ? 0ull - u : u;
}

// Issue priority of a wave from its lanes' positions at the start of a
// trajectory: lanes on or beyond the domain's edge take the lookup's clamping
// path, and beyond a corner the corner rule too, at most steps, so their
// waves run the longest.  Where each wave's trajectories are the only work it
// has left to hide latency with (the chain forward: 262,144 points, 4 waves
// per SIMD), the kernel ends with its slowest waves; raising their priority
// lets them issue first when several waves are ready (C5 chain forward 95 ->
// 86 us).  Waves with no such lane are set back to the default priority 0.
template <int N>
__device__ __forceinline__ void edge_priority(const float (&x)[N], const float (&y)[N]) {
  bool side = false, corner = false;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const bool xo = !(x[k] > 0.0f && x[k] < 1.0f), yo = !(y[k] > 0.0f && y[k] < 1.0f);
    side |= xo | yo;
    corner |= xo & yo;
  }
  if (__builtin_amdgcn_ballot_w64(corner)) __builtin_amdgcn_s_setprio(3);
  else if (__builtin_amdgcn_ballot_w64(side)) __builtin_amdgcn_s_setprio(2);
  else __builtin_amdgcn_s_setprio(0);
}

// Tetrahedron of the clamped point (xc, yc, zc) in [0,1]^3.  The cube
// coordinates are kept as floats (integers below 2^24, so every sum and
// product here is exact): floor(xc * n) capped at n - 1 as the reference's
// min(floor, n - 1), then the cube id and its parity.
__device__ __forceinline__ int tet_3d(float xc, float yc, float zc, float fx, float fy, float fz,
                                      float fxy) {
  const float si = fminf(__builtin_floorf(xc * fx), fx - 1.0f);
  const float sj = fminf(__builtin_floorf(yc * fy), fy - 1.0f);
  const float sk = fminf(__builtin_floorf(zc * fz), fz - 1.0f);
  float x = fmaf(xc, fx, -si);
  float y = fmaf(yc, fy, -sj);
  const float z = fmaf(zc, fz, -sk);
  const uint32_t cube = (uint32_t)fmaf(sk, fxy, fmaf(sj, fx, si));
  if ((int)(si + sj + sk) & 1) {  // parity of i + j + k == parity of i ^ j ^ k
    const float t = x;
    x = y;
    y = 1.0f - t;
  }
  // First matching test wins, as in the reference's if-chain; evaluated as
  // selects (every lane needs all four tests anyway).  The reference tests the
  // signs of (x - y) - z, ((-x) + y) - z, ((x + y) + z) - 2 and
  // ((-x) - y) + z; (-x) + y == -(x - y) and ((-x) - y) + z == z - (x + y) in
  // IEEE arithmetic.  With finite operands and denormals kept (these kernels
  // run with fp32 denormals on: a rounded difference is zero only when the
  // operands are equal and otherwise has the sign of the exact one), a >= b
  // decides "a - b >= 0" exactly, so the outer subtractions are compares.
  const float d = x - y, s = x + y;
  int t = (d >= z) ? 4 : 0;
  t = (-d >= z) ? 3 : t;
  t = (s + z >= 2.0f) ? 2 : t;
  t = (z >= s) ? 1 : t;
  return (int)__umul24(cube, 5u) + t;
}

// Cube (i, j, k) holds tetrahedra 5*(i + j*nx + k*nx*ny) + {0 central, 1..4 corners};
// odd-parity cubes are mirrored by the local remap (x, y) -> (y, 1 - x).
// A wave whose lanes all lie in [0,1]^3 (the meshgrid and most trajectories)
// needs neither the corner rule nor the clamps: as unsigned integers the bit
// patterns of +0 ... 1.0 are exactly 0 ... 0x3f800000, and negative values,
// -0, NaN and infinities compare above.  Meshgrid points on the x = 0 and
// x = 1 faces drift to either side of them, so most waves of a volume warp
// take the clamping path at most steps; there the corner rule's overshoots
// are computed only when some lane lies outside [0,1] on all three axes (the
// reference's overshoot (|p - 1/2| - 1/2) * n is positive only outside
// [0,1]), which costs three compares instead of the nine operations of the
// overshoots and their three compares.
__device__ __forceinline__ int cell_3d(float px, float py, float pz, int nx, int ny, int nz) {
  const float fx = (float)nx, fy = (float)ny, fz = (float)nz;
  const float fxy = (float)(nx * ny);
  const uint32_t bmax = max(max(__float_as_uint(px), __float_as_uint(py)), __float_as_uint(pz));
  if (!__builtin_amdgcn_ballot_w64(bmax > 0x3f800000u)) return tet_3d(px, py, pz, fx, fy, fz, fxy);
  const uint64_t out3 = __builtin_amdgcn_ballot_w64(__float_as_uint(px) > 0x3f800000u) &
                        __builtin_amdgcn_ballot_w64(__float_as_uint(py) > 0x3f800000u) &
                        __builtin_amdgcn_ballot_w64(__float_as_uint(pz) > 0x3f800000u);
  if (out3) {
    const float ox = (fabsf(px - 0.5f) - 0.5f) * fx;
    const float oy = (fabsf(py - 0.5f) - 0.5f) * fy;
    const float oz = (fabsf(pz - 0.5f) - 0.5f) * fz;
    // Beyond a corner (rare): move the axis with the smallest overshoot half
    // a cell inside (cpab_ops_3d.cu:79-88).
    const bool corner = (ox > 0.0f) & (oy > 0.0f) & (oz > 0.0f);
    if (corner) {
      if (ox <= oy && ox <= oz) {
        px = (px < 0.5f) ? 0.5f / fx : 1.0f - 0.5f / fx;
      } else if (oy <= oz) {
        py = (py < 0.5f) ? 0.5f / fy : 1.0f - 0.5f / fy;
      } else {
        pz = (pz < 0.5f) ? 0.5f / fz : 1.0f - 0.5f / fz;
      }
    }
  }
  return tet_3d(fminf(fmaxf(px, 0.0f), 1.0f), fminf(fmaxf(py, 0.0f), 1.0f),
                fminf(fmaxf(pz, 0.0f), 1.0f), fx, fy, fz, fxy);
}

// ---------------------------------------------------------------------------
// Per-cell affine maps.  A cell's row-major [ndim, ndim+1] block (velocity
// field A or one-step map Trels) is held in registers while it is applied.
// ---------------------------------------------------------------------------

template <int D> struct Aff;
template <> struct Aff<1> { float a, b; };
template <> struct Aff<2> { float m[6]; };
template <> struct Aff<3> { float m[12]; };

// Per-cell table loads.  The C ABI limits a tessellation to fewer than 2^24
// cells and a row's table to fewer than 2^30 floats, so the byte offset of an
// entry fits in 32 bits: global loads take it as a VGPR offset from the scalar
// row base (no 64-bit address arithmetic per fetch).  LDS
// tables are passed as address-space-3 pointers so the offsets stay 32-bit
// (one v_mul_u32_u24 per fetch) and the loads become ds_read2_b64 /
// ds_read_b128.
#define CPAB_LDS __attribute__((address_space(3)))
template <typename T> using lds_ptr = const T CPAB_LDS*;
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ lds_ptr<float> as_lds(const float* p) { return (lds_ptr<float>)p; }

// Entry c of a global table of B-byte entries.  Cell ids are below 2^24, so
// the offset is one full-rate v_mul_u32_u24.
template <typename V, uint32_t B>
__device__ __forceinline__ const V* entry(const float* tab, int c) {
  const uint32_t off = __umul24((uint32_t)c, B);
  return reinterpret_cast<const V*>(reinterpret_cast<const char*>(tab) + off);
}

__device__ __forceinline__ Aff<1> load_aff1(const float* tab, int c) {
  const v2f v = *entry<v2f, 8>(tab, c);
  return {v.x, v.y};
}
__device__ __forceinline__ Aff<1> load_aff1(lds_ptr<float> tab, int c) {
  const v2f v = ((lds_ptr<v2f>)tab)[(uint32_t)c];
  return {v.x, v.y};
}
__device__ __forceinline__ Aff<2> load_aff2(const float* tab, int c) {
  const v2f* q = entry<v2f, 24>(tab, c);
  const v2f a = q[0], b = q[1], d = q[2];
  return {{a.x, a.y, b.x, b.y, d.x, d.y}};
}
__device__ __forceinline__ Aff<2> load_aff2(lds_ptr<float> tab, int c) {
  lds_ptr<v2f> q = (lds_ptr<v2f>)tab + __umul24((uint32_t)c, 3u);
  const v2f a = q[0], b = q[1], d = q[2];
  return {{a.x, a.y, b.x, b.y, d.x, d.y}};
}
__device__ __forceinline__ Aff<3> load_aff3(const float* tab, int c) {
  const v4f* q = entry<v4f, 48>(tab, c);
  const v4f a = q[0], b = q[1], d = q[2];
  return {{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, d.x, d.y, d.z, d.w}};
}
__device__ __forceinline__ Aff<3> load_aff3(lds_ptr<float> tab, int c) {
  lds_ptr<v4f> q = (lds_ptr<v4f>)tab + __umul24((uint32_t)c, 3u);
  const v4f a = q[0], b = q[1], d = q[2];
  return {{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, d.x, d.y, d.z, d.w}};
}

// v = M [p; 1] with the reference's nesting fma(m0, x, fma(m1, y, m2)).
__device__ __forceinline__ void apply2(const Aff<2>& M, float px, float py, float& ox, float& oy) {
  ox = fmaf(M.m[0], px, fmaf(M.m[1], py, M.m[2]));
  oy = fmaf(M.m[3], px, fmaf(M.m[4], py, M.m[5]));
}
__device__ __forceinline__ void apply3(const Aff<3>& M, float px, float py, float pz,
                                       float& ox, float& oy, float& oz) {
  ox = fmaf(M.m[0], px, fmaf(M.m[1], py, fmaf(M.m[2], pz, M.m[3])));
  oy = fmaf(M.m[4], px, fmaf(M.m[5], py, fmaf(M.m[6], pz, M.m[7])));
  oz = fmaf(M.m[8], px, fmaf(M.m[9], py, fmaf(M.m[10], pz, M.m[11])));
}

// One explicit-midpoint step with cell A fixed (cpab_ops_2d.cu:269-292,
// cpab_ops_1d.cu:249-266, cpab_ops_3d.cu:247-282).
__device__ __forceinline__ float midpoint1(const Aff<1>& A, float px, float h, float hh) {
  const float v = fmaf(A.a, px, A.b);
  const float pm = fmaf(hh, v, px);
  const float vm = fmaf(A.a, pm, A.b);
  return fmaf(h, vm, px);
}
__device__ __forceinline__ void midpoint2(const Aff<2>& A, float& px, float& py, float h, float hh) {
  float vx, vy, mx, my;
  apply2(A, px, py, vx, vy);
  const float pmx = fmaf(hh, vx, px), pmy = fmaf(hh, vy, py);
  apply2(A, pmx, pmy, mx, my);
  px = fmaf(h, mx, px);
  py = fmaf(h, my, py);
}
__device__ __forceinline__ void midpoint3(const Aff<3>& A, float& px, float& py, float& pz,
                                          float h, float hh) {
  float vx, vy, vz, mx, my, mz;
  apply3(A, px, py, pz, vx, vy, vz);
  const float pmx = fmaf(hh, vx, px), pmy = fmaf(hh, vy, py), pmz = fmaf(hh, vz, pz);
  apply3(A, pmx, pmy, pmz, mx, my, mz);
  px = fmaf(h, mx, px);
  py = fmaf(h, my, py);
  pz = fmaf(h, mz, pz);
}

// ---------------------------------------------------------------------------
// Adjoint step + cell moments for one midpoint step at position p with
// lambda = lambda_{t+1} (cpab_ops_2d.cu:334-382, 1d:301-329, 3d:331-403):
//   M[k][q] += h*lam_k*[pmid;1]_q + (h*h/2)*(A^T lam)_k*[p;1]_q
//   lam     += h*A^T (lam + (h/2) A^T lam)
// `hhh` is (h/2)*h.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void adjoint1(const Aff<1>& A, float px, float h, float hh, float hhh,
                                         float m[2], float& lam) {
  const float v = fmaf(A.a, px, A.b);
  const float pm = fmaf(hh, v, px);
  float at = A.a * lam;
  const float wm = h * lam;
  const float wp = hhh * at;
  m[0] = fmaf(wm, pm, m[0]);
  m[1] = m[1] + wm;
  m[0] = fmaf(wp, px, m[0]);
  m[1] = m[1] + wp;
  const float lmid = fmaf(hh, at, lam);
  at = A.a * lmid;
  lam = fmaf(h, at, lam);
}

__device__ __forceinline__ void adjoint2(const Aff<2>& A, float px, float py, float h, float hh,
                                         float hhh, float m[6], float& lx, float& ly) {
  const float* a = A.m;
  float vx, vy;
  apply2(A, px, py, vx, vy);
  const float pmx = fmaf(hh, vx, px), pmy = fmaf(hh, vy, py);
  float atx = fmaf(a[0], lx, a[3] * ly);
  float aty = fmaf(a[1], lx, a[4] * ly);
  const float wmx = h * lx, wmy = h * ly;
  const float wpx = hhh * atx, wpy = hhh * aty;
  m[0] = fmaf(wmx, pmx, m[0]);
  m[1] = fmaf(wmx, pmy, m[1]);
  m[2] = m[2] + wmx;
  m[3] = fmaf(wmy, pmx, m[3]);
  m[4] = fmaf(wmy, pmy, m[4]);
  m[5] = m[5] + wmy;
  m[0] = fmaf(wpx, px, m[0]);
  m[1] = fmaf(wpx, py, m[1]);
  m[2] = m[2] + wpx;
  m[3] = fmaf(wpy, px, m[3]);
  m[4] = fmaf(wpy, py, m[4]);
  m[5] = m[5] + wpy;
  const float mlx = fmaf(hh, atx, lx), mly = fmaf(hh, aty, ly);
  atx = fmaf(a[0], mlx, a[3] * mly);
  aty = fmaf(a[1], mlx, a[4] * mly);
  lx = fmaf(h, atx, lx);
  ly = fmaf(h, aty, ly);
}

__device__ __forceinline__ void adjoint3(const Aff<3>& A, float px, float py, float pz, float h,
                                         float hh, float hhh, float m[12], float& lx, float& ly,
                                         float& lz) {
  const float* a = A.m;
  float vx, vy, vz;
  apply3(A, px, py, pz, vx, vy, vz);
  const float pmx = fmaf(hh, vx, px), pmy = fmaf(hh, vy, py), pmz = fmaf(hh, vz, pz);
  float atx = fmaf(a[8], lz, fmaf(a[0], lx, a[4] * ly));
  float aty = fmaf(a[9], lz, fmaf(a[1], lx, a[5] * ly));
  float atz = fmaf(a[10], lz, fmaf(a[2], lx, a[6] * ly));
  const float w[3] = {h * lx, h * ly, h * lz};
  const float u[3] = {hhh * atx, hhh * aty, hhh * atz};
  const float pm[3] = {pmx, pmy, pmz};
  const float p[3] = {px, py, pz};
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    m[4 * k + 0] = fmaf(w[k], pm[0], m[4 * k + 0]);
    m[4 * k + 1] = fmaf(w[k], pm[1], m[4 * k + 1]);
    m[4 * k + 2] = fmaf(w[k], pm[2], m[4 * k + 2]);
    m[4 * k + 3] = m[4 * k + 3] + w[k];
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    m[4 * k + 0] = fmaf(u[k], p[0], m[4 * k + 0]);
    m[4 * k + 1] = fmaf(u[k], p[1], m[4 * k + 1]);
    m[4 * k + 2] = fmaf(u[k], p[2], m[4 * k + 2]);
    m[4 * k + 3] = m[4 * k + 3] + u[k];
  }
  const float mlx = fmaf(hh, atx, lx), mly = fmaf(hh, aty, ly), mlz = fmaf(hh, atz, lz);
  atx = fmaf(a[8], mlz, fmaf(a[0], mlx, a[4] * mly));
  aty = fmaf(a[9], mlz, fmaf(a[1], mlx, a[5] * mly));
  atz = fmaf(a[10], mlz, fmaf(a[2], mlx, a[6] * mly));
  lx = fmaf(h, atx, lx);
  ly = fmaf(h, aty, ly);
  lz = fmaf(h, atz, lz);
}

// ---------------------------------------------------------------------------
// Factored adjoint sweep.  With Ã = [A; 0] the (ndim+1)^2 augmented field and
// p̃ = [p; 1], the step above is, in exact arithmetic,
//   lam <- lam + G^T lam,            G = h A_lin + (h^2/2) A_lin^2
//   M   += h lam p̃^T (I + (h/2) Ã^T) + (h^2/2) A_lin^T lam p̃^T
// (p_mid = p + (h/2) Ã p̃, and lam + h A^T (lam + (h/2) A^T lam) = (I + G)^T lam).
// M is linear in lam p̃^T and A is constant inside a cell, so the sweep only
// accumulates S = sum lam p̃^T per cell and the moments follow once per cell
// after all trajectories are summed:
//   M = h S + (h^2/2) (S Ã^T + A_lin^T S)                       (moments_from_s)
// The adjoint step reads G from a per-cell table (adjoint_increment).  Same
// mathematics as cpab_ops_2d.cu:334-382; the rounding differs from the
// reference's op order by a few ulp.
// ---------------------------------------------------------------------------

// Per-cell table of the reverse sweep (16-byte aligned entries of
// RevStride<D>::S floats): G and the inverse of the cell's one-step midpoint
// map p' = E [p; 1], as rows [M | m] with p = M p' + m.
//   1D  [g, M, m, 0]                                              4 floats
//   2D  [g00 g01 g10 g11] [M00 M01 m0 M10] [M11 m1 0 0]             12 floats
//       (the inverse map packed, so that its reads, one of 16 bytes and one
//       of 8, fill no register that goes unused)
//   3D  3 rows [M_r0 M_r1 M_r2 m_r], then G (9 floats), then 0 0 0  24 floats
//       (every float a read fetches is used: a fetched register left unused is
//       reallocated at once, which makes the wave wait for the load there)
template <int D> struct RevStride;
template <> struct RevStride<1> { static constexpr int S = 4; };
template <> struct RevStride<2> { static constexpr int S = 12; };
template <> struct RevStride<3> { static constexpr int S = 24; };

template <int D> struct Adj;
template <> struct Adj<1> { float g; };
template <> struct Adj<2> { float g[4]; };   // row-major g00 g01 g10 g11
template <> struct Adj<3> { float g[9]; };   // row-major

__device__ __forceinline__ Adj<1> load_adj1(const float* tab, int c) { return {*entry<float, 16>(tab, c)}; }
__device__ __forceinline__ Adj<2> load_adj2(const float* tab, int c) {
  const v4f v = *entry<v4f, 48>(tab, c);
  return {{v.x, v.y, v.z, v.w}};
}
__device__ __forceinline__ Adj<1> load_adj1(lds_ptr<float> tab, int c) {
  return {tab[__umul24((uint32_t)c, 4u)]};
}
__device__ __forceinline__ Adj<2> load_adj2(lds_ptr<float> tab, int c) {
  const v4f v = ((lds_ptr<v4f>)tab)[__umul24((uint32_t)c, 3u)];
  return {{v.x, v.y, v.z, v.w}};
}
__device__ __forceinline__ Adj<3> load_adj3(const float* tab, int c) {
  const v4f* q = entry<v4f, 96>(tab, c);
  const v4f a = q[3], b = q[4];
  const float g8 = reinterpret_cast<const float*>(q)[20];
  return {{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, g8}};
}

// Inverse one-step map of a cell, row-major [D, D+1].
template <int D> struct Inv { float m[D * (D + 1)]; };

__device__ __forceinline__ Inv<1> load_inv1(const float* tab, int c) {
  const v2f v = *reinterpret_cast<const v2f*>(entry<float, 16>(tab, c) + 1);
  return {{v.x, v.y}};
}
__device__ __forceinline__ Inv<1> load_inv1(lds_ptr<float> tab, int c) {
  lds_ptr<float> e = tab + __umul24((uint32_t)c, 4u);
  return {{e[1], e[2]}};
}
__device__ __forceinline__ Inv<2> load_inv2(lds_ptr<float> tab, int c) {
  lds_ptr<v4f> q = (lds_ptr<v4f>)tab + __umul24((uint32_t)c, 3u);
  const v4f a = q[1];
  const v2f b = *(lds_ptr<v2f>)(q + 2);
  return {{a.x, a.y, a.z, a.w, b.x, b.y}};
}
__device__ __forceinline__ Inv<2> load_inv2(const float* tab, int c) {
  const v4f* q = entry<v4f, 48>(tab, c);
  const v4f a = q[1];
  const v2f b = *reinterpret_cast<const v2f*>(q + 2);
  return {{a.x, a.y, a.z, a.w, b.x, b.y}};
}
__device__ __forceinline__ Inv<3> load_inv3(const float* tab, int c) {
  const v4f* q = entry<v4f, 96>(tab, c);
  const v4f a = q[0], b = q[1], d = q[2];
  return {{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, d.x, d.y, d.z, d.w}};
}

// p <- M p + m: the position one replay step earlier.
template <int D>
__device__ __forceinline__ void step_back(const Inv<D>& E, float (&p)[D]) {
  float q[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    float acc = E.m[i * (D + 1) + D];
#pragma unroll
    for (int j = D - 1; j >= 0; --j) acc = fmaf(E.m[i * (D + 1) + j], p[j], acc);
    q[i] = acc;
  }
#pragma unroll
  for (int i = 0; i < D; ++i) p[i] = q[i];
}

// Keeps the values in VGPRs at this point of the program (an empty asm
// statement, no instruction): code that computes them cannot be sunk past it,
// e.g. into the join block of a following divergent branch.
template <int N>
__device__ __forceinline__ void pin(float (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) __asm__ volatile("" : "+v"(v[k]));
}

// One reverse step: S += lam (x) [p; 1], then lam += G^T lam.
__device__ __forceinline__ void adjoint_s1(const Adj<1>& G, float px, float s[2], float& lam) {
  s[0] = fmaf(lam, px, s[0]);
  s[1] = s[1] + lam;
  lam = fmaf(G.g, lam, lam);
}
__device__ __forceinline__ void adjoint_s2(const Adj<2>& G, float px, float py, float s[6],
                                           float& lx, float& ly) {
  s[0] = fmaf(lx, px, s[0]);
  s[1] = fmaf(lx, py, s[1]);
  s[2] = s[2] + lx;
  s[3] = fmaf(ly, px, s[3]);
  s[4] = fmaf(ly, py, s[4]);
  s[5] = s[5] + ly;
  const float nx = fmaf(G.g[0], lx, fmaf(G.g[2], ly, lx));
  const float ny = fmaf(G.g[1], lx, fmaf(G.g[3], ly, ly));
  lx = nx;
  ly = ny;
}
__device__ __forceinline__ void adjoint_s3(const Adj<3>& G, float px, float py, float pz,
                                           float s[12], float& lx, float& ly, float& lz) {
  const float l[3] = {lx, ly, lz};
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    s[4 * k + 0] = fmaf(l[k], px, s[4 * k + 0]);
    s[4 * k + 1] = fmaf(l[k], py, s[4 * k + 1]);
    s[4 * k + 2] = fmaf(l[k], pz, s[4 * k + 2]);
    s[4 * k + 3] = s[4 * k + 3] + l[k];
  }
  const float* g = G.g;
  lx = fmaf(g[0], l[0], fmaf(g[3], l[1], fmaf(g[6], l[2], l[0])));
  ly = fmaf(g[1], l[0], fmaf(g[4], l[1], fmaf(g[7], l[2], l[1])));
  lz = fmaf(g[2], l[0], fmaf(g[5], l[1], fmaf(g[8], l[2], l[2])));
}

// G = h A_lin + (h^2/2) A_lin^2 of one cell; `a` is the row-major [D, D+1]
// block of A, `hhh` = (h/2)*h.  Writes the G part of a RevStride<D> entry.
template <int D>
__device__ __forceinline__ void adjoint_increment(const float* a, float h, float hhh, float* g) {
  constexpr int W = D + 1;
  constexpr int RS = D;  // row stride inside the table entry
#pragma unroll
  for (int i = 0; i < D; ++i) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      float sq = 0.0f;
#pragma unroll
      for (int r = 0; r < D; ++r) sq = fmaf(a[i * W + r], a[r * W + j], sq);
      g[i * RS + j] = fmaf(h, a[i * W + j], hhh * sq);
    }
    if (RS > D) g[i * RS + D] = 0.0f;
  }
}

// Inverse of a cell's one-step midpoint map.  With the replay's fp32 step h
// (and h/2, exact), one explicit-midpoint step is, in exact arithmetic,
//   p' = E_lin p + e,  E_lin = I + h A + h (h/2) A^2,  e = h b + h (h/2) A b.
// Its inverse M = E_lin^-1, m = -M e is formed in double and rounded once.
// Writes [M | m] row-major, D rows of D+1.
template <int D>
__device__ __forceinline__ void inverse_step_map(const float* a, float h, float* out) {
  constexpr int W = D + 1;
  const double hd = h, h2 = (double)h * (double)(h * 0.5f);
  double E[3][3] = {}, e[3] = {};
#pragma unroll
  for (int i = 0; i < D; ++i) {
    double ab = 0.0;
#pragma unroll
    for (int r = 0; r < D; ++r) ab += (double)a[i * W + r] * a[r * W + D];
    e[i] = hd * a[i * W + D] + h2 * ab;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      double sq = 0.0;
#pragma unroll
      for (int r = 0; r < D; ++r) sq += (double)a[i * W + r] * a[r * W + j];
      E[i][j] = (i == j ? 1.0 : 0.0) + hd * a[i * W + j] + h2 * sq;
    }
  }
  double M[3][3] = {};
  if (D == 1) {
    M[0][0] = 1.0 / E[0][0];
  } else if (D == 2) {
    const double id = 1.0 / (E[0][0] * E[1][1] - E[0][1] * E[1][0]);
    M[0][0] = E[1][1] * id;
    M[0][1] = -E[0][1] * id;
    M[1][0] = -E[1][0] * id;
    M[1][1] = E[0][0] * id;
  } else {
    const double c00 = E[1][1] * E[2][2] - E[1][2] * E[2][1];
    const double c01 = E[0][2] * E[2][1] - E[0][1] * E[2][2];
    const double c02 = E[0][1] * E[1][2] - E[0][2] * E[1][1];
    const double id = 1.0 / (E[0][0] * c00 + E[1][0] * c01 + E[2][0] * c02);
    M[0][0] = c00 * id;
    M[0][1] = c01 * id;
    M[0][2] = c02 * id;
    M[1][0] = (E[1][2] * E[2][0] - E[1][0] * E[2][2]) * id;
    M[1][1] = (E[0][0] * E[2][2] - E[0][2] * E[2][0]) * id;
    M[1][2] = (E[0][2] * E[1][0] - E[0][0] * E[1][2]) * id;
    M[2][0] = (E[1][0] * E[2][1] - E[1][1] * E[2][0]) * id;
    M[2][1] = (E[0][1] * E[2][0] - E[0][0] * E[2][1]) * id;
    M[2][2] = (E[0][0] * E[1][1] - E[0][1] * E[1][0]) * id;
  }
#pragma unroll
  for (int i = 0; i < D; ++i) {
    double m = 0.0;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      out[i * W + j] = (float)M[i][j];
      m -= M[i][j] * e[j];
    }
    out[i * W + D] = (float)m;
  }
}

// Spectral norm ||M||_2 of the linear part of an inverse one-step map (the
// rounded float entries, row-major [D, D+1]), evaluated in double: the largest
// singular value, from the largest eigenvalue of M^T M (closed form for a
// symmetric 2x2; the trigonometric form for a symmetric 3x3).  A recovered
// position's error is carried to the previous step multiplied by M, so along
// a trajectory of T steps it grows by at most prod ||M_c||_2 <= (max_c ||M_c||_2)^T.
// Rounded up by a relative 1e-9; NaN maps to +inf.
template <int D>
__device__ __forceinline__ float inverse_map_norm(const float* inv) {
  constexpr int W = D + 1;
  double s;
  if (D == 1) {
    s = fabs((double)inv[0]);
  } else if (D == 2) {
    const double a = inv[0], b = inv[1], c = inv[W], d = inv[W + 1];
    const double t = a * a + b * b + c * c + d * d;  // ||M||_F^2
    const double det = a * d - b * c;
    const double disc = sqrt(fmax(t * t - 4.0 * det * det, 0.0));
    s = sqrt(0.5 * (t + disc));
  } else {
    double m[3][3], b[3][3];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) m[i][j] = inv[i * W + j];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) b[i][j] = m[0][i] * m[0][j] + m[1][i] * m[1][j] + m[2][i] * m[2][j];
    const double p1 = b[0][1] * b[0][1] + b[0][2] * b[0][2] + b[1][2] * b[1][2];
    const double q = (b[0][0] + b[1][1] + b[2][2]) / 3.0;
    const double d0 = b[0][0] - q, d1 = b[1][1] - q, d2 = b[2][2] - q;
    const double p2 = d0 * d0 + d1 * d1 + d2 * d2 + 2.0 * p1;
    double lmax = q;
    if (p2 > 0.0) {
      const double p = sqrt(p2 / 6.0), ip = 1.0 / p;
      const double c00 = d0 * ip, c11 = d1 * ip, c22 = d2 * ip;
      const double c01 = b[0][1] * ip, c02 = b[0][2] * ip, c12 = b[1][2] * ip;
      const double det = c00 * (c11 * c22 - c12 * c12) - c01 * (c01 * c22 - c12 * c02) +
                         c02 * (c01 * c12 - c11 * c02);
      const double r = fmin(fmax(0.5 * det, -1.0), 1.0);
      lmax = q + 2.0 * p * cos(acos(r) / 3.0);
    }
    s = sqrt(fmax(lmax, 0.0));
  }
  s *= 1.0 + 1e-9;
  return (s <= 3.0e38) ? (float)s : INFINITY;
}

// Moments of one cell from its accumulated S (both row-major [D, D+1]):
//   M_kq = h S_kq + hhh (sum_{r<D} S_kr A_qr + S_kD A_qD [q<D] + sum_j A_jk S_jq)
template <int D>
__device__ __forceinline__ void moments_from_s(const float* a, const float* s, float h, float hhh,
                                               float* m) {
  constexpr int W = D + 1;
#pragma unroll
  for (int k = 0; k < D; ++k) {
#pragma unroll
    for (int q = 0; q < W; ++q) {
      float t = 0.0f;
      if (q < D) {
#pragma unroll
        for (int r = 0; r < W; ++r) t = fmaf(s[k * W + r], a[q * W + r], t);
      }
#pragma unroll
      for (int j = 0; j < D; ++j) t = fmaf(a[j * W + k], s[j * W + q], t);
      m[k * W + q] = fmaf(h, s[k * W + q], hhh * t);
    }
  }
}

}  // namespace cpab
