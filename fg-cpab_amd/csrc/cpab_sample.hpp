// Border-clamped linear / bilinear / trilinear sampling of one data channel
// and its derivatives, shared by the resampling kernels (interp.hip) and the
// fused transform_data kernels (integrate.hip, adjoint.hip).
//
// Arithmetic follows the reference's eager torch ops one by one
// (cpab/pytorch/interpolation.py:3-159; no fused multiply-add):
// x = g*(W-1); x0 = clamp(floor(x)); xd = x - x0;
// lerp(a, b, t) = a*(1-t) + b*t with the axes reduced x, then y, then z.
// Grid coordinate k indexes data axis k (of the spatial axes).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace cpab {

struct Axis {
  int i0, i1;   // clamped corner indices
  float t;      // fractional weight of i1
};

__device__ __forceinline__ Axis axis_of(float g, int size) {
  const float x = g * (float)(size - 1);
  const float f = floorf(x);
  const float hi = (float)(size - 1);
  // floor -> clamp to [0, size-1] (integer semantics of the reference; done in
  // float first so out-of-range values cannot overflow the conversion).
  const int a = (int)fminf(fmaxf(f, 0.0f), hi);
  const int b = (int)fminf(fmaxf(f + 1.0f, 0.0f), hi);
  return {a, b, x - (float)a};
}

__device__ __forceinline__ float lerp_ref(float a, float b, float t) {
  const float u = 1.0f - t;
  return __fadd_rn(__fmul_rn(a, u), __fmul_rn(b, t));
}

// Offset of (x, y, z) inside one [in[0], in[1](, in[2])] plane (< 2^31, checked
// by the C-ABI layer).
template <int ND>
__device__ __forceinline__ int plane_index(const int* in, int x, int y, int z) {
  if (ND == 1) return x;
  if (ND == 2) return x * in[1] + y;
  return (x * in[1] + y) * in[2] + z;
}

template <int ND>
__device__ __forceinline__ float sample(const int* in, const float* __restrict__ d, const Axis& ax,
                                        const Axis& ay, const Axis& az) {
  if (ND == 1) return lerp_ref(d[ax.i0], d[ax.i1], ax.t);
  if (ND == 2) {
    const float c00 = d[plane_index<2>(in, ax.i0, ay.i0, 0)];
    const float c01 = d[plane_index<2>(in, ax.i0, ay.i1, 0)];
    const float c10 = d[plane_index<2>(in, ax.i1, ay.i0, 0)];
    const float c11 = d[plane_index<2>(in, ax.i1, ay.i1, 0)];
    return lerp_ref(lerp_ref(c00, c10, ax.t), lerp_ref(c01, c11, ax.t), ay.t);
  }
  float c[2][2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        c[a][b][e] = d[plane_index<3>(in, a ? ax.i1 : ax.i0, b ? ay.i1 : ay.i0, e ? az.i1 : az.i0)];
  const float c00 = lerp_ref(c[0][0][0], c[1][0][0], ax.t);
  const float c01 = lerp_ref(c[0][0][1], c[1][0][1], ax.t);
  const float c10 = lerp_ref(c[0][1][0], c[1][1][0], ax.t);
  const float c11 = lerp_ref(c[0][1][1], c[1][1][1], ax.t);
  return lerp_ref(lerp_ref(c00, c10, ay.t), lerp_ref(c01, c11, ay.t), az.t);
}

// d out / d (x, y, z) for one channel with upstream gradient g (before the
// (size-1) chain factor), added into dxyz, and the corner scatter for
// grad_data (gd, may be null).
template <int ND>
__device__ __forceinline__ void sample_grad(const int* in, const float* __restrict__ d,
                                            const Axis& ax, const Axis& ay, const Axis& az,
                                            float g, float* dxyz, float* __restrict__ gd) {
  const float ux = 1.0f - ax.t, uy = 1.0f - ay.t, uz = 1.0f - az.t;
  if (ND == 1) {
    if (dxyz) dxyz[0] += g * (d[ax.i1] - d[ax.i0]);
    if (gd) {
      unsafeAtomicAdd(gd + ax.i0, g * ux);
      unsafeAtomicAdd(gd + ax.i1, g * ax.t);
    }
    return;
  }
  if (ND == 2) {
    const int i00 = plane_index<2>(in, ax.i0, ay.i0, 0), i01 = plane_index<2>(in, ax.i0, ay.i1, 0);
    const int i10 = plane_index<2>(in, ax.i1, ay.i0, 0), i11 = plane_index<2>(in, ax.i1, ay.i1, 0);
    if (dxyz) {
      const float c00 = d[i00], c01 = d[i01], c10 = d[i10], c11 = d[i11];
      const float c0 = lerp_ref(c00, c10, ax.t), c1 = lerp_ref(c01, c11, ax.t);
      dxyz[0] += g * uy * (c10 - c00) + g * ay.t * (c11 - c01);
      dxyz[1] += g * (c1 - c0);
    }
    if (gd) {
      const float g0 = g * uy, g1 = g * ay.t;
      unsafeAtomicAdd(gd + i00, g0 * ux);
      unsafeAtomicAdd(gd + i10, g0 * ax.t);
      unsafeAtomicAdd(gd + i01, g1 * ux);
      unsafeAtomicAdd(gd + i11, g1 * ax.t);
    }
    return;
  }
  int idx[2][2][2];
  float c[2][2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        idx[a][b][e] = plane_index<3>(in, a ? ax.i1 : ax.i0, b ? ay.i1 : ay.i0, e ? az.i1 : az.i0);
        c[a][b][e] = dxyz ? d[idx[a][b][e]] : 0.0f;
      }
  if (dxyz) {
    // Along x: the four (y, z) lines; along y: the two z planes; along z: the two halves.
    const float wyz[2][2] = {{uy * uz, uy * az.t}, {ay.t * uz, ay.t * az.t}};
    float gx = 0.0f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 2; ++e) gx += wyz[b][e] * (c[1][b][e] - c[0][b][e]);
    const float c00 = lerp_ref(c[0][0][0], c[1][0][0], ax.t);
    const float c01 = lerp_ref(c[0][0][1], c[1][0][1], ax.t);
    const float c10 = lerp_ref(c[0][1][0], c[1][1][0], ax.t);
    const float c11 = lerp_ref(c[0][1][1], c[1][1][1], ax.t);
    const float gy = uz * (c10 - c00) + az.t * (c11 - c01);
    const float gz = lerp_ref(c01, c11, ay.t) - lerp_ref(c00, c10, ay.t);
    dxyz[0] += g * gx;
    dxyz[1] += g * gy;
    dxyz[2] += g * gz;
  }
  if (gd) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float w = (a ? ax.t : ux) * (b ? ay.t : uy) * (e ? az.t : uz);
          unsafeAtomicAdd(gd + idx[a][b][e], g * w);
        }
  }
}

}  // namespace cpab

namespace cpab {

// Output-ordered image geometry of the fused transform_data kernels.  Output
// position q = (i0*o1 + i1)*o2 + i2 runs over [o0, o1(, o2)] with the LAST axis
// fastest (the image layout); it integrates the uniform-grid point
// (axes_0[i0], axes_1[i1], axes_2[i2]).  Cpab.uniform_meshgrid
// (cpab/cpab.py:131-144) is the Cartesian product of those per-axis
// coordinates, listed with coordinate 0 fastest (m = i0 + o0*(i1 + o1*i2));
// the kernels read the per-axis vectors, a few KB that stay in cache, instead
// of the meshgrid.
struct ImageShape {
  int o[3];          // output (= meshgrid) sizes, unused axes 1
  int in[3];         // data spatial sizes, unused axes 1
  int C;             // channels
  int nP;            // prod(o)
  int64_t plane_in;  // prod(in)
  double inv_o[3];   // 1.0 / o[k]
  int walk_tiles;    // the fused kernels walk 16 x 4 tiles (tile_index)
};

// q / d for 0 <= q < 2^31 and 1 <= d < 2^31 without the ~40-instruction
// integer division: the double product q * (1/d) is within one of the
// quotient (relative error ~2^-52 on a value below 2^31), and the remainder
// fixes the last unit.  Sets r = q - (q / d) * d.
__device__ __forceinline__ int div_index(int q, int d, double inv_d, int& r) {
  int e = (int)((double)q * inv_d);
  r = q - e * d;
  if (r < 0) { e -= 1; r += d; }
  else if (r >= d) { e += 1; r -= d; }
  return e;
}

// Grid indices of image position q.
template <int ND>
__device__ __forceinline__ void image_index(const ImageShape& s, int q, int (&i)[3]) {
  if (ND == 1) { i[0] = q; i[1] = i[2] = 0; return; }
  if (ND == 2) { i[0] = div_index(q, s.o[1], s.inv_o[1], i[1]); i[2] = 0; return; }
  const int r = div_index(q, s.o[2], s.inv_o[2], i[2]);
  i[0] = div_index(r, s.o[1], s.inv_o[1], i[1]);
}

// Tiled walk of the fused kernels: each run of 64 positions (one wave) is a
// tile of kWalkW along the last axis by kWalkH along the axis before it, which
// keeps a wave's trajectories in few cells and its image reads and writes in
// kWalkW-float runs.  Consecutive tiles step
// 2D: the i0 block, then the i1 block (1024 positions = 64 x 16, i0 x i1);
// 3D: i0, then the i1 block, then the i2 block (1024 = 16 x 4 x 16).
// Needs o[ND-1] % kWalkW == 0 and o[ND-2] % kWalkH == 0 (then the tiles cover
// the grid exactly once).  1 / (o / kWalkH) == kWalkH * (1 / o) exactly:
// scaling by a power of two commutes with rounding.
constexpr int kWalkW = 16;
constexpr int kWalkH = 64 / kWalkW;
static_assert(kWalkW * kWalkH == 64 && (kWalkW & (kWalkW - 1)) == 0, "walk tile");

template <int ND>
__device__ __forceinline__ void tile_index(const ImageShape& s, int m, int (&i)[3]) {
  const int l = m & 63;
  int r0, r1;
  if (ND == 2) {
    const int b1 = div_index(m >> 6, s.o[0] / kWalkH, kWalkH * s.inv_o[0], r0);
    i[0] = r0 * kWalkH + l / kWalkW;
    i[1] = b1 * kWalkW + l % kWalkW;
    i[2] = 0;
    return;
  }
  const int rest = div_index(m >> 6, s.o[0], s.inv_o[0], r0);
  const int b2 = div_index(rest, s.o[1] / kWalkH, kWalkH * s.inv_o[1], r1);
  i[0] = r0;
  i[1] = r1 * kWalkH + l / kWalkW;
  i[2] = b2 * kWalkW + l % kWalkW;
}

// Grid indices of meshgrid position m (coordinate 0 fastest).
template <int ND>
__device__ __forceinline__ void mesh_index(const ImageShape& s, int m, int (&i)[3]) {
  if (ND == 1) { i[0] = m; i[1] = i[2] = 0; return; }
  const int r = div_index(m, s.o[0], s.inv_o[0], i[0]);
  if (ND == 2) { i[1] = r; i[2] = 0; return; }
  i[2] = div_index(r, s.o[1], s.inv_o[1], i[1]);
}

// Image position of grid indices i.
template <int ND>
__device__ __forceinline__ int image_pos(const ImageShape& s, const int (&i)[3]) {
  if (ND == 1) return i[0];
  if (ND == 2) return i[0] * s.o[1] + i[1];
  return (i[0] * s.o[1] + i[1]) * s.o[2] + i[2];
}

// The uniform-grid point with indices i: coordinate k from the k-th per-axis
// vector of `axes` (the vectors concatenated, axis 0 first).
template <int ND>
__device__ __forceinline__ void grid_point(const ImageShape& s, const float* __restrict__ axes,
                                           const int (&i)[3], float (&x)[3]) {
  x[0] = axes[i[0]];
  x[1] = ND >= 2 ? axes[s.o[0] + i[1]] : 0.0f;
  x[2] = ND == 3 ? axes[s.o[0] + s.o[1] + i[2]] : 0.0f;
}

}  // namespace cpab
