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

// Offset of (x, y, z) inside one [in[0], in[1](, in[2])] plane (at most 2^30
// values, checked by the C-ABI layer).
template <int ND>
__device__ __forceinline__ int plane_index(const int* in, int x, int y, int z) {
  if (ND == 1) return x;
  if (ND == 2) return x * in[1] + y;
  return (x * in[1] + y) * in[2] + z;
}

// d[i] for 0 <= i < 2^30, addressed as a 32-bit byte offset from d.  When d
// is the same for the whole wave (one data channel) the load takes d as its
// scalar base and each lane carries one 32-bit offset, instead of a 64-bit
// address per lane and load.
__device__ __forceinline__ float load_at(const float* __restrict__ d, int i) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(d) + ((uint32_t)i << 2));
}

// One data channel as a raw buffer resource: its 64-bit base and byte size sit
// in scalar registers and each lane supplies a 32-bit byte offset (with a
// pointer that the compiler hoists out of a channel loop, the offsets would
// become 64-bit per lane and load).  A read past the size returns 0.
struct ChannelBuf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ ChannelBuf(const float* d, int64_t n)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(d), (short)0,
                                            (int)(uint32_t)min(n * 4, (int64_t)0xFFFFFFFF),
                                            0x00020000)) {}   // dword 3 of a raw gfx9 buffer
  __device__ __forceinline__ float operator()(int i) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)((uint32_t)i << 2), 0, 0));
  }
  // d[i] and d[i + 1] with one 8-byte load (4-byte aligned; the HSA runtime
  // runs the vector memory path in unaligned mode).
  __device__ __forceinline__ float2 pair(int i) const {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)((uint32_t)i << 2), 0, 0);
    const unsigned int lo = v[0], hi = v[1];   // (bit-casting v[k] directly reads v[0] twice)
    return make_float2(__builtin_bit_cast(float, lo), __builtin_bit_cast(float, hi));
  }
};

// A data channel read through load_at.
struct ChannelPtr {
  const float* __restrict__ d;
  __device__ __forceinline__ float operator()(int i) const { return load_at(d, i); }
};

// gd[i] += v (float atomic), addressed like load_at.
__device__ __forceinline__ void add_at(float* __restrict__ gd, int i, float v) {
  unsafeAtomicAdd(reinterpret_cast<float*>(reinterpret_cast<char*>(gd) + ((uint32_t)i << 2)), v);
}

// The 2^ND corner values of one sample from channel src (ChannelBuf or
// ChannelPtr), c[(a << 2) | (b << 1) | e] for the corner
// (a ? x1 : x0, b ? y1 : y0, e ? z1 : z0) (2D: c[(a << 1) | b]).
template <int ND, class Src>
__device__ __forceinline__ void gather(const int* in, const Src& src, const Axis& ax,
                                       const Axis& ay, const Axis& az, float* c) {
  if (ND == 1) {
    c[0] = src(ax.i0);
    c[1] = src(ax.i1);
    return;
  }
  if (ND == 2) {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
        c[(a << 1) | b] = src(plane_index<2>(in, a ? ax.i1 : ax.i0, b ? ay.i1 : ay.i0, 0));
    return;
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 2; ++e)
        c[(a << 2) | (b << 1) | e] =
            src(plane_index<3>(in, a ? ax.i1 : ax.i0, b ? ay.i1 : ay.i0, e ? az.i1 : az.i0));
}

// gather() from a ChannelBuf with the corners paired along the contiguous
// (last) data axis: one 8-byte load reads (.., s) and (.., s + 1) with
// s = min(i0, size - 2) on that axis, which holds both of its corner indices
// (i1 = i0 + 1, or both clamped to 0 or to size - 1).  Needs that axis'
// size >= 2; half the load instructions of gather().
template <int ND>
__device__ __forceinline__ void gather_pairs(const int* in, const ChannelBuf& src, const Axis& ax,
                                             const Axis& ay, const Axis& az, float* c) {
  const Axis& last = ND == 1 ? ax : (ND == 2 ? ay : az);
  const int s = min(last.i0, in[ND - 1] - 2);
  const bool lo_up = last.i0 != s;   // i0 == s + 1 (clamped to size - 1)
  const bool hi_up = last.i1 != s;   // i1 == s + 1
  if (ND == 1) {
    const float2 p = src.pair(s);
    c[0] = lo_up ? p.y : p.x;
    c[1] = hi_up ? p.y : p.x;
    return;
  }
  if (ND == 2) {
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const float2 p = src.pair(plane_index<2>(in, a ? ax.i1 : ax.i0, s, 0));
      c[(a << 1) | 0] = lo_up ? p.y : p.x;
      c[(a << 1) | 1] = hi_up ? p.y : p.x;
    }
    return;
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const float2 p = src.pair(plane_index<3>(in, a ? ax.i1 : ax.i0, b ? ay.i1 : ay.i0, s));
      c[(a << 2) | (b << 1) | 0] = lo_up ? p.y : p.x;
      c[(a << 2) | (b << 1) | 1] = hi_up ? p.y : p.x;
    }
}

// The interpolated value from the corners of gather().
template <int ND>
__device__ __forceinline__ float blend(const float* c, const Axis& ax, const Axis& ay,
                                       const Axis& az) {
  if (ND == 1) return lerp_ref(c[0], c[1], ax.t);
  if (ND == 2) return lerp_ref(lerp_ref(c[0], c[2], ax.t), lerp_ref(c[1], c[3], ax.t), ay.t);
  const float c00 = lerp_ref(c[0], c[4], ax.t);
  const float c01 = lerp_ref(c[1], c[5], ax.t);
  const float c10 = lerp_ref(c[2], c[6], ax.t);
  const float c11 = lerp_ref(c[3], c[7], ax.t);
  return lerp_ref(lerp_ref(c00, c10, ay.t), lerp_ref(c01, c11, ay.t), az.t);
}

template <int ND>
__device__ __forceinline__ float sample(const int* in, const float* __restrict__ d, const Axis& ax,
                                        const Axis& ay, const Axis& az) {
  float c[1 << ND];
  gather<ND>(in, ChannelPtr{d}, ax, ay, az, c);
  return blend<ND>(c, ax, ay, az);
}

// The sample at (ax, ay, az) (blend's value, bit for bit) and its spatial
// gradient d out / d (x, y, z) before the (size-1) chain factor: blend_grad's
// terms without the upstream gradient, which the fused transform_data forward
// stores so that its backward seeds a pixel's adjoint from two or three
// coalesced reads instead of the corner reads.  In 1D/3D g times these equals
// blend_grad's result bit for bit; in 2D the x term is g (uy dx0 + ty dx1)
// where blend_grad rounds (g uy) dx0 + (g ty) dx1.
template <int ND>
__device__ __forceinline__ float sample_spatial_grad(const int* in, const float* __restrict__ d,
                                                     const Axis& ax, const Axis& ay,
                                                     const Axis& az, float* grad) {
  float c[1 << ND];
  gather<ND>(in, ChannelPtr{d}, ax, ay, az, c);
  if (ND == 1) {
    grad[0] = c[1] - c[0];
    return lerp_ref(c[0], c[1], ax.t);
  }
  const float uy = 1.0f - ay.t;
  if (ND == 2) {
    const float c0 = lerp_ref(c[0], c[2], ax.t), c1 = lerp_ref(c[1], c[3], ax.t);
    grad[0] = uy * (c[2] - c[0]) + ay.t * (c[3] - c[1]);
    grad[1] = c1 - c0;
    return lerp_ref(c0, c1, ay.t);
  }
  const float uz = 1.0f - az.t;
  const float wyz[2][2] = {{uy * uz, uy * az.t}, {ay.t * uz, ay.t * az.t}};
  float gx = 0.0f;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int e = 0; e < 2; ++e) gx += wyz[b][e] * (c[4 | (b << 1) | e] - c[(b << 1) | e]);
  const float c00 = lerp_ref(c[0], c[4], ax.t);
  const float c01 = lerp_ref(c[1], c[5], ax.t);
  const float c10 = lerp_ref(c[2], c[6], ax.t);
  const float c11 = lerp_ref(c[3], c[7], ax.t);
  grad[0] = gx;
  grad[1] = uz * (c10 - c00) + az.t * (c11 - c01);
  grad[2] = lerp_ref(c01, c11, ay.t) - lerp_ref(c00, c10, ay.t);
  return lerp_ref(lerp_ref(c00, c10, ay.t), lerp_ref(c01, c11, ay.t), az.t);
}

// d out / d (x, y, z) for one channel with upstream gradient g (before the
// (size-1) chain factor) from the corners of gather(), added into dxyz.
template <int ND>
__device__ __forceinline__ void blend_grad(const float* c, const Axis& ax, const Axis& ay,
                                           const Axis& az, float g, float* dxyz) {
  if (ND == 1) {
    dxyz[0] += g * (c[1] - c[0]);
    return;
  }
  const float uy = 1.0f - ay.t;
  if (ND == 2) {
    const float c00 = c[0], c01 = c[1], c10 = c[2], c11 = c[3];
    const float c0 = lerp_ref(c00, c10, ax.t), c1 = lerp_ref(c01, c11, ax.t);
    dxyz[0] += g * uy * (c10 - c00) + g * ay.t * (c11 - c01);
    dxyz[1] += g * (c1 - c0);
    return;
  }
  const float uz = 1.0f - az.t;
  // Along x: the four (y, z) lines; along y: the two z planes; along z: the two halves.
  const float wyz[2][2] = {{uy * uz, uy * az.t}, {ay.t * uz, ay.t * az.t}};
  float gx = 0.0f;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int e = 0; e < 2; ++e) gx += wyz[b][e] * (c[4 | (b << 1) | e] - c[(b << 1) | e]);
  const float c00 = lerp_ref(c[0], c[4], ax.t);
  const float c01 = lerp_ref(c[1], c[5], ax.t);
  const float c10 = lerp_ref(c[2], c[6], ax.t);
  const float c11 = lerp_ref(c[3], c[7], ax.t);
  const float gy = uz * (c10 - c00) + az.t * (c11 - c01);
  const float gz = lerp_ref(c01, c11, ay.t) - lerp_ref(c00, c10, ay.t);
  dxyz[0] += g * gx;
  dxyz[1] += g * gy;
  dxyz[2] += g * gz;
}

// Where the corner scatter of grad_data adds: float atomics into one channel's
// plane (the deterministic backward brings its own sink with the same add()).
struct FloatScatter {
  float* __restrict__ p;
  __device__ __forceinline__ bool on() const { return p != nullptr; }
  __device__ __forceinline__ FloatScatter channel(int64_t off) const { return {p + off}; }
  __device__ __forceinline__ void add(int i, float v) const { add_at(p, i, v); }
};

// The corner scatter of grad_data: g times each corner's weight added into gd
// (gd.add(plane index, value)).
template <int ND, typename G>
__device__ __forceinline__ void scatter_to(const int* in, const G& gd, const Axis& ax,
                                           const Axis& ay, const Axis& az, float g) {
  const float ux = 1.0f - ax.t, uy = 1.0f - ay.t, uz = 1.0f - az.t;
  if (ND == 1) {
    gd.add(ax.i0, g * ux);
    gd.add(ax.i1, g * ax.t);
    return;
  }
  if (ND == 2) {
    const float g0 = g * uy, g1 = g * ay.t;
    gd.add(plane_index<2>(in, ax.i0, ay.i0, 0), g0 * ux);
    gd.add(plane_index<2>(in, ax.i1, ay.i0, 0), g0 * ax.t);
    gd.add(plane_index<2>(in, ax.i0, ay.i1, 0), g1 * ux);
    gd.add(plane_index<2>(in, ax.i1, ay.i1, 0), g1 * ax.t);
    return;
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float w = (a ? ax.t : ux) * (b ? ay.t : uy) * (e ? az.t : uz);
        gd.add(plane_index<3>(in, a ? ax.i1 : ax.i0, b ? ay.i1 : ay.i0, e ? az.i1 : az.i0), g * w);
      }
}

template <int ND>
__device__ __forceinline__ void scatter(const int* in, float* __restrict__ gd, const Axis& ax,
                                        const Axis& ay, const Axis& az, float g) {
  scatter_to<ND>(in, FloatScatter{gd}, ax, ay, az, g);
}

// blend_grad into dxyz (may be null) and scatter into *gd (may be null).
template <int ND, typename G>
__device__ __forceinline__ void sample_grad_to(const int* in, const float* __restrict__ d,
                                               const Axis& ax, const Axis& ay, const Axis& az,
                                               float g, float* dxyz, const G* gd) {
  if (dxyz) {
    float c[1 << ND];
    gather<ND>(in, ChannelPtr{d}, ax, ay, az, c);
    blend_grad<ND>(c, ax, ay, az, g, dxyz);
  }
  if (gd) scatter_to<ND>(in, *gd, ax, ay, az, g);
}

template <int ND>
__device__ __forceinline__ void sample_grad(const int* in, const float* __restrict__ d,
                                            const Axis& ax, const Axis& ay, const Axis& az,
                                            float g, float* dxyz, float* __restrict__ gd) {
  const FloatScatter sink{gd};
  sample_grad_to<ND>(in, d, ax, ay, az, g, dxyz, gd ? &sink : nullptr);
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
