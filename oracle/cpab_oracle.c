/*
 * TEST INFRASTRUCTURE ONLY -- CPU oracle for the CPAB hot path.  Loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg (as the
 * checker / reference-semantics CPU baseline); the product never links it.
 *
 * A C restatement of the reference's CUDA kernels (cpab/core/cpab_ops_{1d,2d,
 * 3d}.cu) and of cpab/pytorch/interpolation.py, op for op in fp32 (the _f32
 * entry points) plus a float64 twin (_f64) used only to pin the mathematics.
 * Built by oracle/Makefile with -ffp-contract=off -fopenmp.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define CPAB_ORC_MAX_STEPS 100

/* ---- float32: the reference's arithmetic ---- */
#define R float
#define SUF _f32
#define FMA fmaf
#define FLOOR floorf
#define FMIN fminf
#define FMAX fmaxf
#define FABS fabsf
/* exp / log evaluated in double and rounded once (correctly rounded float),
 * the same as the HIP kernels do */
#define EXP(x) ((float)exp((double)(x)))
#define LOG(x) ((float)log((double)(x)))
#include "cpab_oracle_impl.h"
#undef R
#undef SUF
#undef FMA
#undef FLOOR
#undef FMIN
#undef FMAX
#undef FABS
#undef EXP
#undef LOG

/* ---- float64 twin ---- */
#define R double
#define SUF _f64
#define FMA fma
#define FLOOR floor
#define FMIN fmin
#define FMAX fmax
#define FABS fabs
#define EXP exp
#define LOG log
#include "cpab_oracle_impl.h"

int orc_max_steps(void) { return CPAB_ORC_MAX_STEPS; }

/* ---- expm of dT*[A; 0] (cpab_ops_1d.cu:404-429, 2d.cu:537-653, 3d.cu:538-674) ----
 * fp32, nvcc-style contraction of the plain sums (left product fused). */
static int n_squarings(float norm) { return (norm > 0.5f) ? (int)ceilf(log2f(norm * 2.0f)) : 0; }
static float dot3(float x1, float y1, float x2, float y2, float x3, float y3) {
  return fmaf(x3, y3, fmaf(x1, y1, x2 * y2));
}
static float cross2(float x1, float y1, float x2, float y2) { return fmaf(x1, y1, -(x2 * y2)); }

static void expm2(float dT, const float* A, float* o) {
  const float m00 = dT * A[0], m01 = dT * A[1];
  float exprel;
  if (fabsf(m00) > 1e-6f) exprel = (float)expm1((double)m00) / m00;
  else {
    const float m2 = m00 * m00;
    exprel = fmaf((1.0f / 24.0f) * m2, m00, fmaf(1.0f / 6.0f, m2, fmaf(0.5f, m00, 1.0f)));
  }
  o[0] = (float)exp((double)m00);
  o[1] = m01 * exprel;
}

static void expm3(float dT, const float* A, float* o) {
  const float a00 = dT * A[0], a01 = dT * A[1], a02 = dT * A[2];
  const float a10 = dT * A[3], a11 = dT * A[4], a12 = dT * A[5];
  float nsq = fmaf(a00, a00, a01 * a01);
  int ns, k;
  float sc = 1.0f;
  nsq = fmaf(a02, a02, nsq); nsq = fmaf(a10, a10, nsq); nsq = fmaf(a11, a11, nsq); nsq = fmaf(a12, a12, nsq);
  ns = n_squarings(sqrtf(nsq));
  for (k = 0; k < ns; ++k) sc *= 0.5f;
  {
    const float m00 = a00 * sc, m01 = a01 * sc, m02 = a02 * sc, m10 = a10 * sc, m11 = a11 * sc, m12 = a12 * sc;
    const float s00 = fmaf(m00, m00, m01 * m10), s01 = fmaf(m00, m01, m01 * m11);
    const float s02 = fmaf(m00, m02, m01 * m12), s10 = fmaf(m10, m00, m11 * m10);
    const float s11 = fmaf(m10, m01, m11 * m11), s12 = fmaf(m10, m02, m11 * m12);
    const float c12 = 1.0f / 12.0f;
    const float p00 = fmaf(c12, s00, fmaf(0.5f, m00, 1.0f)), p01 = fmaf(0.5f, m01, c12 * s01);
    const float p02 = fmaf(0.5f, m02, c12 * s02), p10 = fmaf(0.5f, m10, c12 * s10);
    const float p11 = fmaf(c12, s11, fmaf(0.5f, m11, 1.0f)), p12 = fmaf(0.5f, m12, c12 * s12);
    const float q00 = fmaf(c12, s00, fmaf(-0.5f, m00, 1.0f)), q01 = fmaf(-0.5f, m01, c12 * s01);
    const float q02 = fmaf(-0.5f, m02, c12 * s02), q10 = fmaf(-0.5f, m10, c12 * s10);
    const float q11 = fmaf(c12, s11, fmaf(-0.5f, m11, 1.0f)), q12 = fmaf(-0.5f, m12, c12 * s12);
    const float det = fmaf(q00, q11, -(q01 * q10));
    const float id = 1.0f / det;
    const float i00 = q11 * id, i01 = (-q01) * id, i10 = (-q10) * id, i11 = q00 * id;
    const float i02 = -fmaf(i00, q02, i01 * q12), i12 = -fmaf(i10, q02, i11 * q12);
    float r00 = fmaf(i00, p00, i01 * p10), r01 = fmaf(i00, p01, i01 * p11);
    float r02 = fmaf(i00, p02, i01 * p12) + i02;
    float r10 = fmaf(i10, p00, i11 * p10), r11 = fmaf(i10, p01, i11 * p11);
    float r12 = fmaf(i10, p02, i11 * p12) + i12;
    for (k = 0; k < ns; ++k) {
      const float n00 = fmaf(r00, r00, r01 * r10), n01 = fmaf(r00, r01, r01 * r11);
      const float n02 = fmaf(r00, r02, r01 * r12) + r02;
      const float n10 = fmaf(r10, r00, r11 * r10), n11 = fmaf(r10, r01, r11 * r11);
      const float n12 = fmaf(r10, r02, r11 * r12) + r12;
      r00 = n00; r01 = n01; r02 = n02; r10 = n10; r11 = n11; r12 = n12;
    }
    o[0] = r00; o[1] = r01; o[2] = r02; o[3] = r10; o[4] = r11; o[5] = r12;
  }
}

static void expm4(float dT, const float* A, float* o) {
  float a[12], m[3][4], s[3][3], t[3], p[3][3], q[3][3], pt[3], qt[3], qi[3][3], qit[3], Rm[3][4];
  float nsq, sc = 1.0f, c00, c10, c20, det, id;
  const float c12 = 1.0f / 12.0f;
  int k, r, c, ns;
  for (k = 0; k < 12; ++k) a[k] = dT * A[k];
  nsq = fmaf(a[0], a[0], a[1] * a[1]);
  for (k = 2; k < 12; ++k) nsq = fmaf(a[k], a[k], nsq);
  ns = n_squarings(sqrtf(nsq));
  for (k = 0; k < ns; ++k) sc *= 0.5f;
  for (r = 0; r < 3; ++r) for (c = 0; c < 4; ++c) m[r][c] = a[4 * r + c] * sc;
  for (r = 0; r < 3; ++r) {
    for (c = 0; c < 3; ++c) s[r][c] = dot3(m[r][0], m[0][c], m[r][1], m[1][c], m[r][2], m[2][c]);
    t[r] = dot3(m[r][0], m[0][3], m[r][1], m[1][3], m[r][2], m[2][3]);
  }
  for (r = 0; r < 3; ++r) {
    for (c = 0; c < 3; ++c) {
      if (r == c) {
        p[r][c] = fmaf(c12, s[r][c], fmaf(0.5f, m[r][c], 1.0f));
        q[r][c] = fmaf(c12, s[r][c], fmaf(-0.5f, m[r][c], 1.0f));
      } else {
        p[r][c] = fmaf(0.5f, m[r][c], c12 * s[r][c]);
        q[r][c] = fmaf(-0.5f, m[r][c], c12 * s[r][c]);
      }
    }
    pt[r] = fmaf(0.5f, m[r][3], c12 * t[r]);
    qt[r] = fmaf(-0.5f, m[r][3], c12 * t[r]);
  }
  c00 = cross2(q[1][1], q[2][2], q[1][2], q[2][1]);
  c10 = cross2(q[1][0], q[2][2], q[1][2], q[2][0]);
  c20 = cross2(q[1][0], q[2][1], q[1][1], q[2][0]);
  det = fmaf(q[0][2], c20, fmaf(q[0][0], c00, -(q[0][1] * c10)));
  id = 1.0f / det;
  qi[0][0] = c00 * id;
  qi[0][1] = cross2(q[0][2], q[2][1], q[0][1], q[2][2]) * id;
  qi[0][2] = cross2(q[0][1], q[1][2], q[0][2], q[1][1]) * id;
  qi[1][0] = cross2(q[1][2], q[2][0], q[1][0], q[2][2]) * id;
  qi[1][1] = cross2(q[0][0], q[2][2], q[0][2], q[2][0]) * id;
  qi[1][2] = cross2(q[0][2], q[1][0], q[0][0], q[1][2]) * id;
  qi[2][0] = c20 * id;
  qi[2][1] = cross2(q[0][1], q[2][0], q[0][0], q[2][1]) * id;
  qi[2][2] = cross2(q[0][0], q[1][1], q[0][1], q[1][0]) * id;
  for (r = 0; r < 3; ++r) qit[r] = -dot3(qi[r][0], qt[0], qi[r][1], qt[1], qi[r][2], qt[2]);
  for (r = 0; r < 3; ++r) {
    for (c = 0; c < 3; ++c) Rm[r][c] = dot3(qi[r][0], p[0][c], qi[r][1], p[1][c], qi[r][2], p[2][c]);
    Rm[r][3] = dot3(qi[r][0], pt[0], qi[r][1], pt[1], qi[r][2], pt[2]) + qit[r];
  }
  for (k = 0; k < ns; ++k) {
    float N[3][4];
    for (r = 0; r < 3; ++r) {
      for (c = 0; c < 3; ++c) N[r][c] = dot3(Rm[r][0], Rm[0][c], Rm[r][1], Rm[1][c], Rm[r][2], Rm[2][c]);
      N[r][3] = dot3(Rm[r][0], Rm[0][3], Rm[r][1], Rm[1][3], Rm[r][2], Rm[2][3]) + Rm[r][3];
    }
    memcpy(Rm, N, sizeof(N));
  }
  for (r = 0; r < 3; ++r) for (c = 0; c < 4; ++c) o[4 * r + c] = Rm[r][c];
}

void orc_expm_f32(int ndim, int64_t n, float dT, const float* As, float* Trels) {
  const int P = ndim * (ndim + 1);
  int64_t i;
  for (i = 0; i < n; ++i) {
    if (ndim == 1) expm2(dT, As + P * i, Trels + P * i);
    else if (ndim == 2) expm3(dT, As + P * i, Trels + P * i);
    else expm4(dT, As + P * i, Trels + P * i);
  }
}

/* cell index of single points (tests of the lookup) */
void orc_cells_f32(int ndim, int64_t n, const float* pts, int nx, int ny, int nz, int32_t* out) {
  int64_t i;
  for (i = 0; i < n; ++i) {
    float p[3] = {0, 0, 0};
    int k;
    for (k = 0; k < ndim; ++k) p[k] = pts[k * n + i];
    out[i] = cell_f32(ndim, p, nx, ny, nz);
  }
}
