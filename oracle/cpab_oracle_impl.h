/*
 * TEST INFRASTRUCTURE ONLY -- the parity checker and CPU baseline, never the
 * product.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.
 *
 * Precision-generic body of the CPU oracle, included twice by cpab_oracle.c:
 * R = float (SUF _f32, the reference's arithmetic, op for op) and R = double
 * (SUF _f64, used only to pin the mathematics: finite differences of the
 * midpoint scheme against the adjoint).
 *
 * Each routine restates the reference kernel it cites, in the same operation
 * order; explicit __fmaf_rn calls of the reference are FMA() here, and the
 * reference's plain `a*b + c*d` expressions (contracted by nvcc) are written
 * with the left product fused, FMA(a, b, c*d) -- the same choice the HIP
 * kernels make.  Compile with -ffp-contract=off.
 */

#define CAT_(a, b) a##b
#define CAT(a, b) CAT_(a, b)
#define FN(name) CAT(name, SUF)

/* ---- cell lookup: cpab_ops_1d.cu:52-59, cpab_ops_2d.cu:71-128, cpab_ops_3d.cu:67-131 ---- */

static int FN(cell1d)(R px, int nx) {
  R xc = FMIN(FMAX(px, (R)0), (R)1 - (R)1e-7f);
  int c = (int)FLOOR(xc * (R)nx);
  return c < nx - 1 ? c : nx - 1;
}

static int FN(cell2d)(R px, R py, int nx, int ny) {
  const R fx = (R)nx, fy = (R)ny;
  R xc = FMIN(FMAX(px, (R)0), (R)1 - (R)1e-7f);
  R yc = FMIN(FMAX(py, (R)0), (R)1 - (R)1e-7f);
  int cx = (int)FLOOR(xc * fx), cy = (int)FLOOR(yc * fy);
  if (cx > nx - 1) cx = nx - 1;
  if (cy > ny - 1) cy = ny - 1;
  R lx = FMA(xc, fx, -(R)cx), ly = FMA(yc, fy, -(R)cy);
  int base = (cx + cy * nx) * 4;
  if (px <= 0) {
    if (py <= 0 && py * fy < px * fx) return base;
    if (py >= 1 && FMA(py, fy, -fy) > (-px) * fx) return base + 2;
    return base + 3;
  }
  if (px >= 1) {
    if (py <= 0 && (-py) * fy > FMA(px, fx, -fx)) return base;
    if (py >= 1 && FMA(py, fy, -fy) > FMA(px, fx, -fx)) return base + 2;
    return base + 1;
  }
  if (py <= 0) return base;
  if (py >= 1) return base + 2;
  {
    int bit1 = lx < ly, bit0 = ((R)1 - lx) < ly;
    int tri = (bit1 << 1) | bit0;
    tri ^= (tri >> 1) & 1;
    return base + tri;
  }
}

static int FN(cell3d)(R px, R py, R pz, int nx, int ny, int nz) {
  const R fx = (R)nx, fy = (R)ny, fz = (R)nz;
  R ox = (FABS(px - (R)0.5) - (R)0.5) * fx;
  R oy = (FABS(py - (R)0.5) - (R)0.5) * fy;
  R oz = (FABS(pz - (R)0.5) - (R)0.5) * fz;
  if (ox > 0 && oy > 0 && oz > 0) {
    if (ox <= oy && ox <= oz) px = (px < (R)0.5) ? (R)0.5 / fx : (R)1 - (R)0.5 / fx;
    else if (oy <= oz) py = (py < (R)0.5) ? (R)0.5 / fy : (R)1 - (R)0.5 / fy;
    else pz = (pz < (R)0.5) ? (R)0.5 / fz : (R)1 - (R)0.5 / fz;
  }
  R xc = FMIN(FMAX(px, (R)0), (R)1), yc = FMIN(FMAX(py, (R)0), (R)1), zc = FMIN(FMAX(pz, (R)0), (R)1);
  int i = (int)FLOOR(xc * fx), j = (int)FLOOR(yc * fy), k = (int)FLOOR(zc * fz);
  if (i > nx - 1) i = nx - 1;
  if (j > ny - 1) j = ny - 1;
  if (k > nz - 1) k = nz - 1;
  R x = FMA(xc, fx, -(R)i), y = FMA(yc, fy, -(R)j), z = FMA(zc, fz, -(R)k);
  int c = 5 * (i + j * nx + k * nx * ny);
  if ((i ^ j ^ k) & 1) { R t = x; x = y; y = (R)1 - t; }
  if (((-x) - y) + z >= 0) return c + 1;
  if (((x + y) + z) - (R)2 >= 0) return c + 2;
  if (((-x) + y) - z >= 0) return c + 3;
  if ((x - y) - z >= 0) return c + 4;
  return c;
}

static int FN(cell)(int ndim, const R* p, int nx, int ny, int nz) {
  if (ndim == 1) return FN(cell1d)(p[0], nx);
  if (ndim == 2) return FN(cell2d)(p[0], p[1], nx, ny);
  return FN(cell3d)(p[0], p[1], p[2], nx, ny, nz);
}

/* v = M [p; 1], nested as fma(m0, x, fma(m1, y, fma(m2, z, m3))) (cpab_ops_2d.cu:145-146). */
static void FN(apply)(int ndim, const R* M, const R* p, R* v) {
  int k;
  for (k = 0; k < ndim; ++k) {
    const R* m = M + k * (ndim + 1);
    if (ndim == 1) v[k] = FMA(m[0], p[0], m[1]);
    else if (ndim == 2) v[k] = FMA(m[0], p[0], FMA(m[1], p[1], m[2]));
    else v[k] = FMA(m[0], p[0], FMA(m[1], p[1], FMA(m[2], p[2], m[3])));
  }
}

/* One midpoint step in cell A (cpab_ops_2d.cu:269-292). */
static void FN(midpoint)(int ndim, const R* A, R* p, R h, R hh) {
  R v[3] = {0, 0, 0}, pm[3] = {0, 0, 0}, vm[3] = {0, 0, 0};
  int k;
  FN(apply)(ndim, A, p, v);
  for (k = 0; k < ndim; ++k) pm[k] = FMA(hh, v[k], p[k]);
  FN(apply)(ndim, A, pm, vm);
  for (k = 0; k < ndim; ++k) p[k] = FMA(h, vm[k], p[k]);
}

/* Replay step incl. the adaptive Heun correction (cpab_ops_2d.cu:294-332). */
static void FN(replay_step)(int ndim, const R* As, int c, R* p, R h, R hh, int adaptive,
                            int nx, int ny, int nz) {
  const int P = ndim * (ndim + 1);
  R q[3], v0[3], v1[3];
  int k, ce;
  if (!adaptive) { FN(midpoint)(ndim, As + P * c, p, h, hh); return; }
  for (k = 0; k < ndim; ++k) q[k] = p[k];
  FN(midpoint)(ndim, As + P * c, q, h, hh);
  ce = FN(cell)(ndim, q, nx, ny, nz);
  if (ce == c) { for (k = 0; k < ndim; ++k) p[k] = q[k]; return; }
  FN(apply)(ndim, As + P * c, p, v0);
  FN(apply)(ndim, As + P * ce, q, v1);
  for (k = 0; k < ndim; ++k) p[k] = FMA(hh, v0[k] + v1[k], p[k]);
}

/* A^T lam with the reference's sum order (cpab_ops_2d.cu:352-353, 3d.cu:355-357). */
static void FN(at_lam)(int ndim, const R* A, const R* l, R* out) {
  int q;
  for (q = 0; q < ndim; ++q) {
    if (ndim == 1) out[q] = A[0] * l[0];
    else if (ndim == 2) out[q] = FMA(A[q], l[0], A[3 + q] * l[1]);
    else out[q] = FMA(A[8 + q], l[2], FMA(A[q], l[0], A[4 + q] * l[1]));
  }
}

/* Adjoint step + moments (cpab_ops_2d.cu:334-382, 1d.cu:301-329, 3d.cu:331-403). */
static void FN(adjoint)(int ndim, const R* A, const R* p, R h, R hh, R hhh, R* m, R* l) {
  const int N1 = ndim + 1;
  R v[3], pm[3], at[3], w[3], u[3], lm[3];
  int k, q;
  FN(apply)(ndim, A, p, v);
  for (k = 0; k < ndim; ++k) pm[k] = FMA(hh, v[k], p[k]);
  FN(at_lam)(ndim, A, l, at);
  for (k = 0; k < ndim; ++k) { w[k] = h * l[k]; u[k] = hhh * at[k]; }
  for (k = 0; k < ndim; ++k) {
    for (q = 0; q < ndim; ++q) m[k * N1 + q] = FMA(w[k], pm[q], m[k * N1 + q]);
    m[k * N1 + ndim] = m[k * N1 + ndim] + w[k];
  }
  for (k = 0; k < ndim; ++k) {
    for (q = 0; q < ndim; ++q) m[k * N1 + q] = FMA(u[k], p[q], m[k * N1 + q]);
    m[k * N1 + ndim] = m[k * N1 + ndim] + u[k];
  }
  for (k = 0; k < ndim; ++k) lm[k] = FMA(hh, at[k], l[k]);
  FN(at_lam)(ndim, A, lm, at);
  for (k = 0; k < ndim; ++k) l[k] = FMA(h, at[k], l[k]);
}

/* ---- forward with Trels (cpab_ops_2d.cu:164-230, cpab_ops_3d.cu:169-241) ----
 * cells (nullable): [n_theta, nP, T] cell index used at each step.
 * path (nullable): [n_theta, T, ndim, nP] the position each step looks up. */
void FN(orc_forward_trels)(int ndim, int64_t nP, int64_t n_theta, int batched, int T, int nx,
                           int ny, int nz, int adaptive, const R* points, const R* Trels,
                           const R* As, R* out, int32_t* cells, R* path) {
  const int P = ndim * (ndim + 1);
  const int nC = ndim == 2 ? 4 * nx * ny : 5 * nx * ny * nz;
  const R h = (R)1 / (R)T, hh = (R)0.5 * h;
  int64_t b;
#pragma omp parallel for collapse(2) schedule(static)
  for (b = 0; b < n_theta; ++b) {
    for (int64_t i = 0; i < nP; ++i) {
      const R* pts = points + (batched ? b * ndim * nP : 0);
      const R* Tb = Trels + b * (int64_t)nC * P;
      const R* Ab = As + b * (int64_t)nC * P;
      R p[3], s[3], v0[3], v1[3];
      int k, t;
      for (k = 0; k < ndim; ++k) p[k] = pts[i + k * nP];
      for (t = 0; t < T; ++t) {
        int c = FN(cell)(ndim, p, nx, ny, nz);
        if (cells) cells[(b * nP + i) * T + t] = c;
        if (path)
          for (k = 0; k < ndim; ++k) path[((b * T + t) * ndim + k) * nP + i] = p[k];
        FN(apply)(ndim, Tb + P * c, p, s);
        if (adaptive) {
          int ce = FN(cell)(ndim, s, nx, ny, nz);
          if (ce != c) {
            FN(apply)(ndim, Ab + P * c, p, v0);
            FN(apply)(ndim, Ab + P * ce, s, v1);
            for (k = 0; k < ndim; ++k) s[k] = FMA(hh, v0[k] + v1[k], p[k]);
          }
        }
        for (k = 0; k < ndim; ++k) p[k] = s[k];
      }
      for (k = 0; k < ndim; ++k) out[(b * ndim + k) * nP + i] = p[k];
    }
  }
}

/* ---- midpoint trajectory endpoint: the map the backward differentiates ----
 * (phase 1 of cpab_ops_2d.cu:426-440).  cells (nullable): [n_theta, nP, T];
 * path (nullable): [n_theta, T, ndim, nP] the position each step looks up. */
void FN(orc_forward_midpoint)(int ndim, int64_t nP, int64_t n_theta, int batched, int T, int nx,
                              int ny, int nz, int adaptive, const R* points, const R* As, R* out,
                              int32_t* cells, R* path) {
  const int P = ndim * (ndim + 1);
  const int nC = ndim == 1 ? nx : ndim == 2 ? 4 * nx * ny : 5 * nx * ny * nz;
  const R h = (R)1 / (R)T, hh = h * (R)0.5;
  int64_t b;
#pragma omp parallel for collapse(2) schedule(static)
  for (b = 0; b < n_theta; ++b) {
    for (int64_t i = 0; i < nP; ++i) {
      const R* pts = points + (batched ? b * ndim * nP : 0);
      const R* Ab = As + b * (int64_t)nC * P;
      R p[3];
      int k, t;
      for (k = 0; k < ndim; ++k) p[k] = pts[i + k * nP];
      for (t = 0; t < T; ++t) {
        int c = FN(cell)(ndim, p, nx, ny, nz);
        if (cells) cells[(b * nP + i) * T + t] = c;
        if (path)
          for (k = 0; k < ndim; ++k) path[((b * T + t) * ndim + k) * nP + i] = p[k];
        FN(replay_step)(ndim, Ab, c, p, h, hh, adaptive, nx, ny, nz);
      }
      for (k = 0; k < ndim; ++k) out[(b * ndim + k) * nP + i] = p[k];
    }
  }
}

/* ---- fused backward (cpab_ops_2d.cu:384-513 and the 1D / 3D twins) ----
 * The reference replays from checkpoints; the replay is deterministic, so the
 * full stored trajectory used here gives the same positions bit for bit.
 * Per-run flushes of the fp32 local moment are accumulated in double (the
 * reference's global fp32 atomics have no fixed order).
 * moments: [n_theta, nC, P] double, zeroed here.  grad_points nullable. */
void FN(orc_backward)(int ndim, int64_t nP, int64_t n_theta, int batched, int T, int nx, int ny,
                      int nz, int adaptive, const R* points, const R* As, const R* grad_out,
                      double* moments, R* grad_points) {
  const int P = ndim * (ndim + 1);
  const int nC = ndim == 1 ? nx : ndim == 2 ? 4 * nx * ny : 5 * nx * ny * nz;
  const int64_t MR = (int64_t)nC * P;
  const R h = (R)1 / (R)T, hh = h * (R)0.5, hhh = hh * h;
  int64_t b;
  memset(moments, 0, sizeof(double) * n_theta * MR);
#pragma omp parallel
  {
    double* acc = (double*)calloc((size_t)(n_theta * MR), sizeof(double));
    R traj[(CPAB_ORC_MAX_STEPS + 1) * 3];
    int cells[CPAB_ORC_MAX_STEPS];
#pragma omp for collapse(2) schedule(static)
    for (b = 0; b < n_theta; ++b) {
      for (int64_t i = 0; i < nP; ++i) {
        const R* pts = points + (batched ? b * ndim * nP : 0);
        const R* Ab = As + b * MR;
        double* mb = acc + b * MR;
        R p[3], lam[3], m[12];
        int k, t, prev = -1;
        for (k = 0; k < ndim; ++k) p[k] = pts[i + k * nP];
        for (t = 0; t < T; ++t) {
          int c = FN(cell)(ndim, p, nx, ny, nz);
          cells[t] = c;
          for (k = 0; k < ndim; ++k) traj[t * 3 + k] = p[k];
          FN(replay_step)(ndim, Ab, c, p, h, hh, adaptive, nx, ny, nz);
        }
        for (k = 0; k < ndim; ++k) lam[k] = grad_out[(b * ndim + k) * nP + i];
        for (k = 0; k < P; ++k) m[k] = 0;
        for (t = T - 1; t >= 0; --t) {
          int c = cells[t];
          if (c != prev && prev >= 0) {
            for (k = 0; k < P; ++k) { mb[prev * P + k] += (double)m[k]; m[k] = 0; }
          }
          prev = c;
          FN(adjoint)(ndim, Ab + P * c, traj + t * 3, h, hh, hhh, m, lam);
        }
        if (prev >= 0)
          for (k = 0; k < P; ++k) mb[prev * P + k] += (double)m[k];
        if (grad_points)
          for (k = 0; k < ndim; ++k) grad_points[(b * ndim + k) * nP + i] = lam[k];
      }
    }
#pragma omp critical
    {
      int64_t j;
      for (j = 0; j < n_theta * MR; ++j) moments[j] += acc[j];
    }
    free(acc);
  }
}

/* ---- 1D closed form (cpab_ops_1d.cu:103-243) ---- */
static int FN(sgn)(R x) { return (x > 0) - (x < 0); }
static int FN(near0)(R x) { return FABS(x) < (R)1e-7f; }

static R FN(hit_time)(R x, R t, int c, R a, R b, int nx, R* xc, int* cc) {
  const int s = FN(sgn)(t);
  const R inf_t = (R)INFINITY * (R)s;
  const R v = FMA(a, x, b);
  R right, left, vc;
  if (FN(near0)(v)) return inf_t;
  *cc = c + FN(sgn)(v) * s;
  if (*cc < 0 || *cc >= nx) return inf_t;
  right = (R)(c + 1) / (R)nx + (R)1e-7f;
  left = (R)c / (R)nx - (R)1e-7f;
  *xc = (t > 0) ? ((v > 0) ? right : left) : ((v > 0) ? left : right);
  vc = FMA(a, *xc, b);
  if (FN(near0)(vc)) return inf_t;
  if (FN(sgn)(v) != FN(sgn)(vc)) return inf_t;
  if (*xc <= 0 || *xc >= 1) return inf_t;
  if (FN(near0)(a)) return (*xc - x) / b;
  return LOG(vc / v) / a;
}

static R FN(closed_form)(R x, R t, const R* A, int nx) {
  int c = FN(cell1d)(x, nx);
  const int contmax = (c > nx - 1 - c ? c : nx - 1 - c) + 1;
  const int s = FN(sgn)(t);
  int cont = 0;
  for (;;) {
    const R a = A[2 * c], b = A[2 * c + 1];
    R xc = x;
    int cc = c;
    const R thit = FN(hit_time)(x, t, c, a, b, nx, &xc, &cc);
    if ((R)s * thit > (R)s * t) {
      R boa;
      if (FN(near0)(a)) return FMA(t, b, x);
      boa = b / a;
      return FMA(EXP(t * a), x + boa, -boa);
    }
    x = xc;
    c = cc;
    t -= thit;
    if (++cont > contmax) break;
  }
  return x;
}

void FN(orc_forward_closed_1d)(int64_t nP, int64_t n_theta, int batched, int nx, const R* points,
                               const R* As, R* out) {
  int64_t b;
#pragma omp parallel for collapse(2) schedule(static)
  for (b = 0; b < n_theta; ++b)
    for (int64_t i = 0; i < nP; ++i)
      out[b * nP + i] = FN(closed_form)(points[(batched ? b * nP : 0) + i], (R)1,
                                        As + b * 2 * (int64_t)nx, nx);
}

/* ---- A = B theta, fp32 fma in CSR column order ---- */
void FN(orc_affine)(int64_t n_theta, int rows, int d, const R* theta, const int32_t* row_ptr,
                    const int32_t* col_idx, const R* vals, R* As) {
  int64_t b;
  for (b = 0; b < n_theta; ++b)
    for (int r = 0; r < rows; ++r) {
      R acc = 0;
      for (int k = row_ptr[r]; k < row_ptr[r + 1]; ++k) acc = FMA(vals[k], theta[b * d + col_idx[k]], acc);
      As[b * rows + r] = acc;
    }
}

/* ---- dtheta = B^T M, fma in CSC row order ---- */
void FN(orc_project)(int64_t n_theta, int D, int d, const R* M, const int32_t* col_ptr,
                     const int32_t* row_idx, const R* vals, R* grad) {
  int64_t b;
  for (b = 0; b < n_theta; ++b)
    for (int j = 0; j < d; ++j) {
      R acc = 0;
      for (int k = col_ptr[j]; k < col_ptr[j + 1]; ++k) acc = FMA(vals[k], M[b * D + row_idx[k]], acc);
      grad[b * d + j] = acc;
    }
}

/* ---- transform_data resampling (cpab/pytorch/interpolation.py:3-159) ----
 * Forward follows the reference's eager torch ops one by one:
 *   x = g*(W-1); x0 = clamp(floor(x)); x1 = clamp(floor(x)+1); xd = x - x0;
 *   lerp(a, b, t) = a*(1-t) + b*t, reduced along x, then y, then z.
 * data [B, C, *in]; grid [B, ndim, nP] with p = i0 + o0*(i1 + o1*i2);
 * out [B, C, *out] (last axis fastest). */
static void FN(axis)(R g, int64_t size, int64_t* a, int64_t* b, R* t) {
  const R x = g * (R)(size - 1);
  const R f = FLOOR(x);
  int64_t lo = (int64_t)f, hi = lo + 1;
  if (lo < 0) lo = 0;
  if (lo > size - 1) lo = size - 1;
  if (hi < 0) hi = 0;
  if (hi > size - 1) hi = size - 1;
  *a = lo;
  *b = hi;
  *t = x - (R)lo;
}

static R FN(lerp)(R a, R b, R t) { return a * ((R)1 - t) + b * t; }

static int64_t FN(out_index)(int ndim, const int64_t* os, int64_t p) {
  /* point p -> row-major output offset within one [*out] plane */
  if (ndim == 1) return p;
  if (ndim == 2) { int64_t i0 = p % os[0], i1 = p / os[0]; return i0 * os[1] + i1; }
  {
    int64_t i0 = p % os[0], r = p / os[0], i1 = r % os[1], i2 = r / os[1];
    return (i0 * os[1] + i1) * os[2] + i2;
  }
}

static int64_t FN(didx)(int ndim, const int64_t* is, int64_t bc, int64_t x, int64_t y, int64_t z) {
  if (ndim == 1) return bc * is[0] + x;
  if (ndim == 2) return (bc * is[0] + x) * is[1] + y;
  return ((bc * is[0] + x) * is[1] + y) * is[2] + z;
}

void FN(orc_interp_forward)(int ndim, int64_t B, int64_t C, const int64_t* is, const int64_t* os,
                            const R* data, const R* grid, R* out) {
  int64_t nP = 1, b;
  int k;
  for (k = 0; k < ndim; ++k) nP *= os[k];
#pragma omp parallel for collapse(2) schedule(static)
  for (b = 0; b < B; ++b)
    for (int64_t p = 0; p < nP; ++p) {
      int64_t lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
      R t[3] = {0, 0, 0};
      int kk;
      for (kk = 0; kk < ndim; ++kk) FN(axis)(grid[(b * ndim + kk) * nP + p], is[kk], &lo[kk], &hi[kk], &t[kk]);
      for (int64_t ch = 0; ch < C; ++ch) {
        const int64_t bc = b * C + ch;
        R v;
        if (ndim == 1) {
          v = FN(lerp)(data[FN(didx)(1, is, bc, lo[0], 0, 0)], data[FN(didx)(1, is, bc, hi[0], 0, 0)], t[0]);
        } else if (ndim == 2) {
          R c00 = data[FN(didx)(2, is, bc, lo[0], lo[1], 0)], c01 = data[FN(didx)(2, is, bc, lo[0], hi[1], 0)];
          R c10 = data[FN(didx)(2, is, bc, hi[0], lo[1], 0)], c11 = data[FN(didx)(2, is, bc, hi[0], hi[1], 0)];
          v = FN(lerp)(FN(lerp)(c00, c10, t[0]), FN(lerp)(c01, c11, t[0]), t[1]);
        } else {
          R c[2][2][2], c00, c01, c10, c11;
          int a1, a2, a3;
          for (a1 = 0; a1 < 2; ++a1) for (a2 = 0; a2 < 2; ++a2) for (a3 = 0; a3 < 2; ++a3)
            c[a1][a2][a3] = data[FN(didx)(3, is, bc, a1 ? hi[0] : lo[0], a2 ? hi[1] : lo[1], a3 ? hi[2] : lo[2])];
          c00 = FN(lerp)(c[0][0][0], c[1][0][0], t[0]);
          c01 = FN(lerp)(c[0][0][1], c[1][0][1], t[0]);
          c10 = FN(lerp)(c[0][1][0], c[1][1][0], t[0]);
          c11 = FN(lerp)(c[0][1][1], c[1][1][1], t[0]);
          v = FN(lerp)(FN(lerp)(c00, c10, t[1]), FN(lerp)(c01, c11, t[1]), t[2]);
        }
        out[bc * nP + FN(out_index)(ndim, os, p)] = v;
      }
    }
}

/* Backward: d out / d grid (analytic derivative of the lerps, times the
 * (size-1) chain factor) and the scatter of grad_out onto the corners.
 * grad_grid / grad_data nullable; grad_data is overwritten. */
void FN(orc_interp_backward)(int ndim, int64_t B, int64_t C, const int64_t* is, const int64_t* os,
                             const R* data, const R* grid, const R* gout, R* grad_grid,
                             R* grad_data) {
  int64_t nP = 1, nd = B * C, b;
  int k;
  for (k = 0; k < ndim; ++k) { nP *= os[k]; nd *= is[k]; }
  if (grad_data) memset(grad_data, 0, sizeof(R) * nd);
  for (b = 0; b < B; ++b)
    for (int64_t p = 0; p < nP; ++p) {
      int64_t lo[3] = {0, 0, 0}, hi[3] = {0, 0, 0};
      R t[3] = {0, 0, 0}, u[3], d[3] = {0, 0, 0};
      int kk;
      for (kk = 0; kk < ndim; ++kk) {
        FN(axis)(grid[(b * ndim + kk) * nP + p], is[kk], &lo[kk], &hi[kk], &t[kk]);
        u[kk] = (R)1 - t[kk];
      }
      for (int64_t ch = 0; ch < C; ++ch) {
        const int64_t bc = b * C + ch;
        const R g = gout[bc * nP + FN(out_index)(ndim, os, p)];
        if (ndim == 1) {
          int64_t i0 = FN(didx)(1, is, bc, lo[0], 0, 0), i1 = FN(didx)(1, is, bc, hi[0], 0, 0);
          d[0] += g * (data[i1] - data[i0]);
          if (grad_data) { grad_data[i0] += g * u[0]; grad_data[i1] += g * t[0]; }
        } else if (ndim == 2) {
          int64_t i00 = FN(didx)(2, is, bc, lo[0], lo[1], 0), i01 = FN(didx)(2, is, bc, lo[0], hi[1], 0);
          int64_t i10 = FN(didx)(2, is, bc, hi[0], lo[1], 0), i11 = FN(didx)(2, is, bc, hi[0], hi[1], 0);
          R c00 = data[i00], c01 = data[i01], c10 = data[i10], c11 = data[i11];
          R c0 = FN(lerp)(c00, c10, t[0]), c1 = FN(lerp)(c01, c11, t[0]);
          d[0] += g * u[1] * (c10 - c00) + g * t[1] * (c11 - c01);
          d[1] += g * (c1 - c0);
          if (grad_data) {
            R g0 = g * u[1], g1 = g * t[1];
            grad_data[i00] += g0 * u[0]; grad_data[i10] += g0 * t[0];
            grad_data[i01] += g1 * u[0]; grad_data[i11] += g1 * t[0];
          }
        } else {
          int64_t idx[2][2][2];
          R c[2][2][2], gx = 0, c00, c01, c10, c11;
          int a1, a2, a3;
          for (a1 = 0; a1 < 2; ++a1) for (a2 = 0; a2 < 2; ++a2) for (a3 = 0; a3 < 2; ++a3) {
            idx[a1][a2][a3] = FN(didx)(3, is, bc, a1 ? hi[0] : lo[0], a2 ? hi[1] : lo[1], a3 ? hi[2] : lo[2]);
            c[a1][a2][a3] = data[idx[a1][a2][a3]];
          }
          {
            R wyz[2][2];
            wyz[0][0] = u[1] * u[2]; wyz[0][1] = u[1] * t[2]; wyz[1][0] = t[1] * u[2]; wyz[1][1] = t[1] * t[2];
            for (a2 = 0; a2 < 2; ++a2) for (a3 = 0; a3 < 2; ++a3) gx += wyz[a2][a3] * (c[1][a2][a3] - c[0][a2][a3]);
          }
          c00 = FN(lerp)(c[0][0][0], c[1][0][0], t[0]);
          c01 = FN(lerp)(c[0][0][1], c[1][0][1], t[0]);
          c10 = FN(lerp)(c[0][1][0], c[1][1][0], t[0]);
          c11 = FN(lerp)(c[0][1][1], c[1][1][1], t[0]);
          d[0] += g * gx;
          d[1] += g * (u[2] * (c10 - c00) + t[2] * (c11 - c01));
          d[2] += g * (FN(lerp)(c01, c11, t[1]) - FN(lerp)(c00, c10, t[1]));
          if (grad_data)
            for (a1 = 0; a1 < 2; ++a1) for (a2 = 0; a2 < 2; ++a2) for (a3 = 0; a3 < 2; ++a3)
              grad_data[idx[a1][a2][a3]] += g * ((a1 ? t[0] : u[0]) * (a2 ? t[1] : u[1]) * (a3 ? t[2] : u[2]));
        }
      }
      if (grad_grid)
        for (kk = 0; kk < ndim; ++kk) grad_grid[(b * ndim + kk) * nP + p] = d[kk] * (R)(is[kk] - 1);
    }
}

#undef FN
