/*
 * A plain C caller of libcpab_hip.so: the calls a non-Python host (a C, C++,
 * cgo or JNI binding) makes for one transform_grid forward + backward, its
 * own device memory and stream from the HIP runtime's C API, no torch.
 * 2D tessellation [4, 4] (64 cells) with the identity basis (theta is the
 * cells' affine parameters, A = theta), 2 thetas, 1000 shared points.
 *
 * cpab_c_caller_run(path) writes theta, points, grad_out and the library's
 * outputs (forward points, moments, point adjoints) as float32 to `path` and
 * returns 0, or 1 after a library or HIP error (message on stderr).  Built as
 * a shared library (tests/c_abi/Makefile) that tests/test_gpu_c_abi.py loads
 * into its own process, which already uses the GPU, and checks against the
 * oracle; with -DCPAB_C_CALLER_MAIN it is a program taking the path as its
 * argument.
 */
#include <stdio.h>
#include <stdlib.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "cpab_hip.h"

enum { NDIM = 2, NCX = 4, NCY = 4, NC = 4 * NCX * NCY, PPC = 6, D = NC * PPC, NTHETA = 2,
       NP = 1000, T = 50 };

static int hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return 1;
  fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return 0;
}

static int cpab_ok(int rc, const char* what) {
  if (rc == CPAB_OK) return 1;
  fprintf(stderr, "%s failed (%d): %s\n", what, rc, cpab_last_error_string());
  return 0;
}

/* xorshift32 in [0, 1) */
static float uniform(uint32_t* s) {
  *s ^= *s << 13;
  *s ^= *s >> 17;
  *s ^= *s << 5;
  return (float)(*s >> 8) * (1.0f / 16777216.0f);
}

static int to_device(void** dst, const void* src, size_t bytes) {
  return hip_ok(hipMalloc(dst, bytes), "hipMalloc") &&
         hip_ok(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

static int write_back(FILE* f, const void* dev, size_t n) {
  float* h = (float*)malloc(n * sizeof(float));
  int ok = h && hip_ok(hipMemcpy(h, dev, n * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy D2H") &&
           fwrite(h, sizeof(float), n, f) == n;
  free(h);
  return ok;
}

int cpab_c_caller_run(const char* path) {
  static float theta[NTHETA * D], points[NDIM * NP], grad_out[NTHETA * NDIM * NP], vals[D];
  static int32_t row_ptr[D + 1], col_idx[D];
  uint32_t s = 12345u;
  for (int i = 0; i < NTHETA * D; ++i) theta[i] = 0.6f * (uniform(&s) - 0.5f);
  for (int i = 0; i < NDIM * NP; ++i) points[i] = uniform(&s);
  for (int i = 0; i < NTHETA * NDIM * NP; ++i) grad_out[i] = uniform(&s) - 0.5f;
  for (int r = 0; r < D; ++r) {  /* B = I as CSR */
    row_ptr[r] = r;
    col_idx[r] = r;
    vals[r] = 1.0f;
  }
  row_ptr[D] = D;
  if (cpab_abi_version() < 300) {
    fprintf(stderr, "unexpected ABI version %d\n", cpab_abi_version());
    return 1;
  }

  void *d_theta, *d_points, *d_gout, *d_rp, *d_ci, *d_vals, *d_As, *d_Tr, *d_out, *d_mom, *d_gp,
      *d_ws;
  const size_t table = (size_t)NTHETA * NC * NDIM * (NDIM + 1) * sizeof(float);
  if (!to_device(&d_theta, theta, sizeof theta) || !to_device(&d_points, points, sizeof points) ||
      !to_device(&d_gout, grad_out, sizeof grad_out) || !to_device(&d_rp, row_ptr, sizeof row_ptr) ||
      !to_device(&d_ci, col_idx, sizeof col_idx) || !to_device(&d_vals, vals, sizeof vals) ||
      !hip_ok(hipMalloc(&d_As, table), "hipMalloc") || !hip_ok(hipMalloc(&d_Tr, table), "hipMalloc") ||
      !hip_ok(hipMalloc(&d_out, sizeof grad_out), "hipMalloc") ||
      !hip_ok(hipMalloc(&d_mom, (size_t)NTHETA * NC * PPC * sizeof(float)), "hipMalloc") ||
      !hip_ok(hipMalloc(&d_gp, sizeof grad_out), "hipMalloc"))
    return 1;
  hipStream_t stream;
  if (!hip_ok(hipStreamCreate(&stream), "hipStreamCreate")) return 1;

  /* forward: A = B theta and the per-step maps, then the integrator */
  if (!cpab_ok(cpab_affine_expm(NDIM, NTHETA, NC, D, (const float*)d_theta, (const int32_t*)d_rp,
                                (const int32_t*)d_ci, (const float*)d_vals, 1.0f / T,
                                (float*)d_As, (float*)d_Tr, stream),
               "cpab_affine_expm") ||
      !cpab_ok(cpab_forward(NDIM, NP, NTHETA, 0, T, NCX, NCY, 1, 0, (const float*)d_points,
                            (const float*)d_Tr, (const float*)d_As, (float*)d_out, stream),
               "cpab_forward"))
    return 1;
  /* backward: moments and point adjoints with a caller-owned workspace */
  const int64_t ws = cpab_backward_workspace_size(NDIM, NP, NTHETA, NC);
  if (ws <= 0) {
    fprintf(stderr, "cpab_backward_workspace_size: %s\n", cpab_last_error_string());
    return 1;
  }
  if (!hip_ok(hipMalloc(&d_ws, (size_t)ws), "hipMalloc") ||
      !cpab_ok(cpab_backward(NDIM, NP, NTHETA, 0, T, NCX, NCY, 1, 0, (const float*)d_points,
                             (const float*)d_As, (const float*)d_gout, (float*)d_mom,
                             (float*)d_gp, d_ws, ws, stream),
               "cpab_backward") ||
      !hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize"))
    return 1;

  FILE* f = fopen(path, "wb");
  if (!f) {
    perror(path);
    return 1;
  }
  const int ok = fwrite(theta, sizeof(float), NTHETA * D, f) == NTHETA * D &&
                 fwrite(points, sizeof(float), NDIM * NP, f) == NDIM * NP &&
                 fwrite(grad_out, sizeof(float), NTHETA * NDIM * NP, f) == NTHETA * NDIM * NP &&
                 write_back(f, d_out, NTHETA * NDIM * NP) && write_back(f, d_mom, NTHETA * NC * PPC) &&
                 write_back(f, d_gp, NTHETA * NDIM * NP);
  fclose(f);
  hipFree(d_theta); hipFree(d_points); hipFree(d_gout); hipFree(d_rp); hipFree(d_ci);
  hipFree(d_vals); hipFree(d_As); hipFree(d_Tr); hipFree(d_out); hipFree(d_mom); hipFree(d_gp);
  hipFree(d_ws);
  hipStreamDestroy(stream);
  if (!ok) {
    fprintf(stderr, "writing %s failed\n", path);
    return 1;
  }
  return 0;
}

#ifdef CPAB_C_CALLER_MAIN
int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: %s OUTPUT\n", argv[0]);
    return 2;
  }
  return cpab_c_caller_run(argv[1]);
}
#endif
