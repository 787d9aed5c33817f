// Measures the fp32 VALU ceiling that the integrator kernels run against:
// 8 or 16 independent non-packed FMA chains per lane (v_fma_f32 / v_fmac_f32,
// built with packed fp32 ops disabled like the library), 8 workgroups of 256
// lanes per CU.  Prints achieved TFLOP/s and cycles per wave64 instruction
// per SIMD at the reported peak clock.  Each lane writes one float.
//   make -C fg-cpab_amd/csrc probe && fg-cpab_amd/cpab/lib/probe_valu_rate
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                 \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

template <int CH>
__global__ __launch_bounds__(256) void fma_chains(float* out, int iters, float a, float b) {
  float x[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) x[c] = threadIdx.x * 1e-3f + c;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < CH; ++c) x[c] = fmaf(x[c], a, b);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) s += x[c];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

template <int CH>
static void run(const hipDeviceProp_t& p, float* out, int blocks, int iters) {
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (int rep = 0; rep < 3; ++rep) {
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL(fma_chains<CH>, dim3(blocks), dim3(256), 0, 0, out, iters, 0.999f, 1e-4f);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double lanes = (double)blocks * 256;
    const double wave_instr = lanes / 64 * iters * CH;
    const double flops = lanes * iters * CH * 2;
    const double simds = 4.0 * p.multiProcessorCount;
    printf("fma chains=%d run %d: %.3f ms  %.1f TFLOP/s  %.2f cycles per wave64 FMA per SIMD at %d MHz\n",
           CH, rep, ms, flops / ms / 1e9, ms * 1e-3 * p.clockRate * 1e3 * simds / wave_instr,
           p.clockRate / 1000);
  }
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  hipDeviceProp_t p;
  CHECK(hipGetDeviceProperties(&p, 0));
  printf("device %s, %d CUs, peak clock %d MHz\n", p.gcnArchName, p.multiProcessorCount,
         p.clockRate / 1000);
  const int blocks = p.multiProcessorCount * 8, iters = 4096;
  float* out = nullptr;
  CHECK(hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)));
  run<8>(p, out, blocks, iters);
  run<16>(p, out, blocks, iters);
  float h = 0.f;
  CHECK(hipMemcpy(&h, out, sizeof(float), hipMemcpyDeviceToHost));
  printf("checksum %g\n", h);
  CHECK(hipFree(out));
  return 0;
}
