// mfma_clock.hip -- sustained v_mfma_f32_32x32x16_f16 rate and shader clock on a
// full chip: 256 workgroups x 4 waves (one wave per SIMD), 8 independent
// accumulators per wave, operands all-ones or random fp16.  Measurement helper for
// the GEMM's roofline (not part of the library).  Build: make -C .. mfma_clock
#include <hip/hip_runtime.h>
#include <stdio.h>
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));
template <int MODE>
__global__ __launch_bounds__(256) void p32(const h8* src, float* out, int iters, unsigned long long* clk) {
  h8 a[2], b[8];
  const int t = blockIdx.x * 256 + threadIdx.x;
  for (int i = 0; i < 2; ++i) a[i] = MODE ? src[(t * 10 + i) % 65536] : (h8){1, 1, 1, 1, 1, 1, 1, 1};
  for (int i = 0; i < 8; ++i) b[i] = MODE ? src[(t * 10 + 2 + i) % 65536] : (h8){1, 1, 1, 1, 1, 1, 1, 1};
  f16v acc[8];
  for (int i = 0; i < 8; ++i) for (int e = 0; e < 16; ++e) acc[i][e] = 0;
  unsigned long long c0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          acc[rb * 4 + cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[rb], b[ks * 4 + cb], acc[rb * 4 + cb], 0, 0, 0);
  }
  unsigned long long c1 = __builtin_readcyclecounter(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0; for (int i = 0; i < 8; ++i) s += acc[i][0] + acc[i][15];
  out[t] = s;
  if (threadIdx.x == 0) { clk[blockIdx.x * 2] = c1 - c0; clk[blockIdx.x * 2 + 1] = r1 - r0; }
}
__global__ void fillr(h8* p, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x; if (i >= n) return;
  h8 v; for (int j = 0; j < 8; ++j) { unsigned z = (i * 8 + j) * 2654435761u; z ^= z >> 13; v[j] = (_Float16)(((int)(z & 2047) - 1024) / 256.0f); }
  p[i] = v;
}
int main() {
  float* out; hipMalloc(&out, 1 << 24);
  h8* src; hipMalloc(&src, 65536 * 16); fillr<<<256, 256>>>(src, 65536);
  unsigned long long* clk; hipMalloc(&clk, 256 * 16);
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  const int iters = 2000;
  auto run = [&](auto kern, const char* name) {
    kern<<<256, 256>>>(src, out, iters, clk); hipDeviceSynchronize();
    hipEventRecord(e0); kern<<<256, 256>>>(src, out, iters, clk); hipEventRecord(e1); hipEventSynchronize(e1);
    float ms; hipEventElapsedTime(&ms, e0, e1);
    double n = (double)iters * 16;  // MFMAs per wave
    unsigned long long h[512]; hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost);
    double ghz = 0; for (int b = 0; b < 256; ++b) ghz += h[2 * b] / (h[2 * b + 1] * 10.0); ghz /= 256;
    printf("%-20s %.1f TFLOPS  %.2f ns/MFMA  clk %.2f GHz  %.1f cycles/MFMA\n", name, 2.0 * 32 * 32 * 16 * n * 1024 / (ms * 1e-3) / 1e12,
           ms * 1e6 / n, ghz, ms * 1e6 / n * ghz);
  };
  run(p32<0>, "32x32x16 const");
  run(p32<1>, "32x32x16 random");
  run(p32<0>, "32x32x16 const");
  run(p32<1>, "32x32x16 random");
  hipError_t st = hipDeviceSynchronize();
  printf("status %s\n", hipGetErrorString(st));
  return st == hipSuccess ? 0 : 3;
}
