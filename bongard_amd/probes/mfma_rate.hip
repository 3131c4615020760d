// Measurement probe, not part of the library: MFMA-only throughput and shader clock.
// 256 workgroups x 4 waves (one wave per SIMD), each wave issuing independent fp8 MFMAs on
// register operands (random bytes), either 16 x v_mfma_f32_32x32x64_f8f6f4 or
// 32 x v_mfma_f32_16x16x128_f8f6f4 per iteration (same FLOPs), the two forms alternating.
// Reports TFLOP/s and the mean shader clock (s_memtime over the 100 MHz s_memrealtime).
// Build and run on the MI355X box:
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//     -o /tmp/mfma_rate bongard_amd/probes/mfma_rate.hip && /tmp/mfma_rate
#include <hip/hip_runtime.h>
#include <cstdio>
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
template <int MODE>
__global__ __launch_bounds__(256) void k(const int* seed, int iters, float* out, unsigned long long* clk) {
  const int lane = threadIdx.x & 63;
  v8i a[2], b[2];
  for (int i = 0; i < 8; ++i) {
    a[0][i] = seed[(lane * 8 + i) & 1023]; a[1][i] = seed[(lane * 8 + i + 512) & 1023];
    b[0][i] = seed[(lane * 8 + i + 256) & 1023]; b[1][i] = seed[(lane * 8 + i + 768) & 1023];
  }
  const unsigned long long t0 = clock64(), r0 = wall_clock64();
  float s = 0.f;
  if constexpr (MODE == 0) {
    v16f c[16];
    for (int j = 0; j < 16; ++j) for (int e = 0; e < 16; ++e) c[j][e] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        c[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[j & 1], b[(j >> 1) & 1], c[j], 0, 0, 0, 0, 0, 0);
    }
    for (int j = 0; j < 16; ++j) for (int e = 0; e < 16; ++e) s += c[j][e];
  } else {
    v4f c[32];
    for (int j = 0; j < 32; ++j) for (int e = 0; e < 4; ++e) c[j][e] = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 32; ++j)
        c[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[j & 1], b[(j >> 1) & 1], c[j], 0, 0, 0, 0, 0, 0);
    }
    for (int j = 0; j < 32; ++j) for (int e = 0; e < 4; ++e) s += c[j][e];
  }
  const unsigned long long t1 = clock64(), r1 = wall_clock64();
  out[blockIdx.x * 256 + threadIdx.x] = s;
  if (threadIdx.x == 0) { clk[2 * blockIdx.x] = t1 - t0; clk[2 * blockIdx.x + 1] = r1 - r0; }
}
int main() {
  int* seed; float* out; unsigned long long* clk;
  hipMalloc(&seed, 4096); hipMalloc(&out, 256 * 256 * 4); hipMalloc(&clk, 256 * 16);
  int h[1024]; unsigned x = 12345u;
  for (int i = 0; i < 1024; ++i) { x = x * 1664525u + 1013904223u; h[i] = (int)(x & 0x7B7B7B7Bu); }
  hipMemcpy(seed, h, 4096, hipMemcpyHostToDevice);
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  for (int r8 = 0; r8 < 10; ++r8) {
    const int mode = r8 & 1, rep = r8 >> 1;
    const int iters = 20000;
    {
      hipEventRecord(e0);
      if (mode == 0) hipLaunchKernelGGL(k<0>, dim3(256), dim3(256), 0, 0, seed, iters, out, clk);
      else hipLaunchKernelGGL(k<1>, dim3(256), dim3(256), 0, 0, seed, iters, out, clk);
      hipEventRecord(e1); hipEventSynchronize(e1);
      float ms; hipEventElapsedTime(&ms, e0, e1);
      unsigned long long hc[512]; hipMemcpy(hc, clk, sizeof(hc), hipMemcpyDeviceToHost);
      double ghz = 0; for (int b = 0; b < 256; ++b) ghz += (double)hc[2 * b] / (double)hc[2 * b + 1] * 0.1;
      ghz /= 256;
      const double flop = 256.0 * 4 * iters * 16 * 131072.0;
      printf("%s rep %d: %.3f ms  %.1f TFLOP/s  clock %.3f GHz\n", mode ? "16x16x128" : "32x32x64 ", rep, ms, flop / (ms * 1e-3) / 1e12, ghz);
      fflush(stdout);
    }
  }
  return 0;
}
