// Measurement probe, not part of the library: the bandwidth of direct-to-LDS loads (the
// GEMM main loop's load path). 256 workgroups of four waves (one per CU); every wave streams
// 1 KB chunks (buffer_load_dwordx4 ... lds) from a region into a private LDS ring, Q loads
// in flight between waits. Build and run on the MI355X box:
//   hipcc --offload-arch=gfx950 -O3 -o /tmp/l2_lds_bw bongard_amd/probes/l2_lds_bw.hip
//   /tmp/l2_lds_bw
// Modes:
//  0: all workgroups read the same region (size R)
//  1: workgroups of an XCD (blockIdx % 8) share a region of size R (8 regions)
//  2: each workgroup its own region of size R
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 make_srd(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xFFFFu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}
__device__ __forceinline__ void dma16(i32x4 srd, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" : : "s"(m0v), "v"(voff), "s"(srd), "s"(so) : "memory");
}
template <int Q>
__global__ __launch_bounds__(256) void bw(const uint8_t* src, uint64_t region, int mode, int iters, uint32_t* sink) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[4 * Q * 1024];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint64_t base = 0;
  if (mode == 1) base = (uint64_t)(blockIdx.x % 8) * region;
  if (mode == 2) base = (uint64_t)blockIdx.x * region;
  const i32x4 srd = make_srd(src + base, (uint32_t)region);
  const uint32_t lds = (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)ring) + wid * Q * 1024;
  const uint32_t nchunks = (uint32_t)(region / 1024);
  // wave w of workgroup b starts at a different chunk so the 4 waves cover distinct data
  uint32_t c = (wid * 97 + (mode == 0 ? blockIdx.x * 13 : 0)) % nchunks;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      dma16(srd, lds + q * 1024, lane * 16, c * 1024);
      c += 4; if (c >= nchunks) c -= nchunks;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if (threadIdx.x == 0 && iters < 0) sink[blockIdx.x] = ring[0];
}
int main(int argc, char** argv) {
  const uint64_t total = 512ull << 20;
  uint8_t* buf = nullptr;
  uint32_t* sink = nullptr;
  if (hipMalloc(&buf, total) != hipSuccess || hipMemset(buf, 1, total) != hipSuccess ||
      hipMalloc(&sink, 4096) != hipSuccess) {
    fprintf(stderr, "allocation failed\n");
    return 1;
  }
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  struct Cfg { int mode; uint64_t region; const char* what; };
  std::vector<Cfg> cfgs = {{0, 4ull << 20, "all WGs one 4 MB region"}, {0, 1ull << 20, "all WGs one 1 MB region"},
                           {1, 2ull << 20, "per-XCD 2 MB region"}, {2, 1ull << 20, "per-WG 1 MB region (256 MB total)"},
                           {2, 64ull << 10, "per-WG 64 KB region (16 MB total)"}};
  for (auto cf : cfgs) {
    for (int q : {4, 8, 16}) {
      const int iters = 2000 / q * 4;
      auto launch = [&]() {
        if (q == 4) hipLaunchKernelGGL(bw<4>, dim3(256), dim3(256), 0, 0, buf, cf.region, cf.mode, iters, sink);
        if (q == 8) hipLaunchKernelGGL(bw<8>, dim3(256), dim3(256), 0, 0, buf, cf.region, cf.mode, iters, sink);
        if (q == 16) hipLaunchKernelGGL(bw<16>, dim3(256), dim3(256), 0, 0, buf, cf.region, cf.mode, iters, sink);
      };
      launch(); hipDeviceSynchronize();
      hipEventRecord(e0); for (int r = 0; r < 5; ++r) launch(); hipEventRecord(e1); hipEventSynchronize(e1);
      float ms; hipEventElapsedTime(&ms, e0, e1);
      const double bytes = 5.0 * 256 * 4 * (double)iters * q * 1024;
      printf("%-36s Q=%2d: %6.2f TB/s (%.1f B/clk/CU at 2 GHz)\n", cf.what, q, bytes / (ms * 1e-3) / 1e12, bytes / (ms * 1e-3) / 256 / 2e9);
      fflush(stdout);
    }
  }
  return 0;
}
