// Practical HBM read ceiling of the GPU this runs on: a streaming-read kernel
// (16-byte loads, 4 or 8 in flight per thread, grid-stride, one word written
// per workgroup) over buffers of the sizes the decode path streams (k_front
// reads about 45 MB per launch, k_bounds about 151 MB), each size rotated over
// 8 copies so that no launch finds its data in L2 or the Infinity Cache.
// Reported beside the published 8 TB/s peak the rooflines are priced
// against: it shows what a kernel with nothing but coalesced reads reaches at
// each size, launch ramp included.
//
// Build and run (no arguments):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       strict-topk-overlap_amd/stk_harness/hbm_probe.hip -o /tmp/hbm_probe && /tmp/hbm_probe
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                 \
      return 1;                                                               \
    }                                                                         \
  } while (0)

template <int UNR>
__global__ __launch_bounds__(256) void k_read(const uint4* __restrict__ p, size_t n16,
                                              uint32_t* out) {
  uint32_t acc = 0;
  const size_t stride = (size_t)gridDim.x * blockDim.x * UNR;
  for (size_t base = (size_t)blockIdx.x * blockDim.x * UNR + threadIdx.x; base < n16;
       base += stride) {
    uint4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const size_t i = base + (size_t)u * blockDim.x;
      v[u] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x12345678u) out[blockIdx.x] = acc;   // keeps the loads alive
}

int main() {
  const size_t sizes[] = {16u << 20, 45u << 20, 151u << 20, 1024u << 20};
  constexpr int kCopies = 8, kReps = 64;
  const int grids[] = {1024, 2048, 4096, 8192};
  uint32_t* out = nullptr;
  CHECK(hipMalloc(&out, 8192 * sizeof(uint32_t)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  printf("%10s %6s %4s %10s %8s\n", "MB", "grid", "unr", "us", "TB/s");
  for (size_t bytes : sizes) {
    uint4* buf[kCopies];
    for (int c = 0; c < kCopies; ++c) {
      CHECK(hipMalloc(&buf[c], bytes));
      CHECK(hipMemset(buf[c], c + 1, bytes));
    }
    const size_t n16 = bytes / 16;
    double best = 1e30;
    for (int grid : grids) {
      for (int unr : {4, 8}) {
        auto launch = [&](int c) {
          if (unr == 4)
            hipLaunchKernelGGL(k_read<4>, dim3(grid), dim3(256), 0, 0, buf[c], n16, out);
          else
            hipLaunchKernelGGL(k_read<8>, dim3(grid), dim3(256), 0, 0, buf[c], n16, out);
        };
        for (int w = 0; w < 16; ++w) launch(w % kCopies);
        CHECK(hipDeviceSynchronize());
        CHECK(hipEventRecord(e0, 0));
        for (int r = 0; r < kReps; ++r) launch(r % kCopies);
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        CHECK(hipGetLastError());
        float ms = 0.f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        const double us = ms * 1e3 / kReps;
        best = us < best ? us : best;
        printf("%10.1f %6d %4d %10.2f %8.2f\n", bytes / 1e6, grid, unr, us,
               bytes / (us * 1e-6) / 1e12);
      }
    }
    printf("best %.1f MB: %.2f us, %.2f TB/s\n", bytes / 1e6, best, bytes / (best * 1e-6) / 1e12);
    fflush(stdout);
    for (int c = 0; c < kCopies; ++c) CHECK(hipFree(buf[c]));
  }
  CHECK(hipFree(out));
  return 0;
}
