// What an agent-scope release costs a streaming reduction on one MI355X:
// the library's split parts each publish their partial with one (an L2
// write-back on gfx950, whose L2s are per XCD and not coherent with each
// other). Not part of the library (kept outside csrc/, so the library's
// source digest does not cover it): build and run it on its own,
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//     ragged-mlir_amd/microbench/bench_release_cost.hip -o /tmp/release_cost && /tmp/release_cost
// One kernel: a grid of 256 threads per workgroup, each workgroup summing its
// own contiguous slice of a 2 GiB buffer of 1.0f with 16-byte loads. Every
// `period` bytes of its slice, a workgroup stores its running sum to its own
// slot, waits for the store (barrier), and its thread 0 issues a fence: agent
// scope (a release as the split parts do it), workgroup scope (the control:
// no write-back), or none. The table gives µs per launch (mean of 20 after 3
// warm-ups, HIP events) and GB/s for each fence and period, at two grids
// (1,536 workgroups: the library worker's resident grid; 4,096), and checks
// every workgroup's sum.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                         \
  do {                                                                                   \
    hipError_t e_ = (x);                                                                 \
    if (e_ != hipSuccess) {                                                              \
      std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      std::exit(1);                                                                      \
    }                                                                                    \
  } while (0)

constexpr int kBlock = 256;

enum Fence { kNone = 0, kWorkgroup = 1, kAgent = 2 };

template <int FENCE>
__global__ __launch_bounds__(kBlock) void k_stream(const float4* __restrict__ in, long long per_block,
                                                   long long period, float* slots, float* sums) {
  const long long begin = (long long)blockIdx.x * per_block;
  const long long end = begin + per_block;
  float acc = 0.f;
  long long next = period > 0 ? begin + period : end;
  // Every thread runs every iteration (the loads are guarded), so the
  // barriers below are reached by the whole workgroup together.
  for (long long base = begin; base < end; base += kBlock) {
    const long long i = base + threadIdx.x;
    if (i < end) {
      const float4 v = in[i];
      acc += (v.x + v.y) + (v.z + v.w);
    }
    if (FENCE != kNone && base + kBlock >= next) {
      // The slice's next `period` elements are read: publish the running
      // sum, as a split part does.
      slots[(long long)blockIdx.x * kBlock + threadIdx.x] = acc;
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
      if (threadIdx.x == 0) {
        if (FENCE == kAgent) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        else __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      }
      __syncthreads();
      next += period;
    }
  }
  __shared__ float part[kBlock];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int s = kBlock / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) part[threadIdx.x] += part[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) sums[blockIdx.x] = part[0];
}

template <int FENCE>
static float time_launch(const float4* in, long long per_block, long long period, int grid, float* slots,
                         float* sums) {
  hipEvent_t start, stop;
  CHECK(hipEventCreate(&start));
  CHECK(hipEventCreate(&stop));
  for (int i = 0; i < 3; ++i) k_stream<FENCE><<<grid, kBlock>>>(in, per_block, period, slots, sums);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(start));
  const int launches = 20;
  for (int i = 0; i < launches; ++i) k_stream<FENCE><<<grid, kBlock>>>(in, per_block, period, slots, sums);
  CHECK(hipEventRecord(stop));
  CHECK(hipEventSynchronize(stop));
  float ms = 0.f;
  CHECK(hipEventElapsedTime(&ms, start, stop));
  CHECK(hipEventDestroy(start));
  CHECK(hipEventDestroy(stop));
  return ms * 1000.f / launches;
}

__global__ void k_fill(float4* p, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
    p[i] = make_float4(1.f, 1.f, 1.f, 1.f);
}

int main() {
  const long long bytes = 2LL << 30;
  const long long n = bytes / 16;   // float4 elements
  float4* in = nullptr;
  CHECK(hipMalloc(&in, bytes));
  k_fill<<<4096, 256>>>(in, n);
  CHECK(hipGetLastError());
  const int grids[2] = {1536, 4096};
  const int max_grid = 4096;
  float *slots = nullptr, *sums = nullptr;
  CHECK(hipMalloc(&slots, sizeof(float) * kBlock * max_grid));
  CHECK(hipMalloc(&sums, sizeof(float) * max_grid));
  CHECK(hipDeviceSynchronize());
  std::printf("| grid | slice KiB | fence | period KiB | releases per launch | µs | GB/s |\n");
  std::printf("|---:|---:|---|---:|---:|---:|---:|\n");
  std::vector<float> host(max_grid);
  for (int grid : grids) {
    const long long per_block = n / grid;   // float4 per workgroup (whole slices only)
    const double moved = (double)per_block * grid * 16;
    const long long periods_kib[4] = {0, 1024, 512, 256};
    for (long long pk : periods_kib) {
      const long long period = pk * 1024 / 16;   // float4 per publication
      for (int fence = 0; fence < 3; ++fence) {
        if ((pk == 0) != (fence == kNone)) continue;
        float us = 0.f;
        if (fence == kNone) us = time_launch<kNone>(in, per_block, 0, grid, slots, sums);
        else if (fence == kWorkgroup) us = time_launch<kWorkgroup>(in, per_block, period, grid, slots, sums);
        else us = time_launch<kAgent>(in, per_block, period, grid, slots, sums);
        CHECK(hipMemcpy(host.data(), sums, sizeof(float) * grid, hipMemcpyDeviceToHost));
        for (int b = 0; b < grid; ++b) {
          if (host[b] != (float)(per_block * 4)) {
            std::fprintf(stderr, "workgroup %d sum %f, expected %f\n", b, host[b], (double)(per_block * 4));
            return 1;
          }
        }
        const long long releases = period > 0 ? (per_block / period) * grid : 0;
        const char* name = fence == kNone ? "none" : fence == kWorkgroup ? "workgroup" : "agent";
        std::printf("| %d | %lld | %s | %lld | %lld | %.1f | %.0f |\n", grid, per_block * 16 / 1024, name, pk,
                    releases, us, moved / (us * 1e-6) / 1e9);
        std::fflush(stdout);
      }
    }
  }
  CHECK(hipFree(in));
  CHECK(hipFree(slots));
  CHECK(hipFree(sums));
  return 0;
}
