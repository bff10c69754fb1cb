// Ticket hand-out rate on one MI355X: the evidence behind k_worker taking its
// tickets from 16 interleaved counters and k_classify reserving one run of
// queue positions per class and workgroup. Not part of the library: build
// and run it on its own,
//   hipcc --offload-arch=gfx950 -O3 ragged-mlir_amd/microbench/bench_ticket_counters.hip -o /tmp/tickets && /tmp/tickets
// Each of `grid` workgroups (256 threads) takes tickets until `total` are
// handed out: thread 0 adds 1 to counter (blockIdx % lanes), and the ticket
// is (old value) * lanes + lane, as in k_worker. Counters sit 256 bytes
// apart. Every workgroup's loop ends once its counter passes total / lanes,
// so every launch drains. The kernel writes nothing but its counters.
#include <hip/hip_runtime.h>

#include <cstdio>

constexpr int kStride = 32;   // int64 slots between counters: 256 bytes

__global__ __launch_bounds__(256) void take_tickets(unsigned long long* counters, int lanes, long long total,
                                                    unsigned long long* taken) {
  __shared__ long long ticket_s;
  const int lane = blockIdx.x % lanes;
  unsigned long long mine = 0;
  for (;;) {
    if (threadIdx.x == 0) ticket_s = (long long)atomicAdd(counters + lane * kStride, 1ull) * lanes + lane;
    __syncthreads();
    const long long ticket = ticket_s;
    __syncthreads();
    if (ticket >= total) break;
    ++mine;
  }
  if (threadIdx.x == 0) atomicAdd(taken, mine);
}

static int check(hipError_t err, const char* what) {
  if (err != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(err));
    return 1;
  }
  return 0;
}

int main() {
  const long long total = 32768;
  const int grids[] = {256, 1024, 1536};
  const int lane_counts[] = {1, 2, 4, 8, 16, 32};
  unsigned long long* counters = nullptr;
  unsigned long long* taken = nullptr;
  const size_t counter_bytes = sizeof(unsigned long long) * kStride * 32;
  if (check(hipMalloc(&counters, counter_bytes), "hipMalloc") || check(hipMalloc(&taken, 8), "hipMalloc")) return 1;
  hipEvent_t start, stop;
  if (check(hipEventCreate(&start), "event") || check(hipEventCreate(&stop), "event")) return 1;
  std::printf("tickets %lld; median of 5 launches\n%8s %6s %10s %12s\n", total, "grid", "lanes", "us", "ns/ticket");
  for (int grid : grids) {
    for (int lanes : lane_counts) {
      float times[5];
      for (int rep = 0; rep < 5; ++rep) {
        if (check(hipMemset(counters, 0, counter_bytes), "memset") || check(hipMemset(taken, 0, 8), "memset")) return 1;
        hipEventRecord(start);
        take_tickets<<<grid, 256>>>(counters, lanes, total, taken);
        hipEventRecord(stop);
        if (check(hipEventSynchronize(stop), "launch")) return 1;
        hipEventElapsedTime(&times[rep], start, stop);
        unsigned long long got = 0;
        if (check(hipMemcpy(&got, taken, 8, hipMemcpyDeviceToHost), "copy")) return 1;
        if ((long long)got != total) {
          std::fprintf(stderr, "grid %d lanes %d: %llu tickets taken, expected %lld\n", grid, lanes, got, total);
          return 1;
        }
      }
      for (int i = 1; i < 5; ++i)
        for (int j = i; j > 0 && times[j] < times[j - 1]; --j) {
          const float t = times[j];
          times[j] = times[j - 1];
          times[j - 1] = t;
        }
      const double us = times[2] * 1e3;
      std::printf("%8d %6d %10.1f %12.2f\n", grid, lanes, us, us * 1e3 / (double)total);
    }
  }
  hipFree(counters);
  hipFree(taken);
  return 0;
}
