// Streaming ceilings of one MI355X: what a plain HBM read and a plain copy
// reach with the access shapes the library's kernels use, so that each
// kernel's GB/s can be read against what this device streams, not only
// against the 8 TB/s peak. Not part of the library (kept outside csrc/, so
// the library's source digest does not cover it): build and run it on its
// own,
//   hipcc --offload-arch=gfx950 -O3 ragged-mlir_amd/microbench/bench_stream_ceiling.hip -o /tmp/ceiling && /tmp/ceiling
// Four kernels over buffers of 1.0f (256 threads per workgroup, 16-byte
// loads, U loads in flight per thread before they are summed):
//  * read_stride: grid-stride read, every round of the grid covers
//    grid x 256 x U consecutive vectors;
//  * read_span: each workgroup reads one contiguous span of `span` bytes
//    (the streaming worker's and block-per-segment's block mapping: one
//    workgroup per 128 KiB segment is C2's mean);
//  * copy_stride: grid-stride copy, U loads then U stores;
//  * copy_held: the register-resident softmax's shape without its
//    arithmetic: a workgroup holds one 64 KiB item (16 loads of 16 bytes per
//    thread, each wave's 16 loads one contiguous 16 KiB span), then stores
//    it, items grid-stride; non-temporal loads and stores (nt), or the
//    default cache policy.
// Every shape is checked on the host to divide the buffer exactly before its
// launch, so every load and store is in bounds and every loop ends. The read
// kernels write one partial sum per workgroup, which the host checks against
// the element count.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

template <int U>
__global__ __launch_bounds__(256) void read_stride(const float4* in, long long vectors, float* partial) {
  const long long stride = (long long)gridDim.x * 256;
  float acc = 0.f;
  for (long long base = (long long)blockIdx.x * 256 + threadIdx.x; base < vectors; base += stride * U) {
    float4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = in[base + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) acc += (x[u].x + x[u].y) + (x[u].z + x[u].w);
  }
  __shared__ float sum_s[256];
  sum_s[threadIdx.x] = acc;
  __syncthreads();
  for (int half = 128; half > 0; half >>= 1) {
    if ((int)threadIdx.x < half) sum_s[threadIdx.x] += sum_s[threadIdx.x + half];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = sum_s[0];
}

template <int U>
__global__ __launch_bounds__(256) void read_span(const float4* in, long long span_vectors, float* partial) {
  const float4* span = in + (long long)blockIdx.x * span_vectors;
  float acc = 0.f;
  for (long long base = threadIdx.x; base < span_vectors; base += 256 * U) {
    float4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = span[base + u * 256];
#pragma unroll
    for (int u = 0; u < U; ++u) acc += (x[u].x + x[u].y) + (x[u].z + x[u].w);
  }
  __shared__ float sum_s[256];
  sum_s[threadIdx.x] = acc;
  __syncthreads();
  for (int half = 128; half > 0; half >>= 1) {
    if ((int)threadIdx.x < half) sum_s[threadIdx.x] += sum_s[threadIdx.x + half];
    __syncthreads();
  }
  if (threadIdx.x == 0) partial[blockIdx.x] = sum_s[0];
}

template <int U>
__global__ __launch_bounds__(256) void copy_stride(const float4* in, float4* out, long long vectors) {
  const long long stride = (long long)gridDim.x * 256;
  for (long long base = (long long)blockIdx.x * 256 + threadIdx.x; base < vectors; base += stride * U) {
    float4 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = in[base + u * stride];
#pragma unroll
    for (int u = 0; u < U; ++u) out[base + u * stride] = x[u];
  }
}

typedef float v4f __attribute__((ext_vector_type(4)));   // the nontemporal builtins take clang vectors

template <bool NT>
__global__ __launch_bounds__(256) void copy_held(const v4f* in, v4f* out, long long items) {
  constexpr int kRows = 16;                      // loads per thread
  constexpr long long kItemVectors = 256 * kRows;   // 64 KiB
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  for (long long item = blockIdx.x; item < items; item += gridDim.x) {
    const long long base = item * kItemVectors + (long long)wave * 64 * kRows + lane;
    v4f x[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      if constexpr (NT) x[i] = __builtin_nontemporal_load(in + base + i * 64);
      else x[i] = in[base + i * 64];
    }
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      if constexpr (NT) __builtin_nontemporal_store(x[i], out + base + i * 64);
      else out[base + i * 64] = x[i];
    }
  }
}

__global__ void fill_ones(float4* p, long long vectors) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < vectors) p[i] = make_float4(1.f, 1.f, 1.f, 1.f);
}

static int check(hipError_t err, const char* what) {
  if (err != hipSuccess) {
    std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(err));
    return 1;
  }
  return 0;
}

// Median of 7 launches (after one warm-up) of `launch`, in microseconds.
template <class Launch>
static int time_median(Launch&& launch, hipEvent_t start, hipEvent_t stop, double* us) {
  std::vector<float> ms;
  launch();
  if (check(hipDeviceSynchronize(), "warm-up")) return 1;
  for (int rep = 0; rep < 7; ++rep) {
    if (check(hipEventRecord(start), "record")) return 1;
    launch();
    if (check(hipEventRecord(stop), "record") || check(hipEventSynchronize(stop), "launch")) return 1;
    float t = 0.f;
    if (check(hipEventElapsedTime(&t, start, stop), "elapsed")) return 1;
    ms.push_back(t);
  }
  std::sort(ms.begin(), ms.end());
  *us = ms[3] * 1e3;
  return 0;
}

static int check_partials(const float* partial_d, int count, double expected, const char* what) {
  std::vector<float> host(count);
  if (check(hipMemcpy(host.data(), partial_d, sizeof(float) * count, hipMemcpyDeviceToHost), "copy partials")) return 1;
  double total = 0;
  for (float v : host) total += v;
  if (total != expected) {
    std::fprintf(stderr, "%s: partial sums add to %.0f, expected %.0f\n", what, total, expected);
    return 1;
  }
  return 0;
}

int main() {
  const long long kMiB = 1ll << 20;
  const long long sizes[] = {512 * kMiB, 1024 * kMiB};
  const long long max_bytes = 1024 * kMiB;
  float4* in = nullptr;
  float4* out = nullptr;
  float* partial = nullptr;
  const int max_grid = 1 << 16;
  if (check(hipMalloc(&in, max_bytes), "hipMalloc in") || check(hipMalloc(&out, max_bytes), "hipMalloc out") ||
      check(hipMalloc(&partial, sizeof(float) * max_grid), "hipMalloc partial"))
    return 1;
  const long long max_vectors = max_bytes / 16;
  fill_ones<<<(unsigned)((max_vectors + 255) / 256), 256>>>(in, max_vectors);
  if (check(hipDeviceSynchronize(), "fill")) return 1;
  hipEvent_t start, stop;
  if (check(hipEventCreate(&start), "event") || check(hipEventCreate(&stop), "event")) return 1;
  hipDeviceProp_t props;
  if (check(hipGetDeviceProperties(&props, 0), "properties")) return 1;
  const int cus = props.multiProcessorCount;
  std::printf("device %s, %d CUs; median of 7 launches after one warm-up; GB/s = bytes moved / time\n",
              props.gcnArchName, cus);
  std::printf("%-12s %9s %6s %3s %10s %9s %8s\n", "kernel", "MiB", "grid", "U", "span KiB", "us", "GB/s");

  for (long long bytes : sizes) {
    const long long vectors = bytes / 16;
    // Grid-stride read: 2, 4 and 8 workgroups per CU.
    for (int per_cu : {2, 4, 8}) {
      const int grid = cus * per_cu;
      for (int u : {4, 8, 16}) {
        const long long round = (long long)grid * 256 * u;
        if (vectors % round != 0) continue;   // every round whole: no load past the buffer
        double us = 0;
        auto launch = [&] {
          if (u == 4) read_stride<4><<<grid, 256>>>(in, vectors, partial);
          if (u == 8) read_stride<8><<<grid, 256>>>(in, vectors, partial);
          if (u == 16) read_stride<16><<<grid, 256>>>(in, vectors, partial);
        };
        if (time_median(launch, start, stop, &us) || check_partials(partial, grid, (double)vectors * 4, "read_stride"))
          return 1;
        std::printf("%-12s %9lld %6d %3d %10s %9.1f %8.0f\n", "read_stride", bytes / kMiB, grid, u, "-", us,
                    bytes / us * 1e-3);
      }
    }
    // One workgroup per contiguous span.
    for (long long span_kib : {32ll, 128ll, 512ll}) {
      const long long span_vectors = span_kib * 1024 / 16;
      const long long grid = vectors / span_vectors;
      if (grid > max_grid || vectors % span_vectors != 0) continue;
      for (int u : {4, 8}) {
        if (span_vectors % (256ll * u) != 0) continue;   // whole rounds inside each span
        double us = 0;
        auto launch = [&] {
          if (u == 4) read_span<4><<<(unsigned)grid, 256>>>(in, span_vectors, partial);
          if (u == 8) read_span<8><<<(unsigned)grid, 256>>>(in, span_vectors, partial);
        };
        if (time_median(launch, start, stop, &us) ||
            check_partials(partial, (int)grid, (double)vectors * 4, "read_span"))
          return 1;
        std::printf("%-12s %9lld %6lld %3d %10lld %9.1f %8.0f\n", "read_span", bytes / kMiB, grid, u, span_kib, us,
                    bytes / us * 1e-3);
      }
    }
    // Grid-stride copy (bytes read + bytes written).
    for (int per_cu : {2, 4, 8}) {
      const int grid = cus * per_cu;
      for (int u : {4, 8}) {
        const long long round = (long long)grid * 256 * u;
        if (vectors % round != 0) continue;
        double us = 0;
        auto launch = [&] {
          if (u == 4) copy_stride<4><<<grid, 256>>>(in, out, vectors);
          if (u == 8) copy_stride<8><<<grid, 256>>>(in, out, vectors);
        };
        if (time_median(launch, start, stop, &us)) return 1;
        std::printf("%-12s %9lld %6d %3d %10s %9.1f %8.0f\n", "copy_stride", bytes / kMiB, grid, u, "-", us,
                    2.0 * bytes / us * 1e-3);
      }
    }
    // Held 64 KiB items (bytes is a multiple of 64 KiB: whole items only).
    const long long items = bytes / (64 * 1024);
    for (int per_cu : {2, 4}) {
      const int grid = cus * per_cu;
      for (int nt : {1, 0}) {
        double us = 0;
        auto launch = [&] {
          const v4f* src = reinterpret_cast<const v4f*>(in);
          v4f* dst = reinterpret_cast<v4f*>(out);
          if (nt) copy_held<true><<<grid, 256>>>(src, dst, items);
          else copy_held<false><<<grid, 256>>>(src, dst, items);
        };
        if (time_median(launch, start, stop, &us)) return 1;
        std::printf("%-12s %9lld %6d %3d %10s %9.1f %8.0f\n", nt ? "copy_held_nt" : "copy_held", bytes / kMiB, grid, 16,
                    "64", us, 2.0 * bytes / us * 1e-3);
      }
    }
  }
  return check(hipFree(in), "hipFree") | check(hipFree(out), "hipFree") | check(hipFree(partial), "hipFree");
}
