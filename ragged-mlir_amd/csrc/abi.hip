// Host implementation of the C ABI in include/ragged_hip.h.
//
// Replaces the reference's CUDA Driver API launcher (runtime/Driver.cpp):
// instead of loading a generated cubin and resolving kernels by name, a
// module selects one of the ahead-of-time compiled gfx950 kernel
// specialisations; instead of a launch plan with relocated memref
// descriptors, one by-value Params struct carries every pointer and size.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/ragged_hip.h"
#include "device.hpp"
#include "table.hpp"

#ifndef RG_SOURCE_DIGEST
#define RG_SOURCE_DIGEST "unknown"
#endif

namespace {

thread_local std::string g_error;

int fail(int status, const char* fmt, ...) {
  char buffer[512];
  va_list args;
  va_start(args, fmt);
  vsnprintf(buffer, sizeof buffer, fmt, args);
  va_end(args);
  g_error = buffer;
  return status;
}

int hip_fail(hipError_t err, const char* what) {
  return fail(RG_E_DEVICE, "%s: %s (%d): %s", what, hipGetErrorName(err), (int)err, hipGetErrorString(err));
}

constexpr int64_t kI64Max = INT64_MAX;
constexpr uint64_t kAlign = 256;
constexpr int64_t kGridMax = 2147483647;

// Class boundaries and part size in bytes of segment data; row thresholds
// follow from the row size (see rg_spec_defaults).
constexpr int64_t kWaveBytes = 8 << 10;     // one wave64 reads up to 8 KiB
constexpr int64_t kBlockBytes = 512 << 10;  // one workgroup reads up to 512 KiB
constexpr int64_t kPartBytes = 256 << 10;   // a split part is 256 KiB of rows

int element_bytes(int dtype) { return dtype == RG_BF16 ? 2 : 4; }

// Geometry of a specialisation: elements per access and mapping, plus the
// table index (see table.hpp).
struct Geometry {
  int vec;
  bool flat;
  int index;
};

// Rows one workgroup of the register-resident softmax holds, or 0 when the
// specialisation has no such worker (flat mapping, or more than 256 lanes per
// row). Mirrors fused_rows() and row_geo() of the device code.
int64_t fused_capacity(int dtype, int d, int vec, bool flat, bool f32_logits) {
  if (flat) return 0;
  const int64_t lanes = (d + vec - 1) / vec;
  if (lanes > rg::kBlock) return 0;
  int lpr = 1;
  while (lpr < lanes) lpr <<= 1;
  const int store = (dtype == RG_F32 || f32_logits) ? 4 : 2;
  const int rpt = std::min(32, 256 / (vec * store));
  return (int64_t)(rg::kBlock / lpr) * rpt;
}

Geometry choose_geometry(int dtype, int d, bool vectorize) {
  const int widest = 16 / element_bytes(dtype);   // 4 f32 or 8 bf16 per 16 B
  if (!vectorize) return {1, false, 0};
  if (d < widest && widest % d == 0) return {widest, true, dtype == RG_BF16 ? 4 : 3};
  int vec = 1;
  while (vec * 2 <= widest && d % (vec * 2) == 0) vec *= 2;
  int index = vec == 1 ? 0 : vec == 2 ? 1 : vec == 4 ? 2 : 3;
  return {vec, false, index};
}

int next_pow2_capped(int64_t value, int cap) {
  int p = 1;
  while (p < value && p < cap) p <<= 1;
  return p;
}

// Feature tiles of a ROW launch with groups of `g` threads.
int64_t feature_tiles(int d, int vec, bool flat, int g) {
  if (flat) return 1;
  const int64_t lanes = (d + vec - 1) / vec;
  const int lpr = next_pow2_capped(lanes, g);
  return (lanes + lpr - 1) / lpr;
}

int combine_features_host(int d) { return next_pow2_capped(d, rg::kCombineFeatures); }

bool mul_ok(int64_t a, int64_t b, int64_t* out) { return !__builtin_mul_overflow(a, b, out) && *out >= 0; }
bool add_ok(int64_t a, int64_t b, int64_t* out) { return !__builtin_add_overflow(a, b, out) && *out >= 0; }

// Workspace of the allocation-free entry point (rg_run_static): one array
// per device, held by the loaded code object until the process ends. Host
// code never passes `scratch` itself to a kernel or a copy: its host-side
// name is not a device address. Its device address is resolved once per
// device with hipGetSymbolAddress (set_up_static_scratch, called by
// rg_module_create with that device current) and only that address is used.
constexpr uint64_t kStaticScratchBytes = RG_STATIC_WORKSPACE_BYTES;
constexpr int kMaxDevices = 64;
constexpr size_t kScratchCounterBytes = (size_t)rg::kTicketStride * 8 * (1 + 2 * rg::kTicketLanes);
static_assert(kStaticScratchBytes % 256 == 0 && kStaticScratchBytes >= kScratchCounterBytes,
              "RG_STATIC_WORKSPACE_BYTES: a multiple of 256 bytes that holds at least the counters");
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices];          // device address of `scratch` on each device, or null
// A call on the device's static workspace failed after it had launched
// something, so its counters may be set: the next call first launches
// k_reset.
bool g_scratch_dirty[kMaxDevices];
// Test control (rg_test_interrupt_static): the next rg_run_static stops after
// this many launches and fails, as a launch error would; -1: off.
int g_interrupt_after = -1;

}  // namespace

static __device__ __align__(256) unsigned char scratch[RG_STATIC_WORKSPACE_BYTES];

// Resolve `scratch` on the current device `device` (once); RG_OK or the HIP error.
static int set_up_static_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(RG_E_INVALID, "device ordinal %d out of range", device);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[device]) return RG_OK;
  void* address = nullptr;
  const hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
  if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(scratch)");
  if (!address || (reinterpret_cast<uintptr_t>(address) & (kAlign - 1)) != 0)
    return fail(RG_E_DEVICE, "static workspace of device %d is not 256-byte aligned", device);
  // A workspace is all-zero before its first call (every call leaves its
  // counters at zero again); the loader zero-fills the array, this makes
  // sure of the counter region.
  const hipError_t zero = hipMemset(address, 0, kScratchCounterBytes);
  if (zero != hipSuccess) return hip_fail(zero, "hipMemset(static workspace counters)");
  g_scratch[device] = address;
  return RG_OK;
}

static void* static_scratch(int device, bool* dirty) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  *dirty = g_scratch_dirty[device];
  return g_scratch[device];
}

static void set_scratch_dirty(int device, bool dirty) {
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  g_scratch_dirty[device] = dirty;
}

// Event pool of a profiling session: launches+1 events per recorded call.
struct Profile {
  bool active = false;
  int max_calls = 0;
  std::vector<hipEvent_t> events;
  std::vector<int> call_first;     // first event index of each call
  std::vector<int> call_roles;     // roles of every launch, concatenated
  std::vector<int> call_launches;  // launches of each call
};

struct rg_module {
  int device;
  rg_spec spec;
  Geometry geometry;
  const rg::KernelSet* kernels;
  const void* roles[RG_ROLE_COUNT];
  int64_t resident[RG_ROLE_COUNT];
  uint32_t lds[RG_ROLE_COUNT];
  bool fused;                 // softmax through k_softmax_fused
  int64_t spin_ticks;         // wall-clock ticks of a chunk's bounded wait
  int64_t drain_ticks;        // wall-clock ticks of a worker split part's (deferred chunk's) wait for its statistics
  int64_t fold_ticks;         // wall-clock bound of a fold whose inputs are all published before it starts
  int64_t clock_khz;          // wall-clock rate
  int64_t* trace;             // item timeline buffer (diagnostics) or null
  int64_t trace_cap;
  mutable Profile profile;
};

// One past the last byte of the register-resident softmax's arena (the pair
// table through the deferred list), 256-byte aligned.
static uint64_t arena_end(const rg_plan* plan) {
  const uint64_t end = plan->buffer_offset[RG_BUF_DEFERRED] + plan->buffer_bytes[RG_BUF_DEFERRED];
  return (end + kAlign - 1) / kAlign * kAlign;
}

extern "C" {

int rg_abi_version(void) { return RG_ABI_VERSION; }

const char* rg_build_info(void) {
  return "target=gfx950;abi=2;flags=-O3 -packed-fp32-ops;source=" RG_SOURCE_DIGEST;
}

const char* rg_last_error(void) { return g_error.c_str(); }

int rg_device_query(int ordinal, rg_device_props* out) {
  if (!out) return fail(RG_E_INVALID, "rg_device_query: null output");
  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, ordinal);
  if (err != hipSuccess) return hip_fail(err, "hipGetDeviceProperties");
  std::memset(out, 0, sizeof *out);
  out->ordinal = ordinal;
  out->cu_count = prop.multiProcessorCount;
  int xcc = 0;
  if (hipDeviceGetAttribute(&xcc, hipDeviceAttributeNumberOfXccs, ordinal) != hipSuccess || xcc <= 0) xcc = 1;
  out->xcd_count = xcc;
  out->wave_size = prop.warpSize;
  out->l2_bytes = prop.l2CacheSize;
  // HIP reports no last-level cache size; MI350-series (gfx950) carries a
  // 256 MiB Infinity Cache.
  out->mall_bytes = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? (int64_t)256 << 20 : 0;
  out->lds_per_cu = prop.maxSharedMemoryPerMultiProcessor;
  out->global_mem_bytes = (int64_t)prop.totalGlobalMem;
  std::snprintf(out->arch, sizeof out->arch, "%s", prop.gcnArchName);
  return RG_OK;
}

int rg_spec_defaults(rg_spec* spec) {
  if (!spec) return fail(RG_E_INVALID, "rg_spec_defaults: null spec");
  if (spec->feature_dim < 1 || spec->feature_dim > 1024) return fail(RG_E_INVALID, "feature_dim must be in [1, 1024]");
  if (spec->dtype != RG_F32 && spec->dtype != RG_BF16) return fail(RG_E_INVALID, "dtype must be f32 or bf16");
  const int64_t row = (int64_t)spec->feature_dim * element_bytes(spec->dtype);
  const bool default_wave = spec->t_wave < 0;
  const Geometry geo = choose_geometry(spec->dtype, spec->feature_dim, spec->vectorize != 0);
  // Segments one lane (flat mapping, D below the vector width) or one group
  // of the lanes that hold a row (rows of at most half a wave's lanes)
  // reduces on its own; the wave class adds those one wave reads in one
  // pass (kWaveBytes).
  const int64_t lanes = (spec->feature_dim + geo.vec - 1) / geo.vec;
  spec->alone_rows = geo.flat ? std::max<int64_t>(1, rg::kLaneElems / spec->feature_dim)
                   : lanes <= rg::kWave / 2 ? rg::kGroupRows : 0;
  if (default_wave) spec->t_wave = std::max<int64_t>({1, spec->alone_rows, kWaveBytes / row});
  // Softmax with a register-resident worker: a block-class segment and a
  // split chunk are exactly what one workgroup holds in registers.
  const int64_t capacity = spec->op == RG_OP_SOFTMAX
      ? fused_capacity(spec->dtype, spec->feature_dim, geo.vec, geo.flat,
                       spec->has_mask != 0 || spec->scale != 1.0f)
      : 0;
  if (capacity > 0) {
    if (spec->t_block < 0) spec->t_block = capacity;
    if (spec->part_rows < 0) spec->part_rows = capacity;
    // The wave class stays with the streaming worker, below the block class.
    if (default_wave) spec->t_wave = std::max<int64_t>(0, std::min<int64_t>(spec->t_wave, spec->t_block - 1));
  }
  if (spec->t_block < 0) spec->t_block = std::max<int64_t>(spec->t_wave + 1, kBlockBytes / row);
  if (spec->part_rows < 0) spec->part_rows = std::max<int64_t>(1, kPartBytes / row);
  return RG_OK;
}

int rg_spec_uses_fused(const rg_spec* spec_in) {
  if (!spec_in) return fail(RG_E_INVALID, "rg_spec_uses_fused: null spec");
  rg_spec spec = *spec_in;
  const int status = rg_spec_defaults(&spec);
  if (status) return status;
  if (spec.op != RG_OP_SOFTMAX) return 0;
  // The register-resident softmax runs when one workgroup can hold a block
  // segment and a split chunk.
  const Geometry geo = choose_geometry(spec.dtype, spec.feature_dim, spec.vectorize != 0);
  const int64_t capacity = fused_capacity(spec.dtype, spec.feature_dim, geo.vec, geo.flat,
                                          spec.has_mask != 0 || spec.scale != 1.0f);
  return capacity > 0 && spec.t_block <= capacity && spec.part_rows <= capacity ? 1 : 0;
}

int rg_module_create(int device, const rg_spec* spec_in, rg_module** out) {
  if (!spec_in || !out) return fail(RG_E_INVALID, "rg_module_create: null argument");
  *out = nullptr;
  rg_spec spec = *spec_in;
  if (spec.op < RG_OP_SUM || spec.op > RG_OP_SOFTMAX) return fail(RG_E_INVALID, "op must be sum, max or softmax");
  if (spec.offsets_dtype != RG_I32 && spec.offsets_dtype != RG_I64)
    return fail(RG_E_INVALID, "offsets dtype must be i32 or i64");
  int status = rg_spec_defaults(&spec);
  if (status) return status;
  if (spec.has_mask && spec.op != RG_OP_SOFTMAX) return fail(RG_E_INVALID, "an additive mask is only defined for softmax");
  if (!(spec.scale == spec.scale) || spec.scale > 3.402823466e38f || spec.scale < -3.402823466e38f)
    return fail(RG_E_INVALID, "scale must be a finite f32");
  if (spec.t_wave < 0 || spec.t_block <= spec.t_wave || spec.part_rows < 1)
    return fail(RG_E_INVALID, "thresholds must satisfy 0 <= t_wave < t_block and part_rows >= 1");

  hipDeviceProp_t prop;
  hipError_t err = hipGetDeviceProperties(&prop, device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(RG_E_UNSUPPORTED, "device %d is %s; this library holds gfx950 code only", device, prop.gcnArchName);

  rg_module* module = new (std::nothrow) rg_module();
  if (!module) return fail(RG_E_INVALID, "out of host memory");
  module->device = device;
  module->spec = spec;
  module->geometry = choose_geometry(spec.dtype, spec.feature_dim, spec.vectorize != 0);
  const int g = module->geometry.index;
  if (spec.op == RG_OP_SUM) module->kernels = rg::kernels_sum(spec.dtype, spec.offsets_dtype, g);
  else if (spec.op == RG_OP_MAX) module->kernels = rg::kernels_max(spec.dtype, spec.offsets_dtype, g);
  else module->kernels = rg::kernels_softmax(spec.dtype, spec.offsets_dtype, g, spec.has_mask != 0);
  const rg::KernelSet& k = *module->kernels;
  if (!k.naive || k.vec != module->geometry.vec || k.flat != module->geometry.flat) {
    delete module;
    return fail(RG_E_INVALID, "no compiled kernel for this dtype/feature geometry");
  }
  // k_classify initialises what a call uses; every classified call's last
  // workgroup returns the counters to zero (RG_ROLE_INIT and
  // RG_ROLE_DEFERRED stay empty: the register-resident softmax needs no
  // slot fill and drains its deferred chunks and wave class itself).
  module->roles[RG_ROLE_CLASSIFY] = rg::kernel_classify(spec.offsets_dtype);
  module->roles[RG_ROLE_WORKER] = k.worker;
  // RG_ROLE_SPLIT_NORMALIZE stays empty: k_worker normalises split parts.
  module->roles[RG_ROLE_NAIVE] = k.naive;
  const bool f32_logits = spec.has_mask != 0 || spec.scale != 1.0f;
  const void* fused = f32_logits ? k.fused_f32 : k.fused;
  module->fused = fused && rg_spec_uses_fused(&spec) == 1;
  module->roles[RG_ROLE_FUSED] = module->fused ? fused : nullptr;

  int previous = 0;
  err = hipGetDevice(&previous);
  if (err == hipSuccess) err = hipSetDevice(device);
  if (err != hipSuccess) {
    delete module;
    return hip_fail(err, "hipSetDevice");
  }
  // The allocation-free entry point's workspace on this device (the device
  // is current here).
  const int scratch_status = set_up_static_scratch(device);
  if (scratch_status != RG_OK) {
    (void)hipSetDevice(previous);
    delete module;
    return scratch_status;
  }
  int clock_khz = 0;
  if (err == hipSuccess) err = hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, device);
  // A chunk waits at most 2 ms for the rest of its segment before deferring.
  module->clock_khz = std::max(clock_khz, 1000);
  module->spin_ticks = module->clock_khz * 2;
  // A worker's split part waits at most 1 s for its segment's statistics
  // before it is left to the grid's last workgroup (the wait normally ends
  // in microseconds).
  module->drain_ticks = module->clock_khz * 1000;
  // A fold whose every input was published before it started (a tree
  // group's last arriver, the last workgroup's drain) normally succeeds at
  // once; it polls for at most 1 s.
  module->fold_ticks = module->clock_khz * 1000;
  for (int role = 0; role < RG_ROLE_COUNT && err == hipSuccess; ++role) {
    module->resident[role] = 0;
    module->lds[role] = 0;
    if (!module->roles[role]) continue;
    hipFuncAttributes attributes;
    err = hipFuncGetAttributes(&attributes, module->roles[role]);
    if (err != hipSuccess) break;
    module->lds[role] = (uint32_t)attributes.sharedSizeBytes;
    int per_cu = 0;
    const int threads = role == RG_ROLE_CLASSIFY ? rg::kClassifyBlock : rg::kBlock;
    err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, module->roles[role], threads, 0);
    if (err != hipSuccess) break;
    module->resident[role] = (int64_t)std::max(per_cu, 1) * prop.multiProcessorCount;
  }
  (void)hipSetDevice(previous);
  if (err != hipSuccess) {
    delete module;
    return hip_fail(err, "kernel occupancy query");
  }
  *out = module;
  return RG_OK;
}

static void release_events(Profile& profile) {
  for (hipEvent_t event : profile.events) (void)hipEventDestroy(event);
  profile.events.clear();
  profile.call_first.clear();
  profile.call_roles.clear();
  profile.call_launches.clear();
}

void rg_module_destroy(rg_module* module) {
  if (module) release_events(module->profile);
  delete module;
}

int rg_profile_start(rg_module* module, int max_calls) {
  if (!module || max_calls < 1 || max_calls > 100000) return fail(RG_E_INVALID, "rg_profile_start: bad argument");
  Profile& profile = module->profile;
  release_events(profile);
  profile.active = true;
  profile.max_calls = max_calls;
  return RG_OK;
}

int rg_profile_stop(rg_module* module, double* role_ms, int64_t* role_launches, double* call_ms, int64_t* calls) {
  if (!module || !role_ms || !role_launches || !call_ms || !calls) return fail(RG_E_INVALID, "rg_profile_stop: null");
  Profile& profile = module->profile;
  profile.active = false;
  for (int r = 0; r < RG_ROLE_COUNT; ++r) {
    role_ms[r] = 0;
    role_launches[r] = 0;
  }
  *call_ms = 0;
  *calls = (int64_t)profile.call_first.size();
  hipError_t err = hipSuccess;
  if (!profile.events.empty()) err = hipEventSynchronize(profile.events.back());
  size_t role_index = 0;
  for (size_t c = 0; c < profile.call_first.size() && err == hipSuccess; ++c) {
    const int first = profile.call_first[c], launches = profile.call_launches[c];
    for (int i = 0; i < launches && err == hipSuccess; ++i) {
      float ms = 0;
      err = hipEventElapsedTime(&ms, profile.events[first + i], profile.events[first + i + 1]);
      const int role = profile.call_roles[role_index++];
      role_ms[role] += ms;
      role_launches[role] += 1;
    }
    float total = 0;
    if (err == hipSuccess) err = hipEventElapsedTime(&total, profile.events[first], profile.events[first + launches]);
    *call_ms += total;
  }
  release_events(profile);
  if (err != hipSuccess) return hip_fail(err, "rg_profile_stop");
  return RG_OK;
}

int rg_module_set_spin_limit(rg_module* module, int64_t microseconds) {
  if (!module || microseconds < -1 || microseconds > 10000000)
    return fail(RG_E_INVALID, "rg_module_set_spin_limit: limit must be -1 (defaults) or in [0, 10 s]");
  if (microseconds < 0) {
    module->spin_ticks = module->clock_khz * 2;
    module->drain_ticks = module->clock_khz * 1000;
    return RG_OK;
  }
  module->spin_ticks = module->clock_khz * microseconds / 1000;
  module->drain_ticks = module->spin_ticks;
  return RG_OK;
}

int rg_module_set_trace(rg_module* module, void* buffer, int64_t records) {
  if (!module || records < 0 || (buffer && records == 0))
    return fail(RG_E_INVALID, "rg_module_set_trace: bad argument");
  module->trace = static_cast<int64_t*>(buffer);
  module->trace_cap = buffer ? records : 0;
  return RG_OK;
}

int rg_device_clock_khz(int device, int64_t* khz) {
  if (!khz) return fail(RG_E_INVALID, "rg_device_clock_khz: null argument");
  int rate = 0;
  const hipError_t err = hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, device);
  if (err != hipSuccess) return hip_fail(err, "hipDeviceGetAttribute");
  *khz = rate;
  return RG_OK;
}

int rg_module_resident(const rg_module* module, int role, int64_t* blocks) {
  if (!module || !blocks || role < 0 || role >= RG_ROLE_COUNT) return fail(RG_E_INVALID, "rg_module_resident: bad argument");
  *blocks = module->resident[role];
  return RG_OK;
}

int rg_plan_create(const rg_module* module, int64_t n, int64_t b, int schedule, rg_plan* plan) {
  if (!module || !plan) return fail(RG_E_INVALID, "rg_plan_create: null argument");
  if (n < 0 || b < 0) return fail(RG_E_INVALID, "N and B must be nonnegative");
  if (b == 0 && n != 0) return fail(RG_E_INVALID, "B=0 requires N=0");
  if (schedule != RG_CLASSIFIED && schedule != RG_BLOCK_PER_SEGMENT && schedule != RG_SHORT_SEGMENTS)
    return fail(RG_E_INVALID, "unknown schedule");
  if (schedule == RG_SHORT_SEGMENTS && (module->spec.t_wave < 1 || module->spec.alone_rows < 1))
    return fail(RG_E_INVALID, "this specialisation has no short-segment schedule");
  if (schedule == RG_BLOCK_PER_SEGMENT && module->spec.debug_visits)
    return fail(RG_E_INVALID, "debug visits require the classified schedule");
  const rg_spec& spec = module->spec;
  const int d = spec.feature_dim;
  const Geometry& geo = module->geometry;
  int64_t nd;
  if (!mul_ok(n, d, &nd) || !mul_ok(nd, element_bytes(spec.dtype), &nd))
    return fail(RG_E_INVALID, "N*D bytes overflow signed i64");
  std::memset(plan, 0, sizeof *plan);
  plan->schedule = schedule;
  plan->n = n;
  plan->b = b;
  plan->t_wave = spec.t_wave;
  plan->t_block = spec.t_block;
  plan->part_rows = spec.part_rows;
  plan->vec = geo.vec;
  plan->flat = geo.flat ? 1 : 0;
  if (b == 0) return RG_OK;

  auto add_launch = [&](int role, int64_t gx, int64_t gy, int block = rg::kBlock) {
    const int i = plan->launches++;
    plan->roles[i] = role;
    plan->grid[i][0] = (uint32_t)std::min<int64_t>(std::max<int64_t>(gx, 1), kGridMax);
    plan->grid[i][1] = (uint32_t)std::max<int64_t>(gy, 1);
    plan->grid[i][2] = 1;
    plan->block[i] = (uint32_t)block;
    plan->lds_bytes[i] = module->lds[role];
  };
  const int64_t tiles_block = feature_tiles(d, geo.vec, geo.flat, rg::kBlock);
  if (schedule == RG_BLOCK_PER_SEGMENT) {
    add_launch(RG_ROLE_NAIVE, b, tiles_block);
    return RG_OK;
  }
  if (schedule == RG_SHORT_SEGMENTS) {
    // Workgroups for grid-stride batches of at most B wave-class segments:
    // the fewest segments a workgroup takes per batch is one per wave.
    const int64_t wave_batch_min = geo.flat ? rg::kBlock : rg::kWavesPerBlock;
    const int64_t stride_grid = (b + wave_batch_min - 1) / wave_batch_min;
    // Batches of segments in order, grid-stride: no counters, no workspace.
    add_launch(RG_ROLE_WORKER, std::min(module->resident[RG_ROLE_WORKER], stride_grid), 1);
    return RG_OK;
  }

  // Workspace: every buffer at a 256-byte aligned offset of one allocation.
  const int64_t b_split = std::min<int64_t>(b, n / (spec.t_block + 1));
  const int64_t items_cap = b_split ? n / spec.part_rows + b_split : 0;
  plan->b_split = b_split;
  plan->items_cap = items_cap;
  const bool softmax = spec.op == RG_OP_SOFTMAX;
  int64_t sizes[RG_WORKSPACE_BUFFERS] = {0};
  int64_t value;
  if (!mul_ok(b, 3 * 8, &value)) return fail(RG_E_INVALID, "queue bytes overflow");
  sizes[RG_BUF_QUEUE] = value;
  if (!mul_ok(items_cap, 8, &sizes[RG_BUF_ITEM_POS]) || !mul_ok(b_split, 8, &sizes[RG_BUF_PART_BEGIN]))
    return fail(RG_E_INVALID, "split table bytes overflow");
  int64_t stat_bytes, item_bytes;
  if (!mul_ok(items_cap, (int64_t)d * 4, &item_bytes) || !mul_ok(b_split, (int64_t)d * 4, &stat_bytes))
    return fail(RG_E_INVALID, "split workspace bytes overflow");
  sizes[RG_BUF_COUNTERS] = (int64_t)rg::kTicketStride * 8 * (1 + 2 * rg::kTicketLanes);
  if (!module->fused) {
    // Part arrivals per split segment (the worker's last part combines).
    if (!mul_ok(b_split, 4, &sizes[RG_BUF_SEG_ARRIVE])) return fail(RG_E_INVALID, "arrival bytes overflow");
    sizes[RG_BUF_PARTIALS] = item_bytes;
    if (softmax) {
      sizes[RG_BUF_PARTIAL_SUMS] = item_bytes;
      sizes[RG_BUF_STATS_MAX] = stat_bytes;
      sizes[RG_BUF_STATS_SUM] = stat_bytes;
      // Split parts (x feature tiles) whose wait for their statistics ran
      // out, normalised by the worker's last workgroup.
      if (!mul_ok(items_cap, tiles_block * 8, &sizes[RG_BUF_DEFERRED])) return fail(RG_E_INVALID, "deferred bytes overflow");
    }
  } else {
    // Register-resident softmax: item descriptors, published (m, s) pairs
    // and the merge counters; no item_pos / part_begin tables.
    sizes[RG_BUF_ITEM_POS] = 0;
    sizes[RG_BUF_PART_BEGIN] = 0;
    if (!mul_ok(b, (int64_t)sizeof(rg::Item), &sizes[RG_BUF_BLOCK_ITEMS]) ||
        !mul_ok(items_cap, (int64_t)sizeof(rg::Item), &sizes[RG_BUF_ITEMS]) ||
        !mul_ok(items_cap, 8, &sizes[RG_BUF_DEFERRED]) || !mul_ok(items_cap, 4, &sizes[RG_BUF_ARRIVE]) ||
        !mul_ok(item_bytes, 2, &sizes[RG_BUF_PAIRS]) ||
        !mul_ok(rg::tree_group_rows(items_cap), (int64_t)d * 8, &sizes[RG_BUF_FINAL_PAIRS]))
      return fail(RG_E_INVALID, "fused softmax workspace bytes overflow");
    // The work ticket counter counts tickets in 32 bits (the high half
    // counts deferred chunks): items, segments and the wave-class batches
    // stay far below 2^32.
    if (b + items_cap > ((int64_t)1 << 31))
      return fail(RG_E_INVALID, "register-resident softmax: more than 2^31 segments and chunks in one call; run this "
                                "input through the naive program");
    // A merge folds a segment's pairs through one buffer resource, whose
    // offsets are 32-bit: the whole pair table stays below 2 GiB.
    if (sizes[RG_BUF_PAIRS] > INT32_MAX)
      return fail(RG_E_INVALID, "register-resident softmax: the pair table of this plan exceeds 2 GiB "
                                "(items_cap x feature_dim x 8 bytes); run this input through the naive program");
  }
  plan->fused = module->fused ? 1 : 0;
  if (spec.debug_visits && !mul_ok(b, 4, &sizes[RG_BUF_VISITS])) return fail(RG_E_INVALID, "visits bytes overflow");
  // The counters at offset 0 of every plan, then the register-resident
  // softmax's arena -- the slots that hold zero between its calls (pairs,
  // group rows, arrival and reader counters, deferred list) -- at one offset
  // for every plan, then the rest, each 256-byte aligned.
  static const int kOrder[RG_WORKSPACE_BUFFERS] = {
      RG_BUF_COUNTERS, RG_BUF_PAIRS, RG_BUF_FINAL_PAIRS, RG_BUF_ARRIVE, RG_BUF_DEFERRED, RG_BUF_QUEUE,
      RG_BUF_ITEM_POS, RG_BUF_PART_BEGIN, RG_BUF_PARTIALS, RG_BUF_PARTIAL_SUMS, RG_BUF_STATS_MAX,
      RG_BUF_STATS_SUM, RG_BUF_VISITS, RG_BUF_SEG_ARRIVE, RG_BUF_ITEMS, RG_BUF_BLOCK_ITEMS};
  int64_t end = 0;
  for (int k = 0; k < RG_WORKSPACE_BUFFERS; ++k) {
    const int i = kOrder[k];
    const int64_t offset = (end + (int64_t)kAlign - 1) / (int64_t)kAlign * (int64_t)kAlign;
    plan->buffer_offset[i] = (uint64_t)offset;
    plan->buffer_bytes[i] = (uint64_t)sizes[i];
    if (!add_ok(offset, sizes[i], &end)) return fail(RG_E_INVALID, "workspace bytes overflow signed i64");
  }
  plan->workspace_bytes = (uint64_t)((end + (int64_t)kAlign - 1) / (int64_t)kAlign * (int64_t)kAlign);

  const int classify_block = b >= rg::kClassifyLarge ? rg::kClassifyBlock : rg::kBlock;
  int64_t classify_grid = (b + classify_block - 1) / classify_block;
  if (module->fused) {
    // k_classify also zeroes what the workspace's last call left nonzero in
    // the register-resident softmax's arena (about a third of the arena in
    // a call over long segments): workgroups for 64 KiB of it each, at most
    // 1024, beyond the segments' own.
    const int64_t arena = (int64_t)(arena_end(plan) - plan->buffer_offset[RG_BUF_PAIRS]);
    classify_grid = std::max(classify_grid, std::min<int64_t>(1024, (arena + 65535) / 65536));
  }
  add_launch(RG_ROLE_CLASSIFY, classify_grid, 1, classify_block);
  if (module->fused) {
    // The block and split classes held in registers, then the wave class in
    // the streaming worker's batches and the deferred chunks, in one
    // persistent launch: one resident wave of workgroups (the waits assume
    // the grid is co-resident), fewer when there is less work.
    add_launch(RG_ROLE_FUSED, std::min(module->resident[RG_ROLE_FUSED], std::max<int64_t>(1, b + items_cap)), 1);
    return RG_OK;
  }
  // One persistent worker drains the wave, block and split queues (as many
  // workgroups as are resident, fewer when there is less work: a ticket is
  // a split part, a block segment or a batch of wave segments).
  const int64_t tickets = items_cap * tiles_block + b;
  add_launch(RG_ROLE_WORKER, std::min(module->resident[RG_ROLE_WORKER], std::max<int64_t>(tickets, 1)), 1);
  return RG_OK;
}

}  // extern "C"

// Enqueue `plan` with `workspace` (rg_run, rg_run_static). `profiled`: the
// call may record HIP events (rg_profile_start), which creates them; the
// allocation-free entry point passes false.
static int enqueue(const char* entry, const rg_module* module, const rg_plan* plan, const void* values,
                   const void* offsets, void* out, const float* mask, void* workspace, uint64_t workspace_bytes,
                   void* stream, bool profiled, int* launched = nullptr, int stop_after = -1) {
  if (launched) *launched = 0;
  if (!module || !plan) return fail(RG_E_INVALID, "%s: null module or plan", entry);
  const rg_spec& spec = module->spec;
  if ((mask != nullptr) != (spec.has_mask != 0)) return fail(RG_E_INVALID, "mask presence must match the module");
  if (plan->launches == 0) return RG_OK;
  // N = 0 leaves values (and a softmax output) empty, possibly null.
  if (!offsets || (plan->n > 0 && (!values || !out)) || (spec.op != RG_OP_SOFTMAX && !out))
    return fail(RG_E_INVALID, "%s: null tensor pointer", entry);
  if (plan->workspace_bytes && (!workspace || workspace_bytes < plan->workspace_bytes))
    return fail(RG_E_WORKSPACE, "workspace of %llu bytes is smaller than the plan's %llu",
                (unsigned long long)workspace_bytes, (unsigned long long)plan->workspace_bytes);
  if (plan->workspace_bytes && ((uintptr_t)workspace & (kAlign - 1)) != 0)
    return fail(RG_E_WORKSPACE, "workspace must be %llu-byte aligned", (unsigned long long)kAlign);
  rg::Params p;
  std::memset(&p, 0, sizeof p);
  p.values = values;
  p.offsets = offsets;
  p.out = out;
  p.mask = mask;
  p.n = plan->n;
  p.b = plan->b;
  p.d = spec.feature_dim;
  p.scale = spec.scale;
  p.has_scale = spec.scale != 1.0f;
  p.t_wave = plan->t_wave;
  p.t_block = plan->t_block;
  p.part_rows = plan->part_rows;
  p.items_cap = plan->items_cap;
  p.b_split = plan->b_split;
  p.min_len = -1;
  p.max_len = -1;
  char* base = static_cast<char*>(workspace);
  auto buffer = [&](int index) -> void* {
    return plan->buffer_bytes[index] ? base + plan->buffer_offset[index] : nullptr;
  };
  p.short_segments = plan->schedule == RG_SHORT_SEGMENTS ? 1 : 0;
  p.alone_rows = spec.alone_rows;
  if (plan->schedule == RG_CLASSIFIED) {
    p.drain_ticks = module->drain_ticks;
    p.counters = static_cast<int64_t*>(buffer(RG_BUF_COUNTERS));
    p.queue = static_cast<int64_t*>(buffer(RG_BUF_QUEUE));
    p.item_pos = static_cast<int64_t*>(buffer(RG_BUF_ITEM_POS));
    p.part_begin = static_cast<int64_t*>(buffer(RG_BUF_PART_BEGIN));
    p.partials = static_cast<float*>(buffer(RG_BUF_PARTIALS));
    p.partial_sums = static_cast<float*>(buffer(RG_BUF_PARTIAL_SUMS));
    p.stats_max = static_cast<float*>(buffer(RG_BUF_STATS_MAX));
    p.stats_sum = static_cast<float*>(buffer(RG_BUF_STATS_SUM));
    p.visits = static_cast<int32_t*>(buffer(RG_BUF_VISITS));
    p.deferred = static_cast<int64_t*>(buffer(RG_BUF_DEFERRED));
    p.arrive = static_cast<int32_t*>(buffer(RG_BUF_ARRIVE));
    p.seg_arrive = static_cast<int32_t*>(buffer(RG_BUF_SEG_ARRIVE));
    p.items = static_cast<rg::Item*>(buffer(RG_BUF_ITEMS));
    p.block_items = static_cast<rg::Item*>(buffer(RG_BUF_BLOCK_ITEMS));
    p.pairs = static_cast<uint64_t*>(buffer(RG_BUF_PAIRS));
    p.final_pairs = static_cast<uint64_t*>(buffer(RG_BUF_FINAL_PAIRS));
    // A segment waits only if the grid can hold all its chunks at once; a
    // margin of 1/8 covers workgroups that are slow to become resident.
    p.wait_parts = std::max<int64_t>(1, module->resident[RG_ROLE_FUSED] * 7 / 8);
    p.spin_ticks = module->spin_ticks;
    p.fold_ticks = module->fold_ticks;
    if (plan->fused) {
      // The arena: from the pair table to the end of the deferred list.
      const uint64_t first = plan->buffer_offset[RG_BUF_PAIRS];
      p.arena = static_cast<unsigned char*>(workspace) + first;
      p.arena_bytes = (int64_t)(arena_end(plan) - first);
    }
    p.trace = module->trace;
    p.trace_cap = module->trace_cap;
  }
  int previous = 0;
  hipError_t err = hipGetDevice(&previous);
  if (err == hipSuccess && previous != module->device) err = hipSetDevice(module->device);
  if (err != hipSuccess) return hip_fail(err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Profile& profile = module->profile;
  const bool record = profiled && profile.active && (int)profile.call_first.size() < profile.max_calls;
  auto mark = [&]() {
    hipEvent_t event;
    if (err == hipSuccess) err = hipEventCreate(&event);
    if (err == hipSuccess) {
      profile.events.push_back(event);
      err = hipEventRecord(event, s);
    }
  };
  if (record) {
    profile.call_first.push_back((int)profile.events.size());
    profile.call_launches.push_back(plan->launches);
    for (int i = 0; i < plan->launches; ++i) profile.call_roles.push_back(plan->roles[i]);
  }
  for (int i = 0; i < plan->launches && err == hipSuccess; ++i) {
    const void* fn = module->roles[plan->roles[i]];
    if (!fn) {
      err = hipErrorInvalidDeviceFunction;
      break;
    }
    if (stop_after >= 0 && i >= stop_after) {
      if (previous != module->device) (void)hipSetDevice(previous);
      return fail(RG_E_DEVICE, "%s: interrupted after %d launches (test control)", entry, i);
    }
    if (record) mark();
    p.tiles = (int32_t)plan->grid[i][1];
    void* args[] = {&p};
    if (err == hipSuccess)
      err = hipLaunchKernel(fn, dim3(plan->grid[i][0], plan->grid[i][1], plan->grid[i][2]), dim3(plan->block[i]),
                            args, 0, s);
    if (err == hipSuccess && launched) ++*launched;
  }
  if (record) mark();
  if (previous != module->device) (void)hipSetDevice(previous);
  if (err != hipSuccess) return hip_fail(err, "hipLaunchKernel");
  return RG_OK;
}

extern "C" {

int rg_run(const rg_module* module, const rg_plan* plan, const void* values, const void* offsets, void* out,
           const float* mask, void* workspace, uint64_t workspace_bytes, void* stream) {
  return enqueue("rg_run", module, plan, values, offsets, out, mask, workspace, workspace_bytes, stream, true);
}

int rg_run_static(const rg_module* module, const rg_plan* plan, const void* values, const void* offsets, void* out,
                  const float* mask, void* stream) {
  if (!module || !plan) return fail(RG_E_INVALID, "rg_run_static: null module or plan");
  if (module->spec.debug_visits)
    return fail(RG_E_INVALID, "rg_run_static: a debug_visits module keeps its counters after a call; use rg_run "
                              "with a zeroed workspace per call");
  if (plan->workspace_bytes > kStaticScratchBytes)
    return fail(RG_E_WORKSPACE,
                "rg_run_static: the plan needs %llu bytes of workspace; the static workspace holds at most %llu "
                "(use rg_run with a caller-allocated workspace)",
                (unsigned long long)plan->workspace_bytes, (unsigned long long)kStaticScratchBytes);
  bool dirty = false;
  void* base = static_scratch(module->device, &dirty);
  if (!base) return fail(RG_E_DEVICE, "rg_run_static: no static workspace address for device %d", module->device);
  if (dirty && plan->workspace_bytes) {
    // An earlier call failed part way: its counters back to zero first.
    int previous = 0;
    hipError_t err = hipGetDevice(&previous);
    if (err == hipSuccess && previous != module->device) err = hipSetDevice(module->device);
    if (err != hipSuccess) return hip_fail(err, "hipSetDevice");
    rg::Params p;
    std::memset(&p, 0, sizeof p);
    p.counters = static_cast<int64_t*>(base);
    void* args[] = {&p};
    err = hipLaunchKernel(rg::kernel_reset(), dim3(1), dim3(rg::kBlock), args, 0, static_cast<hipStream_t>(stream));
    if (previous != module->device) (void)hipSetDevice(previous);
    if (err != hipSuccess) return hip_fail(err, "rg_run_static: static workspace reset");
    set_scratch_dirty(module->device, false);
  }
  int launched = 0;
  int stop_after = -1;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    std::swap(stop_after, g_interrupt_after);
  }
  const int status = enqueue("rg_run_static", module, plan, values, offsets, out, mask,
                             plan->workspace_bytes ? base : nullptr, plan->workspace_bytes, stream, false, &launched,
                             stop_after);
  if (status != RG_OK && launched > 0) set_scratch_dirty(module->device, true);
  return status;
}

int rg_test_interrupt_static(int launches) {
  if (launches < -1 || launches >= RG_MAX_LAUNCHES)
    return fail(RG_E_INVALID, "rg_test_interrupt_static: launches must be -1 or in [0, %d)", RG_MAX_LAUNCHES);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  g_interrupt_after = launches;
  return RG_OK;
}

int rg_check_offsets(int device, int offsets_dtype, const void* offsets, int64_t n, int64_t b, int64_t min_len,
                     int64_t max_len, int64_t* status, void* stream) {
  if (!offsets || !status) return fail(RG_E_INVALID, "rg_check_offsets: null pointer");
  if (offsets_dtype != RG_I32 && offsets_dtype != RG_I64) return fail(RG_E_INVALID, "offsets dtype must be i32 or i64");
  if (n < 0 || b < 0 || b == kI64Max) return fail(RG_E_INVALID, "N and B must be nonnegative and B+1 representable");
  rg::Params p;
  std::memset(&p, 0, sizeof p);
  p.offsets = offsets;
  p.n = n;
  p.b = b;
  p.status = status;
  p.min_len = min_len;
  p.max_len = max_len;
  int previous = 0;
  hipError_t err = hipGetDevice(&previous);
  if (err == hipSuccess && previous != device) err = hipSetDevice(device);
  if (err != hipSuccess) return hip_fail(err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* args[] = {&p};
  err = hipLaunchKernel(rg::kernel_offsets_init(), dim3(1), dim3(rg::kBlock), args, 0, s);
  if (err == hipSuccess) {
    const int64_t blocks = (b + 1 + rg::kBlock - 1) / rg::kBlock;
    if (blocks > kGridMax) err = hipErrorInvalidValue;
    else err = hipLaunchKernel(rg::kernel_offsets_check(offsets_dtype), dim3((uint32_t)blocks), dim3(rg::kBlock), args, 0, s);
  }
  if (previous != device) (void)hipSetDevice(previous);
  if (err != hipSuccess) return hip_fail(err, "offsets check launch");
  return RG_OK;
}

}  // extern "C"
