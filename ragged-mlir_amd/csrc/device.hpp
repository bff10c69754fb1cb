// Device building blocks for segmented sum / max / softmax on CDNA4 (gfx950).
//
// Data layout: values is a packed row-major [N, D] array of f32 or bf16,
// offsets is [B+1] i32/i64, out is [B, D] (sum, max) or [N, D] (softmax).
// Reductions run along N per feature column in f32.
//
// Thread mapping. Every access is a vector of VEC adjacent elements (16 B
// when the row allows it). Two mappings exist:
//  * ROW  (VEC divides D): a row is read by LPR lanes (LPR = next power of
//    two of D/VEC, capped by the group size G); the group covers G/LPR rows
//    per step and lane (row_lane, feat_lane) owns features
//    (tile*LPR + feat_lane)*VEC .. +VEC.
//  * FLAT (D < VEC, D divides VEC): a segment's rows are a contiguous run of
//    L*D elements, so the group reads it as a flat array of 16 B vectors,
//    masking the partial vectors at either end. Component c of every vector
//    belongs to feature c % D, so D=1 and D=2 still use full 16 B loads.
// Reductions across lanes use xor butterflies within a wave64 and LDS only
// across the waves of a workgroup.
//
// Numerics follow the reference's docs/semantics.md: f32 accumulation, sum
// with per-lane compensated (Kahan) addition whose correction is cleared
// when the total is not finite (ToGPU.cpp:377-387), max with IEEE maximum
// (NaN propagates: v_maximum3_f32), softmax as exp(x - max) / sum with
// -inf entries carrying zero mass and NaN / +inf / all -inf columns NaN.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace rg {

enum : int { OP_SUM = 0, OP_MAX = 1, OP_SOFTMAX = 2 };

constexpr int kWave = 64;
constexpr int kBlock = 256;            // threads of every workgroup-level worker
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kUnroll = 4;             // rows (or flat vectors) loaded per lane before folding
constexpr int kCombineFeatures = 64;   // consecutive features per split-combine pass
constexpr int kLaneElems = 64;         // classified worker: flat elements one lane reduces alone
constexpr int kGroupRows = 32;         // classified worker: rows one lane group walks alone
// The classified worker's work tickets come from kTicketLanes counters,
// kTicketStride i64 (256 bytes) apart, after the first kTicketStride slots
// (the class counts and the other per-call counters):
// atomics on one address serialise at about 12.5 ns each on MI355X, on 16
// addresses at about 1 ns per ticket.
constexpr int kTicketLanes = 16;
// k_classify reserves queue runs with one atomic per class per workgroup,
// and those atomics serialise: from kClassifyLarge segments on it runs
// kClassifyBlock-thread workgroups (fewer atomics), below that kBlock ones
// (more workgroups for the per-segment descriptor writes).
constexpr int kClassifyBlock = 1024;
constexpr int kClassifyWaves = kClassifyBlock / kWave;
constexpr int64_t kClassifyLarge = 16384;
constexpr int kTicketStride = 32;
constexpr int kDirect = 16;            // register-resident softmax: chunks merged by all-read
constexpr int kTreeGroup = 16;         // register-resident softmax: chunks per first-level tree group
constexpr int kGroupRowSlot = 10;      // counters slot: final_pairs rows reserved by tree-merged segments
constexpr int kDoneSlot = 11;          // counters slot: workgroups of the call's last kernel finished
// counters slot: the state of the register-resident softmax's arena (the
// slots its merges poll, which must hold zero while unpublished): 0 = the
// workspace is as allocated (all zero); 1 = not known to be zero (another
// plan's buffers overlap it); v >= 2 = its first v - 2 bytes are zero but for
// the kDirtyRanges byte ranges at slots kDirtySlot.. (the pairs and group
// rows the last call published). The call's last workgroup sets them
// (reset_counters); k_classify zeroes what a plan's arena needs.
constexpr int kCleanSlot = 12;
constexpr int kDrainSlot = 13;         // counters slot: deferred chunks claimed by the register-resident softmax's drain
constexpr int kDirtySlot = 14;         // counters slots 14-19: [begin, end) byte ranges of the arena left nonzero
constexpr int kDirtyRanges = 3;
constexpr int kDirectDone = 64;        // up to this many active workgroups count out on kDoneSlot alone
constexpr int32_t kStatsReady = -1;     // seg_arrive[k] once a split segment's softmax statistics are published

// Rows of final_pairs (register-resident softmax): one per first-level group
// of every segment merged by tree. Such a segment has more than kDirect of
// the items_cap chunks, so there are at most items_cap / (kDirect + 1) of
// them and items_cap / kTreeGroup + that many groups.
__host__ __device__ constexpr int64_t tree_group_rows(int64_t items_cap) {
  return items_cap / kTreeGroup + items_cap / (kDirect + 1) + 1;
}

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }
__device__ __forceinline__ float pos_inf() { return __builtin_inff(); }
// IEEE-754 maximum: NaN if either operand is NaN (v_maximum3_f32 on gfx950).
__device__ __forceinline__ float fmax_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fast_exp(float x) { return __expf(x); }
// exp(x) to 1.25 ulp (measured on MI355X over [-104, 89]) in eight
// instructions, one of them transcendental: the product x log2(e) is split
// exactly with fused multiply-adds (p + d, p the f32 product with log2(e)
// rounded to f32, d the rounding error plus x times the rest of log2(e)),
// then 2^(p + d) = 2^p (1 + d ln 2), exact to far below an ulp as |d| <
// 2^-16. __expf rounds x log2(e) to f32 first: 16 ulp at x = -20. ±inf
// and NaN arguments give 2^p itself (0, inf, NaN).
constexpr float kLog2eHi = 1.44269502162933349609375f;   // log2(e) rounded to f32
constexpr float kLog2eLo = 1.925962989091090e-8f;        // log2(e) - kLog2eHi
constexpr float kLn2 = 0.693147180559945309f;
__device__ __forceinline__ float exp_split(float x) {
  const float p = x * kLog2eHi;
  const float lo = __builtin_fmaf(x, kLog2eHi, -p);
  const float d = __builtin_fmaf(x, kLog2eLo, lo);
  const float r = __builtin_amdgcn_exp2f(p);
  const float y = __builtin_fmaf(r, d * kLn2, r);
  return __builtin_isfinite(p) ? y : r;
}

// exp of a softmax output (and of what scales one) for data of type T: f32
// outputs take exp_split, bf16 outputs the fast form, far below their
// rounding.
template <class T>
__device__ __forceinline__ float exp_out(float x) {
  if constexpr (std::is_same<T, float>::value) return exp_split(x);
  else return __expf(x);
}
// exp(x - ref) over rows of type T that share a column reference ref: bf16
// rows as 2^(x log2(e) - ref log2(e)), one FMA into v_exp_f32 with
// shift = -ref log2(e) computed once per column (the error of the rounded
// shift, below 2^-24 |ref| log2(e) in the exponent, is far below a bf16
// ulp); f32 rows through exp_split(x - ref). ±inf and NaN follow x - ref:
// inf - inf and NaN give NaN, x - inf gives 0.
template <class T>
struct ExpShift {
  float ref = 0.f, shift = 0.f;
  ExpShift() = default;
  __device__ explicit ExpShift(float r) : ref(r), shift(-r * kLog2eHi) {}
  __device__ float operator()(float x) const {
    if constexpr (std::is_same<T, float>::value) return exp_split(x - ref);
    else return __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2eHi, shift));
  }
};

// The softmax output y = exp(x - M) / S of one column with statistics
// (M, S), rounded once to T. bf16 outputs: y = 2^(x log2(e) - c) with
// c = M log2(e) + log2(S), one FMA into v_exp_f32 per element (c is rounded
// once per column; its error, below 2^-24 |c| in the exponent, is far below
// a bf16 ulp), so no intermediate value can underflow before the output does.
// f32 outputs: exp_split(x - M) * (1 / S), the reference's exp(x - m) / s
// (ToGPU.cpp:712-733) with the division as a rounded reciprocal. Special
// columns follow IEEE arithmetic: M = -inf (only -inf, S = 0), NaN M or S
// give NaN everywhere; x = -inf in a finite column gives 0.
template <class T>
struct Normalizer {
  float a = 0.f, b = 0.f;   // bf16: a = -c; f32: a = M, b = 1 / S
  Normalizer() = default;
  __device__ Normalizer(float a_, float b_) : a(a_), b(b_) {}
  __device__ static Normalizer of(float m, float s) {
    if constexpr (std::is_same<T, float>::value) return Normalizer(m, 1.0f / s);
    else return Normalizer(-__builtin_fmaf(m, kLog2eHi, __builtin_amdgcn_logf(s)), 0.f);
  }
  __device__ float operator()(float x) const {
    if constexpr (std::is_same<T, float>::value) return exp_split(x - a) * b;
    else return __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2eHi, a));
  }
};

// Workgroup-wide OR of `x` for the kBlock-thread workgroups of every kernel
// here: one ballot per wave, one LDS flag per wave, two barriers. HIP's
// __syncthreads_or reads the workgroup size from the dispatch packet first
// (three 16-bit global loads and a wait for them), a full memory round trip
// per call that lands on the critical path of every poll of a waiting chunk.
// Every thread of the workgroup must call it (it contains barriers).
__device__ __forceinline__ bool block_any(bool x) {
  __shared__ int any_s[kWavesPerBlock];
  const bool wave_any = __ballot(x) != 0;
  if ((threadIdx.x & (kWave - 1)) == 0) any_s[threadIdx.x / kWave] = wave_any ? 1 : 0;
  __syncthreads();
  int any = 0;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) any |= any_s[w];
  // No wave may overwrite its flag (next call) before every wave has read it.
  __syncthreads();
  return any != 0;
}

// One work item of the register-resident softmax: a whole segment (k < 0)
// or chunk c of `parts` of a long segment at split-queue position k.
struct Item {
  int64_t start;   // first row
  int64_t seg;     // original segment id
  int32_t rows;    // rows of the item
  int32_t k;       // split-queue position (a tree-merged chunk: its segment's first final_pairs row), -1 for a whole segment
  int32_t c;       // chunk index within the segment
  int32_t parts;   // chunks of the segment
};

// Everything a kernel needs, passed by value as the single kernel argument.
struct Params {
  const void* values;      // [N, D] f32 | bf16
  const void* offsets;     // [B+1] i32 | i64
  void* out;               // [B, D] or [N, D]
  const float* mask;       // [N, D] f32 or null
  int64_t n, b;
  int32_t d;
  float scale;
  int32_t has_scale;
  int32_t tiles;           // feature tiles of this launch (grid.y)
  int64_t t_wave;          // longest segment of the wave class (rows)
  int64_t t_block;         // longest segment of the block class (rows)
  int64_t part_rows;       // rows per split part
  int64_t items_cap;       // capacity of the split item tables
  int64_t b_split;         // capacity of the split queue / statistics rows
  int64_t* counters;       // slots 0-13: wave (reduced alone), block, split segment
                           //      counts; split items; work ticket; deferred
                           //      chunks (register-resident softmax) or split
                           //      parts (worker softmax); tree items; the wave
                           //      count of a register-resident softmax; the rest
                           //      of the wave class; the split-part normalisation
                           //      ticket; final_pairs rows reserved; done lanes
                           //      finished; the arena's clean extent; deferred
                           //      chunks claimed. Then the worker's ticket lanes
                           //      and the done lanes (kTicketStride apart)
  int64_t* queue;          // [3, B] original segment ids per class
  int64_t* item_pos;       // [items_cap] split-queue position of each item
  int64_t* part_begin;     // [B] first item of each split-queue position
  float* partials;         // [items_cap, D] part result / part softmax reference
  float* partial_sums;     // [items_cap, D] part softmax mass
  float* stats_max;        // [B_split, D] combined softmax reference
  float* stats_sum;        // [B_split, D] combined softmax mass
  int32_t* visits;         // [B] or null (debug)
  int64_t* deferred;       // [items_cap] 1 + item of each chunk left to the drain, 0 while unwritten
                           // (register-resident softmax); [items_cap * tiles] split parts left
                           // to the last workgroup (worker softmax)
  int32_t* arrive;         // [items_cap] register-resident softmax: a tree group's chunk arrivals
                           // (at the group's first item); a segment's readers of its merged
                           // statistics (first item of a direct segment, second of a tree one)
  int32_t* seg_arrive;     // [B_split] part arrivals per split segment (worker)
  Item* items;             // [items_cap] split chunks (register-resident softmax)
  Item* block_items;       // [B] whole segments (register-resident softmax)
  uint64_t* pairs;         // [items_cap, D] published (m, s) of each chunk
  uint64_t* final_pairs;   // [tree_group_rows(items_cap), D] (M, S) of each group of a tree-merged segment
  int64_t spin_ticks;      // wall-clock ticks a chunk waits for its segment before deferring
  int64_t drain_ticks;     // wall-clock bound of a split part's (a deferred chunk's) wait for its segment's statistics
  int64_t fold_ticks;      // wall-clock bound of a fold whose every input is published before it starts
  unsigned char* arena;    // register-resident softmax: pairs, final_pairs, arrive and deferred, contiguous
  int64_t arena_bytes;     // their bytes (a multiple of 256), 0 for every other plan
  int64_t wait_parts;      // longest segment (in chunks) whose chunks wait for each other
  int64_t* trace;          // [trace_cap, 8] item timeline or null (diagnostics)
  int64_t trace_cap;
  int64_t* status;         // [7] checked-offsets status
  int64_t min_len, max_len;  // checked-offsets hints, -1 when absent
  int32_t short_segments;  // worker: every segment in order as wave class (no queues)
  int64_t alone_rows;      // wave-class segments a lane / lane group reduces alone
};

// ---------------------------------------------------------------------------
// Element access: VEC elements of T as f32.

template <class T> struct Elem;

template <> struct Elem<float> {
  static constexpr int kBytes = 4;
  __device__ static float get(const float* p) { return *p; }
  __device__ static void put(float* p, float v) { *p = v; }
  template <int V>
  __device__ static void load(const float* p, float (&x)[V]) {
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "unsupported vector width");
    if constexpr (V == 8) {
      float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else if constexpr (V == 4) {
      float4 r = *reinterpret_cast<const float4*>(p);
      x[0] = r.x; x[1] = r.y; x[2] = r.z; x[3] = r.w;
    } else if constexpr (V == 2) {
      float2 r = *reinterpret_cast<const float2*>(p);
      x[0] = r.x; x[1] = r.y;
    } else {
      x[0] = *p;
    }
  }
  template <int V>
  __device__ static void store(float* p, const float (&x)[V]) {
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "unsupported vector width");
    if constexpr (V == 8) {
      *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
      *reinterpret_cast<float4*>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
    } else if constexpr (V == 4) {
      *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    } else if constexpr (V == 2) {
      *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
    } else {
      *p = x[0];
    }
  }
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// Round-to-nearest-even f32 -> bf16 pair in one v_cvt_pk_bf16_f32; NaN stays NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2_t pair = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(pair, bf16x2_t));
}

template <> struct Elem<__bf16> {
  static constexpr int kBytes = 2;
  __device__ static float get(const __bf16* p) {
    return __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
  }
  __device__ static void put(__bf16* p, float v) { *p = (__bf16)v; }
  template <int V>
  __device__ static void load(const __bf16* p, float (&x)[V]) {
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "unsupported vector width");
    if constexpr (V == 8) {
      uint4 r = *reinterpret_cast<const uint4*>(p);
      x[0] = bf16_lo(r.x); x[1] = bf16_hi(r.x); x[2] = bf16_lo(r.y); x[3] = bf16_hi(r.y);
      x[4] = bf16_lo(r.z); x[5] = bf16_hi(r.z); x[6] = bf16_lo(r.w); x[7] = bf16_hi(r.w);
    } else if constexpr (V == 4) {
      uint2 r = *reinterpret_cast<const uint2*>(p);
      x[0] = bf16_lo(r.x); x[1] = bf16_hi(r.x); x[2] = bf16_lo(r.y); x[3] = bf16_hi(r.y);
    } else if constexpr (V == 2) {
      uint32_t r = *reinterpret_cast<const uint32_t*>(p);
      x[0] = bf16_lo(r); x[1] = bf16_hi(r);
    } else {
      x[0] = get(p);
    }
  }
  template <int V>
  __device__ static void store(__bf16* p, const float (&x)[V]) {
    if constexpr (V == 8) {
      *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]),
                                                pack_bf16(x[4], x[5]), pack_bf16(x[6], x[7]));
    } else if constexpr (V == 4) {
      *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]));
    } else if constexpr (V == 2) {
      *reinterpret_cast<uint32_t*>(p) = pack_bf16(x[0], x[1]);
    } else {
      put(p, x[0]);
    }
  }
};

template <int V>
__device__ __forceinline__ void load_mask(const float* p, float (&x)[V]) {
  Elem<float>::load<V>(p, x);
}

template <class OffT>
__device__ __forceinline__ int64_t offset_at(const Params& p, int64_t i) {
  return (int64_t)static_cast<const OffT*>(p.offsets)[i];
}

// ---------------------------------------------------------------------------
// Per-feature accumulation state.

template <int OP> struct State;

// Compensated sum (ToGPU.cpp:377-387): the correction is cleared whenever the
// running total is not finite, so inf and NaN propagate unchanged.
template <> struct State<OP_SUM> {
  float s, c;
  __device__ void init() { s = 0.f; c = 0.f; }
  __device__ void fold(float x) {
    float y = x - c;
    float t = s + y;
    float e = (t - s) - y;
    c = __builtin_fabsf(t) < pos_inf() ? e : 0.f;
    s = t;
  }
  __device__ float total() const { return s; }
  __device__ void merge(const State& o) { s = s + o.s; c = 0.f; }
  static constexpr float kIdentity = 0.f;
};

template <> struct State<OP_MAX> {
  float m;
  __device__ void init() { m = neg_inf(); }
  __device__ void fold(float x) { m = fmax_nan(m, x); }
  __device__ void merge(const State& o) { m = fmax_nan(m, o.m); }
};

// Softmax statistics: reference m and mass s = sum exp(x - m).
// -inf entries carry no mass. NaN (IEEE maximum) or +inf (inf - inf) make s
// NaN, which poisons the whole column as the contract requires.
template <> struct State<OP_SOFTMAX> {
  float m, s;
  __device__ void init() { m = neg_inf(); s = 0.f; }
  __device__ void fold(float x) {
    float mn = fmax_nan(m, x);
    float next = s * fast_exp(m - mn) + fast_exp(x - mn);
    s = mn == neg_inf() ? s : next;
    m = mn;
  }
  __device__ static float rescaled(float m, float s, float to) {
    return m == neg_inf() ? s : s * fast_exp(m - to);
  }
  __device__ void merge(const State& o) {
    float mn = fmax_nan(m, o.m);
    s = rescaled(m, s, mn) + rescaled(o.m, o.s, mn);
    m = mn;
  }
};

template <int OP, int V>
__device__ __forceinline__ void init_all(State<OP> (&st)[V]) {
#pragma unroll
  for (int v = 0; v < V; ++v) st[v].init();
}

// ---------------------------------------------------------------------------
// Cross-lane combination.

// The value of lane (lane ^ MASK), MASK a power of two below 64, through
// gfx950's lane-crossing operations instead of ds_bpermute (an LDS-crossbar
// access with a per-lane address): DPP quad permutes for 1 and 2, a
// ds_swizzle bit-mode exchange for 4, DPP row_ror:8 for 8 (a rotation by
// half a 16-lane row is the xor), and v_permlane16_swap / v_permlane32_swap
// for 16 and 32 (each swap returns both halves; a lane takes its partner's).
// Every mask is the exact xor exchange, so reductions built on it associate
// as an xor butterfly and every lane of a group ends with the same bits.
template <int MASK>
__device__ __forceinline__ float xor_lane(float v) {
  static_assert(MASK > 0 && MASK < 64 && (MASK & (MASK - 1)) == 0, "mask must be a power of two below 64");
  const int x = __float_as_int(v);
  if constexpr (MASK == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
  if constexpr (MASK == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
  if constexpr (MASK == 4) return __int_as_float(__builtin_amdgcn_ds_swizzle(x, (4 << 10) | 0x1F));   // and 0x1F, xor 4
  if constexpr (MASK == 8) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
  if constexpr (MASK == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return __int_as_float((int)((threadIdx.x & 16) ? r[0] : r[1]));
  }
  if constexpr (MASK == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return __int_as_float((int)((threadIdx.x & 32) ? r[0] : r[1]));
  }
}

// Butterfly over the lanes whose index agrees modulo `stride` (a uniform
// power of two): fn(mask-level callable) is applied at every compile-time
// mask from stride to 32, each step behind one uniform branch.
template <class Step>
__device__ __forceinline__ void xor_butterfly(int stride, Step&& step) {
  if (stride <= 1) step(std::integral_constant<int, 1>{});
  if (stride <= 2) step(std::integral_constant<int, 2>{});
  if (stride <= 4) step(std::integral_constant<int, 4>{});
  if (stride <= 8) step(std::integral_constant<int, 8>{});
  if (stride <= 16) step(std::integral_constant<int, 16>{});
  if (stride <= 32) step(std::integral_constant<int, 32>{});
}

// Lane `src`'s value (src wave-uniform) in every lane, through the scalar
// unit (v_readlane) instead of an LDS-crossbar broadcast.
__device__ __forceinline__ int64_t lane_value(int64_t v, int src) {
  const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, src);
  const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), src);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int lane_value(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

template <int MASK, int OP>
__device__ __forceinline__ State<OP> shfl_xor(const State<OP>& a) {
  State<OP> r;
  if constexpr (OP == OP_SUM) {
    r.s = xor_lane<MASK>(a.s);
    r.c = 0.f;
  } else if constexpr (OP == OP_MAX) {
    r.m = xor_lane<MASK>(a.m);
  } else {
    r.m = xor_lane<MASK>(a.m);
    r.s = xor_lane<MASK>(a.s);
  }
  return r;
}

// Combine lanes whose lane index agrees modulo `stride` (a power of two < 64):
// afterwards every lane holds the combination over its residue class.
template <int OP, int V>
__device__ __forceinline__ void wave_reduce_stride(State<OP> (&st)[V], int stride) {
  xor_butterfly(stride, [&](auto mask) {
#pragma unroll
    for (int v = 0; v < V; ++v) st[v].merge(shfl_xor<decltype(mask)::value, OP>(st[v]));
  });
}

template <int OP> struct Slots { static constexpr int kCount = OP == OP_SOFTMAX ? 2 : 1; };

template <int OP>
__device__ __forceinline__ void st_write(float* slot, int stride, const State<OP>& a) {
  if constexpr (OP == OP_SUM) { slot[0] = a.s; }
  else if constexpr (OP == OP_MAX) { slot[0] = a.m; }
  else { slot[0] = a.m; slot[stride] = a.s; }
}
template <int OP>
__device__ __forceinline__ State<OP> st_read(const float* slot, int stride) {
  State<OP> a;
  if constexpr (OP == OP_SUM) { a.s = slot[0]; a.c = 0.f; }
  else if constexpr (OP == OP_MAX) { a.m = slot[0]; }
  else { a.m = slot[0]; a.s = slot[stride]; }
  return a;
}

// ---------------------------------------------------------------------------
// Geometry of a group of G threads over a feature tile.

struct RowGeo {
  int lpr;          // lanes per row (power of two, <= G)
  int rows_step;    // rows covered per step = G / lpr
  int row_lane, feat_lane;
  int feature;      // first feature of this lane
  bool active;      // feature < D
};

// Lanes per row for D features read VEC at a time by a group of G threads.
__device__ __forceinline__ int lanes_per_row(int d, int vec, int g) {
  int lanes = (d + vec - 1) / vec;
  int p = 1;
  while (p < lanes && p < g) p <<= 1;
  return p;
}

template <int VEC>
__device__ __forceinline__ RowGeo row_geo(int d, int g, int t, int tile) {
  RowGeo geo;
  geo.lpr = lanes_per_row(d, VEC, g);
  geo.rows_step = g / geo.lpr;
  geo.row_lane = t / geo.lpr;
  geo.feat_lane = t % geo.lpr;
  geo.feature = (tile * geo.lpr + geo.feat_lane) * VEC;
  geo.active = geo.feature < d;
  return geo;
}

}  // namespace rg
