// Register-resident softmax: one persistent kernel over a dynamic queue of
// work items, each read from HBM once and written once.
//
// Items (descriptors written by k_classify): every chunk of every
// split-class segment (ceil(L / part_rows) chunks, contiguous in the queue),
// then every block-class segment. A 256-thread workgroup takes the next item
// with one atomic ticket (and prefetches the following descriptor while it
// finishes) and holds its rows in registers (RPT rows per thread), as loaded:
//   1. m = column max of the rows (IEEE maximum: NaN propagates);
//   2. s = column sum of exp(x - m);
//   3. whole segment: y = exp(x - m) / s from the held rows.  Chunk of a
//      longer segment: publish (m, s), get the segment's merged (M, S) and
//      write y = exp(x - M) / S from the held rows (Normalizer: every output
//      one rounding of an f32 value).
// Merging is deterministic (folds in chunk order). Up to kDirect chunks:
// every chunk reads all published pairs itself. Longer: the last chunk of
// each group of kGroup folds the group and publishes it, every chunk folds
// the group results, and those segments are dequeued first. A chunk waits
// for its segment with a bounded spin: since items are dequeued in order
// and a workgroup holds an unstarted ticket only when it cannot wait or all
// chunks of its segment are handed out, every chunk it waits for is started
// by a running workgroup whenever the device holds all chunks of the
// segment at once. Segments with more chunks than that (wait_parts), and
// chunks whose spin limit passes, skip the wait: they drop their registers
// and are re-read by the kernel's drain once every ticket is handed out. A
// wait for chunks not yet handed out also ends when the ticket counter
// stalls (fewer workgroups resident than the plan assumed: another process
// on the device). No wait is unbounded.
//
// After the items, the same tickets hand out the wave class in the
// streaming worker's batches (a ticket per short segment would serialise the
// kernel on its counter), then the workgroups drain the deferred chunks; the
// last workgroup out drains what is left and returns the counters to zero.
// One launch after k_classify does the whole call.
//
// Every slot a merge polls (pairs, group rows, group arrival counters, the
// deferred list: the arena) holds zero while unpublished, so a pair that is
// not yet visible is never taken for a published one. A workspace is zero
// when allocated; the call returns the counters and the deferred list to
// zero itself, and its last workgroup records the byte ranges of the pairs
// and group rows it published, which the next call's k_classify zeroes with
// many workgroups before this kernel starts (zeroing them here, by each
// segment's last reader, cost this kernel 3.5%).
//
// Reference semantics: docs/semantics.md (softmax row), the reference's
// online statistics and merge algebra (ToGPU.cpp:486-557, 435-472) restated
// as an exact two-pass over registers.
#pragma once

#include <type_traits>

#include "worker.hpp"

namespace rg {

constexpr int kGroup = kTreeGroup;   // chunks merged per first-level group
// Sleep between two polls of a waiting chunk, in units of 64 clocks (about
// 1.7 us at 64). A waiter's fold takes LDS, barriers and issue slots from
// the workgroups that share its CU; on MI355X, C5 runs 1.5-2% faster at 32
// to 127 than at 2. Polling feature 0 of each slot between folds (128x
// fewer bytes) was 8% slower: the extra round trip delays every wake-up.
constexpr int kPollSleep = 64;

// The work ticket counter (counters[4]) holds two counts: tickets handed out
// after the first round (low 32 bits) and chunks deferred to the drain (high
// 32 bits; a deferral adds 2^32 and takes its deferred-list slot from the old
// value). The first round of tickets is the workgroup index -- a thousand
// first fetches from one address would serialise the launch (~12.5 ns each:
// the last workgroup started 12 us late; C5's kernel 15 us faster without
// them) -- and a fetch returning k hands out ticket gridDim.x + k. Every
// ticket fetch also tells a workgroup how many chunks were deferred by then,
// and a workgroup that leaves having seen none -- the common case -- leaves
// without a further round trip. The plan keeps tickets below 2^32.
constexpr uint64_t kTicketMask = 0xffffffffull;
constexpr int kDeferShift = 32;

// Buffer addressing: a wave-uniform 128-bit resource (base in SGPRs) per
// chunk, covering exactly the chunk's bytes, and one per-thread byte offset
// plus a per-row stride. A row past the chunk is out of the resource's range:
// its load returns 0 (replaced by -inf before use) and its store is dropped
// by the hardware, so no load or store is predicated. Lanes without a
// feature (D below a power of two) get an offset that is always out of range.
using Rsrc = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;   // raw 32-bit data format (gfx9 family)

constexpr int kOutOfRange = 0x7ff00000;  // byte offset beyond any chunk resource

// Item descriptors are read through the constant address space: they are
// written by k_classify before this kernel starts and never during it, so
// the loads go through the scalar cache into SGPRs (no VGPRs held while a
// prefetch is in flight).
typedef __attribute__((address_space(4))) const Item ConstItem;
typedef __attribute__((address_space(4))) const int64_t ConstI64;

__device__ __forceinline__ Item load_item(ConstItem* item) {
  Item it;
  it.start = item->start;
  it.seg = item->seg;
  it.rows = item->rows;
  it.k = item->k;
  it.c = item->c;
  it.parts = item->parts;
  return it;
}

// A copy of a uniform flag the compiler cannot relate to other tests of the
// same flag: stops it from duplicating the code between two such tests.
__device__ __forceinline__ bool opaque(bool flag) {
  int v = __builtin_amdgcn_readfirstlane((int)flag);
  asm volatile("" : "+s"(v));
  return v != 0;
}

// A workgroup-uniform 64-bit value (from LDS) in SGPRs.
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ Rsrc make_rsrc(const void* base, int64_t bytes) {
  const int records = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, records, kRsrcWord3);
}

// Cache policy of the row loads and stores: nontemporal (the nt bit). Every
// row is read once and written once; on MI355X streaming them this way
// moves about 5% more bytes per second than the default policy (measured on
// a 1 GiB copy and on this kernel). The stores also carry sc1 (device
// scope): the output is written through rather than left dirty in the
// XCDs' L2 caches for the end-of-kernel writeback (C5: calls about 1% faster,
// five of five alternating rounds on two boxes; sc1 on the loads as well was
// neutral).
constexpr int kStreamAux = 2;
constexpr int kStoreAux = kStreamAux | 16;

// Load / store BYTES (2, 4, 8 or 16) as 32-bit words (2 bytes in the low half).
template <int BYTES>
__device__ __forceinline__ void buffer_load(Rsrc r, int voffset, int soffset, uint32_t* w) {
  static_assert(BYTES == 2 || BYTES == 4 || BYTES == 8 || BYTES == 16 || BYTES == 32, "unsupported width");
  if constexpr (BYTES == 32) {
    buffer_load<16>(r, voffset, soffset, w);
    buffer_load<16>(r, voffset + 16, soffset, w + 4);
  } else if constexpr (BYTES == 16) {
    auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, kStreamAux);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (BYTES == 8) {
    auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voffset, soffset, kStreamAux);
    w[0] = v[0]; w[1] = v[1];
  } else if constexpr (BYTES == 4) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, kStreamAux);
  } else {
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, voffset, soffset, kStreamAux);
  }
}

template <int BYTES>
__device__ __forceinline__ void buffer_store(Rsrc r, int voffset, int soffset, const uint32_t* w) {
  static_assert(BYTES == 2 || BYTES == 4 || BYTES == 8 || BYTES == 16, "unsupported width");
  if constexpr (BYTES == 16) {
    __attribute__((ext_vector_type(4))) unsigned v = {w[0], w[1], w[2], w[3]};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voffset, soffset, kStoreAux);
  } else if constexpr (BYTES == 8) {
    __attribute__((ext_vector_type(2))) unsigned v = {w[0], w[1]};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, voffset, soffset, kStoreAux);
  } else if constexpr (BYTES == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(w[0], r, voffset, soffset, kStoreAux);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)w[0], r, voffset, soffset, kStoreAux);
  }
}

// VEC elements of S as 32-bit words: unpack to f32 / pack from f32.
template <class S, int VEC> struct Words {
  static constexpr int kBytes = VEC * (int)sizeof(S);
  static constexpr int kCount = kBytes >= 4 ? kBytes / 4 : 1;
  __device__ static float get(const uint32_t* w, int i) {
    if constexpr (sizeof(S) == 4) return __uint_as_float(w[i]);
    else return (i & 1) ? bf16_hi(w[i >> 1]) : bf16_lo(w[i >> 1]);
  }
  __device__ static void set(uint32_t* w, const float (&x)[VEC]) {
    if constexpr (sizeof(S) == 4) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) w[i] = __float_as_uint(x[i]);
    } else if constexpr (VEC == 1) {
      w[0] = pack_bf16(x[0], 0.f) & 0xffffu;
    } else {
#pragma unroll
      for (int i = 0; i < kCount; ++i) w[i] = pack_bf16(x[2 * i], x[2 * i + 1]);
    }
  }
  // -inf in every element (identity of the column max, zero mass).
  __device__ static void fill_neg_inf(uint32_t* w) {
#pragma unroll
    for (int i = 0; i < kCount; ++i) w[i] = sizeof(S) == 4 ? 0xff800000u : 0xff80ff80u;
  }
};

// Column reduction over the lanes of a workgroup that share a feature lane
// (ROW mapping, lpr lanes per row): xor butterfly within each wave, then one
// LDS pass across the four waves. Every thread receives its features' total.
template <bool MAX, int VEC>
__device__ __forceinline__ void block_allreduce(float (&v)[VEC], int lpr, int feat_lane, float* lds) {
  const int t = threadIdx.x, lane = t & (kWave - 1), w = t / kWave;
  auto combine = [](float a, float b) { return MAX ? fmax_nan(a, b) : a + b; };
  xor_butterfly(lpr, [&](auto mask) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = combine(v[i], xor_lane<decltype(mask)::value>(v[i]));
  });
  const int rep = lpr < kWave ? lpr : kWave;
  if (lane < rep) {
    float* slot = lds + (w * kWave + lane) * VEC;
#pragma unroll
    for (int i = 0; i < VEC; ++i) slot[i] = v[i];
  }
  __syncthreads();
  if (lpr <= kWave) {
    // Every wave holds every feature lane: fold waves 0..3 in order, at
    // fixed offsets from one base address.
    const float* base = lds + feat_lane * VEC;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float acc = base[i];
#pragma unroll
      for (int ww = 1; ww < kWavesPerBlock; ++ww) acc = combine(acc, base[ww * kWave * VEC + i]);
      v[i] = acc;
    }
  } else {
    // A row spans lpr / 64 waves: feature lane fl lives in every
    // (lpr/64)-th wave starting at fl / 64.
    const int stride = lpr / kWave;
    // Opaque: keeps the compiler from precomputing (and spilling) these
    // addresses across the caller's loop for this rarely taken branch.
    int offset = ((feat_lane / kWave) * kWave + (feat_lane & (kWave - 1))) * VEC;
    asm volatile("" : "+v"(offset));
    const float* base = lds + offset;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float acc = base[i];
      for (int ww = feat_lane / kWave + stride; ww < kWavesPerBlock; ww += stride)
        acc = combine(acc, base[(ww - feat_lane / kWave) * kWave * VEC + i]);
      v[i] = acc;
    }
  }
  __syncthreads();
}

// Statistics shared between workgroups travel only through agent-scope
// atomic stores and loads (coherent across the XCDs' L2 caches), so no
// L2-wide writeback or invalidate is needed. Each (m, s) pair of a feature is
// one 64-bit store into a slot that holds zero until then: a published pair
// is never zero (a finite m comes with s >= 1, as the column's largest row
// contributes exp(0); m = -inf and NaN have nonzero bits), so a reader polls
// the data itself instead of a separate flag, and a pair that is not yet
// visible reads as unpublished, never as a stale value. A publisher that
// bumps a counter waits for its stores to complete (s_waitcnt vmcnt(0))
// before the barrier after which one thread updates the counter.
__device__ __forceinline__ uint64_t pack_pair(float m, float s) {
  return ((uint64_t)__float_as_uint(s) << 32) | __float_as_uint(m);
}
__device__ __forceinline__ float pair_m(uint64_t v) { return __uint_as_float((uint32_t)v); }
__device__ __forceinline__ float pair_s(uint64_t v) { return __uint_as_float((uint32_t)(v >> 32)); }
__device__ __forceinline__ bool pair_ready(uint64_t v) { return v != 0; }
__device__ __forceinline__ void store_pair(uint64_t* p, float m, float s) {
  __hip_atomic_store(p, pack_pair(m, s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait for this wave's outstanding vector memory operations (vmcnt = 0).
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Segments of at most kDirect chunks merge directly: every chunk reads all
// chunks' pairs. Longer ones fold groups of kGroup chunks (last arriver) and
// every chunk then folds the segment's group rows.
constexpr int kBatch = 8;            // pair loads in flight per thread

// Pair loads of a fold go through one wave-uniform resource over the slots
// it reads: the slot's byte offset is uniform (an SGPR), the feature's is
// per lane, so kBatch loads in flight hold only their results in VGPRs (64-bit
// per-lane addresses would take as many again, and the fused kernel, which
// holds its rows meanwhile, would spill). The cache policy is sc1, the
// agent-scope coherence of a relaxed atomic load on gfx950; every poll is
// separated from the next by a barrier (a fence), so the compiler cannot
// reuse an earlier load's value.
constexpr int kPairAux = 16;

__device__ __forceinline__ uint64_t load_pair_at(Rsrc r, int voffset, int soffset) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voffset, soffset, kPairAux);
  return ((uint64_t)v[1] << 32) | v[0];
}

// acc <- merge of (acc, part): the larger reference and the masses rescaled
// to it. ACCURATE (f32 outputs) rescales with exp_split (1.25 ulp), else with
// __expf, whose error (up to ~16 f32 ulp for large differences) is far
// below a bf16 output's rounding.
template <bool ACCURATE>
__device__ __forceinline__ void merge_stats(State<OP_SOFTMAX>& acc, const State<OP_SOFTMAX>& part) {
  if constexpr (!ACCURATE) {
    acc.merge(part);
  } else {
    const float mn = fmax_nan(acc.m, part.m);
    const float a = acc.m == neg_inf() ? acc.s : acc.s * exp_split(acc.m - mn);
    const float b = part.m == neg_inf() ? part.s : part.s * exp_split(part.m - mn);
    acc.s = a + b;
    acc.m = mn;
  }
}

// One thread's fold of `count` slots, slot_bytes apart, starting voff bytes
// into resource r, in slot order, kBatch loads at a time; ok turns false if
// a slot is still unpublished.
template <bool ACCURATE>
__device__ __forceinline__ State<OP_SOFTMAX> fold_range(Rsrc r, int voff, int count, int slot_bytes, bool& ok) {
  State<OP_SOFTMAX> acc;
  acc.init();
  for (int i0 = 0; i0 < count; i0 += kBatch) {
    uint64_t v[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) v[j] = i0 + j < count ? load_pair_at(r, voff, (i0 + j) * slot_bytes) : 0;
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      if (i0 + j < count) {
        ok = ok && pair_ready(v[j]);
        State<OP_SOFTMAX> part;
        part.m = pair_m(v[j]);
        part.s = pair_s(v[j]);
        merge_stats<ACCURATE>(acc, part);
      }
    }
  }
  return acc;
}

// Whole workgroup: fold `count` slots (stride apart) of every feature into
// (lds_m[f], lds_s[f]). R threads per feature (the largest power of two with
// R * d <= 256 and R <= count) fold R contiguous ranges of slots at once;
// the R range results are folded in range order through `stage` (R * d
// pairs). The association depends only on (count, d): deterministic. True,
// after a barrier, when every slot was published.
// The thread index through an opaque copy: values derived from it inside a
// persistent kernel's loop are recomputed where they are used (a few
// integer instructions) instead of being hoisted before the loop and kept
// in registers the held rows need, or spilled.
__device__ __forceinline__ int local_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// A fold reads at most (count - 1) * stride + 1 slots of d pairs from base:
// a segment's chunks or groups, far below 2^31 bytes (the plan checks it).
template <bool ACCURATE>
__device__ __forceinline__ bool fold_block(const uint64_t* base, int64_t count, int64_t stride, int d, float* lds_m,
                                           float* lds_s, uint64_t* stage) {
  const int t = local_tid();
  int r = 1;
  while (2 * r * d <= kBlock && 2 * r <= count) r *= 2;
  bool ok = true;
  const int slot_bytes = (int)(stride * d * 8);
  const Rsrc pairs = make_rsrc(base, ((count - 1) * stride * d + d) * 8);
  if (r == 1) {
    for (int f = t; f < d; f += kBlock) {
      const State<OP_SOFTMAX> st = fold_range<ACCURATE>(pairs, f * 8, (int)count, slot_bytes, ok);
      lds_m[f] = st.m;
      lds_s[f] = st.s;
    }
    return !block_any(!ok);
  }
  if (t < r * d) {
    const int part = t / d, f = t - part * d;
    const int lo = (int)(count * part / r), hi = (int)(count * (part + 1) / r);
    const State<OP_SOFTMAX> st = fold_range<ACCURATE>(pairs, lo * slot_bytes + f * 8, hi - lo, slot_bytes, ok);
    stage[t] = pack_pair(st.m, st.s);
  }
  const bool all = !block_any(!ok);
  if (all && t < d) {
    State<OP_SOFTMAX> acc;
    acc.init();
    for (int q = 0; q < r; ++q) {
      State<OP_SOFTMAX> part;
      part.m = pair_m(stage[q * d + t]);
      part.s = pair_s(stage[q * d + t]);
      merge_stats<ACCURATE>(acc, part);
    }
    lds_m[t] = acc.m;
    lds_s[t] = acc.s;
  }
  __syncthreads();
  return all;
}

// fold_block until every slot is published or `ticks` of wall clock pass
// (thread 0 decides, so the workgroup agrees); false when it gave up.
template <bool ACCURATE>
__device__ __forceinline__ bool poll_fold(const uint64_t* base, int64_t count, int d, int64_t ticks, float* lds_m,
                                          float* lds_s, uint64_t* stage) {
  const long long start = wall_clock64();
  for (;;) {
    if (fold_block<ACCURATE>(base, count, 1, d, lds_m, lds_s, stage)) return true;
    bool give_up = false;
    if (threadIdx.x == 0) give_up = wall_clock64() - start >= ticks;
    if (block_any(give_up)) return false;
    __builtin_amdgcn_s_sleep(2);
  }
}

// A wait also ends, before its budget, once the segment still has chunks
// not handed out (ticket counter <= last_ticket, both counting the tickets
// after the first round) and the ticket counter has
// not moved over an interval of spin_ticks / kStallDivisor (100 us with the
// default budget): every workgroup that could take them is then busy
// (waiting, or another process holds the CUs), so waiting longer gains
// nothing. In a free device the counter moves every few hundred
// nanoseconds and a wait lasts 10-25 us, so the counter -- the kernel's
// hottest atomic, which hundreds of polling waiters would slow for
// everyone -- is read only by waits already one interval long, once per
// interval.
constexpr int kStallDivisor = 20;

// fold_block until every slot is published, the wall-clock budget ends or
// the ticket counter stalls before the segment's last chunk is handed out
// (the decisions are thread 0's, so the workgroup agrees); false when the
// wait gave up.
template <bool ACCURATE>
__device__ __forceinline__ bool wait_fold(const uint64_t* base, int64_t count, int d, int64_t spin_ticks,
                                          const int64_t* tickets, int64_t last_ticket, float* lds_m, float* lds_s,
                                          uint64_t* stage) {
  const long long start = wall_clock64();
  const long long interval = spin_ticks / kStallDivisor;
  long long next_check = start + interval;
  int64_t seen = -1;
  for (;;) {
    if (fold_block<ACCURATE>(base, count, 1, d, lds_m, lds_s, stage)) return true;
    bool give_up = false;
    if (threadIdx.x == 0) {
      const long long now = wall_clock64();
      give_up = now - start >= spin_ticks;
      if (!give_up && now >= next_check) {
        const int64_t handed = (int64_t)((uint64_t)__hip_atomic_load(const_cast<int64_t*>(tickets), __ATOMIC_RELAXED,
                                                                     __HIP_MEMORY_SCOPE_AGENT) & kTicketMask);
        give_up = handed == seen && handed <= last_ticket;
        seen = handed;
        next_check = now + interval;
      }
    }
    if (block_any(give_up)) return false;
    __builtin_amdgcn_s_sleep(kPollSleep);
  }
}

// A value the compiler cannot see through, made where it is used: constants
// of rarely taken branches inside the persistent loop are then not hoisted
// out of it and held in registers (or spilled) while the rows are live.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// A chunk's segment: its first item and its merged statistics (the chunks'
// pairs of a direct segment, the group rows of a tree one).
struct SegmentStats {
  const uint64_t* base;   // first slot of the statistics a reader folds
  int64_t count;          // slots (chunks or groups) they span, d pairs each
};
__device__ __forceinline__ SegmentStats segment_stats(const Params& p, int64_t idx, int32_t c, int32_t parts,
                                                      int32_t k) {
  SegmentStats st;
  if (parts <= kDirect) {
    st.base = p.pairs + (idx - c) * p.d;
    st.count = parts;
  } else {
    st.base = p.final_pairs + (int64_t)k * p.d;
    st.count = (parts + kGroup - 1) / kGroup;
  }
  return st;
}

// Counter-based first level of a long segment's merge: the last chunk of
// each group of kGroup folds the group and publishes it in the segment's
// row gbase + group of final_pairs. Every chunk of the group stored its pair
// (agent scope), waited for the stores to complete and only then counted
// itself, so the fold normally succeeds at once; a pair not yet visible
// reads as zero and the fold polls again (a fold that never completes
// within fold_ticks publishes NaN: the segment's output is then NaN, never
// silently wrong). It returns the group's counter to zero (every chunk of
// the group has counted). The segment's chunks then
// fold its groups' rows directly, as a directly merged segment folds its
// chunks' pairs: no second counter level, whose store, atomic, fold and
// store again would sit on every chunk's wait.
template <bool ACCURATE>
__device__ __forceinline__ void tree_merge(const Params& p, int64_t slot, int64_t first, int64_t parts, int64_t gbase, int* flag_s,
                           float* lds_m, float* lds_s, uint64_t* stage) {
  const int t = local_tid();
  const int d = p.d;
  const int64_t group = (slot - first) / kGroup;
  const int64_t gfirst = first + group * kGroup;
  const int64_t gsize = parts - group * kGroup < kGroup ? parts - group * kGroup : kGroup;
  // Every read of *flag_s is followed by a barrier before its next write.
  wait_stores();
  __syncthreads();
  if (t == 0) *flag_s = atomicAdd(p.arrive + gfirst, 1) == gsize - 1;
  __syncthreads();
  const bool last_in_group = *flag_s != 0;
  __syncthreads();
  if (!last_in_group) return;
  const bool ok = poll_fold<ACCURATE>(p.pairs + gfirst * d, gsize, d, p.fold_ticks, lds_m, lds_s, stage);
  for (int f = t; f < d; f += kBlock) {
    const float nan = __uint_as_float(opaque_u32(0x7fc00000u));
    store_pair(p.final_pairs + (gbase + group) * d + f, ok ? lds_m[f] : nan, ok ? lds_s[f] : nan);
  }
  if (t == 0) p.arrive[gfirst] = 0;
}

template <class T, class OffT, int VEC, int RPT, bool MASK, bool STORE_F32>
__device__ __forceinline__ void drain_and_finish(const Params& p, int64_t active, bool seen, float* lds_m, float* lds_s,
                                 uint64_t* stage, int* flag_s, int64_t* claim_s);

template <class T, class OffT, int VEC, int RPT, bool MASK, bool STORE_F32>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4))) void k_softmax_fused(Params p) {
  // Rows stay as loaded (T) unless the input transform (scale, mask) makes
  // f32 logits that must not be rounded back to T.
  using Store = typename std::conditional<STORE_F32, float, T>::type;
  using In = Words<T, VEC>;
  using Reg = Words<Store, VEC>;
  // f32 outputs: merges rescale with the accurate exp, and pass 1 sums
  // with a compensated (Kahan) add per thread, as the reference's online
  // statistics do (ToGPU.cpp:377-387, 509-603).
  constexpr bool kAccurate = std::is_same<T, float>::value;
  // lds: reductions, then the segment's merged max per feature, then the
  // normaliser's first constant; lds_s: the merged sum, then its second.
  __shared__ float lds[kBlock * VEC];
  __shared__ float lds_s[kBlock * VEC];
  __shared__ uint64_t stage[kBlock];    // partial folds of the segment merge
  __shared__ float own_m[kBlock * VEC];   // this item's column max and sum
  __shared__ float own_s[kBlock * VEC];
  __shared__ int64_t next_s;
  __shared__ int flag_s;
  __shared__ int64_t stamp_s[5];    // item timeline (diagnostics), thread 0 only
  const int t = threadIdx.x;
  const RowGeo g = row_geo<VEC>(p.d, kBlock, t, 0);
  // Rows of this thread inside an item: row0 + i * rstep. Where a row fits
  // in one wave (lpr <= 64), each wave holds its own run of consecutive rows,
  // so a wave's RPT loads read one contiguous span: on MI355X a 64 KiB item
  // read as 4 KiB-strided 1 KiB pieces per wave moves 5.2 TB/s, read as one
  // 16 KiB span per wave 6.05 TB/s (measured on a held-item copy). Wider rows
  // keep one row per workgroup step.
  const bool wave_rows = g.lpr <= kWave;
  const int rstep = wave_rows ? kWave / g.lpr : g.rows_step;
  const int row0 = wave_rows ? (t / kWave) * RPT * rstep + (t % kWave) / g.lpr : g.row_lane;
  // First row of this wave (uniform): row groups wholly past the item are
  // skipped per wave.
  const int wave_row0 = wave_rows ? __builtin_amdgcn_readfirstlane((t / kWave) * RPT * rstep) : 0;
  // Ticket order: chunks of segments merged by tree (top of the item
  // array), chunks of segments merged directly (bottom), block-class
  // segments; then the wave class (after this loop). k_classify counts a
  // register-resident program's wave class in counters[7] instead of
  // counters[0], so the last term is 0. It stays: without it the compiler
  // allocates this kernel's scalar registers differently and it runs slower.
  // The class counts were written by k_classify and stay fixed during this
  // kernel: read through the constant address space they load into SGPRs
  // (scalar loads) instead of occupying vector registers, which the held
  // rows need.
  const ConstI64* counts = (const ConstI64*)p.counters;
  const int64_t n_tree = counts[6] < p.items_cap ? counts[6] : p.items_cap;
  const int64_t n_direct = counts[3] < p.items_cap - n_tree ? counts[3] : p.items_cap - n_tree;
  const int64_t n_split = n_tree + n_direct;
  const int64_t n_block = counts[1] < p.b ? counts[1] : p.b;
  const int64_t total = n_split + n_block + counts[0];
  const int64_t d = p.d;
  // Byte offsets inside an item: per thread, and the stride between a
  // thread's rows.
  const int voff_in = g.active ? (row0 * p.d + g.feature) * (int)sizeof(T) : kOutOfRange;
  const int step_in = rstep * p.d * (int)sizeof(T);
  const int voff_mask = g.active ? (row0 * p.d + g.feature) * 4 : kOutOfRange;
  const int step_mask = rstep * p.d * 4;
  // Index of a chunk ticket in the item (and pair) arrays.
  auto index_of = [&](int64_t ticket) -> int64_t {
    return ticket < n_tree ? p.items_cap - n_tree + ticket : ticket - n_tree;
  };
  ConstItem* items = (ConstItem*)p.items;
  ConstItem* block_items = (ConstItem*)p.block_items;
  auto item_at = [&](int64_t ticket) -> Item {
    if (ticket < n_split) return load_item(items + index_of(ticket));
    if (ticket < n_split + n_block) return load_item(block_items + (ticket - n_split));
    return load_item(block_items + (p.b - 1 - (ticket - n_split - n_block)));
  };
  if (t == 0) next_s = 0;
  __syncthreads();
  int64_t ticket = blockIdx.x;
  Item it;
  if (ticket < total) it = item_at(ticket);
  while (ticket < total) {
    const bool chunk = it.k >= 0;
    const bool may_wait = chunk && it.parts <= p.wait_parts;
    // Next ticket: taken while this item loads once every chunk has been
    // handed out (this ticket is past them), else when this item starts its
    // stores. Chunks of one segment therefore start together, and a ticket
    // held but not started never belongs to a segment its holder waits for:
    // waits only run down to chunks that are started.
    const bool early = ticket >= n_split;
    __syncthreads();
    unsigned long long taken = 0;
    if (t == 0 && early) taken = atomicAdd((unsigned long long*)(p.counters + 4), 1ull);
    // Timeline stamps are unconditional (cheap); only the record is optional.
    if (t == 0) stamp_s[0] = wall_clock64();
    const int rows = it.rows;
    const int64_t start = it.start;
    const int64_t chunk_elems = (int64_t)rows * d;
    int voff = voff_in, voff_m = voff_mask;
    asm volatile("" : "+v"(voff), "+v"(voff_m));
    const Rsrc in = make_rsrc(static_cast<const T*>(p.values) + start * d, chunk_elems * (int64_t)sizeof(T));
    // 1. Rows into registers (all loads in flight at once), column max.
    //    The loads issue at the highest wave priority (s_setprio 3), so a
    //    workgroup starting an item is not held behind the exponentials of
    //    the waves sharing its SIMD: on MI355X this keeps more of the item
    //    stream in flight (C5: kernel 2-3% faster). The stores below do the
    //    same; the merges run at the base priority (raising them too gave
    //    back most of the gain).
    uint32_t data[RPT][Reg::kCount];
    if constexpr (!STORE_F32) {
      __builtin_amdgcn_s_setprio(3);
#pragma unroll
      for (int i = 0; i < RPT; ++i) buffer_load<In::kBytes>(in, voff + i * step_in, 0, data[i]);
      __builtin_amdgcn_s_setprio(0);
    } else {
      const Rsrc mk = make_rsrc(MASK ? p.mask + start * d : nullptr, MASK ? chunk_elems * 4 : 0);
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
#pragma clang fp contract(off)
        uint32_t raw[In::kCount];
        buffer_load<In::kBytes>(in, voff + i * step_in, 0, raw);
        float x[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) x[v] = In::get(raw, v);
        if (p.has_scale) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = x[v] * p.scale;
        }
        if constexpr (MASK) {
          uint32_t mw[VEC];
          buffer_load<VEC * 4>(mk, voff_m + i * step_mask, 0, mw);
#pragma unroll
          for (int v = 0; v < VEC; ++v) x[v] = x[v] + __uint_as_float(mw[v]);
        }
        Reg::set(data[i], x);
      }
    }
    // Next ticket, while the loads are in flight. A workgroup that could
    // wait for its segment takes it early only once every chunk of the
    // segment has been handed out; otherwise after the wait. So a ticket
    // held but not started never belongs to a segment its holder waits
    // for, and waits only run down to chunks that are started.
    if (t == 0 && opaque(early)) next_s = (int64_t)taken;
    // Rows past the item (and featureless lanes) read 0: make them -inf,
    // the identity of the max and a zero mass.
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      if (!(g.active && row0 < rows - i * rstep)) Reg::fill_neg_inf(data[i]);
    }
    // Row groups wholly past the item (wave-uniform) skip the arithmetic below.
    auto live = [&](int i) { return i == 0 || wave_row0 + i * rstep < rows; };
    float m[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) m[v] = neg_inf();
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) m[v] = fmax_nan(m[v], Reg::get(data[i], v));
    }
    // Keep the rows packed across the reduction: without this the compiler
    // keeps every unpacked f32 value alive until pass 2.
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
      for (int w = 0; w < Reg::kCount; ++w) asm volatile("" : "+v"(data[i][w]));
    }
    block_allreduce<true, VEC>(m, g.lpr, g.feat_lane, lds);
    if (t == 0) stamp_s[1] = wall_clock64();
    // The reduction's barrier published next_s: prefetch the next item.
    int64_t next = 0;
    Item next_it;
    if (opaque(early)) {
      next = (int64_t)((uint64_t)uniform64(next_s) & kTicketMask) + gridDim.x;
      if (next < total) next_it = item_at(next);
    }
    // 2. Column sums of exp(x - m); the rows stay as loaded. A column of
    //    only -inf has no mass: its reference is taken as 0 so that every
    //    term is 0, not NaN.
    float sum[VEC];
    ExpShift<T> ex[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      ex[v] = ExpShift<T>(m[v] == neg_inf() ? 0.f : m[v]);
      sum[v] = 0.f;
    }
    if constexpr (kAccurate) {
      // Every term is in [0, 1] (or NaN): the correction is finite
      // wherever the sum is.
      float comp[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) comp[v] = 0.f;
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        if (!live(i)) continue;
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
#pragma clang fp contract(off)
          const float y = ex[v](Reg::get(data[i], v)) - comp[v];
          const float t = sum[v] + y;
          comp[v] = (t - sum[v]) - y;
          sum[v] = t;
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        if (!live(i)) continue;
#pragma unroll
        for (int v = 0; v < VEC; ++v) sum[v] += ex[v](Reg::get(data[i], v));
      }
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
      for (int w = 0; w < Reg::kCount; ++w) asm volatile("" : "+v"(data[i][w]));
    }
    block_allreduce<false, VEC>(sum, g.lpr, g.feat_lane, lds);
    if (t == 0) stamp_s[2] = wall_clock64();
    // The item's column statistics leave registers for LDS: the merge below
    // then holds nothing but the rows.
    if (row0 == 0 && g.active) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        own_m[g.feature + v] = m[v];
        own_s[g.feature + v] = sum[v];
      }
    }
    __syncthreads();
    // 3. The segment's statistics (M, S) per column -- the item's own for a
    //    whole segment -- as the normaliser's constants into lds / lds_s.
    bool defer = false;
    if (!chunk) {
      for (int f = t; f < d; f += kBlock) {
        const Normalizer<T> n = Normalizer<T>::of(own_m[f], own_s[f]);
        lds[f] = n.a;
        lds_s[f] = n.b;
      }
    } else {
      const int64_t idx = index_of(ticket);
      const int64_t first = idx - it.c;
      const int64_t parts = it.parts;
      for (int f = local_tid(); f < d; f += kBlock) store_pair(p.pairs + idx * d + f, own_m[f], own_s[f]);
      const bool direct = parts <= kDirect;
      if (!direct) tree_merge<kAccurate>(p, idx, first, parts, it.k, &flag_s, lds, lds_s, stage);
      if (!may_wait) {
        defer = true;        // more chunks than the device surely holds at once
      } else {
        const int64_t last_ticket = ticket - it.c + parts - 1 - gridDim.x;
        const int64_t* tickets = p.counters + 4;
        const bool ready = direct ? wait_fold<kAccurate>(p.pairs + first * d, parts, p.d, p.spin_ticks, tickets,
                                                         last_ticket, lds, lds_s, stage)
                                  : wait_fold<kAccurate>(p.final_pairs + it.k * d, (parts + kGroup - 1) / kGroup,
                                                         p.d, p.spin_ticks, tickets, last_ticket, lds, lds_s, stage);
        defer = !ready;
        // Same thread wrote lds[f] / lds_s[f] in the fold: no barrier needed.
        if (ready) {
          for (int f = t; f < d; f += kBlock) {
            const Normalizer<T> n = Normalizer<T>::of(lds[f], lds_s[f]);
            lds[f] = n.a;
            lds_s[f] = n.b;
          }
        }
      }
      if (t == 0 && defer) {
        const int64_t slot = (int64_t)(atomicAdd((unsigned long long*)(p.counters + 4), 1ull << kDeferShift) >>
                                       kDeferShift);
        if (slot < p.items_cap)
          __hip_atomic_store(p.deferred + slot, idx + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    if (t == 0 && !opaque(early)) taken = atomicAdd((unsigned long long*)(p.counters + 4), 1ull);
    if (t == 0) stamp_s[3] = wall_clock64();
    if (!defer) {
      // 4. y = exp(x - M) / S from the held rows; rows past the item are
      //    dropped by the resource's range check.
      const Rsrc out = make_rsrc(static_cast<T*>(p.out) + start * d, chunk_elems * (int64_t)sizeof(T));
      asm volatile("" : "+v"(voff));
      Normalizer<T> norm[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) norm[v] = g.active ? Normalizer<T>(lds[g.feature + v], lds_s[g.feature + v])
                                                       : Normalizer<T>();
      __builtin_amdgcn_s_setprio(3);
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        if (!live(i)) continue;
        float y[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) y[v] = norm[v](Reg::get(data[i], v));
        uint32_t w[In::kCount];
        In::set(w, y);
        buffer_store<In::kBytes>(out, voff + i * step_in, 0, w);
      }
      __builtin_amdgcn_s_setprio(0);
      if (p.visits && t == 0 && it.c == 0) atomicAdd(p.visits + it.seg, 1);
    }
    if (!opaque(early)) {
      if (t == 0) next_s = (int64_t)taken;
      __syncthreads();
      next = (int64_t)((uint64_t)uniform64(next_s) & kTicketMask) + gridDim.x;
      if (next < total) next_it = item_at(next);
    }
    if (opaque(p.trace && ticket < p.trace_cap) && t == 0) {
      int64_t* r = p.trace + ticket * 8;
      r[0] = ticket;
      r[1] = stamp_s[0];
      r[2] = stamp_s[1];
      r[3] = stamp_s[2];
      r[4] = stamp_s[3];
      r[5] = wall_clock64();
      r[6] = __smid();
      r[7] = (opaque(chunk) ? (it.parts <= kDirect ? 1 : 2) : 0) + (defer ? 4 : 0) + ((int64_t)rows << 8);
    }
    ticket = next;
    it = next_it;
  }
  // The wave class, in the streaming worker's batches: the rest of the wave
  // class one segment per wave (counters[8]), then the segments one lane
  // group reduces alone (counters[7]). Their tickets follow the items'; this
  // workgroup holds its first.
  {
    const int64_t n_coop = counts[8] < p.b ? counts[8] : p.b;
    const int64_t n_wave = counts[7] < p.b ? counts[7] : p.b;
    const int64_t batch = wave_batch_size<false, VEC>(p.d);
    const int64_t n_coop_batches = (n_coop + kWavesPerBlock - 1) / kWavesPerBlock;
    const int64_t tail = total + n_coop_batches + (n_wave + batch - 1) / batch;
    while (ticket < tail) {
      const int64_t i = ticket - total;
      if (i < n_coop_batches) coop_batch<OP_SOFTMAX, T, OffT, VEC, false, MASK>(p, i, n_coop);
      else wave_batch<OP_SOFTMAX, T, OffT, VEC, false, MASK>(p, i - n_coop_batches, n_wave, false);
      __syncthreads();
      if (t == 0) next_s = (int64_t)atomicAdd((unsigned long long*)(p.counters + 4), 1ull);
      __syncthreads();
      ticket = (int64_t)((uint64_t)uniform64(next_s) & kTicketMask) + gridDim.x;
    }
  }
  // The last ticket fetch (next_s, as fetched) counted the chunks deferred
  // by then.
  __shared__ int64_t claim_s;
  const bool seen = ((uint64_t)uniform64(next_s) >> kDeferShift) != 0;
  drain_and_finish<T, OffT, VEC, RPT, MASK, STORE_F32>(p, gridDim.x, seen, lds, lds_s, stage, &flag_s, &claim_s);
}

// A deferred chunk (item idx): fold its segment's statistics (bounded by
// `ticks`), then re-read its rows and write y = exp(x - M) / S with the
// register path's arithmetic (the same Normalizer from the same fold), so
// its bits do not depend on whether it waited. When the statistics do not
// appear in time it returns false having written nothing -- unless `must` (the last
// workgroup, after every other has finished: nothing can publish later),
// which then writes NaN, so that a lost publication is never silent.
template <class T, int VEC, int RPT, bool MASK, bool STORE_F32>
__device__ __forceinline__ bool finish_deferred(const Params& p, int64_t idx, int64_t ticks, bool must, float* lds_m, float* lds_s,
                                uint64_t* stage) {
  using Store = typename std::conditional<STORE_F32, float, T>::type;
  using In = Words<T, VEC>;
  using Reg = Words<Store, VEC>;
  const int t = threadIdx.x;
  const Item it = p.items[idx];
  const SegmentStats st = segment_stats(p, idx, it.c, it.parts, it.k);
  const bool ok = poll_fold<std::is_same<T, float>::value>(st.base, st.count, p.d, ticks, lds_m, lds_s, stage);
  if (!ok && !must) return false;
  for (int f = t; f < p.d; f += kBlock) {
    const float nan = __builtin_nanf("");
    const Normalizer<T> n = ok ? Normalizer<T>::of(lds_m[f], lds_s[f]) : Normalizer<T>(nan, nan);
    lds_m[f] = n.a;
    lds_s[f] = n.b;
  }
  __syncthreads();
  const RowGeo g = row_geo<VEC>(p.d, kBlock, t, 0);
  if constexpr (MASK) {
    // Masked logits: one row step at a time (holding the mask's words as
    // well would spill the register path's rows).
    if (g.active) {
      Normalizer<T> norm[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) norm[v] = Normalizer<T>(lds_m[g.feature + v], lds_s[g.feature + v]);
      T* out = static_cast<T*>(p.out);
      for (int64_t r = it.start + g.row_lane; r < it.start + it.rows; r += g.rows_step) {
        float x[VEC];
        load_input<T, VEC, MASK>(p, r * p.d + g.feature, x);
#pragma unroll
        for (int v = 0; v < VEC; ++v) x[v] = norm[v](x[v]);
        Elem<T>::template store<VEC>(out + r * p.d + g.feature, x);
      }
    }
    if (p.visits && t == 0 && it.c == 0) atomicAdd(p.visits + it.seg, 1);
    __syncthreads();
    return true;
  }
  // The chunk's rows as the register path holds them (the same row
  // mapping, every load in flight at once, the same input transform), so
  // each output takes the register path's arithmetic and bits.
  const bool wave_rows = g.lpr <= kWave;
  const int rstep = wave_rows ? kWave / g.lpr : g.rows_step;
  const int row0 = wave_rows ? (t / kWave) * RPT * rstep + (t % kWave) / g.lpr : g.row_lane;
  const int wave_row0 = wave_rows ? __builtin_amdgcn_readfirstlane((t / kWave) * RPT * rstep) : 0;
  const int voff = g.active ? (row0 * p.d + g.feature) * (int)sizeof(T) : kOutOfRange;
  const int step = rstep * p.d * (int)sizeof(T);
  const int64_t elems = (int64_t)it.rows * p.d;
  const Rsrc in = make_rsrc(static_cast<const T*>(p.values) + it.start * p.d, elems * (int64_t)sizeof(T));
  uint32_t data[RPT][Reg::kCount];
  if constexpr (!STORE_F32) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) buffer_load<In::kBytes>(in, voff + i * step, 0, data[i]);
  } else {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma clang fp contract(off)
      uint32_t raw[In::kCount];
      buffer_load<In::kBytes>(in, voff + i * step, 0, raw);
      float x[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) x[v] = In::get(raw, v);
      if (p.has_scale) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) x[v] = x[v] * p.scale;
      }
      Reg::set(data[i], x);
    }
  }
  Normalizer<T> norm[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) norm[v] = g.active ? Normalizer<T>(lds_m[g.feature + v], lds_s[g.feature + v])
                                                   : Normalizer<T>();
  const Rsrc out = make_rsrc(static_cast<T*>(p.out) + it.start * p.d, elems * (int64_t)sizeof(T));
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    if (i != 0 && wave_row0 + i * rstep >= it.rows) continue;
    float y[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) y[v] = norm[v](Reg::get(data[i], v));
    uint32_t w[In::kCount];
    In::set(w, y);
    buffer_store<In::kBytes>(out, voff + i * step, 0, w);
  }
  if (p.visits && t == 0 && it.c == 0) atomicAdd(p.visits + it.seg, 1);
  __syncthreads();
  return true;
}

// Deferred chunks, once this workgroup's tickets have run out (every item is
// then handed out, and every holder publishes its pair before it waits, so
// every deferred chunk's statistics appear). A workgroup whose last ticket
// fetch counted deferred chunks (`seen`) claims entries of the deferred list
// in order while any is listed and finishes each (an entry whose statistics
// do not appear within drain_ticks is left for the last workgroup); it then
// counts out once its stores are complete. A workgroup that saw none counts
// out at once: deferrals after its fetch are left to the others. The last
// workgroup out finishes every entry still listed (all pairs are published
// by then), returns the list and the counters to zero and records what the
// call left nonzero in the arena.
template <class T, class OffT, int VEC, int RPT, bool MASK, bool STORE_F32>
__device__ __forceinline__ void drain_and_finish(const Params& p, int64_t active, bool seen, float* lds_m, float* lds_s,
                                 uint64_t* stage, int* flag_s, int64_t* claim_s) {
  const int t = threadIdx.x;
  unsigned long long* claimed = (unsigned long long*)(p.counters + kDrainSlot);
  unsigned long long* word = (unsigned long long*)(p.counters + 4);
  const unsigned long long cap = (unsigned long long)p.items_cap;
  auto listed = [&]() {
    const unsigned long long n = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> kDeferShift;
    return n < cap ? n : cap;
  };
  while (seen) {
    __syncthreads();
    if (t == 0) {
      // One fetch-and-add per claim (a compare-and-swap loop serialises
      // the claimers: ~1 us per entry with a thousand of them). A claim
      // past the entries listed so far is given up; an entry listed later
      // at that position is finished by the last workgroup.
      const unsigned long long c = atomicAdd(claimed, 1ull);
      const int64_t mine = c < listed() ? (int64_t)c : -1;
      // The entry's writer reserved it before storing it: wait for the store.
      int64_t entry = 0;
      if (mine >= 0) {
        const long long t0 = wall_clock64();
        while ((entry = __hip_atomic_load(p.deferred + mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0 &&
               wall_clock64() - t0 < p.fold_ticks)
          __builtin_amdgcn_s_sleep(2);
      }
      *claim_s = mine < 0 ? -1 : (entry > 0 ? ((mine << 32) | (entry - 1)) : -2);
    }
    __syncthreads();
    const int64_t claim = *claim_s;
    if (claim == -1) break;
    if (claim == -2) continue;    // never written in time: the last workgroup sees it
    const int64_t slot = claim >> 32, idx = claim & 0xffffffffll;
    if (finish_deferred<T, VEC, RPT, MASK, STORE_F32>(p, idx, p.drain_ticks, false, lds_m, lds_s, stage) && t == 0)
      __hip_atomic_store(p.deferred + slot, (int64_t)-1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // A workgroup that deferred or finished a chunk took part in the drain
  // (its own deferral precedes its last fetch): its list stores must be
  // visible to the last workgroup before it counts out.
  if (!last_out(p, flag_s, active, seen)) return;
  const int64_t listed_n = (int64_t)listed();
  // The list read kBlock entries per round trip (one thread each); the
  // entries still unfinished (normally none) are then finished one by one.
  __shared__ int64_t sweep_s[kBlock];
  for (int64_t j0 = 0; j0 < listed_n; j0 += kBlock) {
    __syncthreads();
    sweep_s[t] = j0 + t < listed_n
                     ? __hip_atomic_load(p.deferred + j0 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                     : 0;
    if (j0 + t < listed_n) p.deferred[j0 + t] = 0;     // the list returns to zero
    __syncthreads();
    if (!block_any(sweep_s[t] > 0)) continue;
    for (int k = 0; k < kBlock; ++k) {
      const int64_t entry = sweep_s[k];
      if (entry > 0) (void)finish_deferred<T, VEC, RPT, MASK, STORE_F32>(p, entry - 1, p.fold_ticks, true, lds_m, lds_s, stage);
    }
  }
  // What this call left nonzero in the arena, for the next call's
  // k_classify: the pairs of the direct chunks (bottom of the pair table)
  // and of the tree chunks (top), and the group rows.
  int64_t dirty[2 * kDirtyRanges];
  {
    const int64_t n_tree = p.counters[6] < p.items_cap ? p.counters[6] : p.items_cap;
    const int64_t n_direct = p.counters[3] < p.items_cap - n_tree ? p.counters[3] : p.items_cap - n_tree;
    const int64_t rows_cap = tree_group_rows(p.items_cap);
    const int64_t rows = p.counters[kGroupRowSlot] < rows_cap ? p.counters[kGroupRowSlot] : rows_cap;
    const int64_t pairs = p.pairs ? (const unsigned char*)p.pairs - p.arena : 0;
    const int64_t finals = p.final_pairs ? (const unsigned char*)p.final_pairs - p.arena : 0;
    const int64_t slot = (int64_t)p.d * 8;
    dirty[0] = pairs;
    dirty[1] = pairs + n_direct * slot;
    dirty[2] = pairs + (p.items_cap - n_tree) * slot;
    dirty[3] = pairs + p.items_cap * slot;
    dirty[4] = finals;
    dirty[5] = finals + rows * slot;
  }
  __syncthreads();
  reset_counters(p, dirty);
}

}  // namespace rg
