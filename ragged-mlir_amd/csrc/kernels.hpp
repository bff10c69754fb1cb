// Worker kernels for segmented sum / max / softmax on gfx950.
//
// Schedules (the same arithmetic in both):
//  * block per segment ("naive"): grid.x walks segments, one 256-thread
//    workgroup each (reference: the direct schedule, ToGPU.cpp:1283-1349).
//  * classified: k_classify bins every segment by length into a wave64
//    queue, a workgroup queue and a split queue (reference: ToGPU.cpp:
//    901-998, with wave64 thresholds) and initialises the per-segment state
//    the call uses; one persistent worker (worker.hpp) drains the queues
//    (ToGPU.cpp:999-1045), and the call's last workgroup returns the
//    counters to zero for the next call (last_out, reset_counters). A
//    split segment is cut into ceil(L / part_rows) parts -- proportional to
//    its length instead of the reference's fixed 8 -- each processed by one
//    workgroup; the last part folds them (ToGPU.cpp:399-472) and, for
//    softmax, the worker then writes the probabilities (ToGPU.cpp:279-281).
#pragma once

#include <type_traits>

#include "device.hpp"

namespace rg {

// ---------------------------------------------------------------------------
// Input transformation: f32(value) * scale + mask (docs/mask-abi.md:28-43).

// bf16 values are scaled unconditionally (p.scale is 1 without one, and
// x * 1 is x exactly): a branch here would end the basic block after every
// load, and the conversion of the loaded words could then not move below
// the next load -- each load of an unrolled loop would wait for the one
// before. f32 values need no conversion, and skip the multiply.
template <class T, int VEC, bool MASK>
__device__ __forceinline__ void load_input(const Params& p, int64_t element, float (&x)[VEC]) {
#pragma clang fp contract(off)
  Elem<T>::template load<VEC>(static_cast<const T*>(p.values) + element, x);
  if (!std::is_same<T, float>::value || p.has_scale) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = x[v] * p.scale;
  }
  if constexpr (MASK) {
    float m[VEC];
    load_mask<VEC>(p.mask + element, m);
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = x[v] + m[v];
  }
}

template <class T, bool MASK>
__device__ __forceinline__ float load_input1(const Params& p, int64_t element) {
#pragma clang fp contract(off)
  float x = Elem<T>::get(static_cast<const T*>(p.values) + element) * p.scale;
  if constexpr (MASK) x = x + p.mask[element];
  return x;
}

// Identity element a masked-off component folds in: it changes nothing.
template <int OP> __device__ __forceinline__ float fold_identity() {
  return OP == OP_SUM ? 0.f : neg_inf();
}

// ---------------------------------------------------------------------------
// ROW mapping traversal of rows [r0, r1) by a group with geometry `g`.

template <int OP, class T, int VEC, bool MASK>
__device__ __forceinline__ void fold_rows(const Params& p, const RowGeo& g, int64_t r0, int64_t r1,
                                          State<OP> (&st)[VEC]) {
  if (!g.active) return;
  const int64_t step = g.rows_step;
  int64_t r = r0 + g.row_lane;
  const int64_t d = p.d;
  for (; r + (kUnroll - 1) * step < r1; r += kUnroll * step) {
    float x[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) load_input<T, VEC, MASK>(p, (r + u * step) * d + g.feature, x[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) st[v].fold(x[u][v]);
    }
  }
  for (; r < r1; r += step) {
    float x[VEC];
    load_input<T, VEC, MASK>(p, r * d + g.feature, x);
#pragma unroll
    for (int v = 0; v < VEC; ++v) st[v].fold(x[v]);
  }
}

// Softmax normalisation of rows [r0, r1): out = exp(x - m) * (1 / s).
template <class T, int VEC, bool MASK>
__device__ __forceinline__ void normalize_rows(const Params& p, const RowGeo& g, int64_t r0, int64_t r1,
                                               const float (&m)[VEC], const float (&inv)[VEC]) {
  if (!g.active) return;
  const int64_t step = g.rows_step;
  const int64_t d = p.d;
  T* out = static_cast<T*>(p.out);
  int64_t r = r0 + g.row_lane;
  for (; r + (kUnroll - 1) * step < r1; r += kUnroll * step) {
    float x[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) load_input<T, VEC, MASK>(p, (r + u * step) * d + g.feature, x[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) x[u][v] = exp_out<T>(x[u][v] - m[v]) * inv[v];
      Elem<T>::template store<VEC>(out + (r + u * step) * d + g.feature, x[u]);
    }
  }
  for (; r < r1; r += step) {
    float x[VEC];
    load_input<T, VEC, MASK>(p, r * d + g.feature, x);
#pragma unroll
    for (int v = 0; v < VEC; ++v) x[v] = exp_out<T>(x[v] - m[v]) * inv[v];
    Elem<T>::template store<VEC>(out + r * d + g.feature, x);
  }
}

// ---------------------------------------------------------------------------
// FLAT mapping traversal of elements [lo, hi) (= rows [r0, r1) times D).

// The elements of vector j one by one, each index clamped into [lo, hi)
// (lo < hi): no load leaves the segment, and with no branch between them
// the VEC loads are in flight together. Components outside [lo, hi) hold
// a copy of an element inside; callers mask them.
template <class T, int VEC, bool MASK>
__device__ __forceinline__ void load_partial(const Params& p, int64_t j, int64_t lo, int64_t hi, float (&x)[VEC]) {
#pragma unroll
  for (int c = 0; c < VEC; ++c) {
    const int64_t e = j * VEC + c;
    x[c] = load_input1<T, MASK>(p, e < lo ? lo : (e < hi ? e : hi - 1));
  }
}
// Vector j covers elements [j*VEC, j*VEC + VEC); component c is feature c % D.

template <int OP, class T, int VEC, bool MASK>
__device__ __forceinline__ void fold_flat(const Params& p, int g, int t, int64_t lo, int64_t hi,
                                          State<OP> (&st)[VEC]) {
  if (lo >= hi) return;
  const int64_t full_lo = (lo + VEC - 1) / VEC, full_hi = hi / VEC;
  // Up to two partial vectors: the one holding lo and the one holding hi-1.
  const int64_t head = lo / VEC, tail = (hi - 1) / VEC;
  const bool head_partial = lo % VEC != 0 || (head == tail && hi % VEC != 0);
  const bool tail_partial = hi % VEC != 0 && tail != head;
  if ((head_partial && t == 0) || (tail_partial && t == 1)) {
    const int64_t j = t == 0 ? head : tail;
    float x[VEC];
    load_partial<T, VEC, MASK>(p, j, lo, hi, x);
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int64_t e = j * VEC + c;
      st[c].fold(e >= lo && e < hi ? x[c] : fold_identity<OP>());
    }
  }
  int64_t j = full_lo + t;
  for (; j + (kUnroll - 1) * g < full_hi; j += kUnroll * g) {
    float x[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) load_input<T, VEC, MASK>(p, (j + u * g) * VEC, x[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int c = 0; c < VEC; ++c) st[c].fold(x[u][c]);
    }
  }
  for (; j < full_hi; j += g) {
    float x[VEC];
    load_input<T, VEC, MASK>(p, j * VEC, x);
#pragma unroll
    for (int c = 0; c < VEC; ++c) st[c].fold(x[c]);
  }
}

template <class T, int VEC, bool MASK>
__device__ __forceinline__ void normalize_flat(const Params& p, int g, int t, int64_t lo, int64_t hi,
                                               const float (&m)[VEC], const float (&inv)[VEC]) {
  if (lo >= hi) return;
  T* out = static_cast<T*>(p.out);
  const int64_t full_lo = (lo + VEC - 1) / VEC, full_hi = hi / VEC;
  const int64_t head = lo / VEC, tail = (hi - 1) / VEC;
  const bool head_partial = lo % VEC != 0 || (head == tail && hi % VEC != 0);
  const bool tail_partial = hi % VEC != 0 && tail != head;
  if ((head_partial && t == 0) || (tail_partial && t == 1)) {
    const int64_t j = t == 0 ? head : tail;
    float x[VEC];
    load_partial<T, VEC, MASK>(p, j, lo, hi, x);
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int64_t e = j * VEC + c;
      if (e >= lo && e < hi) Elem<T>::put(out + e, exp_out<T>(x[c] - m[c]) * inv[c]);
    }
  }
  for (int64_t j = full_lo + t; j < full_hi; j += g) {
    float x[VEC];
    load_input<T, VEC, MASK>(p, j * VEC, x);
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[c] = exp_out<T>(x[c] - m[c]) * inv[c];
    Elem<T>::template store<VEC>(out + j * VEC, x);
  }
}

// In FLAT mode component c holds feature c % D (D a power of two dividing
// VEC): fold components D.. into 0..D-1, each target in increasing c. The
// target is selected among the constant indices t < c, so no register
// array is indexed by a run-time value (which would place it in scratch).
template <int OP, int VEC>
__device__ __forceinline__ void merge_components(State<OP> (&st)[VEC], int d) {
#pragma unroll
  for (int c = 1; c < VEC; ++c) {
#pragma unroll
    for (int t = 0; t < c; ++t) {
      if (c >= d && (c & (d - 1)) == t) st[t].merge(st[c]);
    }
  }
}

// x[c] = x[c % D] for every component (D a power of two dividing VEC), with
// constant register indices only.
template <int VEC>
__device__ __forceinline__ void spread_components(float (&x)[VEC], int d) {
#pragma unroll
  for (int c = 1; c < VEC; ++c) {
#pragma unroll
    for (int t = 0; t < c; ++t) {
      if (c >= d && (c & (d - 1)) == t) x[c] = x[t];
    }
  }
}

// ---------------------------------------------------------------------------
// Workgroup reduction (G = kBlock) over lanes that share a feature lane:
// lanes agree modulo `lpr`. Every thread ends with the total for its own
// feature lane. `lds` holds kBlock * VEC * 2 floats.

template <int OP, int VEC>
__device__ __forceinline__ void block_reduce(State<OP> (&st)[VEC], int lpr, int feat_lane, float* lds) {
  constexpr int S = Slots<OP>::kCount;
  const int t = threadIdx.x, lane = t & (kWave - 1), w = t / kWave;
  if (lpr < kWave) wave_reduce_stride<OP, VEC>(st, lpr);
  const int rep = lpr < kWave ? lpr : kWave;
  if (lane < rep) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) st_write<OP>(lds + ((w * kWave + lane) * VEC + v) * S, 1, st[v]);
  }
  __syncthreads();
  State<OP> acc[VEC];
  if (t < lpr) {
    if (lpr <= kWave) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = st_read<OP>(lds + (t * VEC + v) * S, 1);
      for (int ww = 1; ww < kWavesPerBlock; ++ww) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v].merge(st_read<OP>(lds + ((ww * kWave + t) * VEC + v) * S, 1));
      }
    } else {
      const int wpr = lpr / kWave;              // waves per row
      const int w0 = t / kWave, l0 = t & (kWave - 1);
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = st_read<OP>(lds + ((w0 * kWave + l0) * VEC + v) * S, 1);
      for (int ww = w0 + wpr; ww < kWavesPerBlock; ww += wpr) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v].merge(st_read<OP>(lds + ((ww * kWave + l0) * VEC + v) * S, 1));
      }
    }
  }
  __syncthreads();
  if (t < lpr) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) st_write<OP>(lds + (t * VEC + v) * S, 1, acc[v]);
  }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < VEC; ++v) st[v] = st_read<OP>(lds + (feat_lane * VEC + v) * S, 1);
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Storing a reduction result / finishing softmax statistics.

template <class T, int VEC>
__device__ __forceinline__ void store_vec(T* dst, const float (&x)[VEC]) {
  Elem<T>::template store<VEC>(dst, x);
}

template <int OP>
__device__ __forceinline__ float value_of(const State<OP>& a) {
  if constexpr (OP == OP_SUM) return a.s;
  else return a.m;
}

template <int OP, int VEC>
__device__ __forceinline__ void result_of(const State<OP> (&st)[VEC], float (&x)[VEC]) {
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    if constexpr (OP == OP_SUM) x[v] = st[v].s;
    else x[v] = st[v].m;
  }
}

template <int VEC>
__device__ __forceinline__ void softmax_factors(const State<OP_SOFTMAX> (&st)[VEC], float (&m)[VEC],
                                                float (&inv)[VEC]) {
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    m[v] = st[v].m;
    inv[v] = 1.0f / st[v].s;
  }
}

// ---------------------------------------------------------------------------
// Whole-segment processing by a workgroup (block class, naive schedule) or
// by one wave (wave class). `g` = group size, `t` = thread index in group.

template <int OP, class T, int VEC, bool FLAT, bool MASK, bool BLOCK>
__device__ __forceinline__ void process_segment(const Params& p, int64_t s, int64_t start, int64_t end,
                                                int tile, float* lds) {
  constexpr int G = BLOCK ? kBlock : kWave;
  const int t = BLOCK ? threadIdx.x : (threadIdx.x & (kWave - 1));
  State<OP> st[VEC];
  init_all<OP, VEC>(st);
  if constexpr (FLAT) {
    const int64_t lo = start * p.d, hi = end * p.d;
    fold_flat<OP, T, VEC, MASK>(p, G, t, lo, hi, st);
    merge_components<OP, VEC>(st, p.d);
    if constexpr (BLOCK) block_reduce<OP, VEC>(st, 1, 0, lds);
    else wave_reduce_stride<OP, VEC>(st, 1);
    if constexpr (OP == OP_SOFTMAX) {
      float m[VEC], inv[VEC];
      softmax_factors<VEC>(st, m, inv);
      // Component c of every vector belongs to feature c % D.
      spread_components<VEC>(m, p.d);
      spread_components<VEC>(inv, p.d);
      normalize_flat<T, VEC, MASK>(p, G, t, lo, hi, m, inv);
    } else if (t == 0) {
      float x[VEC];
      result_of<OP, VEC>(st, x);
      T* out = static_cast<T*>(p.out) + s * p.d;
#pragma unroll
      for (int f = 0; f < VEC; ++f) {
        if (f < p.d) Elem<T>::put(out + f, x[f]);
      }
    }
  } else {
    const RowGeo g = row_geo<VEC>(p.d, G, t, tile);
    fold_rows<OP, T, VEC, MASK>(p, g, start, end, st);
    if constexpr (BLOCK) block_reduce<OP, VEC>(st, g.lpr, g.feat_lane, lds);
    else if (g.lpr < kWave) wave_reduce_stride<OP, VEC>(st, g.lpr);
    if constexpr (OP == OP_SOFTMAX) {
      float m[VEC], inv[VEC];
      softmax_factors<VEC>(st, m, inv);
      normalize_rows<T, VEC, MASK>(p, g, start, end, m, inv);
    } else if (g.row_lane == 0 && g.active) {
      float x[VEC];
      result_of<OP, VEC>(st, x);
      store_vec<T, VEC>(static_cast<T*>(p.out) + s * p.d + g.feature, x);
    }
  }
  if (p.visits && tile == 0 && t == 0) atomicAdd(p.visits + s, 1);
}

template <class OffT>
__device__ __forceinline__ void segment_rows(const Params& p, int64_t s, int64_t& start, int64_t& end) {
  // Clamp to [0, N] so that offsets that break the (unchecked) validated
  // contract can give wrong answers but never address outside values/out.
  start = offset_at<OffT>(p, s);
  end = offset_at<OffT>(p, s + 1);
  start = start < 0 ? 0 : (start > p.n ? p.n : start);
  end = end < start ? start : (end > p.n ? p.n : end);
}

// ---------------------------------------------------------------------------
// Kernels.

template <int OP, class T, class OffT, int VEC, bool FLAT, bool MASK>
__global__ __launch_bounds__(kBlock) void k_naive(Params p) {
  __shared__ float lds[kBlock * VEC * 2];
  for (int64_t s = blockIdx.x; s < p.b; s += gridDim.x) {
    int64_t start, end;
    segment_rows<OffT>(p, s, start, end);
    process_segment<OP, T, VEC, FLAT, MASK, true>(p, s, start, end, blockIdx.y, lds);
  }
}

// Rows of split item `item`: its part of its segment.
template <class OffT>
__device__ __forceinline__ void item_rows(const Params& p, int64_t item, int64_t& k, int64_t& s, int64_t& part,
                                          int64_t& start, int64_t& end) {
  k = p.item_pos[item];
  s = p.queue[2 * p.b + k];
  part = item - p.part_begin[k];
  int64_t seg_start, seg_end;
  segment_rows<OffT>(p, s, seg_start, seg_end);
  start = seg_start + part * p.part_rows;
  start = start > seg_end ? seg_end : start;
  end = start + p.part_rows > seg_end ? seg_end : start + p.part_rows;
}

// Features folded at once when a split segment's parts are combined:
// threads = part lanes x feature lanes (consecutive features, coalesced).
__device__ __forceinline__ int combine_features(int d) {
  int f = 1;
  while (f < d && f < kCombineFeatures) f <<= 1;
  return f;
}

// Workgroups of a persistent grid that take part in a call with `work`
// units: at most one per unit, at least one (it returns the counters to
// zero).
__device__ __forceinline__ int64_t active_workgroups(int64_t work) {
  const int64_t grid = gridDim.x;
  return work < 1 ? 1 : (work < grid ? work : grid);
}

// End of a classified call's last kernel: every active workgroup (blockIdx <
// `active`, all of whom read the counters first) counts itself out
// (once its stores are complete when `drain`: what the last workgroup then
// reads must be published); returns true in the last one. Up to
// kDirectDone workgroups count at counters[kDoneSlot] alone; more count in
// two levels, because atomics on one address serialise (about 12.5 ns each
// on MI355X): workgroup w at lane w % kTicketLanes (the done lanes,
// kTicketStride apart after the ticket lanes), the last of each lane at
// counters[kDoneSlot]. The last workgroup may still use the workspace; it
// then calls reset_counters. With `drain` the count is a release at agent
// scope (stores complete, then an L2 writeback, as in split_part) and the
// last workgroup acquires: what the others wrote is visible to it.
__device__ __forceinline__ bool last_out(const Params& p, int* flag_s, int64_t active, bool drain) {
  if (drain) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): this workgroup's stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    if (drain) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const unsigned count = (unsigned)active;
    bool last = false;
    if (count <= kDirectDone) {
      // Few workgroups: one counter serialises them in under a microsecond,
      // and the last one learns it one round trip sooner.
      last = atomicAdd((unsigned long long*)(p.counters + kDoneSlot), 1ull) == count - 1;
    } else {
      const unsigned lanes = kTicketLanes;
      const unsigned lane = blockIdx.x % lanes;
      const unsigned long long in_lane = (count - lane + lanes - 1) / lanes;   // active workgroups w = lane (mod lanes)
      unsigned long long* lane_counter =
          (unsigned long long*)(p.counters + kTicketStride * (1 + kTicketLanes + lane));
      if (atomicAdd(lane_counter, 1ull) == in_lane - 1)
        last = atomicAdd((unsigned long long*)(p.counters + kDoneSlot), 1ull) == lanes - 1;
    }
    if (last && drain) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    *flag_s = last ? 1 : 0;
  }
  __syncthreads();
  return *flag_s != 0;
}

// Every counter of the workspace back to zero, so the next call's
// k_classify starts from zero (the workspace's contract: all-zero before its
// first call, left so by every call), and the arena's state recorded: a
// register-resident softmax call leaves its arena zero but for `dirty` (the
// byte ranges of the pairs and group rows it published, which the next
// call's k_classify zeroes); any other call's buffers overlap that region,
// so it records the arena as unknown (1). A debug specialisation (visits
// set) keeps its counters for inspection instead; its workspace is fresh
// per call.
__device__ __forceinline__ void reset_counters(const Params& p, const int64_t* dirty = nullptr) {
  if (p.visits) return;
  const int t = threadIdx.x;
  if (t < kTicketStride) {
    int64_t v = 0;
    if (t == kCleanSlot) v = dirty ? p.arena_bytes + 2 : 1;
    else if (dirty && t >= kDirtySlot && t < kDirtySlot + 2 * kDirtyRanges) v = dirty[t - kDirtySlot];
    p.counters[t] = v;
  }
  if (t < 2 * kTicketLanes) p.counters[kTicketStride * (1 + t)] = 0;
}

#ifdef RG_PROLOGUE_KERNELS
// Defined in exactly one translation unit (kernels_common.hip).

// A workspace's counters back to their between-calls state (zero, the
// arena's clean extent none) after a call that failed part way may have left
// them set: the allocation-free entry point launches it on its static
// workspace before the next call on that device. One workgroup.
__global__ __launch_bounds__(kBlock) void k_reset(Params p) {
  const int t = threadIdx.x;
  if (t < kTicketStride) p.counters[t] = t == kCleanSlot ? 1 : 0;
  if (t < 2 * kTicketLanes) p.counters[kTicketStride * (1 + t)] = 0;
}

// Bin segments: wave (L <= t_wave), block (L <= t_block), split (longer).
// Per wave and class: ballot, rank by mbcnt, one atomic add reserves the
// wave's run of queue positions, so a wave's segments of one class sit in
// consecutive positions in segment order (classified-abi.md:56-66).
template <class OffT>
__global__ __launch_bounds__(kClassifyBlock) void k_classify(Params p) {
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int waves = (int)(blockDim.x / kWave);   // kWavesPerBlock or kClassifyWaves
  const int lane = threadIdx.x & (kWave - 1);
  const bool active = s < p.b;
  int64_t length = 0, start = 0;
  if (active) {
    int64_t end;
    segment_rows<OffT>(p, s, start, end);
    length = end - start;
  }
  // Run 0: wave-class segments one lane / lane group reduces alone (front
  // of the wave queue); run 3: the rest of the wave class, one wave each
  // (back of the wave queue); runs 1, 2: block and split classes.
  const int cls = length <= p.t_wave ? (length <= p.alone_rows ? 0 : 3) : (length <= p.t_block ? 1 : 2);
  if (active && p.visits) p.visits[s] = 0;
  // Register-resident softmax: its merges poll the arena's slots, which must
  // hold zero (unpublished) when it starts. The workspace's last call
  // recorded what it left nonzero (kCleanSlot, kDirtySlot): every thread of
  // the launch -- the plan gives it workgroups for this beyond the segments'
  // -- zeroes those ranges, and the part of this plan's arena beyond the
  // extent known to be zero, before the kernel that polls them starts. A
  // workspace as allocated is all zero.
  if (p.arena_bytes > 0) {
    // The workgroups past the segments' zero the arena alone, so that the
    // classification's workgroups are not held up by it (they do not even
    // read the record); without such workgroups every thread takes a share.
    const int64_t classifying = (p.b + blockDim.x - 1) / blockDim.x;
    const bool extra = gridDim.x > classifying;
    const int64_t first = extra ? classifying * blockDim.x : 0;
    const int64_t mark = !extra || (int64_t)blockIdx.x >= classifying ? p.counters[kCleanSlot] : 0;
    if (mark != 0) {
      const int64_t clean = mark == 1 ? 0 : (mark - 2 < p.arena_bytes ? mark - 2 : p.arena_bytes);
      {
        const int64_t threads = (int64_t)gridDim.x * blockDim.x - first;
        const int64_t tid = s - first;
        // [lo, hi) widened to 16-byte words: the bytes it adds are zero
        // already or zeroed here, and stay inside the arena (its size and
        // the clean extent are multiples of 256). Non-temporal stores: the
        // lines are not read again before the next kernel, and dirty L2
        // lines would be written back at this kernel's end.
        auto zero = [&](int64_t lo, int64_t hi) {
          lo = lo < 0 ? 0 : lo & ~(int64_t)15;
          hi = hi > p.arena_bytes ? p.arena_bytes : (hi + 15) & ~(int64_t)15;
          typedef unsigned words4 __attribute__((ext_vector_type(4)));
          words4* words = reinterpret_cast<words4*>(p.arena + lo);
          const words4 zero4 = {0u, 0u, 0u, 0u};
          for (int64_t i = tid; i < (hi - lo) / 16; i += threads) __builtin_nontemporal_store(zero4, words + i);
        };
        zero(clean, p.arena_bytes);
        if (mark >= 2) {
          for (int r = 0; r < kDirtyRanges; ++r) {
            const int64_t lo = p.counters[kDirtySlot + 2 * r], hi = p.counters[kDirtySlot + 2 * r + 1];
            if (lo < clean) zero(lo, hi < clean ? hi : clean);
          }
        }
      }
    }
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  // Queue runs: the workgroup (kBlock threads, or kClassifyBlock for many
  // segments) reserves each class's run with one atomic (not one per wave:
  // atomics on one counter serialise at the memory side, about 12.5 ns each,
  // so fewer and larger workgroups reserve faster), and each wave takes its part
  // of the run in wave order, so a wave's (and the workgroup's) segments of
  // one class sit in consecutive positions in segment order
  // (classified-abi.md:56-66).
  //
  // The register-resident softmax (p.items set) also reserves its split
  // segments' items in the same round of atomics: the direct chunks (runs
  // 4), the tree chunks (5) and the tree segments' group rows (6), each
  // workgroup's total with one atomic and each segment's range at its
  // exclusive prefix within the workgroup, in segment order. A reservation
  // per segment after the queue's would be one more dependent round trip,
  // and its result would also wait for the queue stores issued before it
  // (vmcnt counts loads and stores in issue order).
  __shared__ long long run_s[7][kClassifyWaves];
  const int wave = threadIdx.x / kWave;
  uint64_t ballots[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    ballots[c] = __ballot(active && cls == c);
    if (lane == 0) run_s[c][wave] = (long long)__popcll(ballots[c]);
  }
  const bool split_items = p.items != nullptr;
  const long long split_parts = split_items && active && cls == 2 ? (length + p.part_rows - 1) / p.part_rows : 0;
  const bool tree = split_parts > kDirect;
  long long split_before[3] = {0, 0, 0};   // direct parts, tree parts, group rows of the wave's lanes below
  if (split_items && ballots[2] != 0) {
    const long long mine3[3] = {tree ? 0 : split_parts, tree ? split_parts : 0,
                                tree ? (split_parts + kTreeGroup - 1) / kTreeGroup : 0};
#pragma unroll
    for (int r = 0; r < 3; ++r) {
      long long x = mine3[r];
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const long long y = __shfl_up(x, off, kWave);
        if (lane >= off) x += y;
      }
      split_before[r] = x - mine3[r];
      if (lane == kWave - 1) run_s[4 + r][wave] = x;
    }
  } else if (split_items && lane == 0) {
    run_s[4][wave] = run_s[5][wave] = run_s[6][wave] = 0;
  }
  __syncthreads();
  if (threadIdx.x < (split_items ? 7 : 4)) {
    const int c = threadIdx.x;
    long long total = 0;
    for (int w = 0; w < waves; ++w) total += run_s[c][w];
    // Run 3 is counted in counters[8]. A register-resident softmax
    // (block_items set) counts run 0 in counters[7]: k_softmax_fused takes
    // the wave class after its items from counters[7] and [8], and its item
    // count, which adds counters[0], sees none. Its split reservations:
    // direct chunks in counters[3], tree chunks (from the top of the item
    // array) in counters[6], group rows in counters[kGroupRowSlot].
    const int slot = c == 3 ? 8 : c == 0 && p.block_items ? 7 : c == 4 ? 3 : c == 5 ? 6 : c == 6 ? kGroupRowSlot : c;
    long long base = total ? (long long)atomicAdd((unsigned long long*)(p.counters + slot), (unsigned long long)total) : 0;
    for (int w = 0; w < waves; ++w) {
      const long long count = run_s[c][w];
      run_s[c][w] = base;
      base += count;
    }
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool mine = active && cls == c;
    const uint64_t ballot = ballots[c];
    if (ballot == 0) continue;
    const int64_t pos = run_s[c][wave] + __popcll(ballot & below);
    // A class holds at most B segments; only counters a failed call left set
    // could reserve past that, and nothing is written there.
    if (mine && pos < p.b) p.queue[c == 3 ? p.b - 1 - pos : c * p.b + pos] = s;
    // Register-resident softmax: whole block-class segments are items too.
    if (mine && c == 1 && p.block_items && pos < p.b) p.block_items[pos] = Item{start, s, (int32_t)length, -1, 0, 1};
    if (c != 2) continue;
    // Split segments reserve ceil(L / part_rows) consecutive items. Valid
    // offsets never put more than b_split segments in the split queue;
    // clamped invalid ones could, so never index past it. The
    // register-resident softmax (p.items set) takes segments of more than
    // kDirect chunks from the top of the item array, so they are dequeued
    // first, while every workgroup of the grid is still free to hold one.
    long long first = 0, parts = 0, gbase = 0;
    bool fits = true;
    if (mine && split_items) {
      // Reserved before the queue position was known: a segment past b_split
      // (clamped invalid offsets only) still owns its items, written empty.
      const bool owned = pos < p.b_split;
      parts = split_parts;
      if (tree) {
        const long long above = run_s[5][wave] + split_before[1];
        first = (long long)p.items_cap - above - parts;
        // The segment's rows of final_pairs, one per group of kTreeGroup.
        const long long groups = (parts + kTreeGroup - 1) / kTreeGroup;
        gbase = run_s[6][wave] + split_before[2];
        fits = owned && first >= 0 && gbase + groups <= tree_group_rows(p.items_cap);
      } else {
        first = run_s[4][wave] + split_before[0];
        fits = owned && first + parts <= p.items_cap;
      }
      if (owned && p.part_begin) p.part_begin[pos] = first;
      if (owned && p.seg_arrive) p.seg_arrive[pos] = 0;
    } else if (mine && pos < p.b_split) {
      // Streaming worker: a reserved item must name a queued segment, so the
      // reservation waits for the queue position.
      parts = (length + p.part_rows - 1) / p.part_rows;
      first = (long long)atomicAdd((unsigned long long*)(p.counters + 3), (unsigned long long)parts);
      fits = first + parts <= p.items_cap;
      if (p.part_begin) p.part_begin[pos] = first;
      // The segment's part arrivals start at zero (streaming worker; the
      // register-resident softmax's counters are in its arena).
      if (p.seg_arrive) p.seg_arrive[pos] = 0;
    }
    if (p.items) {
      // Item descriptors. An allocation that does not fit the array (only
      // inconsistent offsets make one) becomes empty items that touch no
      // memory. Up to kDirect chunks: each lane writes its own segment's.
      auto describe = [&](int64_t i, long long f, long long count, long long k, long long seg, long long seg_start,
                          long long seg_rows, bool whole) {
        const int64_t c = i - f;
        const int64_t rows = seg_rows - c * p.part_rows < p.part_rows ? seg_rows - c * p.part_rows : p.part_rows;
        Item item{0, seg, 0, -1, 1, 1};
        if (whole) item = Item{seg_start + c * p.part_rows, seg, (int32_t)rows, (int32_t)k, (int32_t)c, (int32_t)count};
        p.items[i] = item;
      };
      if (parts > 0 && parts <= kDirect) {
        const int64_t lo = first > 0 ? first : 0;
        const int64_t last = first + parts < p.items_cap ? first + parts : p.items_cap;
        for (int64_t i = lo; i < last; ++i) describe(i, first, parts, pos, s, start, length, fits);
      }
      uint64_t todo = __ballot(parts > kDirect);
      while (todo) {
        const int src = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1;
        const long long f = lane_value((int64_t)first, src), count = lane_value((int64_t)parts, src);
        const int64_t lo = f > 0 ? f : 0;
        const int64_t last = f + count < p.items_cap ? f + count : p.items_cap;
        // A tree-merged chunk's k: its segment's first row of final_pairs.
        const long long k = lane_value((int64_t)gbase, src), seg = lane_value((int64_t)s, src);
        const long long seg_start = lane_value((int64_t)start, src);
        const long long seg_rows = lane_value((int64_t)length, src);
        const bool whole = lane_value((int)fits, src) != 0;
        for (int64_t i = lo + lane; i < last; i += kWave) describe(i, f, count, k, seg, seg_start, seg_rows, whole);
      }
      continue;
    }
    // Split pipeline: the whole wave writes each split segment's entries.
    uint64_t todo = __ballot(parts > 0);
    while (todo) {
      const int src = __ffsll((unsigned long long)todo) - 1;
      todo &= todo - 1;
      const long long f = lane_value((int64_t)first, src), count = lane_value((int64_t)parts, src);
      const long long k = lane_value((int64_t)pos, src);
      const int64_t last = f + count < p.items_cap ? f + count : p.items_cap;
      for (int64_t i = f + lane; i < last; i += kWave) {
        if (p.item_pos) p.item_pos[i] = k;
      }
    }
  }
}

// Checked mode (checked-abi.md): earliest offending index per condition.
__global__ __launch_bounds__(kBlock) void k_offsets_init(Params p) {
  if (threadIdx.x < 7) p.status[threadIdx.x] = INT64_MAX;
}

template <class OffT>
__global__ __launch_bounds__(kBlock) void k_offsets_check(Params p) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i > p.b) return;
  long long* status = reinterpret_cast<long long*>(p.status);
  const int64_t o = offset_at<OffT>(p, i);
  if (i == 0 && o != 0) atomicMin(status + 0, 0ll);
  if (i == p.b && o != p.n) atomicMin(status + 1, (long long)p.b);
  if (o < 0) atomicMin(status + 2, (long long)i);
  if (o > p.n) atomicMin(status + 3, (long long)i);
  if (i < p.b) {
    const int64_t next = offset_at<OffT>(p, i + 1);
    if (next < o) {
      atomicMin(status + 4, (long long)i);
    } else if (o >= 0 && next <= p.n) {
      const int64_t length = next - o;   // both ends in [0, N] and ordered: no overflow
      if (p.min_len >= 0 && length < p.min_len) atomicMin(status + 5, (long long)i);
      if (p.max_len >= 0 && length > p.max_len) atomicMin(status + 6, (long long)i);
    }
  }
}

#endif  // RG_PROLOGUE_KERNELS

}  // namespace rg
