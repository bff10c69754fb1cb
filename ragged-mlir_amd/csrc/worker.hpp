// The classified schedule's worker for sum, max and the softmax that has no
// register-resident worker (small or unvectorised feature widths).
//
// k_classify bins every segment into the wave, block and split queues
// (reference ToGPU.cpp:901-998, wave64 thresholds). The reference then runs
// one persistent kernel chain per class on forked streams
// (ToGPU.cpp:999-1045, Driver.cpp:299-353). Here one persistent launch
// drains all of them by atomic ticket (16 interleaved ticket counters: one
// address serialises atomics), longest work first:
//   1. the parts of split segments; the part that arrives last at its
//      segment's counter folds every part in part order (deterministic) and
//      writes the result (sum, max) or the merged statistics (softmax) --
//      the reference's split_combine (ToGPU.cpp:399-472) without a separate
//      launch;
//   2. block-class segments, one workgroup each;
//   3. wave-class segments longer than alone_rows, one wave each (queued
//      from the back of the wave queue);
//   4. batches of wave-class segments of at most alone_rows rows, each
//      reduced alone by one lane (flat mapping, D below the vector width) or
//      by the group of lanes that holds a row -- a batch costs one pass of
//      the wave instead of one wave-wide reduction per segment.
// Softmax, once a workgroup's tickets run out: the split parts'
// probabilities (the reference's split_normalize, ToGPU.cpp:279-281), from
// a counter of their own, each after its segment's statistics are out.
// The short-segment schedule runs only step 4, over every segment in order.
#pragma once

#include "kernels.hpp"

namespace rg {

// kLaneElems (flat elements one lane reduces on its own) is in device.hpp.

// Agent-scope stores / loads of the split partials: parts run on any XCD,
// and the last arriver must see every part's values.
__device__ __forceinline__ void publish(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fetch(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Feature tiles of a group of G threads (ROW mapping): lanes per row is
// capped by G, and the remaining lanes of a row are further tiles.
template <int VEC>
__device__ __forceinline__ int tiles_of(int d, int g) {
  const int lanes = (d + VEC - 1) / VEC;
  const int lpr = lanes_per_row(d, VEC, g);
  return (lanes + lpr - 1) / lpr;
}

// Vectors j0 .. j1 (elements j*VEC .. j*VEC + VEC - 1) of the flat input,
// U at a time: body(j, x) for each. Whole vectors are loaded U at a time
// with no branch between the loads, so they are all in flight together; in
// the last round, short of U, a load past jv re-reads vector jv (in cache)
// and is not passed on. The one vector that reaches past the array's last
// element (N*D not a multiple of VEC) is read element by element, so no
// load leaves the array.
template <int U, class T, int VEC, bool MASK, class Body>
__device__ __forceinline__ void flat_vectors(const Params& p, int64_t j0, int64_t j1, Body&& body) {
  const int64_t total = p.n * p.d, full = total / VEC;
  const int64_t jv = j1 < full ? j1 : full - 1;     // last whole vector
  int64_t j = j0;
  for (; j + (U - 1) <= jv; j += U) {
    float x[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) load_input<T, VEC, MASK>(p, (j + u) * VEC, x[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) body(j + u, x[u]);
  }
  if (j <= jv) {
    float x[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) load_input<T, VEC, MASK>(p, (j + u <= jv ? j + u : jv) * VEC, x[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j + u <= jv) body(j + u, x[u]);
    }
  }
  if (j1 > jv) {
    float x[VEC];
    load_partial<T, VEC, MASK>(p, j1, j1 * VEC, total, x);   // components past the array are masked by body
    body(j1, x);
  }
}

// ---------------------------------------------------------------------------
// One lane reduces elements [lo, hi) of a flat-mapped segment: aligned
// VEC-element vectors, components outside [lo, hi) masked. Component c of
// every vector is feature c % D (D divides VEC).

template <int OP, class T, int VEC, bool MASK>
__device__ __forceinline__ void lane_fold(const Params& p, int64_t lo, int64_t hi, State<OP> (&st)[VEC]) {
  init_all<OP, VEC>(st);
  if (lo >= hi) return;
  flat_vectors<8, T, VEC, MASK>(p, lo / VEC, (hi - 1) / VEC, [&](int64_t j, const float (&x)[VEC]) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int64_t e = j * VEC + c;
      st[c].fold(e >= lo && e < hi ? x[c] : fold_identity<OP>());
    }
  });
}

// Combines the components of each feature in place: component c holds
// feature c % d (d a power of two dividing VEC). Afterwards every component
// holds the combination of its feature's components, so no register array
// is indexed by a run-time value.
template <bool MAX, int VEC>
__device__ __forceinline__ void fold_residues(float (&x)[VEC], int d) {
#pragma unroll
  for (int off = VEC / 2; off >= 1; off /= 2) {
    if (off >= d) {
#pragma unroll
      for (int c = 0; c < off; ++c) x[c] = MAX ? fmax_nan(x[c], x[c + off]) : x[c] + x[c + off];
    }
  }
#pragma unroll
  for (int off = 1; off < VEC; off *= 2) {
    if (off >= d) {
#pragma unroll
      for (int c = 0; c < off; ++c) x[c + off] = x[c];
    }
  }
}

// A softmax column sum of exp terms in [0, 1]: compensated (Kahan) for f32
// outputs, as the reference's statistics are (ToGPU.cpp:377-387, 509-603),
// plain for bf16 outputs (far below their rounding).
template <class T>
struct ExpSum {
  float s = 0.f, c = 0.f;
  __device__ void add(float e) {
    if constexpr (std::is_same<T, float>::value) {
#pragma clang fp contract(off)
      const float y = e - c;
      const float t = s + y;
      c = (t - s) - y;
      s = t;
    } else {
      s += e;
    }
  }
};

// Vectors a lane holds in registers for a short flat segment (48 floats).
template <int VEC>
constexpr int kLaneVectors = 48 / VEC;

// Softmax of a flat-mapped segment of at most kLaneVectors whole vectors by
// one lane, held in registers: all loads in one round, then column max,
// exp(x - ref) in place, column sums and the stores. A column of only -inf
// has no mass (ref 0). Vectors past j1 re-read vector j1 and are not used.
template <class T, int VEC, bool MASK>
__device__ __forceinline__ void lane_softmax_held(const Params& p, int64_t lo, int64_t hi, int64_t j0, int64_t j1) {
  constexpr int K = kLaneVectors<VEC>;
  const int d = p.d;
  float x[K][VEC];
#pragma unroll
  for (int u = 0; u < K; ++u) load_input<T, VEC, MASK>(p, (j0 + u <= j1 ? j0 + u : j1) * VEC, x[u]);
  auto inside = [&](int u, int c) {
    const int64_t e = (j0 + u) * VEC + c;
    return j0 + u <= j1 && e >= lo && e < hi;
  };
  float m[VEC], ref[VEC], s[VEC], inv[VEC];
  ExpSum<T> acc[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) m[c] = neg_inf();
#pragma unroll
  for (int u = 0; u < K; ++u) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) m[c] = inside(u, c) ? fmax_nan(m[c], x[u][c]) : m[c];
  }
  fold_residues<true, VEC>(m, d);
#pragma unroll
  for (int c = 0; c < VEC; ++c) ref[c] = m[c] == neg_inf() ? 0.f : m[c];
#pragma unroll
  for (int u = 0; u < K; ++u) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      x[u][c] = exp_out<T>(x[u][c] - ref[c]);
      acc[c].add(inside(u, c) ? x[u][c] : 0.f);
    }
  }
#pragma unroll
  for (int c = 0; c < VEC; ++c) s[c] = acc[c].s;
  fold_residues<false, VEC>(s, d);
#pragma unroll
  for (int c = 0; c < VEC; ++c) inv[c] = fast_exp(m[c] - m[c]) / s[c];   // 1 / s, or NaN for an all -inf column
  T* out = static_cast<T*>(p.out);
#pragma unroll
  for (int u = 0; u < K; ++u) {
    if (j0 + u > j1) break;
    const int64_t j = j0 + u;
    float y[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) y[c] = x[u][c] * inv[c];
    if (j * VEC >= lo && j * VEC + VEC <= hi) {
      Elem<T>::template store<VEC>(out + j * VEC, y);   // a whole vector of this segment
    } else {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        if (inside(u, c)) Elem<T>::put(out + j * VEC + c, y[c]);
      }
    }
  }
}

// Softmax of a flat-mapped segment by one lane: column max, column sum of
// exp(x - ref) and the normalised values. A segment of at most kLaneVectors
// whole vectors is held in registers (one read); a longer one, or the one
// that reaches the array's partial last vector, takes three passes over
// its elements (re-read from cache). A column of only -inf has no mass.
template <class T, int VEC, bool MASK>
__device__ __forceinline__ void lane_softmax(const Params& p, int64_t lo, int64_t hi) {
  if (lo >= hi) return;
  const int d = p.d;
  const int64_t j0 = lo / VEC, j1 = (hi - 1) / VEC;
  if (j1 - j0 < kLaneVectors<VEC> && j1 < p.n * p.d / VEC) {
    lane_softmax_held<T, VEC, MASK>(p, lo, hi, j0, j1);
    return;
  }
  // Every pass visits the segment's vectors four at a time (four loads in
  // flight per lane).
  auto pass = [&](auto&& body) { flat_vectors<4, T, VEC, MASK>(p, j0, j1, body); };
  float m[VEC];   // per component; component c is feature c % d
#pragma unroll
  for (int c = 0; c < VEC; ++c) m[c] = neg_inf();
  pass([&](int64_t j, const float (&x)[VEC]) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int64_t e = j * VEC + c;
      if (e >= lo && e < hi) m[c] = fmax_nan(m[c], x[c]);
    }
  });
  fold_residues<true, VEC>(m, d);
  float ref[VEC], s[VEC];
  ExpSum<T> acc[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) ref[c] = m[c] == neg_inf() ? 0.f : m[c];
  pass([&](int64_t j, const float (&x)[VEC]) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int64_t e = j * VEC + c;
      if (e >= lo && e < hi) acc[c].add(exp_out<T>(x[c] - ref[c]));
    }
  });
#pragma unroll
  for (int c = 0; c < VEC; ++c) s[c] = acc[c].s;
  fold_residues<false, VEC>(s, d);
  float inv[VEC];
#pragma unroll
  for (int c = 0; c < VEC; ++c) inv[c] = fast_exp(m[c] - m[c]) / s[c];   // 1 / s, or NaN for an all -inf column
  T* out = static_cast<T*>(p.out);
  pass([&](int64_t j, const float (&in)[VEC]) {
    float x[VEC];
#pragma unroll
    for (int c = 0; c < VEC; ++c) x[c] = exp_out<T>(in[c] - ref[c]) * inv[c];
    if (j * VEC >= lo && j * VEC + VEC <= hi) {
      Elem<T>::template store<VEC>(out + j * VEC, x);   // a whole vector of this segment
    } else {
#pragma unroll
      for (int c = 0; c < VEC; ++c) {
        const int64_t e = j * VEC + c;
        if (e >= lo && e < hi) Elem<T>::put(out + e, x[c]);
      }
    }
  });
}

// A wave-class segment reduced by one lane (flat mapping).
template <int OP, class T, int VEC, bool MASK>
__device__ __forceinline__ void lane_segment(const Params& p, int64_t s, int64_t start, int64_t end) {
  const int64_t lo = start * p.d, hi = end * p.d;
  if constexpr (OP == OP_SOFTMAX) {
    lane_softmax<T, VEC, MASK>(p, lo, hi);
  } else {
    State<OP> st[VEC];
    lane_fold<OP, T, VEC, MASK>(p, lo, hi, st);
    merge_components<OP, VEC>(st, p.d);
    T* out = static_cast<T*>(p.out) + s * p.d;
#pragma unroll
    for (int f = 0; f < VEC; ++f) {
      if (f < p.d) Elem<T>::put(out + f, value_of<OP>(st[f]));
    }
  }
  if (p.visits) atomicAdd(p.visits + s, 1);
}

// A wave-class segment in the row mapping reduced by a group of lanes that
// together hold one row (lane `feature_lane` owns features feature_lane*VEC
// .. +VEC): every lane walks all rows of the segment on its own, so no lane
// waits for another; eight rows' loads in flight per lane.
template <int OP, class T, int VEC, bool MASK>
__device__ __forceinline__ void group_segment(const Params& p, int64_t s, int64_t start, int64_t end,
                                              int feature_lane) {
  const int64_t d = p.d;
  const int64_t f0 = (int64_t)feature_lane * VEC;
  if (f0 < d) {
    // Rows past the segment re-read its last row (in cache) instead of
    // branching around the load, so the eight loads issue back to back.
    auto rows = [&](auto&& body) {
      for (int64_t r = start; r < end; r += 8) {
        float x[8][VEC];
#pragma unroll
        for (int u = 0; u < 8; ++u) load_input<T, VEC, MASK>(p, (r + u < end ? r + u : end - 1) * d + f0, x[u]);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (r + u < end) body(r + u, x[u]);
        }
      }
    };
    if constexpr (OP == OP_SOFTMAX) {
      float m[VEC], ref[VEC], inv[VEC];
      ExpSum<T> sum[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) m[v] = neg_inf();
      rows([&](int64_t, const float (&x)[VEC]) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) m[v] = fmax_nan(m[v], x[v]);
      });
#pragma unroll
      for (int v = 0; v < VEC; ++v) ref[v] = m[v] == neg_inf() ? 0.f : m[v];
      rows([&](int64_t, const float (&x)[VEC]) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) sum[v].add(exp_out<T>(x[v] - ref[v]));
      });
#pragma unroll
      for (int v = 0; v < VEC; ++v) inv[v] = fast_exp(m[v] - m[v]) / sum[v].s;   // NaN for an all -inf column
      T* out = static_cast<T*>(p.out);
      rows([&](int64_t r, const float (&x)[VEC]) {
        float y[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) y[v] = exp_out<T>(x[v] - ref[v]) * inv[v];
        Elem<T>::template store<VEC>(out + r * d + f0, y);
      });
    } else {
      State<OP> st[VEC];
      init_all<OP, VEC>(st);
      rows([&](int64_t, const float (&x)[VEC]) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) st[v].fold(x[v]);
      });
      float y[VEC];
      result_of<OP, VEC>(st, y);
      Elem<T>::template store<VEC>(static_cast<T*>(p.out) + s * d + f0, y);
    }
  }
  if (p.visits && feature_lane == 0) atomicAdd(p.visits + s, 1);
}

// ---------------------------------------------------------------------------
// Split parts: the part's fold into partials[item] (agent scope), then the
// last part of the segment to arrive folds all of them in part order.

template <int OP, class T, class OffT, int VEC, bool FLAT, bool MASK>
__device__ __forceinline__ void split_part(const Params& p, int64_t item, int tile, float* lds, int* flag_s) {
  const int t = threadIdx.x;
  int64_t k, s, part, start, end;
  item_rows<OffT>(p, item, k, s, part, start, end);
  State<OP> st[VEC];
  init_all<OP, VEC>(st);
  if constexpr (FLAT) {
    fold_flat<OP, T, VEC, MASK>(p, kBlock, t, start * p.d, end * p.d, st);
    merge_components<OP, VEC>(st, p.d);
    block_reduce<OP, VEC>(st, 1, 0, lds);
    if (t == 0) {
#pragma unroll
      for (int f = 0; f < VEC; ++f) {
        if (f < p.d) {
          publish(p.partials + item * p.d + f, value_of<OP>(st[f]));
          if constexpr (OP == OP_SOFTMAX) publish(p.partial_sums + item * p.d + f, st[f].s);
        }
      }
    }
  } else {
    const RowGeo g = row_geo<VEC>(p.d, kBlock, t, tile);
    fold_rows<OP, T, VEC, MASK>(p, g, start, end, st);
    block_reduce<OP, VEC>(st, g.lpr, g.feat_lane, lds);
    if (g.row_lane == 0 && g.active) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        if (g.feature + v < p.d) {
          publish(p.partials + item * p.d + g.feature + v, value_of<OP>(st[v]));
          if constexpr (OP == OP_SOFTMAX) publish(p.partial_sums + item * p.d + g.feature + v, st[v].s);
        }
      }
    }
  }
  // Arrival: once this part's stores have completed (every thread waits
  // for its own, then the barrier), count it at the segment. The segment's
  // parts are the items [first, stop) that exist: valid offsets always give
  // all of them; offsets that break the contract can reserve items past
  // items_cap, which are never run, so the target counts only those below.
  int64_t seg_start, seg_end;
  segment_rows<OffT>(p, s, seg_start, seg_end);
  const int64_t all_parts = (seg_end - seg_start + p.part_rows - 1) / p.part_rows;
  const int tiles = FLAT ? 1 : tiles_of<VEC>(p.d, kBlock);
  const int64_t first = p.part_begin[k];
  const int64_t stop = first + all_parts < p.items_cap ? first + all_parts : p.items_cap;
  //
  // Ordering (the LLVM AMDGPU memory model for gfx942/gfx950): the arrival
  // is a release at agent scope -- every thread's stores complete
  // (s_waitcnt vmcnt(0)) before the barrier, then thread 0's release fence
  // (buffer_wbl2 sc1: the XCD's L2 written back) precedes the atomic -- and
  // the last arriver acquires at agent scope (buffer_inv sc1) before the
  // barrier after which its threads read the other parts' partials. Parts
  // run on any XCD, each with its own L2.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  if (t == 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const bool last = atomicAdd(p.seg_arrive + k, 1) == (stop - first) * tiles - 1;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    *flag_s = last;
  }
  __syncthreads();
  const bool last = *flag_s != 0;
  __syncthreads();
  if (!last) return;
  // Combine: threads = part lanes x features, LDS tree over part lanes, the
  // parts folded in order within each lane and lanes in order.
  const int ft = combine_features(p.d);
  const int pl_count = kBlock / ft;
  const int fl = t % ft, pl = t / ft;
  for (int64_t f0 = 0; f0 < p.d; f0 += ft) {
    const int64_t f = f0 + fl;
    State<OP> acc;
    acc.init();
    if (f < p.d) {
      // Contiguous runs of parts per lane keep the fold in part order.
      const int64_t count = stop - first;
      const int64_t lo = first + count * pl / pl_count, hi = first + count * (pl + 1) / pl_count;
      for (int64_t item2 = lo; item2 < hi; ++item2) {
        if constexpr (OP == OP_SUM) {
          acc.fold(fetch(p.partials + item2 * p.d + f));
        } else {
          State<OP> part_st;
          part_st.m = fetch(p.partials + item2 * p.d + f);
          if constexpr (OP == OP_SOFTMAX) part_st.s = fetch(p.partial_sums + item2 * p.d + f);
          acc.merge(part_st);
        }
      }
    }
    st_write<OP>(lds + t, kBlock, acc);
    __syncthreads();
    if (pl == 0 && f < p.d) {
      for (int q = 1; q < pl_count; ++q) acc.merge(st_read<OP>(lds + q * ft + fl, kBlock));
      if constexpr (OP == OP_SOFTMAX) {
        publish(p.stats_max + k * p.d + f, acc.m);
        publish(p.stats_sum + k * p.d + f, acc.s);
      } else {
        Elem<T>::put(static_cast<T*>(p.out) + s * p.d + f, value_of<OP>(acc));
      }
    }
    __syncthreads();
  }
  if constexpr (OP != OP_SOFTMAX) {
    if (p.visits && t == 0) atomicAdd(p.visits + s, 1);
  } else {
    // The statistics are complete once every thread's stores are: release
    // the segment's parts to their normalisation (normalize_part), with
    // the same agent-scope release as the arrival above.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    if (t == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __hip_atomic_store(p.seg_arrive + k, kStatsReady, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Softmax probabilities of split part `item` (feature tile `tile`) with its
// segment's combined statistics (ToGPU.cpp:279-281), once the segment's last
// part has published them. With `wait`, the workgroup waits for them for at
// most drain_ticks and returns false, having written nothing, if they are
// still out: the caller defers the part (k_worker). The wait normally ends
// well before: every part was handed to a running workgroup before any
// workgroup gets here, and a part never waits. Without `wait` the statistics
// must already be published.
template <class T, class OffT, int VEC, bool FLAT, bool MASK>
__device__ __forceinline__ bool normalize_part(const Params& p, int64_t item, int tile, bool wait) {
  const int t = threadIdx.x;
  int64_t k, s, part, start, end;
  item_rows<OffT>(p, item, k, s, part, start, end);
  if (wait) {
    bool ready = true;
    if (t == 0) {
      const long long t0 = wall_clock64();
      while (__hip_atomic_load(p.seg_arrive + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != kStatsReady) {
        if (wall_clock64() - t0 >= p.drain_ticks) {
          ready = false;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      // Acquire at agent scope: the statistics read below were released
      // before the flag.
      if (ready) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    if (block_any(!ready)) return false;
  }
  float m[VEC], inv[VEC];
  if constexpr (FLAT) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int f = c % p.d;
      m[c] = fetch(p.stats_max + k * p.d + f);
      inv[c] = 1.0f / fetch(p.stats_sum + k * p.d + f);
    }
    normalize_flat<T, VEC, MASK>(p, kBlock, t, start * p.d, end * p.d, m, inv);
  } else {
    const RowGeo g = row_geo<VEC>(p.d, kBlock, t, tile);
    if (g.active) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        m[v] = fetch(p.stats_max + k * p.d + g.feature + v);
        inv[v] = 1.0f / fetch(p.stats_sum + k * p.d + g.feature + v);
      }
      normalize_rows<T, VEC, MASK>(p, g, start, end, m, inv);
    }
  }
  if (p.visits && part == 0 && tile == 0 && t == 0) atomicAdd(p.visits + s, 1);
  return true;
}

// ---------------------------------------------------------------------------
// Wave-class batches: in the flat mapping 64 segments per wave, one per
// lane; in the row mapping one per group of the G lanes that hold a row
// (64 / G per wave), or one per wave when a row needs more than a wave.

template <bool FLAT, int VEC>
__device__ __forceinline__ int wave_group(int d) {
  return FLAT ? 1 : (tiles_of<VEC>(d, kWave) == 1 ? lanes_per_row(d, VEC, kWave) : kWave);
}

template <bool FLAT, int VEC>
__device__ __forceinline__ int64_t wave_batch_size(int d) {
  return (int64_t)(kWave / wave_group<FLAT, VEC>(d)) * kWavesPerBlock;
}

// Batch `index` of the wave-class segments reduced alone: queue positions
// index*batch .. of the first n_wave (every segment in order if `direct`).
template <int OP, class T, class OffT, int VEC, bool FLAT, bool MASK>
__device__ __forceinline__ void wave_batch(const Params& p, int64_t index, int64_t n_wave, bool direct) {
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1), w = t / kWave;
  const int tiles_wave = FLAT ? 1 : tiles_of<VEC>(p.d, kWave);
  const int group = wave_group<FLAT, VEC>(p.d);
  const int per_wave = kWave / group;
  // Wave w takes per_wave positions, one per group.
  const int64_t pos = index * per_wave * kWavesPerBlock + w * per_wave + lane / group;
  const bool have = pos < n_wave;
  int64_t s = 0, start = 0, end = 0;
  if (have) {
    s = direct ? pos : p.queue[pos];
    segment_rows<OffT>(p, s, start, end);
  }
  // Reduced by its own lane (flat mapping) or lane group (rows narrower
  // than a wave) when at most alone_rows long, else by the whole wave (only
  // `direct` batches hold such segments: k_classify queues them apart).
  const bool alone = have && (FLAT || group < kWave) && end - start <= p.alone_rows;
  if (alone) {
    if constexpr (FLAT) lane_segment<OP, T, VEC, MASK>(p, s, start, end);
    else group_segment<OP, T, VEC, MASK>(p, s, start, end, lane % group);
  }
  uint64_t todo = __ballot(have && !alone && lane % group == 0);   // one bit per group
  while (todo) {
    const int src = __ffsll((unsigned long long)todo) - 1;
    todo &= todo - 1;
    const int64_t ss = lane_value(s, src);
    const int64_t a = lane_value(start, src), b = lane_value(end, src);
    for (int tile = 0; tile < tiles_wave; ++tile) process_segment<OP, T, VEC, FLAT, MASK, false>(p, ss, a, b, tile, nullptr);
  }
}

// Batch `index` of the rest of the wave class (queued from the back, n_coop
// segments): one segment per wave, reduced by the whole wave.
template <int OP, class T, class OffT, int VEC, bool FLAT, bool MASK>
__device__ __forceinline__ void coop_batch(const Params& p, int64_t index, int64_t n_coop) {
  const int w = threadIdx.x / kWave;
  const int64_t pos = index * kWavesPerBlock + w;
  if (pos >= n_coop) return;
  const int64_t s = p.queue[p.b - 1 - pos];
  int64_t start, end;
  segment_rows<OffT>(p, s, start, end);
  const int tiles_wave = FLAT ? 1 : tiles_of<VEC>(p.d, kWave);
  for (int tile = 0; tile < tiles_wave; ++tile) process_segment<OP, T, VEC, FLAT, MASK, false>(p, s, start, end, tile, nullptr);
}

template <int OP, class T, class OffT, int VEC, bool FLAT, bool MASK>
__global__ __launch_bounds__(kBlock) void k_worker(Params p) {
  __shared__ float lds[kBlock * VEC * 2];
  __shared__ int64_t ticket_s;
  __shared__ int flag_s;
  const int t = threadIdx.x;
  const int tiles_block = FLAT ? 1 : tiles_of<VEC>(p.d, kBlock);
  // Ticket order: split parts (x feature tiles), block-class segments,
  // wave-class segments one per wave, batches of wave-class segments
  // reduced alone.
  const int64_t batch = wave_batch_size<FLAT, VEC>(p.d);
  // Short-segment schedule: every segment, in order, is wave class; no
  // counters, grid-stride batches.
  const bool direct = p.short_segments != 0;
  const int64_t n_items = direct ? 0 : (p.counters[3] < p.items_cap ? p.counters[3] : p.items_cap);
  const int64_t n_parts = n_items * tiles_block;
  const int64_t n_block = direct ? 0 : p.counters[1];
  const int64_t n_coop = direct ? 0 : p.counters[8];
  const int64_t n_coop_batches = (n_coop + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t n_wave = direct ? p.b : p.counters[0];
  // Every segment reduced alone (all in run 0): the batches take segment ids
  // in order, as the short-segment schedule does, without the queue.
  const bool in_order = direct || n_wave == p.b;
  const int64_t n_batches = (n_wave + batch - 1) / batch;
  const int64_t before_alone = n_parts + n_block + n_coop_batches;
  const int64_t total = before_alone + n_batches;
  // The workgroups that take tickets: at most one per ticket (the grid is
  // sized to the device, the tickets to the input). The others leave now
  // and touch no counter -- also when they start after the call's last
  // workgroup has reset the counters, as they then read no tickets at all.
  const int64_t active = direct ? gridDim.x : active_workgroups(total);
  if (blockIdx.x >= active) return;
  // Tickets interleave over the lanes: lane k hands out k, k + lanes, ...
  // to the workgroups blockIdx = k (mod lanes), every lane has at least one.
  const int lanes = active < kTicketLanes ? (int)active : kTicketLanes;
  const int lane_id = (int)(blockIdx.x % lanes);
  unsigned long long* counter = (unsigned long long*)(p.counters + kTicketStride * (1 + lane_id));
  // Tickets are static (grid-stride, as in the short-segment schedule) when
  // every ticket is a batch of segments in order: batches are alike, so
  // the hand-out atomic's round trip buys no balance.
  const bool static_tickets = direct || in_order;
  // The first round of tickets is the workgroup index (a round of first
  // fetches would queue on each lane's counter); a lane's fetch returning c
  // then hands out active + c * lanes + lane.
  int64_t next = blockIdx.x;
  bool first = true;
  for (;;) {
    int64_t ticket = next;
    if (!static_tickets && !first) {
      __syncthreads();
      if (t == 0) ticket_s = active + (int64_t)atomicAdd(counter, 1ull) * lanes + lane_id;
      __syncthreads();
      ticket = (int64_t)(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)ticket_s >> 32)) << 32) |
                         __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)ticket_s));
    }
    first = false;
    next += gridDim.x;
    if (ticket >= total) break;
    if (ticket < n_parts) {
      split_part<OP, T, OffT, VEC, FLAT, MASK>(p, ticket / tiles_block, (int)(ticket % tiles_block), lds, &flag_s);
    } else if (ticket < n_parts + n_block) {
      const int64_t s = p.queue[p.b + (ticket - n_parts)];
      int64_t start, end;
      segment_rows<OffT>(p, s, start, end);
      // (process_segment counts a visit at tile 0 only.)
      for (int tile = 0; tile < tiles_block; ++tile) process_segment<OP, T, VEC, FLAT, MASK, true>(p, s, start, end, tile, lds);
    } else if (ticket < before_alone) {
      coop_batch<OP, T, OffT, VEC, FLAT, MASK>(p, ticket - n_parts - n_block, n_coop);
    } else {
      wave_batch<OP, T, OffT, VEC, FLAT, MASK>(p, ticket - before_alone, n_wave, in_order);
    }
  }
  // Softmax: the split parts' probabilities, from a counter of their own,
  // once this workgroup's tickets have run out (so every part has been
  // handed out). A part whose statistics are not out within drain_ticks is
  // deferred (counters[5] entries of `deferred`, agent scope); the last
  // workgroup out (last_out) normalises those: by then every part has run
  // and every segment's statistics are published. That workgroup then
  // returns the counters to zero for the next call.
  if (direct) return;
  if constexpr (OP == OP_SOFTMAX) {
    if (n_parts > 0) {
      for (;;) {
        __syncthreads();
        if (t == 0) ticket_s = (int64_t)atomicAdd((unsigned long long*)(p.counters + 9), 1ull);
        __syncthreads();
        const int64_t i = (int64_t)(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)ticket_s >> 32))
                                     << 32) |
                                    __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)ticket_s));
        if (i >= n_parts) break;
        if (!normalize_part<T, OffT, VEC, FLAT, MASK>(p, i / tiles_block, (int)(i % tiles_block), true) && t == 0) {
          const int64_t slot = (int64_t)atomicAdd((unsigned long long*)(p.counters + 5), 1ull);
          if (slot < n_parts) __hip_atomic_store(p.deferred + slot, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
  if (!last_out(p, &flag_s, active, OP == OP_SOFTMAX && n_parts > 0)) return;
  if constexpr (OP == OP_SOFTMAX) {
    if (n_parts > 0) {
      const int64_t deferred = __hip_atomic_load(p.counters + 5, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int64_t count = deferred < n_parts ? deferred : n_parts;
      for (int64_t j = 0; j < count; ++j) {
        const int64_t i = __hip_atomic_load(p.deferred + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        (void)normalize_part<T, OffT, VEC, FLAT, MASK>(p, i / tiles_block, (int)(i % tiles_block), false);
      }
      __syncthreads();
    }
  }
  reset_counters(p);
}

}  // namespace rg
