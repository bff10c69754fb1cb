// Register-resident softmax: one persistent kernel over a dynamic queue of
// work items, each read from HBM once and written once.
//
// Items (built by k_classify): every chunk of every split-class segment
// (ceil(L / part_rows) chunks, contiguous in the queue), then every
// block-class segment. A 256-thread workgroup takes the next item with one
// atomic ticket and holds its rows in registers (RPT rows per thread):
//   1. m = column max of the rows (IEEE maximum: NaN propagates);
//   2. e = exp(x - m) replaces x in registers, s = column sum of e;
//   3. whole segment: y = e / s.  Chunk of a longer segment: publish (m, s),
//      get the segment's merged (M, S) and write y = e * exp(m - M) / S.
// Merging is deterministic: the last chunk to arrive in each group of 32
// consecutive chunks folds the group in chunk order, and the last group to
// arrive folds the groups in order and publishes (M, S). A chunk waits for
// that with a bounded spin (relaxed agent-scope polling): since items
// are dequeued in order, every chunk it waits for is already held by a
// running workgroup whenever the device holds all chunks of the segment at
// once. If the spin limit passes (a segment with more chunks than resident
// workgroups, or a shared device), the chunk drops its registers and is
// recorded for k_softmax_deferred, which re-reads it after this kernel.
// No wait is unbounded.
//
// Reference semantics: docs/semantics.md (softmax row), the reference's
// online statistics and merge algebra (ToGPU.cpp:486-557, 435-472) restated
// as an exact two-pass over registers.
#pragma once

#include <type_traits>

#include "kernels.hpp"

namespace rg {

constexpr int kGroup = 32;          // chunks merged per first-level group

// Buffer addressing: a wave-uniform 128-bit resource (base in SGPRs) per
// chunk, covering exactly the chunk's bytes, and one per-thread byte offset
// plus a per-row stride. A row past the chunk is out of the resource's range:
// its load returns 0 (replaced by -inf before use) and its store is dropped
// by the hardware, so no load or store is predicated. Lanes without a
// feature (D below a power of two) get an offset that is always out of range.
using Rsrc = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;   // raw 32-bit data format (gfx9 family)

constexpr int kOutOfRange = 0x7ff00000;  // byte offset beyond any chunk resource

__device__ __forceinline__ Rsrc make_rsrc(const void* base, int64_t bytes) {
  const int records = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, records, kRsrcWord3);
}

// Load / store BYTES (2, 4, 8 or 16) as 32-bit words (2 bytes in the low half).
template <int BYTES>
__device__ __forceinline__ void buffer_load(Rsrc r, int voffset, int soffset, uint32_t* w) {
  static_assert(BYTES == 2 || BYTES == 4 || BYTES == 8 || BYTES == 16 || BYTES == 32, "unsupported width");
  if constexpr (BYTES == 32) {
    buffer_load<16>(r, voffset, soffset, w);
    buffer_load<16>(r, voffset + 16, soffset, w + 4);
  } else if constexpr (BYTES == 16) {
    auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (BYTES == 8) {
    auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voffset, soffset, 0);
    w[0] = v[0]; w[1] = v[1];
  } else if constexpr (BYTES == 4) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, 0);
  } else {
    w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, voffset, soffset, 0);
  }
}

template <int BYTES>
__device__ __forceinline__ void buffer_store(Rsrc r, int voffset, int soffset, const uint32_t* w) {
  static_assert(BYTES == 2 || BYTES == 4 || BYTES == 8 || BYTES == 16, "unsupported width");
  if constexpr (BYTES == 16) {
    __attribute__((ext_vector_type(4))) unsigned v = {w[0], w[1], w[2], w[3]};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voffset, soffset, 0);
  } else if constexpr (BYTES == 8) {
    __attribute__((ext_vector_type(2))) unsigned v = {w[0], w[1]};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, voffset, soffset, 0);
  } else if constexpr (BYTES == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(w[0], r, voffset, soffset, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)w[0], r, voffset, soffset, 0);
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
  for (int mask = lpr; mask < kWave; mask <<= 1) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = combine(v[i], __shfl_xor(v[i], mask, kWave));
  }
  const int rep = lpr < kWave ? lpr : kWave;
  if (lane < rep) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) lds[(w * kWave + lane) * VEC + i] = v[i];
  }
  __syncthreads();
  // Waves holding feature lane fl: all four when lpr <= 64, else every
  // (lpr/64)-th wave starting at fl/64.
  const int stride = lpr <= kWave ? 1 : lpr / kWave;
  const int w0 = lpr <= kWave ? 0 : feat_lane / kWave;
  const int l0 = feat_lane & (kWave - 1);
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float acc = lds[(w0 * kWave + l0) * VEC + i];
    for (int ww = w0 + stride; ww < kWavesPerBlock; ww += stride) acc = combine(acc, lds[(ww * kWave + l0) * VEC + i]);
    v[i] = acc;
  }
  __syncthreads();
}

// Statistics shared between workgroups travel only through agent-scope
// atomic stores and loads (coherent across the XCDs' L2 caches), so no
// L2-wide writeback or invalidate is needed. A publisher waits until its
// stores have completed (s_waitcnt vmcnt(0)) before the barrier after which
// one thread bumps the counter that others test; readers issue their loads
// only after observing that counter.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_agent(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait for this wave's outstanding vector memory operations (vmcnt = 0).
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Fold statistics slots first, first + stride, ... (count of them, each D
// floats of m and s) in order into (m, s) of feature f.
__device__ __forceinline__ void fold_stats(const float* pm, const float* ps, int64_t first, int64_t count,
                                           int64_t stride_items, int d, int f, float& m, float& s) {
  State<OP_SOFTMAX> acc;
  acc.init();
  for (int64_t i = 0; i < count; ++i) {
    State<OP_SOFTMAX> part;
    const int64_t slot = (first + i * stride_items) * d + f;
    part.m = load_agent(pm + slot);
    part.s = load_agent(ps + slot);
    acc.merge(part);
  }
  m = acc.m;
  s = acc.s;
}

// Chunk `item` (position c of P in its segment, first item F) has stored its
// statistics (store_agent). Returns true once (M, S) of the segment is in
// stats_max/stats_sum[k]; false if the spin limit passed first.
__device__ bool merge_and_wait(const Params& p, int64_t item, int64_t k, int64_t first, int64_t parts, int* flag_s) {
  const int t = threadIdx.x;
  const int64_t c = item - first;
  const int64_t group = c / kGroup;
  const int64_t gfirst = first + group * kGroup;
  const int64_t gsize = parts - group * kGroup < kGroup ? parts - group * kGroup : kGroup;
  const int64_t groups = (parts + kGroup - 1) / kGroup;
  // Level 1: the last chunk of the group to arrive folds it into slot gfirst.
  wait_stores();
  __syncthreads();
  if (t == 0) *flag_s = atomicAdd(p.arrive + gfirst, 1) == gsize - 1;
  __syncthreads();
  if (*flag_s) {
    // Each thread owns features t, t+256, ...: it reads every slot of its
    // features before overwriting slot gfirst.
    for (int f = t; f < p.d; f += kBlock) {
      float gm, gs;
      fold_stats(p.partials, p.partial_sums, gfirst, gsize, 1, p.d, f, gm, gs);
      store_agent(p.partials + gfirst * p.d + f, gm);
      store_agent(p.partial_sums + gfirst * p.d + f, gs);
    }
    wait_stores();
    __syncthreads();
    // Level 2: the last group to arrive folds the groups and publishes.
    if (t == 0) *flag_s = atomicAdd(p.seg_arrive + k, 1) == groups - 1;
    __syncthreads();
    if (*flag_s) {
      for (int f = t; f < p.d; f += kBlock) {
        float gm, gs;
        fold_stats(p.partials, p.partial_sums, first, groups, kGroup, p.d, f, gm, gs);
        store_agent(p.stats_max + k * p.d + f, gm);
        store_agent(p.stats_sum + k * p.d + f, gs);
      }
      wait_stores();
      __syncthreads();
      if (t == 0) __hip_atomic_store(p.seg_ready + k, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Wait for the segment's statistics (bounded).
  if (t == 0) {
    const long long start = wall_clock64();
    int ready = load_agent(p.seg_ready + k);
    while (!ready && wall_clock64() - start < p.spin_ticks) {
      __builtin_amdgcn_s_sleep(2);
      ready = load_agent(p.seg_ready + k);
    }
    *flag_s = ready;
  }
  __syncthreads();
  const bool ready = *flag_s != 0;
  __syncthreads();
  return ready;
}

template <class T, class OffT, int VEC, int RPT, bool MASK, bool STORE_F32>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4))) void k_softmax_fused(Params p) {
  // Rows stay as loaded (T) unless the input transform (scale, mask) makes
  // f32 logits that must not be rounded back to T.
  using Store = typename std::conditional<STORE_F32, float, T>::type;
  using In = Words<T, VEC>;
  using Reg = Words<Store, VEC>;
  __shared__ float lds[kBlock * VEC];
  __shared__ int64_t ticket_s;
  __shared__ int flag_s;
  const int t = threadIdx.x;
  const RowGeo g = row_geo<VEC>(p.d, kBlock, t, 0);
  const int64_t n_split = p.counters[3] < p.items_cap ? p.counters[3] : p.items_cap;
  const int64_t n_block = p.counters[1];
  const int64_t total = n_split + n_block;
  const int64_t d = p.d;
  // Byte offsets inside a chunk: per thread, and the stride between a
  // thread's rows.
  const int voff_in = g.active ? (g.row_lane * p.d + g.feature) * (int)sizeof(T) : kOutOfRange;
  const int step_in = g.rows_step * p.d * (int)sizeof(T);
  const int voff_mask = g.active ? (g.row_lane * p.d + g.feature) * 4 : kOutOfRange;
  const int step_mask = g.rows_step * p.d * 4;
  for (;;) {
    if (t == 0) ticket_s = (int64_t)atomicAdd((unsigned long long*)(p.counters + 4), 1ull);
    __syncthreads();
    const int64_t ticket = ticket_s;
    __syncthreads();
    if (ticket >= total) break;
    int64_t s, k = -1, first = 0, parts = 1, start, end;
    const bool chunk = ticket < n_split;
    if (chunk) {
      int64_t part;
      item_rows<OffT>(p, ticket, k, s, part, start, end);
      first = p.part_begin[k];
      int64_t seg_start, seg_end;
      segment_rows<OffT>(p, s, seg_start, seg_end);
      parts = (seg_end - seg_start + p.part_rows - 1) / p.part_rows;
    } else {
      s = p.queue[p.b + (ticket - n_split)];
      segment_rows<OffT>(p, s, start, end);
    }
    const int rows = (int)(end - start);   // at most one chunk: fits a workgroup's registers
    const int64_t chunk_elems = (int64_t)rows * d;
    // Per-item copies of the offsets: computing each row's offset next to
    // its access (instead of hoisting RPT offsets out of the item loop)
    // keeps them out of the register budget.
    int voff = voff_in, voff_m = voff_mask;
    asm volatile("" : "+v"(voff), "+v"(voff_m));
    const Rsrc in = make_rsrc(static_cast<const T*>(p.values) + start * d, chunk_elems * (int64_t)sizeof(T));
    // 1. Rows into registers (all loads in flight at once), column max.
    uint32_t data[RPT][Reg::kCount];
    if constexpr (!STORE_F32) {
#pragma unroll
      for (int i = 0; i < RPT; ++i) buffer_load<In::kBytes>(in, voff + i * step_in, 0, data[i]);
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
    // Rows past the chunk (and featureless lanes) read 0: make them -inf,
    // the identity of the max and a zero mass.
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      if (!(g.active && g.row_lane < rows - i * g.rows_step)) Reg::fill_neg_inf(data[i]);
    }
    float m[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) m[v] = neg_inf();
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) m[v] = fmax_nan(m[v], Reg::get(data[i], v));
    }
    // Keep the rows packed across the reduction: without this the compiler
    // keeps every unpacked f32 value alive until pass 2 (twice the registers,
    // a quarter of the occupancy).
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
#pragma unroll
      for (int w = 0; w < Reg::kCount; ++w) asm volatile("" : "+v"(data[i][w]));
    }
    block_allreduce<true, VEC>(m, g.lpr, g.feat_lane, lds);
    // 2. e = exp(x - m) in place, column sums. A column of only -inf has no
    //    mass: its reference is taken as 0 so that e = 0, not NaN.
    float ref[VEC], sum[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      ref[v] = m[v] == neg_inf() ? 0.f : m[v];
      sum[v] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      float e[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        e[v] = fast_exp(Reg::get(data[i], v) - ref[v]);
        sum[v] += e[v];
      }
      Reg::set(data[i], e);
      // Pack now, so that the f32 values die here rather than after the
      // reduction below.
#pragma unroll
      for (int w = 0; w < Reg::kCount; ++w) asm volatile("" : "+v"(data[i][w]));
    }
    block_allreduce<false, VEC>(sum, g.lpr, g.feat_lane, lds);
    // 3. Scale factor per column: exp(m - M) / S.
    float factor[VEC];
    bool ready = true;
    if (!chunk) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) factor[v] = fast_exp(m[v] - m[v]) / sum[v];
    } else {
      if (g.row_lane == 0 && g.active) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          store_agent(p.partials + ticket * d + g.feature + v, m[v]);
          store_agent(p.partial_sums + ticket * d + g.feature + v, sum[v]);
        }
      }
      ready = merge_and_wait(p, ticket, k, first, parts, &flag_s);
      if (ready && g.active) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float big_m = load_agent(p.stats_max + k * d + g.feature + v);
          const float big_s = load_agent(p.stats_sum + k * d + g.feature + v);
          factor[v] = fast_exp(m[v] - big_m) / big_s;
        }
      }
    }
    if (!ready) {
      if (t == 0) {
        const int64_t slot = (int64_t)atomicAdd((unsigned long long*)(p.counters + 5), 1ull);
        if (slot < p.items_cap) p.deferred[slot] = ticket;
      }
      continue;
    }
    // 4. Normalise from registers; rows past the chunk are dropped by the
    //    resource's range check.
    const Rsrc out = make_rsrc(static_cast<T*>(p.out) + start * d, chunk_elems * (int64_t)sizeof(T));
    asm volatile("" : "+v"(voff));
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      float y[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) y[v] = Reg::get(data[i], v) * factor[v];
      uint32_t w[In::kCount];
      In::set(w, y);
      buffer_store<In::kBytes>(out, voff + i * step_in, 0, w);
    }
    if (p.visits && t == 0 && (!chunk || ticket == first)) atomicAdd(p.visits + s, 1);
  }
}

// Chunks that gave up waiting: re-read and normalise with the segment's
// published statistics (complete once k_softmax_fused has finished).
template <class T, class OffT, int VEC, bool MASK>
__global__ __launch_bounds__(kBlock) void k_softmax_deferred(Params p) {
  const int64_t count = p.counters[5] < p.items_cap ? p.counters[5] : p.items_cap;
  const int t = threadIdx.x;
  const RowGeo g = row_geo<VEC>(p.d, kBlock, t, 0);
  for (int64_t i = blockIdx.x; i < count; i += gridDim.x) {
    const int64_t item = p.deferred[i];
    int64_t k, s, part, start, end;
    item_rows<OffT>(p, item, k, s, part, start, end);
    if (!g.active) continue;
    float m[VEC], inv[VEC];
    Elem<float>::load<VEC>(p.stats_max + k * p.d + g.feature, m);
    Elem<float>::load<VEC>(p.stats_sum + k * p.d + g.feature, inv);
#pragma unroll
    for (int v = 0; v < VEC; ++v) inv[v] = 1.0f / inv[v];
    normalize_rows<T, VEC, MASK>(p, g, start, end, m, inv);
    if (p.visits && t == 0 && part == 0) atomicAdd(p.visits + s, 1);
  }
}

}  // namespace rg
