/* C ABI of libragged_hip.so: segmented sum / max / softmax on gfx950.
 *
 * This library replaces the reference's native launcher
 * (simon-jd/ragged-mlir runtime/Driver.h:21-54 and runtime/bindings.cpp:11-37,
 * the nanobind module ragged._native.DriverModule) together with the kernels
 * the reference generated through MLIR -> NVVM -> PTX
 * (lib/Conversion/ToGPU.cpp). The kernels are hand-written HIP compiled ahead
 * of time for gfx950, so there is no module loading from a code blob: a
 * "module" is a handle on one kernel specialisation (op, dtype, offsets
 * dtype, feature width, mask) on one device.
 *
 * Conventions
 *  - Every function returns RG_OK (0) or a negative RG_E_* status; the
 *    calling thread's message is then available from rg_last_error().
 *  - No function allocates device memory. The caller owns values, offsets,
 *    out, mask and the workspace, and passes raw device pointers.
 *  - rg_run and rg_check_offsets only enqueue work on the given HIP stream;
 *    they never synchronise. On error nothing has been launched.
 *  - All handles are thread-compatible: concurrent calls on one module are
 *    safe (it is immutable after creation).
 */
#ifndef RAGGED_HIP_H
#define RAGGED_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RG_ABI_VERSION 3

enum rg_status {
  RG_OK = 0,
  RG_E_INVALID = -1,      /* bad argument or specialisation */
  RG_E_DEVICE = -2,       /* HIP runtime error (device, launch, occupancy) */
  RG_E_UNSUPPORTED = -3,  /* device is not gfx950 */
  RG_E_WORKSPACE = -4     /* workspace missing or too small for the plan */
};

enum rg_op { RG_OP_SUM = 0, RG_OP_MAX = 1, RG_OP_SOFTMAX = 2 };
enum rg_dtype { RG_F32 = 0, RG_BF16 = 1 };
enum rg_index { RG_I32 = 0, RG_I64 = 1 };
/* RG_SHORT_SEGMENTS: every segment is expected to be at most alone_rows
 * rows (the caller's max_len says so): one worker launch takes the segments
 * in order, with no classification and no workspace. Any input is still
 * computed exactly; a longer segment only runs slower. Not available when
 * alone_rows or t_wave is 0. */
enum rg_schedule { RG_CLASSIFIED = 0, RG_BLOCK_PER_SEGMENT = 1, RG_SHORT_SEGMENTS = 2 };

/* Kernel roles (a plan lists its launches in submission order). */
enum rg_role {
  RG_ROLE_INIT = 0,            /* not launched: k_classify initialises what a call uses */
  RG_ROLE_CLASSIFY = 1,
  RG_ROLE_WAVE = 2,            /* not launched: the wave class runs inside RG_ROLE_WORKER */
  RG_ROLE_BLOCK = 3,           /* not launched: the block class runs inside RG_ROLE_WORKER */
  RG_ROLE_SPLIT_PARTIAL = 4,   /* not launched: split parts run inside RG_ROLE_WORKER */
  RG_ROLE_SPLIT_COMBINE = 5,   /* not launched: the last part of a segment combines, inside RG_ROLE_WORKER */
  RG_ROLE_SPLIT_NORMALIZE = 6, /* not launched: the classified worker normalises split parts */
  RG_ROLE_NAIVE = 7,           /* block-per-segment schedule */
  RG_ROLE_FUSED = 8,           /* softmax: register-resident worker over all block/split items, then the
                                  wave class and the chunks that stopped waiting (re-read) */
  RG_ROLE_DEFERRED = 9,        /* not launched: RG_ROLE_FUSED drains its deferred chunks itself */
  RG_ROLE_WORKER = 10,         /* persistent worker over the wave, block and split queues */
  RG_ROLE_COUNT = 11
};

#define RG_MAX_LAUNCHES 8
#define RG_WORKSPACE_BUFFERS 16

/* A kernel specialisation (ProgramSpec fields that change device code;
 * reference: python/ragged/model.py:129-188). */
typedef struct rg_spec {
  int32_t op;             /* rg_op */
  int32_t dtype;          /* rg_dtype: values and out */
  int32_t offsets_dtype;  /* rg_index */
  int32_t feature_dim;    /* D in [1, 1024] */
  float scale;            /* f32 multiplier of every input (1 = none) */
  int32_t has_mask;       /* softmax only: additive f32 [N, D] mask */
  int32_t vectorize;      /* 0: one element per access (any alignment) */
  int32_t debug_visits;   /* classified only: count final writes per segment */
  int64_t t_wave;         /* wave class: segments of at most t_wave rows; <0: default */
  int64_t t_block;        /* block class: at most t_block rows; <0: default */
  int64_t part_rows;      /* rows per split part; <0: default */
  int64_t alone_rows;     /* output of rg_spec_defaults: wave-class segments of at most this
                             many rows are reduced by one lane (flat mapping) or one group of
                             the lanes that hold a row (rows narrower than half a wave); the
                             rest of the wave class by one wave each */
} rg_spec;

/* Device facts the host cost model and grids use. */
typedef struct rg_device_props {
  int32_t ordinal;
  int32_t cu_count;          /* compute units */
  int32_t xcd_count;         /* accelerator complex dies (own L2 each) */
  int32_t wave_size;
  int64_t l2_bytes;          /* L2 per XCD as reported by the runtime */
  int64_t mall_bytes;        /* last-level (Infinity) cache; 0 if unknown */
  int64_t lds_per_cu;
  int64_t global_mem_bytes;
  char arch[64];             /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} rg_device_props;

/* Resolved launch sequence and workspace layout for one (N, B, schedule)
 * (reference: runtime.py:145-162 scratch layout, layout.py:50-107). */
typedef struct rg_plan {
  int32_t schedule;                       /* rg_schedule */
  int32_t launches;                       /* kernels in submission order */
  int32_t roles[RG_MAX_LAUNCHES];         /* rg_role of each launch */
  uint32_t grid[RG_MAX_LAUNCHES][3];
  uint32_t block[RG_MAX_LAUNCHES];
  uint32_t lds_bytes[RG_MAX_LAUNCHES];    /* static LDS of each kernel */
  uint64_t workspace_bytes;               /* one allocation, buffers 256-B aligned */
  uint64_t buffer_offset[RG_WORKSPACE_BUFFERS];
  uint64_t buffer_bytes[RG_WORKSPACE_BUFFERS];
  int64_t n, b;
  int64_t b_split;                        /* rows of the split statistics */
  int64_t items_cap;                      /* capacity of the split item table */
  int64_t t_wave, t_block, part_rows;
  int32_t vec;                            /* elements per vector access */
  int32_t flat;                           /* 1: flat mapping (D < vec) */
  int32_t fused;                          /* 1: softmax runs the register-resident worker */
} rg_plan;

/* Workspace buffer indices (rg_plan.buffer_offset / buffer_bytes). */
enum rg_buffer {
  RG_BUF_COUNTERS = 0,      /* i64 slots: 0 wave-class segments of at most alone_rows rows, 1 block,
                               2 split counts, 3 split items, 4 work ticket, 5 deferred count
                               (register-resident softmax chunks, or worker softmax split
                               parts), 6 tree items; 7 slot 0's count for a register-resident
                               softmax (whose slot 0 stays 0); 8 the rest of the wave class;
                               9 softmax split-part normalisation ticket; 10 final_pairs rows
                               reserved (register-resident softmax); 11 done lanes finished
                               (of the call's last kernel); 12 the fused softmax arena's state
                               (0: the workspace is as allocated, all zero; 1: unknown, another
                               plan's buffers overlap it; v >= 2: its first v - 2 bytes are zero
                               but for the byte ranges [14, 15), [16, 17), [18, 19) hold: the
                               pairs and group rows the last call published, which the next
                               call's classification zeroes); 13 deferred chunks claimed; then
                               16 ticket counters of the classified worker and 16 done lanes,
                               256 bytes apart from byte 256 (8448 bytes in all). All zero
                               before a call but slots 12 and 14-19; the call's last workgroup
                               leaves them so. */
  RG_BUF_QUEUE = 1,         /* i64[3, B] original segment ids per class; the wave class holds
                               its segments of at most alone_rows rows from the front and the
                               others from the back */
  RG_BUF_ITEM_POS = 2,      /* i64[items_cap] split position of each item */
  RG_BUF_PART_BEGIN = 3,    /* i64[B_split] first item of each split segment */
  RG_BUF_PARTIALS = 4,      /* f32[items_cap, D] */
  RG_BUF_PARTIAL_SUMS = 5,  /* f32[items_cap, D] (softmax) */
  RG_BUF_STATS_MAX = 6,     /* f32[B_split, D] (softmax) */
  RG_BUF_STATS_SUM = 7,     /* f32[B_split, D] (softmax) */
  RG_BUF_VISITS = 8,        /* i32[B] (debug_visits) */
  RG_BUF_DEFERRED = 9,      /* i64[items_cap] 1 + item of each chunk left to the drain, 0 while
                               unwritten (fused softmax); i64[items_cap * feature tiles] split
                               parts left to the worker's last workgroup (worker softmax) */
  RG_BUF_ARRIVE = 10,       /* i32[items_cap] chunk arrivals per 16-chunk group and readers of
                               each segment's merged statistics (fused softmax) */
  RG_BUF_SEG_ARRIVE = 11,   /* i32[B_split] part arrivals per split segment (worker) */
  RG_BUF_ITEMS = 12,        /* 32-byte descriptors [items_cap] of split chunks (fused softmax) */
  RG_BUF_BLOCK_ITEMS = 13,  /* 32-byte descriptors [B] of whole segments (fused softmax) */
  RG_BUF_PAIRS = 14,        /* u64[items_cap, D] published (max, sum) of each chunk (fused softmax) */
  RG_BUF_FINAL_PAIRS = 15   /* u64[rows, D] merged (max, sum) of each 16-chunk group of a long
                               segment (fused softmax) */
};
/* Buffers are laid out at 256-byte aligned offsets: the counters at 0, then
 * the fused softmax's arena (pairs, final pairs, arrive, deferred: the slots
 * that hold zero between its calls) at the same offset in every plan, then
 * the rest. */

typedef struct rg_module rg_module;

/* ABI version of the library (RG_ABI_VERSION). */
int rg_abi_version(void);

/* Identity of the build: target, flags and source digest. */
const char* rg_build_info(void);

/* Message of the last failed call on this thread ("" if none). */
const char* rg_last_error(void);

/* Device facts; replaces the occupancy/L2 queries of runtime.py:165-178. */
int rg_device_query(int ordinal, rg_device_props* out);

/* Fill the default class thresholds and part size of `spec` (fields < 0). */
int rg_spec_defaults(rg_spec* spec);

/* 1 if `spec` (after defaults) runs softmax through the register-resident
 * worker (RG_ROLE_FUSED), 0 if not, <0 on a bad spec. Host only. */
int rg_spec_uses_fused(const rg_spec* spec);

/* Create a kernel specialisation on a device; replaces
 * DriverModule(cubin, target) (Driver.h:23-27, Driver.cpp:178-195). Fails with
 * RG_E_UNSUPPORTED unless the device is gfx950. */
int rg_module_create(int device, const rg_spec* spec, rg_module** out);

/* Release a module; replaces DriverModule.close() (Driver.h:44). Work already
 * enqueued is unaffected (kernels are not unloaded). */
void rg_module_destroy(rg_module* module);

/* Resident workgroups of one role on the whole device (one resident wave
 * of the persistent workers); replaces resident_blocks (Driver.cpp:236-245). */
int rg_module_resident(const rg_module* module, int role, int64_t* blocks);

/* Resolve launches and workspace for N rows, B segments; replaces
 * add_plan (Driver.cpp:272-292). Pure host arithmetic, overflow checked. */
int rg_plan_create(const rg_module* module, int64_t n, int64_t b, int schedule, rg_plan* plan);

/* Enqueue the plan on `stream` (a hipStream_t); replaces run_plan
 * (Driver.cpp:299-353). `workspace` must hold plan->workspace_bytes bytes
 * at a 256-byte aligned address (may be NULL when that is 0); `mask` is NULL
 * unless the module has one.
 *
 * Workspace contract: zero-filled before its first call. Every call
 * initialises the per-segment state it uses and its last workgroup returns
 * the workspace's counters to zero; a fused softmax call also records which
 * bytes of its arena it left nonzero (counters slots 12, 14-19), and the
 * next call's classification zeroes those and whatever part of its plan's
 * arena a call of another plan overwrote.
 * So calls in order on one stream reuse a workspace with no clearing, across
 * plans and modules (a failed rg_run may leave it dirty: zero it again). A
 * module with debug_visits keeps its counters for inspection instead: give
 * each of its calls a zeroed workspace. */
int rg_run(const rg_module* module, const rg_plan* plan, const void* values, const void* offsets,
           void* out, const float* mask, void* workspace, uint64_t workspace_bytes, void* stream);

/* Size of the static workspace rg_run_static uses on each device (64 MiB
 * unless the library is built with another -DRG_STATIC_WORKSPACE_BYTES). */
#ifndef RG_STATIC_WORKSPACE_BYTES
#define RG_STATIC_WORKSPACE_BYTES (64ull << 20)
#endif

/* rg_run without a caller workspace. No counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).
 *
 * The workspace is a static device array of RG_STATIC_WORKSPACE_BYTES per
 * device: every process that loads the library holds it on each device it
 * creates a module on, from the first rg_module_create there until the
 * process ends, whether or not it calls this. Plans whose workspace_bytes
 * exceed it fail with RG_E_WORKSPACE before anything is launched (rg_run
 * takes any size). Every call on a device shares that device's array under
 * rg_run's workspace contract, so results do not depend on earlier calls; a
 * call that fails after launching part of its plan leaves the array marked,
 * and the next call on that device first launches a one-workgroup kernel
 * that returns its counters to zero. Calls that overlap on one device (two
 * streams, or two host threads) race on the array and must be serialised by
 * the caller. Calls no allocating routine: no hipMalloc, no event creation
 * (rg_profile_* does not record these calls). Same kernels and results as
 * rg_run; a debug_visits module is refused (it keeps its counters after a
 * call). Enqueue only. */
int rg_run_static(const rg_module* module, const rg_plan* plan, const void* values, const void* offsets,
                  void* out, const float* mask, void* stream);

/* Test control: the next rg_run_static (any device) stops after `launches`
 * kernel launches of its plan and fails with RG_E_DEVICE, as a launch error
 * there would; -1 turns it off. No counterpart in the reference. */
int rg_test_interrupt_static(int launches);

/* Longest wait, in microseconds, of every softmax wait for statistics that
 * other workgroups publish, before the work is deferred: a register-resident
 * chunk's wait for the rest of its segment (default 2000; deferred chunks
 * are re-read once every item is handed out, by the same kernel), the
 * re-read's own wait, and a streaming worker split part's wait for its
 * segment's statistics (default 1000000; deferred parts are normalised by
 * the worker's last workgroup; a fused softmax's re-read left undone by its
 * wait is finished by that kernel's last workgroup). Results do not depend on it.
 * A test and diagnostics control: 0 makes every such wait that does not
 * succeed at once take the deferred path; -1 restores both defaults. */
int rg_module_set_spin_limit(rg_module* module, int64_t microseconds);

/* Diagnostics: a timeline of the register-resident softmax's work items.
 * With `buffer` (device memory of `records` x 8 int64) set, every later run
 * writes for each ticket t < records the record
 *   {t, start, loaded, reduced, merged, end, hw_id, kind}
 * (device wall-clock ticks at the item's start, after its loads and column
 * max, after its column sums, after the segment merge, after its stores are
 * issued; hw_id = __smid() of the workgroup; kind = 0 whole segment,
 * 1 chunk merged directly, 2 chunk merged by tree, +4 when deferred, plus
 * rows << 8). A null buffer turns it off. No counterpart in the reference:
 * a measurement hook only. */
int rg_module_set_trace(rg_module* module, void* buffer, int64_t records);

/* Rate of the device wall clock the timeline records use, in kHz. */
int rg_device_clock_khz(int device, int64_t* khz);

/* Measurement: while profiling is on, rg_run records a HIP event before
 * every launch and after the last one (no synchronisation), for at most
 * `max_calls` calls. rg_profile_stop waits for those events and returns, per
 * role, the summed kernel milliseconds and launch counts, and the summed
 * whole-call milliseconds. Not thread-safe; measurement only. */
int rg_profile_start(rg_module* module, int max_calls);
int rg_profile_stop(rg_module* module, double* role_ms, int64_t* role_launches, double* call_ms,
                    int64_t* calls);

/* Checked mode: write into status[7] (device i64) the earliest offending
 * index of each offsets condition, INT64_MAX if none (docs/checked-abi.md;
 * replaces the offsets_init / offsets_check kernels, ToGPU.cpp:1067-1189).
 * min_len / max_len < 0 mean "no hint". Enqueue only. */
int rg_check_offsets(int device, int offsets_dtype, const void* offsets, int64_t n, int64_t b,
                     int64_t min_len, int64_t max_len, int64_t* status, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RAGGED_HIP_H */
