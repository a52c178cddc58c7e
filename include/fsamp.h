/*
 * fsamp.h -- C ABI of the MI355X (gfx950) fused top-k + top-p sampler.
 *
 * One call turns [B, V] fp16/bf16 logits into [B] int64 token ids:
 *   exact top-k (k = min(top_k, V), descending value, ties to the lowest token id)
 *   -> fp32 softmax over the k survivors -> inclusive prefix -> keep rank i iff the
 *   exclusive prefix c_i - p_i < top_p (all k when top_p >= 1) -> draw the first kept rank
 *   with c_i >= u * Z_p, Z_p = c_r the prefix at the last kept rank.
 *
 * The entry points replace the reference's pybind11 module `fused_sampling`
 * (csrc/bindings.cpp:16-25).  Conventions shared by every entry point:
 *   - all pointers are device pointers unless stated; nothing is allocated or freed;
 *   - work is enqueued on `stream` and the call returns without synchronising;
 *   - the return value is FSAMP_OK or one of the error codes below
 *     (fsamp_error_string gives the message the reference raises for the same check);
 *   - `dtype` is FSAMP_DTYPE_F16 or FSAMP_DTYPE_BF16; logits are row-major contiguous.
 *
 * Workspace.  Rows are split over `splits` workgroups and the last workgroup of a row to
 * finish merges the row (one launch per call).  That needs `fsamp_workspace_bytes(...)`
 * bytes of device workspace laid out as [per-row counters: round_up(128*B, 256) bytes]
 * [one grid counter: 256 bytes][per-split candidates].  The counter regions must be zero
 * before a call (fsamp_workspace_init zeroes the whole buffer on the stream) and every call
 * leaves them zero again; the candidate region is scratch.  A buffer reused with a larger B
 * must be zeroed again, because the larger counter region overlaps the old candidates.
 * Calls that share one workspace must not run concurrently.  A call whose plan has
 * splits == 1 and that uses no offset counter (fsamp_sample_ex) reads no workspace: ws may
 * then be NULL.
 */
#ifndef FSAMP_H
#define FSAMP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fsamp_dtype { FSAMP_DTYPE_F16 = 0, FSAMP_DTYPE_BF16 = 1 };

enum fsamp_status {
  FSAMP_OK = 0,
  FSAMP_ERR_DTYPE = 1,      /* "logits must be float16 or bfloat16" */
  FSAMP_ERR_SHAPE = 2,      /* "logits must be a contiguous cuda [B, V] tensor" */
  FSAMP_ERR_TOPK_LOW = 3,   /* "top_k must be >= 1" */
  FSAMP_ERR_TOPK_HIGH = 4,  /* "top_k must be <= 1024" */
  FSAMP_ERR_TOPP = 5,       /* "top_p must be in (0, 1]" */
  FSAMP_ERR_WORKSPACE = 6,  /* workspace missing or smaller than fsamp_workspace_bytes() */
  FSAMP_ERR_NULL = 7,       /* a required pointer is NULL */
  FSAMP_ERR_PHASE = 8,      /* "phase must be in [1, 7]" */
  FSAMP_ERR_SPLITS = 9,     /* "splits must be >= 1" (probe) */
  FSAMP_ERR_VOCAB = 10,     /* vocabulary does not fit the workgroup tiling */
  FSAMP_ERR_LAUNCH = 11     /* the HIP runtime reported an error at launch */
};

#define FSAMP_K_MAX 1024

/* Message for a status code (static storage). */
const char* fsamp_error_string(int status);

/* The launch plan for a shape: split count, workgroup size and register tiling.
 * Mirrors make_plan (csrc/fused_sampling.cu:341-364). */
typedef struct fsamp_plan {
  int64_t batch, vocab, k;   /* k = min(top_k, vocab) */
  int32_t splits;            /* workgroups per row */
  int32_t slice;             /* elements per split (a multiple of 8) */
  int32_t threads;           /* workgroup size */
  int32_t chunks;            /* 8-element chunks held in registers per thread */
  int32_t vec;               /* 1 when rows are loaded with 16-byte vector loads */
  int32_t reserved;
  size_t workspace_bytes;
} fsamp_plan;

/* Fill *plan for logits at `logits` (only its alignment is read) of shape [B, V].
 * splits_override > 0 forces the split count (clamped as the reference clamps it). */
int fsamp_make_plan(const void* logits, int64_t B, int64_t V, int64_t top_k,
                    int64_t splits_override, fsamp_plan* plan);

/* Bytes of workspace a call with these arguments needs (0 when the plan has one split). */
size_t fsamp_workspace_bytes(const void* logits, int64_t B, int64_t V, int64_t top_k,
                             int64_t splits_override);

/* Zero `bytes` of workspace on `stream` with a fill kernel (graph-capturable). */
int fsamp_workspace_init(void* ws, size_t bytes, hipStream_t stream);

/*
 * Sample one token per row.  Replaces sample_fused (csrc/fused_sampling.cu:449-458,
 * csrc/bindings.cpp:20) and adds the explicit-uniform form:
 *   u != NULL : u[b] (device, fp32 in [0,1)) is row b's uniform;
 *   u == NULL : the uniform is splitmix64(seed, offset, row) in-kernel, as the reference's
 *               explicit-offset path does (csrc/fused_sampling.cuh:65-71).
 * out: [B] int64 token ids.
 */
int fsamp_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                 double top_p, const float* u, uint64_t seed, uint64_t offset, int64_t* out,
                 void* ws, size_t ws_bytes, int64_t splits_override, hipStream_t stream);

/*
 * Per-row sampling controls and the graph-safe draw of fsamp_sample_ex.  Every pointer may be
 * NULL (the call's scalar value applies).  Device arrays of B entries:
 *   top_k[b]        row b samples from its top min(max(top_k[b], 1), k) ranks: a prefix of
 *                   the call's top-k selection (int32);
 *   top_p[b]        row b's nucleus threshold (fp32): ranks are kept while the exclusive
 *                   prefix is < top_p[b]; >= 1 keeps all, <= 0 keeps rank 0 only;
 *   temperature[b]  row b's softmax runs on (x - max) * (1 / temperature[b]) in fp32;
 *                   temperature[b] <= 0 (or NaN) is greedy: rank 0.
 * offset_counter    device uint64: when u == NULL, the row uniforms are
 *                   splitmix64(seed, *offset_counter, row) and the call adds 4 to the counter
 *                   once every row has drawn (in the kernel, so a captured HIP graph advances
 *                   it on every replay).  The call's `offset` argument is then ignored.  The
 *                   grid counter in the workspace is used, so ws is required.
 * No counterpart in the reference for the per-row arrays (SEMANTICS.md lists them as open);
 * the counter replaces the graph-capturable generator path of sample_fused with offset < 0
 * (csrc/fused_sampling.cu:112-118, :441-447).
 */
typedef struct fsamp_row_params {
  const int32_t* top_k;
  const float* top_p;
  const float* temperature;
  uint64_t* offset_counter;
} fsamp_row_params;

/*
 * fsamp_stages with per-row controls (rows may be NULL: then it is fsamp_stages, or
 * fsamp_sample when keep and renormed are NULL too).  keep / renormed are [B, k] with ranks at
 * or past a row's own k written as 0.
 */
int fsamp_sample_ex(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                    double top_p, const float* u, uint64_t seed, uint64_t offset,
                    const fsamp_row_params* rows, int64_t* out, uint8_t* keep, float* renormed,
                    void* ws, size_t ws_bytes, int64_t splits_override, hipStream_t stream);

/*
 * Debug form of fsamp_sample that also writes, per row and rank i < k,
 *   keep[b*k+i]     = 1 if rank i is inside the nucleus, else 0   (uint8)
 *   renormed[b*k+i] = p_i / Z_p inside the nucleus, else 0       (fp32)
 * Replaces stages_fused (csrc/fused_sampling.cu:503-513, csrc/bindings.cpp:22).
 */
int fsamp_stages(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                 double top_p, const float* u, uint64_t seed, uint64_t offset, int64_t* out,
                 uint8_t* keep, float* renormed, void* ws, size_t ws_bytes,
                 int64_t splits_override, hipStream_t stream);

/*
 * The selected candidate ids, [B, k] int64 in descending value order with ties by
 * ascending id.  Replaces topk_fused (csrc/fused_sampling.cu:460-473, bindings.cpp:21).
 */
int fsamp_topk(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
               int64_t* ids, void* ws, size_t ws_bytes, int64_t splits_override,
               hipStream_t stream);

/*
 * Ablation: run the pipeline up to `phase` (1..7) and stop; phase 7 is fsamp_sample with
 * seed = offset = 0.  Phases: 1 load + keys + maxima, 2 lower bound, 3 candidate filter,
 * 4 workgroup sort, 5 split hand-off, 6 row merge, 7 softmax + cut + draw.
 * Replaces probe_phase (csrc/fused_sampling.cu:475-501, bindings.cpp:23).
 */
int fsamp_probe_phase(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                      double top_p, int64_t phase, int64_t* out, void* ws, size_t ws_bytes,
                      int64_t splits_override, hipStream_t stream);

/* Launch floor: write B zeros.  Replaces probe_noop (csrc/probes.cu:86-94). */
int fsamp_probe_noop(int64_t B, int64_t* out, hipStream_t stream);

/* One full pass, one workgroup per row, argmax ids into out[B].
 * Replaces probe_scan_rowblock (csrc/probes.cu:96-106). */
int fsamp_probe_scan_rowblock(const void* logits, int dtype, int64_t B, int64_t V,
                              int64_t* out, hipStream_t stream);

/* Load-only floor of the sampler's large-batch launch shape (no counterpart in the reference):
 * one 512-thread workgroup per row reads the row with 38 nontemporal 16-byte loads per thread,
 * all in flight at once, and each of its 8 waves writes the largest order key of its share to
 * wave_max[b*8 + w] (device, B*8 uint32).  Needs a 16-byte-aligned base, V % 8 == 0 and
 * V <= 155648 (FSAMP_ERR_VOCAB otherwise). */
int fsamp_probe_load(const void* logits, int dtype, int64_t B, int64_t V, uint32_t* wave_max,
                     hipStream_t stream);

/* One full pass over `splits` workgroups per row, then a per-row merge (two launches);
 * ws needs B*splits*8 bytes.  Replaces probe_scan_split (csrc/probes.cu:108-125). */
int fsamp_probe_scan_split(const void* logits, int dtype, int64_t B, int64_t V,
                           int64_t splits, int64_t* out, void* ws, size_t ws_bytes,
                           hipStream_t stream);

/* Resource usage of every sampler kernel instantiation.  Replaces kernel_attrs
 * (csrc/fused_sampling.cu:515-540). */
typedef struct fsamp_attr_row {
  char name[64];
  int32_t threads;          /* workgroup size */
  int32_t chunks;           /* register chunks per thread */
  int32_t vgprs;            /* hipFuncAttributes::numRegs */
  int32_t scratch_bytes;    /* hipFuncAttributes::localSizeBytes (spill) */
  int32_t lds_bytes;        /* hipFuncAttributes::sharedSizeBytes */
  int32_t blocks_per_cu;    /* hipOccupancyMaxActiveBlocksPerMultiprocessor */
} fsamp_attr_row;

/* Writes up to max_rows rows; *n_rows receives the number of instantiations: every tiling
 * twice, the second time (name suffix ",merge") with the workgroup hand-off and merge that
 * calls with k > 128 and split rows launch. */
int fsamp_kernel_attrs(fsamp_attr_row* rows, int32_t max_rows, int32_t* n_rows);

/* Lane-layout self-test of the wave64 primitives the kernel is built on (DPP moves, swizzle,
 * the fixed-order scan and the bitonic network); writes 12*64 uint32 words to `out` (device).
 * No counterpart in the reference. */
int fsamp_debug_wave_selftest(uint32_t* out, hipStream_t stream);

/* Tuning aid with no counterpart in the reference: fsamp_sample (explicit u) that also records
 * the shader clock (s_memtime) at fixed points of every workgroup into trace[workgroup*32 + i],
 * i < 16, the constant 100 MHz clock (s_memrealtime) at its start and at the end of the
 * sampling tail into slots 16 and 17, and the shader clock at which wave w (w < 14) has its
 * whole share of the slice into slot 18 + w (device, B*splits*32 int64, pre-filled by the
 * caller). */
int fsamp_debug_sample_traced(const void* logits, int dtype, int64_t B, int64_t V,
                              int64_t top_k, double top_p, const float* u, int64_t* out,
                              void* ws, size_t ws_bytes, int64_t splits_override,
                              int64_t* trace, hipStream_t stream);

/* Tuning aid with no counterpart in the reference: force the workgroup size (256, 512 or
 * 1024) that later plans use, or 0 for the automatic choice.  Process-wide, not thread-safe;
 * a plan that cannot be tiled at that size fails with FSAMP_ERR_VOCAB. */
int fsamp_debug_force_threads(int32_t threads);

#ifdef __cplusplus
}
#endif

#endif /* FSAMP_H */
