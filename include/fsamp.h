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
  FSAMP_ERR_LAUNCH = 11,    /* the HIP runtime reported an error at launch */
  FSAMP_ERR_VERSION = 12,   /* fsamp_call.struct_bytes is not sizeof(fsamp_call) */
  FSAMP_ERR_SCRATCH = 13    /* the call needs more than fsamp_sample_noalloc's fixed scratch */
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

/* Bytes of single-buffer workspace a call with these arguments needs: always the counter
 * regions (round_up(128*B, 256) + 256 bytes), plus B*splits*k*8 candidate bytes when the plan
 * splits rows.  Returns 0 only for invalid arguments (fsamp_make_plan gives the reason). */
size_t fsamp_workspace_bytes(const void* logits, int64_t B, int64_t V, int64_t top_k,
                             int64_t splits_override);

/* The two parts of the split workspace that fsamp_run, fsamp_topk_shard take (no counterpart in
 * the reference, which allocates its per-split partials per call and needs no counters):
 *   counters  fsamp_counter_bytes(B) bytes of per-row arrival counters.  They must be zero
 *             before the first call and every call leaves them zero, so one buffer, zeroed once
 *             (fsamp_workspace_init), serves every later call on a stream; calls that run
 *             concurrently (different streams) need their own.
 *   scratch   fsamp_scratch_bytes(...) bytes of per-split candidates, any contents (0 when the
 *             plan has one split: scratch may then be NULL, and counters too).
 * Because the counters never share memory with the candidates, calls of any batch size can
 * share one counter buffer in any order (HIP graphs captured at several sizes included). */
size_t fsamp_counter_bytes(int64_t B);
size_t fsamp_scratch_bytes(const void* logits, int64_t B, int64_t V, int64_t top_k,
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
 * fsamp_sample without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid allocation).  No
 * counterpart in the reference.  Split rows use a fixed scratch that the library holds on each
 * GPU until the process ends (FSAMP_NOALLOC_ROWS * 128 bytes of row tickets plus
 * FSAMP_NOALLOC_CANDIDATE_BYTES of candidates, 4.125 MiB); a call whose plan needs more (a
 * split plan with B > FSAMP_NOALLOC_ROWS, or B*splits*k*8 candidate bytes above the limit)
 * returns FSAMP_ERR_SCRATCH.  Nothing is allocated or freed.  The call takes the device's scratch
 * address once, at its first call on that device (the current device, which `stream` must
 * belong to), and clears the tickets there with a fill kernel on `stream`.  Every call on one
 * GPU shares its scratch: calls that may overlap on one GPU (different streams, concurrent graph
 * replays) race and must be serialised by the caller.
 */
#define FSAMP_NOALLOC_ROWS 1024
#define FSAMP_NOALLOC_CANDIDATE_BYTES (4u << 20)
int fsamp_sample_noalloc(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                         double top_p, const float* u, uint64_t seed, uint64_t offset,
                         int64_t* out, int64_t splits_override, hipStream_t stream);

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
 * the counter is an in-kernel alternative to the reference's generator path (sample_fused
 * with offset < 0 takes torch's Philox state, csrc/fused_sampling.cu:441-447), which
 * fsamp_run's seed_ptr / offset_ptr reproduce exactly.
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
 * One call described in full: every option of the entry points above, with a row stride, the
 * split workspace, and the seed / offset either as values or as device pointers read in the
 * kernel.  The torch binding (fused_sampling) calls this.  Output modes, exactly one of:
 *   out       [B] int64 token ids (keep / renormed [B, k] may be added, as in fsamp_stages);
 *   ids       [B, k] int64 candidate ids (fsamp_topk);
 *   words     [B, k] uint64 sorted candidate words (fsamp_topk_shard).
 * The uniform of row b, when u == NULL, is splitmix64(S, O, b) with
 *   S = seed_ptr ? *seed_ptr : seed,     O = (offset_ptr ? *offset_ptr : 0) + offset,
 * which is how the reference unpacks torch's Philox state (at::cuda::philox::unpack for
 * csrc/fused_sampling.cu:296-300): eager calls pass the generator's (seed, offset) values, a
 * call captured in a HIP graph passes the graph's seed and offset pointers and its offset
 * within the graph, so eager calls and graph replays draw from one generator stream.
 */
typedef struct fsamp_call {
  size_t struct_bytes;             /* sizeof(fsamp_call) (FSAMP_ERR_VERSION otherwise) */
  const void* logits;              /* row b at logits + b*ld elements */
  int32_t dtype;
  int32_t threads_override;        /* 0, or force the workgroup size 256/512/1024 (tuning) */
  int64_t batch, vocab;
  int64_t ld;                      /* elements between rows; 0 means vocab */
  int64_t top_k;
  double top_p;
  int64_t splits_override;
  const float* u;                  /* [B] uniforms in [0,1), or NULL */
  uint64_t seed, offset;
  const int64_t* seed_ptr;         /* device, or NULL */
  const int64_t* offset_ptr;       /* device, or NULL */
  const int32_t* top_k_row;        /* per-row controls as in fsamp_row_params, or NULL */
  const float* top_p_row;
  const float* temperature_row;
  int64_t* out;
  uint8_t* keep;
  float* renormed;
  int64_t* ids;
  uint64_t* words;
  int64_t id_offset;               /* words mode: added to every id (0 <= id_offset, and
                                      id_offset + vocab < 2^32 - 1) */
  void* counters;                  /* split workspace (fsamp_counter_bytes(batch)) */
  size_t counter_bytes;
  void* scratch;                   /* split workspace (fsamp_scratch_bytes(...)) */
  size_t scratch_bytes;
} fsamp_call;

int fsamp_run(const fsamp_call* call, hipStream_t stream);

/*
 * Vocabulary-parallel selection, one shard: logits [B, V_shard] (row stride ld) are columns
 * [id_offset, id_offset + V_shard) of the whole rows.  Writes the shard's top_k candidates of
 * every row as words[b*top_k + i] = (key << 32) | (0xFFFFFFFF - (id_offset + id)), sorted
 * descending (value, then lowest id), the same word the row's split workgroups hand to its
 * merge.  Needs top_k <= V_shard.  Lifts the reference's per-split contract (unsorted top-K per
 * split in partial[B, splits, K], csrc/fused_sampling.cu:156, :242) from workgroups to shards;
 * a tensor-parallel LM head gathers the B x top_k words of every shard (one all-gather) and
 * calls fsamp_merge_sample on the N lists.  Workspace as fsamp_run.
 */
int fsamp_topk_shard(const void* logits, int dtype, int64_t B, int64_t V_shard, int64_t ld,
                     int64_t top_k, int64_t id_offset, uint64_t* words, void* counters,
                     size_t counter_bytes, void* scratch, size_t scratch_bytes,
                     int64_t splits_override, hipStream_t stream);

/*
 * Merge N sorted candidate lists per row and sample: words [B, N, k] (each list as
 * fsamp_topk_shard writes it; a short list ends in zero words, and the N lists of a row must
 * hold at least k candidate words between them) -> the row's top k -> the fp32
 * tail of fsamp_sample (u, or splitmix64(seed, offset, row) when u == NULL) -> out[B] token
 * ids (keep / renormed [B, k] optional), or, with out == NULL, ids [B, k] of the merged top k.
 * dtype says how the keys decode to values.  One wave per row.  Replaces the reference's
 * merge over splits*K partial candidates (merge_sample_kernel / merge_ids_kernel,
 * csrc/fused_sampling.cu:245-329) with N shard lists in place of the splits.
 */
int fsamp_merge_sample(const uint64_t* words, int dtype, int64_t B, int64_t n_lists, int64_t k,
                       double top_p, const float* u, uint64_t seed, uint64_t offset,
                       int64_t* out, uint8_t* keep, float* renormed, int64_t* ids,
                       hipStream_t stream);

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
 * issued as the sampler issues them (6 in flight), and each of its 8 waves writes the largest
 * order key of its share to
 * wave_max[b*8 + w] (device, B*8 uint32).  Needs a 16-byte-aligned base, V % 8 == 0 and
 * V <= 155648 (FSAMP_ERR_VOCAB otherwise). */
int fsamp_probe_load(const void* logits, int dtype, int64_t B, int64_t V, uint32_t* wave_max,
                     hipStream_t stream);

/* Pure streaming-read floor of a whole batch (no counterpart in the reference): the contiguous
 * [B, V] logits read once by short 256-thread workgroups of 4 nontemporal 16-byte loads per
 * thread (16 KB each, as many as the batch needs), each wave writing the largest order key of
 * its 4 KB to wave_max (device, fsamp_probe_stream_words(B, V) uint32).  It bounds what any
 * one-pass kernel can read at, free of a row shape.  Needs a 16-byte-aligned base and
 * V % 8 == 0 (FSAMP_ERR_VOCAB), and n_words >= fsamp_probe_stream_words (FSAMP_ERR_WORKSPACE). */
int64_t fsamp_probe_stream_words(int64_t B, int64_t V);
int fsamp_probe_stream(const void* logits, int dtype, int64_t B, int64_t V, uint32_t* wave_max,
                       int64_t n_words, hipStream_t stream);

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

#ifdef __cplusplus
}
#endif

#endif /* FSAMP_H */
