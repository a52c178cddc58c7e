// fsamp_api.hip -- the C ABI declared in include/fsamp.h: plan, validation, launch.
//
// Host-side counterpart of make_plan / run_fused / sample_fused / topk_fused / stages_fused /
// probe_phase / kernel_attrs (csrc/fused_sampling.cu:331-540).  Everything here is plain C++
// over the HIP runtime: no torch types, no allocation, one kernel launch per sampler call.

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include <algorithm>

#include "fsamp.h"
#include "fsamp_internal.h"

namespace fsamp {
namespace {

size_t round_up(size_t a, size_t b) { return (a + b - 1) / b * b; }

// per-row arrival counters, one 128-byte line each (atomics on one line serialise)
size_t counter_bytes(int64_t B) { return round_up((size_t)B * TICKET_STRIDE * 4u, 256); }
constexpr size_t kGridCounterBytes = 256;  // the grid counter of the graph-safe draw

// Tiling preference forced by fsamp_debug_force_threads (0 = automatic).
int g_force_threads = 0;

// Split count when the caller does not force one: one workgroup per row once the batch alone
// fills half the CUs; below that, splits shorten each workgroup's selection chain (the
// slice's candidates, gather and sort shrink with it) at the price of one more list in the
// row merge.  Measured on MI355X (per call, k=50): V=151936 bf16 at B=1 10.35 / 10.38 /
// 9.97 / 10.45 us for S=4/5/6/7, and with 64-value ties at B=8 16.2 / 13.4 / 12.6 us for
// S=4/5/6; V=128256 fp16 at B=1 9.2 / 9.8 / 9.6 us for S=4/5/6 and at B=64 11.3 / 10.5 us
// for S=2/4.
int auto_splits(int64_t B, int64_t V) {
  if (B >= 128) return 1;
  if (B >= 64) return 4;
  return V > 131072 ? 6 : 4;
}

// Workgroup size for a slice: 256 threads while 8 chunks per thread hold it, then 512 (up to
// 38 chunks, 8 waves with room for the slice in VGPRs), then 1024;
// never fewer threads than k (the slice's lower bound ranks one maximum per thread and the
// candidate sort one candidate per thread).
int preferred_threads(int slice, int K) {
  int want = g_force_threads > 0 ? g_force_threads
             : (slice <= 256 * 8 * 8 ? 256 : (slice <= 512 * 8 * 38 ? 512 : 1024));
  while (want < K) want *= 2;
  return want;
}

// Smallest compiled tiling of the preferred workgroup size that holds `slice` elements; when
// that size has none large enough, the smallest-capacity tiling of any size (unless forced).
const KernelEntry* pick_tiling(int slice, int vec, int K) {
  const int want = preferred_threads(slice, K);
  const KernelEntry* best = nullptr;
  const KernelEntry* any = nullptr;
  for (int i = 0; i < kNumKernels; ++i) {
    const KernelEntry& e = kKernels[i];
    const int64_t cap = (int64_t)e.threads * e.chunks * 8;
    if (e.vec != vec || cap < slice || e.threads < K) continue;
    if (e.threads == want && (best == nullptr || e.chunks < best->chunks)) best = &e;
    if (any == nullptr || cap < (int64_t)any->threads * any->chunks * 8) any = &e;
  }
  if (best != nullptr || g_force_threads > 0) return best;
  return any;
}

int validate(int dtype, int64_t B, int64_t V, int64_t top_k) {
  if (dtype != FSAMP_DTYPE_F16 && dtype != FSAMP_DTYPE_BF16) return FSAMP_ERR_DTYPE;
  if (B < 1 || V < 1 || V > (int64_t)0x7FFFFFF0 || B > (int64_t)0x7FFFFFFF) return FSAMP_ERR_SHAPE;
  if (top_k < 1) return FSAMP_ERR_TOPK_LOW;
  if (std::min(top_k, V) > FSAMP_K_MAX) return FSAMP_ERR_TOPK_HIGH;
  return FSAMP_OK;
}

int make_plan_impl(const void* logits, int64_t B, int64_t V, int64_t top_k, int64_t splits_override,
                   fsamp_plan* pl, const KernelEntry** kern) {
  pl->batch = B;
  pl->vocab = V;
  pl->k = std::min(top_k, V);
  const int K = (int)pl->k;
  const bool vec = ((uintptr_t)logits % 16 == 0) && (V % 8 == 0);
  const int units = (int)((V + 7) / 8);
  int S = splits_override > 0 ? (int)std::min<int64_t>(splits_override, 1 << 20) : auto_splits(B, V);
  // the row's last workgroup merges S*K words in LDS, ranking across at most MAX_SPLITS lists
  S = std::max(1, std::min({S, CAND_CAP / K, MAX_SPLITS, units}));
  const KernelEntry* e = nullptr;
  int slice = 0;
  for (;;) {
    slice = ((units + S - 1) / S) * 8;
    e = pick_tiling(slice, vec ? 1 : 0, K);
    if (e != nullptr) break;
    if (S >= CAND_CAP / K || S >= MAX_SPLITS || S >= units) return FSAMP_ERR_VOCAB;
    ++S;
  }
  S = (int)((V + slice - 1) / slice);  // no empty trailing split
  pl->splits = S;
  pl->slice = slice;
  pl->threads = e->threads;
  pl->chunks = e->chunks;
  pl->vec = vec ? 1 : 0;
  pl->reserved = 0;
  pl->workspace_bytes = counter_bytes(B) + kGridCounterBytes +
                        (S > 1 ? (size_t)B * (size_t)S * (size_t)K * 8u : 0u);
  if (kern) *kern = e;
  return FSAMP_OK;
}

__global__ void fill_zero_kernel(uint32_t* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

int launch(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k, double top_p,
           const float* u, uint64_t seed, uint64_t offset, int64_t* out, int64_t* ids,
           uint8_t* keep, float* renormed, int stop, void* ws, size_t ws_bytes,
           int64_t splits_override, hipStream_t stream, int64_t* trace = nullptr,
           const fsamp_row_params* rows = nullptr) {
  int rc = validate(dtype, B, V, top_k);
  if (rc != FSAMP_OK) return rc;
  if (!(top_p > 0.0 && top_p <= 1.0)) return FSAMP_ERR_TOPP;
  if (logits == nullptr || (out == nullptr && ids == nullptr)) return FSAMP_ERR_NULL;
  if ((keep == nullptr) != (renormed == nullptr)) return FSAMP_ERR_NULL;
  fsamp_plan pl;
  const KernelEntry* e = nullptr;
  rc = make_plan_impl(logits, B, V, top_k, splits_override, &pl, &e);
  if (rc != FSAMP_OK) return rc;
  const bool use_ctr = rows != nullptr && rows->offset_counter != nullptr && u == nullptr;
  if ((pl.splits > 1 || use_ctr) && (ws == nullptr || ws_bytes < pl.workspace_bytes))
    return FSAMP_ERR_WORKSPACE;
  Params p;
  p.logits = static_cast<const uint16_t*>(logits);
  p.out = out;
  p.ids = ids;
  p.keep = keep;
  p.renormed = renormed;
  p.u = u;
  p.seed = seed;
  p.offset = offset;
  p.tickets = static_cast<uint32_t*>(ws);
  p.grid_ticket = ws != nullptr
                      ? reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + counter_bytes(B))
                      : nullptr;
  p.partials = pl.splits > 1 ? reinterpret_cast<uint64_t*>(static_cast<char*>(ws) +
                                                           counter_bytes(B) + kGridCounterBytes)
                             : nullptr;
  p.offset_ctr = use_ctr ? reinterpret_cast<uint64_t*>(rows->offset_counter) : nullptr;
  p.topk_row = rows != nullptr ? rows->top_k : nullptr;
  p.topp_row = rows != nullptr ? rows->top_p : nullptr;
  p.temp_row = rows != nullptr ? rows->temperature : nullptr;
  p.B = (int)B;
  p.V = (int)V;
  p.K = (int)pl.k;
  p.S = pl.splits;
  p.slice = pl.slice;
  p.top_p_f = (float)top_p;
  p.keep_all = top_p >= 1.0 ? 1 : 0;
  p.is_bf16 = dtype == FSAMP_DTYPE_BF16 ? 1 : 0;
  p.vec = pl.vec;
  p.stop = stop;
  p.trace = trace;
  void* args[] = {&p};
  const void* fn = (pl.k > 128 && pl.splits > 1) ? e->fn_merge : e->fn;
  const hipError_t err = hipLaunchKernel(fn, dim3((unsigned)(B * pl.splits)), dim3(e->threads),
                                         args, 0, stream);
  if (err != hipSuccess) return FSAMP_ERR_LAUNCH;
  if (hipGetLastError() != hipSuccess) return FSAMP_ERR_LAUNCH;
  return FSAMP_OK;
}

}  // namespace
}  // namespace fsamp

using namespace fsamp;

extern "C" {

const char* fsamp_error_string(int status) {
  switch (status) {
    case FSAMP_OK: return "ok";
    case FSAMP_ERR_DTYPE: return "logits must be float16 or bfloat16";
    case FSAMP_ERR_SHAPE: return "logits must be a contiguous cuda [B, V] tensor";
    case FSAMP_ERR_TOPK_LOW: return "top_k must be >= 1";
    case FSAMP_ERR_TOPK_HIGH: return "top_k must be <= 1024";
    case FSAMP_ERR_TOPP: return "top_p must be in (0, 1]";
    case FSAMP_ERR_WORKSPACE: return "workspace is missing or smaller than fsamp_workspace_bytes()";
    case FSAMP_ERR_NULL: return "a required pointer is NULL";
    case FSAMP_ERR_PHASE: return "phase must be in [1, 7]";
    case FSAMP_ERR_SPLITS: return "splits must be >= 1";
    case FSAMP_ERR_VOCAB: return "vocabulary too large for the workgroup tiling";
    case FSAMP_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown fsamp status";
  }
}

int fsamp_make_plan(const void* logits, int64_t B, int64_t V, int64_t top_k,
                    int64_t splits_override, fsamp_plan* plan) {
  if (plan == nullptr) return FSAMP_ERR_NULL;
  const int rc = validate(FSAMP_DTYPE_BF16, B, V, top_k);
  if (rc != FSAMP_OK) return rc;
  return make_plan_impl(logits, B, V, top_k, splits_override, plan, nullptr);
}

size_t fsamp_workspace_bytes(const void* logits, int64_t B, int64_t V, int64_t top_k,
                             int64_t splits_override) {
  fsamp_plan pl;
  if (fsamp_make_plan(logits, B, V, top_k, splits_override, &pl) != FSAMP_OK) return 0;
  return pl.workspace_bytes;
}

int fsamp_workspace_init(void* ws, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return FSAMP_OK;
  if (ws == nullptr) return FSAMP_ERR_NULL;
  const size_t n = bytes / 4;
  if (n == 0) return FSAMP_OK;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream,
                     static_cast<uint32_t*>(ws), n);
  return hipGetLastError() == hipSuccess ? FSAMP_OK : FSAMP_ERR_LAUNCH;
}

int fsamp_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                 double top_p, const float* u, uint64_t seed, uint64_t offset, int64_t* out,
                 void* ws, size_t ws_bytes, int64_t splits_override, hipStream_t stream) {
  if (out == nullptr) return FSAMP_ERR_NULL;
  return launch(logits, dtype, B, V, top_k, top_p, u, seed, offset, out, nullptr, nullptr,
                nullptr, 7, ws, ws_bytes, splits_override, stream);
}

int fsamp_sample_ex(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                    double top_p, const float* u, uint64_t seed, uint64_t offset,
                    const fsamp_row_params* rows, int64_t* out, uint8_t* keep, float* renormed,
                    void* ws, size_t ws_bytes, int64_t splits_override, hipStream_t stream) {
  if (out == nullptr) return FSAMP_ERR_NULL;
  return launch(logits, dtype, B, V, top_k, top_p, u, seed, offset, out, nullptr, keep, renormed,
                7, ws, ws_bytes, splits_override, stream, nullptr, rows);
}

int fsamp_stages(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                 double top_p, const float* u, uint64_t seed, uint64_t offset, int64_t* out,
                 uint8_t* keep, float* renormed, void* ws, size_t ws_bytes,
                 int64_t splits_override, hipStream_t stream) {
  if (out == nullptr || keep == nullptr || renormed == nullptr) return FSAMP_ERR_NULL;
  return launch(logits, dtype, B, V, top_k, top_p, u, seed, offset, out, nullptr, keep,
                renormed, 7, ws, ws_bytes, splits_override, stream);
}

int fsamp_topk(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
               int64_t* ids, void* ws, size_t ws_bytes, int64_t splits_override,
               hipStream_t stream) {
  if (ids == nullptr) return FSAMP_ERR_NULL;
  return launch(logits, dtype, B, V, top_k, 1.0, nullptr, 0, 0, nullptr, ids, nullptr, nullptr,
                7, ws, ws_bytes, splits_override, stream);
}

int fsamp_probe_phase(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                      double top_p, int64_t phase, int64_t* out, void* ws, size_t ws_bytes,
                      int64_t splits_override, hipStream_t stream) {
  if (phase < 1 || phase > 7) return FSAMP_ERR_PHASE;
  if (out == nullptr) return FSAMP_ERR_NULL;
  return launch(logits, dtype, B, V, top_k, top_p, nullptr, 0, 0, out, nullptr, nullptr, nullptr,
                (int)phase, ws, ws_bytes, splits_override, stream);
}

int fsamp_debug_force_threads(int32_t threads) {
  if (threads != 0 && threads != 256 && threads != 512 && threads != 1024) return FSAMP_ERR_SHAPE;
  g_force_threads = threads;
  return FSAMP_OK;
}

int fsamp_debug_sample_traced(const void* logits, int dtype, int64_t B, int64_t V,
                               int64_t top_k, double top_p, const float* u, int64_t* out,
                               void* ws, size_t ws_bytes, int64_t splits_override,
                               int64_t* trace, hipStream_t stream) {
  if (out == nullptr || trace == nullptr) return FSAMP_ERR_NULL;
  return launch(logits, dtype, B, V, top_k, top_p, u, 0, 0, out, nullptr, nullptr, nullptr, 7,
                ws, ws_bytes, splits_override, stream, trace);
}

int fsamp_kernel_attrs(fsamp_attr_row* rows, int32_t max_rows, int32_t* n_rows) {
  if (n_rows == nullptr) return FSAMP_ERR_NULL;
  // every tiling twice: the common instantiation, then the one with the workgroup merge
  *n_rows = 2 * kNumKernels;
  for (int i = 0; i < 2 * kNumKernels && i < max_rows; ++i) {
    const KernelEntry& e = kKernels[i % kNumKernels];
    const bool merge = i >= kNumKernels;
    const void* fn = merge ? e.fn_merge : e.fn;
    hipFuncAttributes a;
    if (hipFuncGetAttributes(&a, fn) != hipSuccess) return FSAMP_ERR_LAUNCH;
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, e.threads, 0) != hipSuccess)
      return FSAMP_ERR_LAUNCH;
    fsamp_attr_row& r = rows[i];
    memset(&r, 0, sizeof(r));
    strncpy(r.name, e.name, sizeof(r.name) - 1);
    if (merge) strncat(r.name, ",merge", sizeof(r.name) - 1 - strlen(r.name));
    r.threads = e.threads;
    r.chunks = e.chunks;
    r.vgprs = a.numRegs;
    r.scratch_bytes = (int32_t)a.localSizeBytes;
    r.lds_bytes = (int32_t)a.sharedSizeBytes;
    r.blocks_per_cu = blocks;
  }
  return FSAMP_OK;
}

}  // extern "C"
