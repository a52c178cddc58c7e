// fsamp_api.hip -- the C ABI declared in include/fsamp.h: plan, validation, launch.
//
// Host-side counterpart of make_plan / run_fused / sample_fused / topk_fused / stages_fused /
// probe_phase / kernel_attrs (csrc/fused_sampling.cu:331-540).  Everything here is plain C++
// over the HIP runtime: no torch types, no allocation, one kernel launch per sampler call.

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "fsamp.h"
#include "fsamp_internal.h"

namespace fsamp {
namespace {

size_t round_up(size_t a, size_t b) { return (a + b - 1) / b * b; }

// per-row arrival counters, one 128-byte line each (atomics on one line serialise)
size_t counter_bytes(int64_t B) { return round_up((size_t)B * TICKET_STRIDE * 4u, 256); }
constexpr size_t kGridCounterBytes = 256;  // the grid counter of the in-kernel offset advance

// Split count when the caller does not force one.  Splits shorten each workgroup's selection
// chain (the slice's candidates, gather and sort shrink with it) at the price of one more list
// in the row merge, but a grid of more workgroups than MI355X's 256 CUs runs in two waves (the
// large tilings hold one workgroup per CU), which costs far more than any split saves.  So the
// splits of a batch add up to at most 128 workgroups for k <= 128 (256 for wider k, whose
// selection is longer), and per row at most 8 (V > 196608), 6 (V > 131072), 4 (V > 65536) or
// 1: short rows gain less from a shorter chain than the hand-off and merge cost (V=32000 k=50 at
// B=1 / 16 / 64: 6.2 / 6.7 / 7.8 us unsplit against 8.4 / 8.5 / 9.2 us with 4 splits; V=50304
// at B=1 7.6 against 9.1 us), long ones more (V=256000 at B=1: 9.9 us with 8 splits, 10.3 with
// 6; V=202048: 9.9 against 10.7 us).  For 64 < k <= 128 (two ranks per lane in the merge) at
// most 4: V=151936 k=128 at B=1 / 16, 15.3 / 15.4 us against 15.7 / 16.0 us with 6 splits.
// Measured on MI355X (per call,
// graph replay, from the (threads, splits) sweep): V=151936 bf16 k=50 at B=48 12.2 / 12.0 /
// 18.4 us for S=2/3/6 and at B=96 14.4 / 13.7 / 20.2 us for S=1/2/4; V=128256 fp16 k=50 at
// B=64 12.9 / 11.9 / 12.3 us for S=1/2/4 and at B=96 12.8 / 19.2 us for S=1/4; B=1 k=50 at
// V=151936 10.35 / 9.97 / 10.45 us for S=4/6/7; with 64-value ties at B=8 16.2 / 12.6 us for
// S=4/6; k=256 at B=1..64 with 1024 threads 15.7-16.4 us for S=4, against 16.4-17.1 us for the
// 512-thread plans.
// Rows read element by element (not 16-byte aligned, V % 8 != 0) take the small element
// tilings, which gain from more splits at every row length: up to 8, within 256 workgroups
// (V=50257 k=50 at B = 1 / 16 / 64 / 128: 11.4 / 12.2 / 15.4 / 17.7 us with 8 / 8 / 4 / 2
// splits, against 19.4 / 20.6 / 20.7 / 20.8 us unsplit).
int auto_splits(int64_t B, int64_t V, int K, bool vec) {
  const int64_t grid = K > 128 || !vec ? 256 : 128;
  const int64_t most = K > 128  ? 4
                       : !vec   ? 8
                       : K > 64  ? (V > 65536 ? 4 : 1)
                       : V > 196608 ? 8 : V > 131072 ? 6 : V > 65536 ? 4 : 1;
  return (int)std::max<int64_t>(1, std::min<int64_t>(most, grid / B));
}

// Workgroup size for a slice: 256 threads while 8 chunks per thread hold it, then 512 (up to
// 38 chunks, 8 waves with room for the slice in VGPRs), then 1024; for k > 128, 1024 while 8
// chunks per thread hold the slice (the wide selection's histograms, ranking and merge run over
// the whole workgroup); `force` (a tuning override) replaces the choice; never fewer threads
// than k (the slice's lower bound ranks one maximum per thread and the candidate sort one
// candidate per thread).  A slice that 512 threads would hold in 32 chunks (V = 128256 or
// 131072 in one slice) takes 1024 threads x 16 chunks while the grid has at most 192
// workgroups: measured per call (graph replay) at V=128256 k=50 bf16, 11.6 / 11.9 / 12.7 us
// against 12.8 / 12.6 / 14.4 us at B = 96 / 128 / 192 (sixteen waves per CU keep more loads in
// flight); from B = 224 on the two measure alike at V=128256, and at V=131072 the 512-thread
// tiling is 1-2 us faster.
int preferred_threads(int slice, int K, int force, int64_t grid) {
  int want = force > 0                              ? force
             : K > 128 && slice <= 1024 * 8 * 8     ? 1024
             : slice <= 256 * 8 * 8                 ? 256
             : slice > 512 * 8 * 24 && slice <= 1024 * 8 * 16 && grid <= 192 ? 1024
             : slice <= 512 * 8 * 38                ? 512
                                                    : 1024;
  while (want < K) want *= 2;
  return want;
}

// Smallest compiled tiling of the preferred workgroup size that holds `slice` elements; when
// that size has none large enough, the smallest-capacity tiling of any size (unless forced).
const KernelEntry* pick_tiling(int slice, int vec, int K, int force, int64_t grid) {
  const int want = preferred_threads(slice, K, force, grid);
  const KernelEntry* best = nullptr;
  const KernelEntry* any = nullptr;
  for (int i = 0; i < kNumKernels; ++i) {
    const KernelEntry& e = kKernels[i];
    const int64_t cap = (int64_t)e.threads * e.chunks * 8;
    if (e.vec != vec || cap < slice || e.threads < K) continue;
    if (e.threads == want && (best == nullptr || e.chunks < best->chunks)) best = &e;
    if (any == nullptr || cap < (int64_t)any->threads * any->chunks * 8) any = &e;
  }
  if (best != nullptr || force > 0) return best;
  return any;
}

int validate(int dtype, int64_t B, int64_t V, int64_t top_k) {
  if (dtype != FSAMP_DTYPE_F16 && dtype != FSAMP_DTYPE_BF16) return FSAMP_ERR_DTYPE;
  if (B < 1 || V < 1 || V > (int64_t)0x7FFFFFF0 || B > (int64_t)0x7FFFFFFF) return FSAMP_ERR_SHAPE;
  if (top_k < 1) return FSAMP_ERR_TOPK_LOW;
  if (std::min(top_k, V) > FSAMP_K_MAX) return FSAMP_ERR_TOPK_HIGH;
  return FSAMP_OK;
}

int make_plan_impl(const void* logits, int64_t B, int64_t V, int64_t ld, int64_t top_k,
                   int64_t splits_override, int force_threads, fsamp_plan* pl,
                   const KernelEntry** kern) {
  pl->batch = B;
  pl->vocab = V;
  pl->k = std::min(top_k, V);
  const int K = (int)pl->k;
  const bool vec = ((uintptr_t)logits % 16 == 0) && (V % 8 == 0) && (ld % 8 == 0);
  const int units = (int)((V + 7) / 8);
  int S = splits_override > 0 ? (int)std::min<int64_t>(splits_override, 1 << 20) : auto_splits(B, V, K, vec);
  // the row's last workgroup merges S*K words in LDS, ranking across at most MAX_SPLITS lists
  S = std::max(1, std::min({S, CAND_CAP / K, MAX_SPLITS, units}));
  const KernelEntry* e = nullptr;
  int slice = 0;
  for (;;) {
    slice = ((units + S - 1) / S) * 8;
    e = pick_tiling(slice, vec ? 1 : 0, K, force_threads, B * (int64_t)S);
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

size_t scratch_bytes_of(const fsamp_plan& pl) {
  return pl.splits > 1 ? (size_t)pl.batch * (size_t)pl.splits * (size_t)pl.k * 8u : 0u;
}

__global__ void fill_zero_kernel(uint32_t* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// ---- fixed scratch of fsamp_sample_noalloc ---------------------------------------------------
//
// Device memory the library owns for callers that cannot allocate: FSAMP_NOALLOC_ROWS per-row
// tickets (128 bytes each) followed by FSAMP_NOALLOC_CANDIDATE_BYTES of split candidates, in a
// file-scope array that every GPU the library runs on holds once, until the process ends.  In
// host code `scratch` only names the array (it is no device address): its address on a device
// comes from hipGetSymbolAddress, taken once per device with that device current, and only that
// pointer is ever passed to a kernel.  The tickets must be zero before a call and every call
// leaves them zero; they are cleared once, by a fill kernel, at the first call on a device.
constexpr size_t kFixedTicketBytes = (size_t)FSAMP_NOALLOC_ROWS * TICKET_STRIDE * 4u;
constexpr size_t kFixedScratchBytes = kFixedTicketBytes + FSAMP_NOALLOC_CANDIDATE_BYTES;
static __device__ __align__(256) unsigned char scratch[kFixedScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_fixed_mu;
void* g_fixed_ptr[kMaxDevices] = {};

// The device's copy of `scratch` (set-up on first use), or nullptr on a HIP error.
void* fixed_scratch(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_fixed_mu);
  if (g_fixed_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
      return nullptr;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)(kFixedTicketBytes / 4 / 256)), dim3(256),
                       0, stream, static_cast<uint32_t*>(ptr), kFixedTicketBytes / 4);
    if (hipGetLastError() != hipSuccess) return nullptr;
    g_fixed_ptr[dev] = ptr;
  }
  return g_fixed_ptr[dev];
}

// One sampler launch, whatever entry point it came through.  The workspace arrives in one of
// two forms: a single buffer `ws` laid out as [tickets][grid counter][partials] (the classic
// entry points), or separate `counters` (tickets, persistent and zero between calls) and
// `scratch` (partials, any contents) buffers (fsamp_run and the fixed-scratch entry point).
struct Call {
  const void* logits = nullptr;
  int dtype = FSAMP_DTYPE_BF16;
  int64_t B = 0, V = 0, ld = 0, top_k = 0;
  double top_p = 1.0;
  int64_t splits_override = 0;
  int force_threads = 0;
  const float* u = nullptr;
  uint64_t seed = 0, offset = 0;
  const uint64_t* seed_src = nullptr;
  const uint64_t* offset_src = nullptr;
  uint64_t* offset_ctr = nullptr;  // fsamp_sample_ex's in-kernel counter
  const int32_t* topk_row = nullptr;
  const float* topp_row = nullptr;
  const float* temp_row = nullptr;
  int64_t* out = nullptr;
  int64_t* ids = nullptr;
  uint64_t* words = nullptr;
  uint32_t id_offset = 0;
  uint8_t* keep = nullptr;
  float* renormed = nullptr;
  int stop = 7;
  int64_t* trace = nullptr;
  // workspace, single-buffer form
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // workspace, split form
  bool split_ws = false;
  void* counters = nullptr;
  size_t counters_bytes = 0;
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
};

int launch(const Call& c, hipStream_t stream) {
  int rc = validate(c.dtype, c.B, c.V, c.top_k);
  if (rc != FSAMP_OK) return rc;
  if (c.ld < c.V) return FSAMP_ERR_SHAPE;
  if (!(c.top_p > 0.0 && c.top_p <= 1.0)) return FSAMP_ERR_TOPP;
  const int modes = (c.out != nullptr) + (c.ids != nullptr) + (c.words != nullptr);
  if (c.logits == nullptr || modes != 1) return FSAMP_ERR_NULL;
  if ((c.keep == nullptr) != (c.renormed == nullptr)) return FSAMP_ERR_NULL;
  if (c.keep != nullptr && c.out == nullptr) return FSAMP_ERR_NULL;
  fsamp_plan pl;
  const KernelEntry* e = nullptr;
  rc = make_plan_impl(c.logits, c.B, c.V, c.ld, c.top_k, c.splits_override, c.force_threads, &pl,
                      &e);
  if (rc != FSAMP_OK) return rc;
  if (c.words != nullptr && (uint64_t)c.id_offset + (uint64_t)c.V > 0xFFFFFFFEull)
    return FSAMP_ERR_SHAPE;
  Params p;
  memset(&p, 0, sizeof(p));
  const bool use_ctr = c.offset_ctr != nullptr && c.u == nullptr;
  if (!c.split_ws) {
    if ((pl.splits > 1 || use_ctr) && (c.ws == nullptr || c.ws_bytes < pl.workspace_bytes))
      return FSAMP_ERR_WORKSPACE;
    char* ws = static_cast<char*>(c.ws);
    p.tickets = reinterpret_cast<uint32_t*>(ws);
    p.grid_ticket = ws != nullptr ? reinterpret_cast<uint32_t*>(ws + counter_bytes(c.B)) : nullptr;
    p.partials = pl.splits > 1
                     ? reinterpret_cast<uint64_t*>(ws + counter_bytes(c.B) + kGridCounterBytes)
                     : nullptr;
  } else {
    if (use_ctr) return FSAMP_ERR_WORKSPACE;  // the split form has no grid counter
    if (pl.splits > 1) {
      if (c.counters == nullptr || c.counters_bytes < counter_bytes(c.B) || c.scratch == nullptr ||
          c.scratch_bytes < scratch_bytes_of(pl))
        return FSAMP_ERR_WORKSPACE;
      p.tickets = static_cast<uint32_t*>(c.counters);
      p.partials = static_cast<uint64_t*>(c.scratch);
    }
  }
  p.logits = static_cast<const uint16_t*>(c.logits);
  p.out = c.out;
  p.ids = c.ids;
  p.words = c.words;
  p.id_offset = c.id_offset;
  p.keep = c.keep;
  p.renormed = c.renormed;
  p.u = c.u;
  p.seed = c.seed;
  // the in-kernel counter of fsamp_sample_ex supplies the whole offset
  p.offset = use_ctr ? 0ull : c.offset;
  p.seed_src = c.u == nullptr ? c.seed_src : nullptr;
  p.offset_src = c.u == nullptr ? (use_ctr ? c.offset_ctr : c.offset_src) : nullptr;
  p.offset_ctr = use_ctr ? c.offset_ctr : nullptr;
  p.topk_row = c.topk_row;
  p.topp_row = c.topp_row;
  p.temp_row = c.temp_row;
  p.B = (int)c.B;
  p.V = (int)c.V;
  p.ld = c.ld;
  p.K = (int)pl.k;
  p.S = pl.splits;
  p.slice = pl.slice;
  p.top_p_f = (float)c.top_p;
  p.keep_all = c.top_p >= 1.0 ? 1 : 0;
  p.is_bf16 = c.dtype == FSAMP_DTYPE_BF16 ? 1 : 0;
  p.vec = pl.vec;
  p.stop = c.stop;
  p.trace = c.trace;
  void* args[] = {&p};
  const void* fn = (pl.k > 128 && pl.splits > 1) ? e->fn_merge : e->fn;
  const hipError_t err = hipLaunchKernel(fn, dim3((unsigned)(c.B * pl.splits)), dim3(e->threads),
                                         args, 0, stream);
  if (err != hipSuccess) return FSAMP_ERR_LAUNCH;
  if (hipGetLastError() != hipSuccess) return FSAMP_ERR_LAUNCH;
  return FSAMP_OK;
}

// The classic argument list as a Call (contiguous rows, single-buffer workspace).
Call classic(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k, double top_p,
             const float* u, uint64_t seed, uint64_t offset, void* ws, size_t ws_bytes,
             int64_t splits_override) {
  Call c;
  c.logits = logits;
  c.dtype = dtype;
  c.B = B;
  c.V = V;
  c.ld = V;
  c.top_k = top_k;
  c.top_p = top_p;
  c.u = u;
  c.seed = seed;
  c.offset = offset;
  c.ws = ws;
  c.ws_bytes = ws_bytes;
  c.splits_override = splits_override;
#ifdef FSAMP_TUNE_THREADS
  c.force_threads = FSAMP_TUNE_THREADS;  // tuning builds only: the workgroup size of every call
#endif
  return c;
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
    case FSAMP_ERR_VERSION: return "fsamp_call.struct_bytes does not match this library";
    case FSAMP_ERR_SCRATCH:
      return "the call needs more than fsamp_sample_noalloc's fixed scratch (batch above "
             "FSAMP_NOALLOC_ROWS or split candidates above FSAMP_NOALLOC_CANDIDATE_BYTES)";
    default: return "unknown fsamp status";
  }
}

int fsamp_make_plan(const void* logits, int64_t B, int64_t V, int64_t top_k,
                    int64_t splits_override, fsamp_plan* plan) {
  if (plan == nullptr) return FSAMP_ERR_NULL;
  const int rc = validate(FSAMP_DTYPE_BF16, B, V, top_k);
  if (rc != FSAMP_OK) return rc;
  return make_plan_impl(logits, B, V, V, top_k, splits_override, 0, plan, nullptr);
}

size_t fsamp_workspace_bytes(const void* logits, int64_t B, int64_t V, int64_t top_k,
                             int64_t splits_override) {
  fsamp_plan pl;
  if (fsamp_make_plan(logits, B, V, top_k, splits_override, &pl) != FSAMP_OK) return 0;
  return pl.workspace_bytes;
}

size_t fsamp_counter_bytes(int64_t B) { return B < 1 ? 0 : counter_bytes(B); }

size_t fsamp_scratch_bytes(const void* logits, int64_t B, int64_t V, int64_t top_k,
                           int64_t splits_override) {
  fsamp_plan pl;
  if (fsamp_make_plan(logits, B, V, top_k, splits_override, &pl) != FSAMP_OK) return 0;
  return scratch_bytes_of(pl);
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

int fsamp_run(const fsamp_call* a, hipStream_t stream) {
  if (a == nullptr) return FSAMP_ERR_NULL;
  if (a->struct_bytes != sizeof(fsamp_call)) return FSAMP_ERR_VERSION;
  if (a->threads_override != 0 && a->threads_override != 256 && a->threads_override != 512 &&
      a->threads_override != 1024)
    return FSAMP_ERR_SHAPE;
  if (a->id_offset < 0 || a->id_offset > (int64_t)0xFFFFFFFF) return FSAMP_ERR_SHAPE;
  Call c;
  c.logits = a->logits;
  c.dtype = a->dtype;
  c.B = a->batch;
  c.V = a->vocab;
  c.ld = a->ld == 0 ? a->vocab : a->ld;
  c.top_k = a->top_k;
  c.top_p = a->top_p;
  c.splits_override = a->splits_override;
  c.force_threads = a->threads_override;
  c.u = a->u;
  c.seed = a->seed;
  c.offset = a->offset;
  c.seed_src = reinterpret_cast<const uint64_t*>(a->seed_ptr);
  c.offset_src = reinterpret_cast<const uint64_t*>(a->offset_ptr);
  c.topk_row = a->top_k_row;
  c.topp_row = a->top_p_row;
  c.temp_row = a->temperature_row;
  c.out = a->out;
  c.ids = a->ids;
  c.words = a->words;
  c.id_offset = (uint32_t)a->id_offset;
  c.keep = a->keep;
  c.renormed = a->renormed;
  c.split_ws = true;
  c.counters = a->counters;
  c.counters_bytes = a->counter_bytes;
  c.scratch = a->scratch;
  c.scratch_bytes = a->scratch_bytes;
  return launch(c, stream);
}

int fsamp_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                 double top_p, const float* u, uint64_t seed, uint64_t offset, int64_t* out,
                 void* ws, size_t ws_bytes, int64_t splits_override, hipStream_t stream) {
  if (out == nullptr) return FSAMP_ERR_NULL;
  Call c = classic(logits, dtype, B, V, top_k, top_p, u, seed, offset, ws, ws_bytes,
                   splits_override);
  c.out = out;
  return launch(c, stream);
}

int fsamp_sample_ex(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                    double top_p, const float* u, uint64_t seed, uint64_t offset,
                    const fsamp_row_params* rows, int64_t* out, uint8_t* keep, float* renormed,
                    void* ws, size_t ws_bytes, int64_t splits_override, hipStream_t stream) {
  if (out == nullptr) return FSAMP_ERR_NULL;
  Call c = classic(logits, dtype, B, V, top_k, top_p, u, seed, offset, ws, ws_bytes,
                   splits_override);
  c.out = out;
  c.keep = keep;
  c.renormed = renormed;
  if (rows != nullptr) {
    c.topk_row = rows->top_k;
    c.topp_row = rows->top_p;
    c.temp_row = rows->temperature;
    c.offset_ctr = rows->offset_counter;
  }
  return launch(c, stream);
}

int fsamp_stages(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                 double top_p, const float* u, uint64_t seed, uint64_t offset, int64_t* out,
                 uint8_t* keep, float* renormed, void* ws, size_t ws_bytes,
                 int64_t splits_override, hipStream_t stream) {
  if (out == nullptr || keep == nullptr || renormed == nullptr) return FSAMP_ERR_NULL;
  Call c = classic(logits, dtype, B, V, top_k, top_p, u, seed, offset, ws, ws_bytes,
                   splits_override);
  c.out = out;
  c.keep = keep;
  c.renormed = renormed;
  return launch(c, stream);
}

int fsamp_topk(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
               int64_t* ids, void* ws, size_t ws_bytes, int64_t splits_override,
               hipStream_t stream) {
  if (ids == nullptr) return FSAMP_ERR_NULL;
  Call c = classic(logits, dtype, B, V, top_k, 1.0, nullptr, 0, 0, ws, ws_bytes, splits_override);
  c.ids = ids;
  return launch(c, stream);
}

int fsamp_probe_phase(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                      double top_p, int64_t phase, int64_t* out, void* ws, size_t ws_bytes,
                      int64_t splits_override, hipStream_t stream) {
  if (phase < 1 || phase > 7) return FSAMP_ERR_PHASE;
  if (out == nullptr) return FSAMP_ERR_NULL;
  Call c = classic(logits, dtype, B, V, top_k, top_p, nullptr, 0, 0, ws, ws_bytes,
                   splits_override);
  c.out = out;
  c.stop = (int)phase;
  return launch(c, stream);
}

int fsamp_debug_sample_traced(const void* logits, int dtype, int64_t B, int64_t V,
                               int64_t top_k, double top_p, const float* u, int64_t* out,
                               void* ws, size_t ws_bytes, int64_t splits_override,
                               int64_t* trace, hipStream_t stream) {
  if (out == nullptr || trace == nullptr) return FSAMP_ERR_NULL;
  Call c = classic(logits, dtype, B, V, top_k, top_p, u, 0, 0, ws, ws_bytes, splits_override);
  c.out = out;
  c.trace = trace;
  return launch(c, stream);
}

int fsamp_sample_noalloc(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                         double top_p, const float* u, uint64_t seed, uint64_t offset,
                         int64_t* out, int64_t splits_override, hipStream_t stream) {
  if (out == nullptr) return FSAMP_ERR_NULL;
  int rc = validate(dtype, B, V, top_k);
  if (rc != FSAMP_OK) return rc;
  fsamp_plan pl;
  rc = make_plan_impl(logits, B, V, V, top_k, splits_override, 0, &pl, nullptr);
  if (rc != FSAMP_OK) return rc;
  Call c = classic(logits, dtype, B, V, top_k, top_p, u, seed, offset, nullptr, 0,
                   splits_override);
  c.out = out;
  c.split_ws = true;
  if (pl.splits > 1) {
    if (B > FSAMP_NOALLOC_ROWS || scratch_bytes_of(pl) > FSAMP_NOALLOC_CANDIDATE_BYTES)
      return FSAMP_ERR_SCRATCH;
    char* ptr = static_cast<char*>(fixed_scratch(stream));
    if (ptr == nullptr) return FSAMP_ERR_LAUNCH;
    c.counters = ptr;
    c.counters_bytes = kFixedTicketBytes;
    c.scratch = ptr + kFixedTicketBytes;
    c.scratch_bytes = FSAMP_NOALLOC_CANDIDATE_BYTES;
  }
  return launch(c, stream);
}

int fsamp_topk_shard(const void* logits, int dtype, int64_t B, int64_t V_shard, int64_t ld,
                     int64_t top_k, int64_t id_offset, uint64_t* words, void* counters,
                     size_t counter_bytes, void* scratch, size_t scratch_bytes,
                     int64_t splits_override, hipStream_t stream) {
  if (words == nullptr) return FSAMP_ERR_NULL;
  if (top_k > V_shard && V_shard >= 1) return FSAMP_ERR_TOPK_HIGH;
  fsamp_call a;
  memset(&a, 0, sizeof(a));
  a.struct_bytes = sizeof(a);
  a.logits = logits;
  a.dtype = dtype;
  a.batch = B;
  a.vocab = V_shard;
  a.ld = ld;
  a.top_k = top_k;
  a.top_p = 1.0;
  a.splits_override = splits_override;
  a.words = words;
  a.id_offset = id_offset;
  a.counters = counters;
  a.counter_bytes = counter_bytes;
  a.scratch = scratch;
  a.scratch_bytes = scratch_bytes;
  return fsamp_run(&a, stream);
}

int fsamp_merge_sample(const uint64_t* words, int dtype, int64_t B, int64_t n_lists, int64_t k,
                       double top_p, const float* u, uint64_t seed, uint64_t offset,
                       int64_t* out, uint8_t* keep, float* renormed, int64_t* ids,
                       hipStream_t stream) {
  if (dtype != FSAMP_DTYPE_F16 && dtype != FSAMP_DTYPE_BF16) return FSAMP_ERR_DTYPE;
  if (B < 1 || B > (int64_t)0x7FFFFFFF || n_lists < 1 || n_lists > 4096) return FSAMP_ERR_SHAPE;
  if (k < 1) return FSAMP_ERR_TOPK_LOW;
  if (k > FSAMP_K_MAX) return FSAMP_ERR_TOPK_HIGH;
  if (!(top_p > 0.0 && top_p <= 1.0)) return FSAMP_ERR_TOPP;
  if (words == nullptr || ((out == nullptr) == (ids == nullptr))) return FSAMP_ERR_NULL;
  if ((keep == nullptr) != (renormed == nullptr) || (keep != nullptr && out == nullptr))
    return FSAMP_ERR_NULL;
  Params p;
  memset(&p, 0, sizeof(p));
  p.out = out;
  p.ids = ids;
  p.keep = keep;
  p.renormed = renormed;
  p.u = u;
  p.seed = seed;
  p.offset = offset;
  p.B = (int)B;
  p.K = (int)k;
  p.S = 1;
  p.top_p_f = (float)top_p;
  p.keep_all = top_p >= 1.0 ? 1 : 0;
  p.is_bf16 = dtype == FSAMP_DTYPE_BF16 ? 1 : 0;
  p.stop = 7;
  const int rb = k <= 64 ? 0 : k <= 128 ? 1 : k <= 256 ? 2 : k <= 512 ? 3 : 4;
  int nl = (int)n_lists;
  const uint64_t* w = words;
  void* args[] = {&p, &w, &nl};
  const hipError_t err = hipLaunchKernel(kMergeKernels[rb], dim3((unsigned)B), dim3(64), args, 0,
                                         stream);
  if (err != hipSuccess || hipGetLastError() != hipSuccess) return FSAMP_ERR_LAUNCH;
  return FSAMP_OK;
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
