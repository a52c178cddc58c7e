// fsamp_internal.h -- definitions shared by the sampler kernel and its host launcher.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace fsamp {

constexpr int CAND_CAP = 4096;   // LDS candidate words per workgroup (32 KiB)
constexpr int NSUB = 8;          // LDS sub-histograms in the radix fallback
constexpr int RMAX = (FSAMP_K_MAX + 63) / 64;  // ranks per lane in the tail
constexpr int MAX_SPLITS = 16;  // workgroups per row (the row merge ranks across <= 16 lists)
constexpr int TICKET_STRIDE = 32;  // u32 words between row counters: one 128-byte line each

// Kernel arguments (passed by value as kernarg).
struct Params {
  const uint16_t* logits;  // [B, V] fp16/bf16 bit patterns
  int64_t* out;            // [B] token ids (sample mode / ablation)
  int64_t* ids;            // [B, K] candidate ids (topk mode) or nullptr
  uint8_t* keep;           // [B, K] or nullptr
  float* renormed;         // [B, K] or nullptr
  uint64_t* words;         // [B, K] sorted (key, ~(id_offset + id)) words (shard mode) or nullptr
  const float* u;          // [B] uniforms or nullptr (splitmix64 of seed/offset/row)
  uint64_t seed, offset;
  const uint64_t* seed_src;    // device seed read in the kernel (replaces seed) or nullptr
  const uint64_t* offset_src;  // device base offset read in the kernel (offset is added) or nullptr
  uint64_t* partials;      // workspace: [B, S, K] per-split candidates
  uint32_t* tickets;       // workspace: [B] arrival counters, zero between calls
  uint32_t* grid_ticket;   // workspace: rows that have drawn from *offset_ctr, zero between calls
  uint64_t* offset_ctr;    // graph-safe draw offset advanced in the kernel (device) or nullptr
  const int32_t* topk_row; // per-row k, top_p, temperature (device) or nullptr
  const float* topp_row;
  const float* temp_row;
  int B, V, K, S;
  int64_t ld;              // elements between consecutive rows (>= V)
  uint32_t id_offset;      // added to every id written to words[]
  int slice;               // elements per split, a multiple of 8
  float top_p_f;           // (float)top_p
  int keep_all;            // top_p >= 1: keep every rank
  int is_bf16;
  int vec;                 // rows are 16-byte aligned: dwordx4 loads
  int stop;                // ablation phase (7 = the whole pipeline)
  int64_t* trace;          // per-workgroup phase timestamps (s_memtime) or nullptr
};

struct KernelEntry {
  int threads;
  int chunks;
  int vec;
  const void* fn;        // the common instantiation
  const void* fn_merge;  // with the workgroup hand-off and merge (k > 128, split rows)
  const char* name;
};

// (threads, chunks) register tilings that are compiled; chunks*8 elements per thread.
// Vector-load (16-byte aligned rows) tilings, by workgroup size (each group is compiled in its
// own parts of the build, see fsamp_kernel.hip):
#define FSAMP_KERNEL_LIST_VEC_256(X) \
  X(256, 1) X(256, 2) X(256, 3) X(256, 4) X(256, 5) X(256, 6) X(256, 8) X(256, 12) X(256, 16)
#define FSAMP_KERNEL_LIST_VEC_512(X) \
  X(512, 8) X(512, 12) X(512, 16) X(512, 20) X(512, 24) X(512, 32) X(512, 38)
#define FSAMP_KERNEL_LIST_VEC_1024(X) \
  X(1024, 4) X(1024, 5) X(1024, 6) X(1024, 8) X(1024, 10) X(1024, 12) X(1024, 16) X(1024, 19)
#define FSAMP_KERNEL_LIST_VEC(X) \
  FSAMP_KERNEL_LIST_VEC_256(X) FSAMP_KERNEL_LIST_VEC_512(X) FSAMP_KERNEL_LIST_VEC_1024(X)
// Element-load tilings (rows not 16-byte aligned, V % 8 != 0): small slices only; the planner
// adds splits until a slice fits.
#define FSAMP_KERNEL_LIST_SCALAR(X) \
  X(256, 1) X(256, 2) X(256, 3) X(256, 4) X(256, 6) X(256, 8) X(1024, 4) X(1024, 5) \
  X(1024, 6) X(1024, 8)

// Pipelined load of the large register tilings (vector loads, 512 or fewer threads, at least
// 12,288 vector chunks per workgroup): a thread keeps this many loads in flight, converting chunk
// c before it issues the next load, so that the selection can start before the slice has landed
// (the streaming selection in fsamp_kernel.hip).  0 issues every load at once.  On MI355X a
// 512 x 38 register load of the B=256 batch measured 15.7 us with every load in flight and
// 14.1-14.3 us at depths 4-12; the streaming sampler measured 18.78 / 18.99 us at depths 4 / 6,
// and depths above 6 push the 512 x 38 streaming kernel past 256 VGPRs.
// The 1024-thread tilings stay unpipelined: their streaming form needs more than the 128 VGPRs a
// 1024-thread workgroup may use and measured 30.6 us at B=256 against 19.0 us.
template <int NT, int CH, bool VEC>
constexpr int pipe_depth() {
#ifdef FSAMP_PIPE_DEPTH
  return VEC && NT < 1024 && CH * NT >= 12288 && CH >= 16 ? FSAMP_PIPE_DEPTH : 0;
#else
  return !VEC || NT >= 1024 || CH < 16 || CH * NT < 12288 ? 0 : 4;
#endif
}

// Chunks whose maxima give the streaming selection its lower bound (even: whole pairs), and the
// loads issued at once before the bound so that the pipe does not drain while it is computed.
template <int CH>
constexpr int stream_bound_chunks() {
#ifdef FSAMP_STREAM_BOUND
  return FSAMP_STREAM_BOUND;
#else
  return (CH * 2 / 3) & ~1;
#endif
}

template <int CH>
constexpr int stream_extra_loads() {
#ifdef FSAMP_STREAM_EXTRA
  return FSAMP_STREAM_EXTRA;
#else
  return 4;
#endif
}

extern const KernelEntry kKernels[];
extern const int kNumKernels;
// fsamp_merge_kernel<RB> for RB = 1, 2, 4, 8, 16
extern const void* const kMergeKernels[5];

}  // namespace fsamp
