// fsamp_kernel.hip -- fused top-k + top-p sampler for gfx950 (CDNA4), one launch per call.
//
// Each row of [B, V] fp16/bf16 logits is cut into `S` slices; workgroup (row, split) keeps its
// slice in VGPRs as packed 16-bit order keys (one HBM read), finds the exact top-k of the
// slice and, when S > 1, hands the k candidates to the last workgroup of the row to finish,
// which merges the S lists.  The workgroup that owns the row's final top-k then runs the
// fp32 tail: softmax over the k survivors, prefix, top-p cut on the exclusive prefix and the
// inverse-CDF draw against u * Z_p.
//
// Reference behaviour followed (sathviknookala/llm_sampling_kernel):
//   order key and (key, ~id) packing     csrc/fused_sampling.cuh:8-23 (here -0 and +0 share a
//                                        key so ties follow benchmarks/reference.py:53)
//   exact top-k with lowest-id ties      csrc/fused_sampling.cu:127-243, SEMANTICS.md:150-183
//   split-row selection + row merge      csrc/fused_sampling.cu:143-156, :245-262
//   softmax/prefix/cut/draw              csrc/fused_sampling.cu:264-309, reference.py:55-68
//   key -> value decode                  csrc/fused_sampling.cuh:50-63
//   splitmix64 uniform                   csrc/fused_sampling.cuh:65-71
//
// Selection, MI355X-first (one HBM read; every later step works on registers and LDS):
//   1. every thread issues all of its dwordx4 loads at once (CH chunks of 8 elements, chunk c
//      of thread t at uint4 index c*NT + t: coalesced) and, as each chunk lands, converts it
//      to packed u16 order keys with 16-bit packed integer ops, keeping the chunk maxima
//      (two per VGPR) and the thread maximum;
//   2. L, a lower bound of the slice's k-th largest key: each wave sorts its 64 thread maxima
//      with a DPP bitonic network, publishes its top ceil(k/W), and the k-th largest of those
//      W lists (ranked by binary search) owns k distinct elements >= L;
//   3. elements >= L (typically ~1-2 per qualifying thread) are gathered into per-wave LDS
//      regions as u64 (key << 32 | ~id) words -- unique, so ordering them orders by value and
//      then by ascending id, which is the tie rule -- with one compare per chunk (cached maxima);
//   4. the candidates are ranked by counting (one barrier) into the sorted top-k; if there
//      are more than one per thread (heavy ties), an exact radix select over the registers
//      (two 8-bit LDS histograms restricted to keys >= L, a gather above the threshold and an
//      id-ordered block scan of the tied keys) first reduces them to exactly k.
// No step re-reads HBM.  Rows split over several workgroups hand their sorted top-k to the
// row's last workgroup through write-through atomics and are merged by rank.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "fsamp.h"
#include "fsamp_internal.h"
#include "fsamp_wave.h"

namespace fsamp {

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// One 16-byte load of logits with the nontemporal hint (global_load_dwordx4 ... nt): every
// logit is read exactly once, so the lines are not worth keeping in the caches.  On MI355X a
// 256-workgroup pass over the B=256 batch (38 such loads per thread, all issued at once)
// measured 12.5 us with the hint against 13.9 us without it.
__device__ __forceinline__ uint4 load_stream16(const uint16_t* a) {
  const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a));
  return make_uint4(r.x, r.y, r.z, r.w);
}

// ---- packed 16-bit keys -----------------------------------------------------------------

// Two 16-bit floats -> two order keys, per half: negative b -> 0x10000 - b, non-negative
// b -> b | 0x8000.  Descending value == descending key, -0 and +0 both map to 0x8000, every
// real value maps to a key >= 1 (0 is reserved for padding).  For a negative half
// (b ^ 0xFFFF) + 1 <= 0x8000, so the add never carries into the other half.
__device__ __forceinline__ uint32_t keys2(uint32_t w) {
  const s16x2 v = __builtin_bit_cast(s16x2, w);
  const s16x2 s = v >> (s16x2)(15);
  const uint32_t su = __builtin_bit_cast(uint32_t, s);
  return (w ^ (su | 0x80008000u)) + (su & 0x00010001u);
}

__device__ __forceinline__ uint32_t pkmax(uint32_t a, uint32_t b) {
  const u16x2 x = __builtin_bit_cast(u16x2, a);
  const u16x2 y = __builtin_bit_cast(u16x2, b);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(x, y));
}

__device__ __forceinline__ uint32_t key16(uint16_t b) {
  return (b & 0x8000u) ? ((0x10000u - b) & 0xFFFFu) : (uint32_t)(b | 0x8000u);
}

__device__ __forceinline__ uint64_t pack(uint32_t key, uint32_t id) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - id);
}

__device__ __forceinline__ uint32_t unpack_id(uint64_t w) {
  return 0xFFFFFFFFu - (uint32_t)(w & 0xFFFFFFFFull);
}

// A candidate word with its id moved by `off` (a shard's first column in the whole row): the
// low half is ~id, so ~(id + off) = ~id - off.  Zero words (padding past the slice) stay zero.
__device__ __forceinline__ uint64_t global_word(uint64_t w, uint32_t off) {
  return w == 0ull ? 0ull : w - (uint64_t)off;
}

// key -> fp32 value (the exact bf16/fp16 value; the -0 key decodes to +0)
__device__ __forceinline__ float key_to_float(uint32_t key, int is_bf16) {
  const uint32_t b = (key & 0x8000u) ? (key & 0x7FFFu) : ((0x10000u - key) & 0xFFFFu);
  // both decodes and a select: no branch in the latency-bound tail
  const float as_bf16 = __uint_as_float(b << 16);
  const float as_f16 = (float)__builtin_bit_cast(_Float16, (unsigned short)b);
  return is_bf16 ? as_bf16 : as_f16;
}

// ---- fp32 tail helpers -------------------------------------------------------------------

// e^x for x <= 0: Cody-Waite split by ln2 (16-bit head, tail), degree-7 Taylor polynomial for
// |r| <= ln2/2 by Horner with fma, scale by 2^n from exponent bits; x < -86 gives 0.
// Bit-identical to the CPU oracle's exp, which evaluates the same operations in the same order.
__device__ __forceinline__ float exp_nonpos(float x) {
  // evaluated for every x and selected at the end (no branch); below -86, or for NaN, the
  // intermediate scale is meaningless and the select returns 0
  const bool in_range = x >= -86.0f;
  x = in_range ? x : 0.0f;
  const float n = rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, x);
  r = __builtin_fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.0f / 5040.0f;
  p = __builtin_fmaf(p, r, 1.0f / 720.0f);
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const float e = p * __uint_as_float((uint32_t)(ni + 127) << 23);
  return in_range ? e : 0.0f;
}

// splitmix64 finalizer over (seed, offset, row): 24-bit uniform in [0, 1)
__device__ __forceinline__ float rng_uniform(uint64_t seed, uint64_t offset, uint32_t row) {
  uint64_t z = seed + offset * 0x9E3779B97F4A7C15ull + (uint64_t)row * 0xD1B54A32D192ED03ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z = z ^ (z >> 31);
  return (float)((z >> 40) & 0xFFFFFFull) * (1.0f / 16777216.0f);
}

// ---- LDS layout ----------------------------------------------------------------------------

constexpr int STAGE_SLOTS = 4;  // chunk pairs a thread can stage for the gather

// Wide selection (k > WIDE_MIN on split rows): candidates ranked by key bins d = M - key
// below the slice maximum M.  A bin holding more than WIDE_BIN_MAX candidates (heavy ties,
// where the in-bin ranking is quadratic) or a bound farther than WIDE_BINS keys below M sends
// the slice to the general selection.  On split rows with k = 256 it measured 18.2 us against
// 22.3 us for the general selection and bitonic merge (B=16, V=151936, six splits).
#ifdef FSAMP_WIDE_MIN
constexpr int WIDE_MIN = FSAMP_WIDE_MIN;
#else
constexpr int WIDE_MIN = 128;    // the wide selection and merge serve k > WIDE_MIN
#endif
constexpr int WIDE_BINS = 1024;
constexpr int WIDE_BIN_MAX = 256;

template <int NT>
struct Smem {
  union {
    uint64_t cand[CAND_CAP];   // radix-select candidates; later the row's split lists
    struct {
      uint4 a[STAGE_SLOTS][NT];  // staged chunk pairs: even chunk
      uint4 b[STAGE_SLOTS][NT];  //                     odd chunk
    } st;
  } g;
  uint64_t top[FSAMP_K_MAX];   // gathered candidates, then the sorted top-K of the slice/row
  uint8_t meta[STAGE_SLOTS][NT];  // pair index of each staged pair
  uint8_t ent[NT / 64][64 * STAGE_SLOTS];  // per wave: its staged (lane << 2 | slot) entries
  static_assert(STAGE_SLOTS <= 4, "an entry keeps its slot in two bits");
  union {
    struct {
      uint32_t hist[NSUB * 256];  // radix-fallback histograms (NSUB sub-histograms)
      uint32_t suf[256];          // suffix sums of the folded histogram
    } rx;
    uint32_t lb[1024];            // per-wave sorted thread maxima (lower bound)
    struct {
      uint32_t hist[WIDE_BINS];   // bin counts, then bin ends (bin d: key M - d)
      uint32_t fill[WIDE_BINS];   // candidates per bin
    } wb;
  } u;
  int32_t wsum[2][16];         // per-wave partials for block scans (double-buffered)
  int32_t misc[16];
};

enum { M_HB = 0, M_ABOVE, M_LB, M_GT, M_CNT, M_RED };

// ---- block primitives ----------------------------------------------------------------------

// LDS atomics that many lanes aim at one address serialise.  The two most common bins of the
// wave's active lanes (found by the first active lanes) get one atomic each carrying their
// lane counts -- on tie-heavy data that is every lane -- and the lanes left over, whose bins
// are spread, add 1 each to their own bin in parallel.
__device__ __forceinline__ void wave_add(uint32_t* base, uint32_t bin, bool active) {
  uint64_t todo = __ballot(active);
#pragma unroll
  for (int round = 0; round < 2; ++round) {
    if (todo == 0ull) return;
    const int leader = __builtin_ctzll(todo);
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
    const uint64_t same = __ballot(active && bin == b) & todo;
    if (lane_id() == leader) atomicAdd(&base[b], (uint32_t)__popcll(same));
    todo &= ~same;
  }
  if ((todo >> lane_id()) & 1ull) atomicAdd(&base[bin], 1u);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, xor_lane<1>(v));
  v = max(v, xor_lane<2>(v));
  v = max(v, xor_lane<4>(v));
  v = max(v, xor_lane<8>(v));
  v = max(v, xor_lane<16>(v));
  return max(v, xor_lane<32>(v));
}

// inclusive prefix over the 64 lanes (integers: the association does not matter), by the
// DPP row shifts and row broadcasts of wave_incl_scan_u32 (no LDS round trips)
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  return (int)wave_incl_scan_u32((uint32_t)v);
}

// Exclusive prefix of v over the workgroup in thread order; *total gets the sum.
template <int NT>
__device__ __forceinline__ int block_excl_scan(int v, int* total, int32_t* wsum) {
  constexpr int NW = NT / 64;
  const int lane = lane_id(), wid = threadIdx.x >> 6;
  const int incl = wave_incl_scan_i32(v);
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  int pre = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int s = wsum[w];
    pre += (w < wid) ? s : 0;
    tot += s;
  }
  *total = tot;
  return pre + incl - v;
}

// suf[b] = sum of hist[b'] for b' >= b, computed by wave 0; the caller synchronises after.
__device__ __forceinline__ void suffix256(const uint32_t* hist, uint32_t* suf) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    uint32_t h[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h[j] = hist[255 - (4 * l + j)];
      s += h[j];
    }
    const uint32_t incl = (uint32_t)wave_incl_scan_i32((int)s);
    uint32_t run = incl - s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      run += h[j];
      suf[255 - (4 * l + j)] = run;
    }
  }
}

// The bucket b with suf[b] >= want > suf[b+1]; writes it and above_base + suf[b+1].
template <int NT>
__device__ __forceinline__ void find_bucket(const uint32_t* suf, int want, int above_base,
                                            int32_t* out_bucket, int32_t* out_above) {
  for (int b = threadIdx.x; b < 256; b += NT) {
    const uint32_t here = suf[b];
    const uint32_t next = (b == 255) ? 0u : suf[b + 1];
    if (here >= (uint32_t)want && next < (uint32_t)want) {
      *out_bucket = b;
      *out_above = above_base + (int)next;
    }
  }
}

// The first bin b of h[0..NB) at which the running sum h[0] + ... + h[b] reaches `want`, or -1
// when the whole histogram holds fewer (uniform).  NB / NT consecutive bins per thread, one
// block scan; wsum is the scan's per-wave buffer, *out a word of LDS for the answer.
template <int NT, int NB>
__device__ __forceinline__ int block_first_reach(const uint32_t* h, uint32_t want, int32_t* wsum,
                                                 int32_t* out) {
  constexpr int PER = (NB + NT - 1) / NT;
  const int b0 = (int)threadIdx.x * PER;
  uint32_t loc[PER];
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    loc[j] = b0 + j < NB ? h[b0 + j] : 0u;
    s += loc[j];
  }
  int total = 0;
  uint32_t run = (uint32_t)block_excl_scan<NT>((int)s, &total, wsum);
  if ((uint32_t)total < want) return -1;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (run < want && run + loc[j] >= want) *out = b0 + j;
    run += loc[j];
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*out);
}

// h[b] <- exclusive prefix of cnt[0..NB) at b (bin starts); returns the total (uniform) and
// sets *big when a bin holds more than `cap` (uniform after the closing barrier).
template <int NT, int NB>
__device__ __forceinline__ int block_bin_starts(const uint32_t* cnt, uint32_t* h, uint32_t cap,
                                                int32_t* wsum, bool* big) {
  constexpr int PER = (NB + NT - 1) / NT;
  const int b0 = (int)threadIdx.x * PER;
  uint32_t loc[PER];
  uint32_t s = 0;
  bool over = false;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    loc[j] = b0 + j < NB ? cnt[b0 + j] : 0u;
    s += loc[j];
    over |= loc[j] > cap;
  }
  int total = 0;
  uint32_t run = (uint32_t)block_excl_scan<NT>((int)s, &total, wsum);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if (b0 + j < NB) h[b0 + j] = run;
    run += loc[j];
  }
  *big = __syncthreads_or(over ? 1 : 0) != 0;
  return total;
}

// Output r of the descending merge of two descending lists a[0..K), b[0..K) of unique words
// (zero words pad a short list and sort last): i, the number of a-words among the first r
// outputs, is the first index of the diagonal i + j = r - 1 where a[i] > b[r - 1 - i] fails
// (the predicate only turns from true to false along it), and output r is the larger of
// a[i] and b[r - i].
__device__ __forceinline__ uint64_t merge_path_at(const uint64_t* a, const uint64_t* b, int K,
                                                  int r) {
  int lo = r - K > 0 ? r - K : 0;
  int hi = r < K ? r : K;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] > b[r - 1 - mid]) lo = mid + 1;
    else hi = mid;
  }
  const uint64_t x = lo < K ? a[lo] : 0ull;
  const uint64_t y = r - lo < K ? b[r - lo] : 0ull;
  return x > y ? x : y;
}

// Words grouped by bin in a[0..n) (bin d at [end[d] - cnt[d], end[d]), d = M - key): each word's
// rank in descending word order is its bin's start plus the words of its bin above it; the
// ranks below `keep` are written to out[].  Words are unique, so the ranks are a permutation.
template <int NT>
__device__ __forceinline__ void block_rank_bins(const uint64_t* a, int n, uint32_t M,
                                                const uint32_t* end, const uint32_t* cnt,
                                                int keep, uint64_t* out) {
  for (int i = threadIdx.x; i < n; i += NT) {
    const uint64_t w = a[i];
    const uint32_t d = M - (uint32_t)(w >> 32);
    const int e = (int)end[d];
    const int b = e - (int)cnt[d];
    int r = b;
    int j = b;
    for (; j + 4 <= e; j += 4) {  // four independent reads in flight per step
      const uint64_t a0 = a[j], a1 = a[j + 1], a2 = a[j + 2], a3 = a[j + 3];
      r += (a0 > w ? 1 : 0) + (a1 > w ? 1 : 0) + (a2 > w ? 1 : 0) + (a3 > w ? 1 : 0);
    }
    for (; j < e; ++j) r += a[j] > w ? 1 : 0;
    if (r < keep) out[r] = w;
  }
}

// Fold the NSUB sub-histograms into hist[0..255].
template <int NT>
__device__ __forceinline__ void fold_hist(uint32_t* hist) {
  for (int b = threadIdx.x; b < 256; b += NT) {
    uint32_t v = 0;
#pragma unroll
    for (int q = 0; q < NSUB; ++q) v += hist[q * 256 + b];
    hist[b] = v;
  }
}

template <int NT>
__device__ __forceinline__ void zero_hist(uint32_t* hist) {
  for (int i = threadIdx.x; i < NSUB * 256; i += NT) hist[i] = 0u;
}

// One compare-exchange stage (partner distance J) of a bitonic network over a 64-word segment
// held one word per lane: lanes of a descending block (desc) keep the larger word in the
// lower lane.  For block sizes K < 64 the direction comes from the lane index; K == 64 and
// every larger block take the segment's direction, seg_desc.
template <int K, int J>
__device__ __forceinline__ uint64_t seg_step(uint64_t v, bool seg_desc) {
  const int l = lane_id();
  const bool desc = K < 64 ? ((l & K) == 0) : seg_desc;
  const bool keep_hi = ((l & J) == 0) == desc;
  const uint64_t o = xor_lane64<J>(v);
  return ((o > v) == keep_hi) ? o : v;
}

template <int K, int J>
__device__ __forceinline__ uint64_t seg_merge(uint64_t v, bool seg_desc) {
  v = seg_step<K, J>(v, seg_desc);
  if constexpr (J > 1) v = seg_merge<K, J / 2>(v, seg_desc);
  return v;
}

template <int K>
__device__ __forceinline__ uint64_t seg_levels(uint64_t v, bool seg_desc) {
  if constexpr (K > 2) v = seg_levels<K / 2>(v, seg_desc);
  return seg_merge<K, K / 2>(v, seg_desc);
}

// Descending bitonic sort of a[0..P) in LDS by the whole workgroup, P a power of two >= 64
// (element e of a block of size k runs descending when (e & k) == 0).  Levels up to 64 and,
// in every larger level, the stages of partner distance below 64 run in registers on 64-word
// segments (one word per lane, DPP exchanges, no barrier); only the stages of distance >= 64
// go through LDS, one compare-exchange per thread and pair and a barrier each.
template <int NT>
__device__ __forceinline__ void block_bitonic_sort_desc(uint64_t* a, int P) {
  constexpr int W = NT / 64;
  const int l = lane_id(), w = threadIdx.x >> 6;
  const int nseg = P >> 6;
  for (int sg = w; sg < nseg; sg += W) {
    const uint64_t v = a[sg * 64 + l];
    a[sg * 64 + l] = seg_levels<64>(v, (sg & 1) == 0);
  }
  __syncthreads();
  for (int k = 128; k <= P; k <<= 1) {
    for (int j = k >> 1; j >= 64; j >>= 1) {
      for (int i = threadIdx.x; i < (P >> 1); i += NT) {
        const int e = ((i & ~(j - 1)) << 1) | (i & (j - 1));  // lower element of pair i
        const uint64_t x = a[e], y = a[e + j];
        if ((x < y) == ((e & k) == 0)) {
          a[e] = y;
          a[e + j] = x;
        }
      }
      __syncthreads();
    }
    for (int sg = w; sg < nseg; sg += W) {
      const uint64_t v = a[sg * 64 + l];
      a[sg * 64 + l] = seg_merge<64, 32>(v, ((sg * 64) & k) == 0);
    }
    __syncthreads();
  }
}

// The last level of the descending sort: a[0..P) holds a bitonic sequence (P a power of two
// >= 64), sorted descending by the whole workgroup -- half-cleaner stages of distance >= 64
// through LDS, then the distances below 64 in registers per 64-word segment.
template <int NT>
__device__ __forceinline__ void block_bitonic_merge_desc(uint64_t* a, int P) {
  constexpr int W = NT / 64;
  const int l = lane_id(), w = threadIdx.x >> 6;
  for (int j = P >> 1; j >= 64; j >>= 1) {
    for (int i = threadIdx.x; i < (P >> 1); i += NT) {
      const int e = ((i & ~(j - 1)) << 1) | (i & (j - 1));
      const uint64_t x = a[e], y = a[e + j];
      if (x < y) {
        a[e] = y;
        a[e + j] = x;
      }
    }
    __syncthreads();
  }
  for (int sg = w; sg < (P >> 6); sg += W) a[sg * 64 + l] = seg_merge<64, 32>(a[sg * 64 + l], true);
  __syncthreads();
}

// The descending top 64R of a[0..P) into a[0..64R), P a power of two >= 128R, by the whole
// workgroup: every 64R-word segment is sorted in registers by one wave (DPP network, element
// l*R + i in lane l), then pairs of sorted segments are folded by bitonic top-merges
// (elementwise maximum of one list and the other reversed, then half-cleaners) in
// log2(P/64R) rounds, each round's merges running in parallel across the waves with a
// barrier between rounds.  For k <= 64R this is a fraction of the full sort's work.
template <int NT, int R>
__device__ __forceinline__ void block_top_desc(uint64_t* a, int P) {
  constexpr int W = NT / 64;
  constexpr int SEG = 64 * R;
  const int l = lane_id(), w = threadIdx.x >> 6;
  const int nseg = P / SEG;
  for (int sg = w; sg < nseg; sg += W) {
    uint64_t v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = a[sg * SEG + l * R + i];
    wave_sort_desc_n<R>(v);
#pragma unroll
    for (int i = 0; i < R; ++i) a[sg * SEG + l * R + i] = v[i];
  }
  __syncthreads();
  for (int step = 1; step < nseg; step <<= 1) {
    for (int m = w; m < (nseg >> 1) / step; m += W) {
      const int lo = m * 2 * step, hi = lo + step;
      uint64_t v[R], b_rev[R];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        v[i] = a[lo * SEG + l * R + i];
        b_rev[i] = a[hi * SEG + SEG - 1 - (l * R + i)];
      }
      wave_merge_top<R>(v, b_rev);
#pragma unroll
      for (int i = 0; i < R; ++i) a[lo * SEG + l * R + i] = v[i];
    }
    __syncthreads();
  }
}

// ---- wave-0 selection helpers ------------------------------------------------------------------

constexpr int WSORT_MAX = 256;  // candidates wave 0 sorts in registers (4 words per lane)

// Wave 0: sort the n <= 64*R words of src[] (zero-padded) and store the top `keep` of them to
// dst[] in descending order.
template <int R, typename Load>
__device__ __forceinline__ void wave_sort_store(const Load& src, int n, int keep, uint64_t* dst) {
  const int l = lane_id();
  uint64_t v[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int e = l * R + i;
    v[i] = e < n ? src(e) : 0ull;
  }
  wave_sort_desc_n<R>(v);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int e = l * R + i;
    if (e < keep) dst[e] = v[i];
  }
}

template <typename Load>
__device__ __forceinline__ void wave_sort_topk(const Load& src, int n, int keep, uint64_t* dst) {
  if (n <= 64) wave_sort_store<1>(src, n, keep, dst);
  else if (n <= 128) wave_sort_store<2>(src, n, keep, dst);
  else wave_sort_store<4>(src, n, keep, dst);
}

// Wave 0: the k-th largest (1-based) of the n <= 64*R unique words of src[].
template <int R>
__device__ __forceinline__ uint32_t wave_kth_u32(const uint32_t* src, int n, int k) {
  const int l = lane_id();
  if constexpr (R == 1) {
    const uint32_t w = wave_sort_desc<uint32_t>(l < n ? src[l] : 0u);
    return read_lane_u32(w, k - 1);
  }
  uint64_t v[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int e = l * R + i;
    v[i] = e < n ? (uint64_t)src[e] : 0ull;
  }
  wave_sort_desc_n<R>(v);
  const int e = k - 1;
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (l * R + i == e) mine = (uint32_t)v[i];
  return read_lane_u32(mine, e / R);
}

// Wave 0: copy the n words the row's workgroups handed over (agent-scope loads, which read
// past the per-XCD L2) into LDS, eight loads in flight per lane before the first store.
__device__ __forceinline__ void load_lists(const uint64_t* src, int n, uint64_t* dst) {
  const int l = lane_id();
  for (int i0 = 0; i0 < n; i0 += 8 * 64) {
    uint64_t w[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = i0 + q * 64 + l;
      w[q] = i < n ? __hip_atomic_load(&src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = i0 + q * 64 + l;
      if (i < n) dst[i] = w[q];
    }
  }
}

// Wave 0: merge S descending lists of K words (lists[s*K + i] in LDS, padded with zeros to
// 64*R) into the descending top K, left in a[] (element l*R + i in lane l): list 0 is loaded in
// order, every further list reversed across the lanes and folded in with the bitonic top-merge.
template <int R>
__device__ __forceinline__ void wave_merge_lists(const uint64_t* lists, int S, int K,
                                                 uint64_t (&a)[R]);

// The same merge with the result stored to dst[0..K).  Wide lists (R = 8, 16) use this form:
// with the result array owned here the compiler keeps the network within ~100 VGPRs, where
// passing the caller's array in doubles the register footprint.
template <int R>
__device__ __forceinline__ void wave_merge_lists_dst(const uint64_t* lists, int S, int K,
                                                     uint64_t* dst) {
  const int l = lane_id();
  uint64_t a[R], b[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int f = l * R + i;
    a[i] = f < K ? lists[f] : 0ull;
  }
  for (int s = 1; s < S; ++s) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int e = 64 * R - 1 - (l * R + i);
      b[i] = e < K ? lists[s * K + e] : 0ull;
    }
    wave_merge_top<R>(a, b);
  }
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int e = l * R + i;
    if (e < K) dst[e] = a[i];
  }
}

template <int R>
__device__ __forceinline__ void wave_merge_lists(const uint64_t* lists, int S, int K,
                                                 uint64_t (&a)[R]) {
  const int l = lane_id();
  uint64_t b[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int f = l * R + i;
    a[i] = f < K ? lists[f] : 0ull;
  }
  for (int s = 1; s < S; ++s) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int e = 64 * R - 1 - (l * R + i);
      b[i] = e < K ? lists[s * K + e] : 0ull;
    }
    wave_merge_top<R>(a, b);
  }
}

// ---- the fp32 tail (one wave) ----------------------------------------------------------------

// Runs on wave 0 with the row's top K words sorted descending: rank l*R + j, R = ceil(K/64)
// <= RB, is v[j] of lane l (FROM_LDS false) or top[l*R + j] (FROM_LDS true, for wide K where
// the words stay in LDS).  Per-lane sums are serial, lane values are combined by
// wave_incl_scan_f32's fixed association (z = its last lane; the prefix offset of lane l = its
// value at lane l-1).  The CPU oracle evaluates the same operations in the same order.
// A row's sampling controls, read at kernel start so that their latency hides under the loads.
struct RowCtl {
  float u;       // the row's uniform
  int k;         // ranks the row samples from (<= K): a prefix of the top-K selection
  float top_p;   // nucleus threshold
  int keep_all;  // top_p >= 1
  float inv_t;   // 1 / temperature (exactly 1 when the call has none)
};

// Graph-safe draw: once every row has taken its uniform from *offset_ctr, the last one adds 4
// to it for the next call (lane 0 of the row's finishing wave).
__device__ __forceinline__ void advance_offset(const Params& p) {
  if (p.offset_ctr == nullptr || lane_id() != 0) return;
  const unsigned n = __hip_atomic_fetch_add(p.grid_ticket, 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
  if (n == (unsigned)(p.B - 1)) {
    __hip_atomic_store(p.grid_ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(p.offset_ctr, (uint64_t)4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// wpre (FROM_LDS only, or nullptr): the unnormalised weights exp((x_i - m) * inv_t) of every
// rank i < rc.k, already computed by the whole workgroup with the same operations.
template <int RB, bool FROM_LDS>
__device__ __forceinline__ void sample_tail(const Params& p, const uint64_t (&v)[RB],
                                            const uint64_t* top, const RowCtl& rc, int row,
                                            const float* wpre = nullptr) {
  const int K = rc.k;
  const float u = rc.u;
  const int l = lane_id();
  // ranks per lane; a compile-time 1 for RB = 1 (K <= 64), so that the lane of rank r is r
  // itself rather than an integer division on the draw's critical path
  const int R = RB == 1 ? 1 : (K + 63) >> 6;
  const int base = l * R;
  auto word = [&](int j) -> uint64_t {
    if constexpr (FROM_LDS) return top[base + j];
    else return v[j];
  };
  float w[RB], pr[RB], c[RB];
  const float m = FROM_LDS ? key_to_float((uint32_t)(top[0] >> 32), p.is_bf16)
                           : key_to_float(read_lane_u32((uint32_t)(v[0] >> 32), 0), p.is_bf16);
  // ranks past K (or past R per lane) carry w = p = 0: adding +0 to the non-negative sums
  // leaves them bit-identical, so the guards are selects and the tail runs without branches
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    const bool valid = j < R && base + j < K;
    float e;
    if (FROM_LDS && wpre != nullptr) {
      e = wpre[base + j];
    } else {
      const float x = key_to_float((uint32_t)(word(j) >> 32), p.is_bf16);
      e = exp_nonpos((x - m) * rc.inv_t);
    }
    w[j] = valid ? e : 0.0f;
    s = s + w[j];
  }
  const float z = read_lane_f32(wave_incl_scan_f32(s), 63);
  float tsum = 0.0f;
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    pr[j] = w[j] / z;
    tsum = tsum + pr[j];
  }
  float acc = wave_shr1_f32(wave_incl_scan_f32(tsum));
  int my_drop = K;
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    const int idx = base + j;
    const bool valid = j < R && idx < K;
    acc = acc + pr[j];  // + 0 past the valid ranks
    c[j] = valid ? acc : 0.0f;
    const bool drop = valid && idx >= 1 && my_drop == K && !((c[j] - pr[j]) < rc.top_p);
    my_drop = drop ? idx : my_drop;
  }
  // lanes hold consecutive rank ranges, so the lowest lane with a hit has the first hit
  const uint64_t drops = __ballot(my_drop < K);
  const int first_drop = drops ? __builtin_amdgcn_readlane(my_drop, __builtin_ctzll(drops)) : K;
  const int r = (rc.keep_all || first_drop == K) ? K - 1 : first_drop - 1;
  float mine_c = 0.0f;
#pragma unroll
  for (int j = 0; j < RB; ++j)
    if (j == r - base) mine_c = c[j];
  const float zp = read_lane_f32(mine_c, r / R);
  const float target = u * zp;
  int my_pick = K;
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    const int idx = base + j;
    const bool pick = j < R && idx <= r && my_pick == K && c[j] >= target;
    my_pick = pick ? idx : my_pick;
  }
  const uint64_t hits = __ballot(my_pick < K);
  const int pick = hits ? __builtin_amdgcn_readlane(my_pick, __builtin_ctzll(hits)) : r;
  // the picked word: rank pick is v[pick % R] of lane pick / R (both uniform)
  uint32_t lo32;
  if constexpr (FROM_LDS) {
    lo32 = (uint32_t)top[pick];
  } else {
    const int pl = pick / R, pj = pick - pl * R;
    lo32 = 0;
#pragma unroll
    for (int j = 0; j < RB; ++j)
      if (j == pj) lo32 = (uint32_t)v[j];
    lo32 = read_lane_u32(lo32, pl);
  }
  if (l == 0) p.out[row] = (int64_t)(0xFFFFFFFFu - lo32);
  if (p.keep != nullptr) {
    const size_t rowo = (size_t)row * p.K;  // rows of the outputs are the call's K wide
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int idx = base + j;
      if (j < R && idx < K) {
        p.keep[rowo + idx] = (uint8_t)(idx <= r);
        p.renormed[rowo + idx] = idx <= r ? pr[j] / zp : 0.0f;
      }
    }
    for (int idx = K + l; idx < p.K; idx += 64) {  // ranks past the row's own k
      p.keep[rowo + idx] = 0;
      p.renormed[rowo + idx] = 0.0f;
    }
  }
}

// Wave 0, after the slice's (or row's) top K words are in v[] blocked by RB (element l*RB + i
// in lane l, zeros past the end): the candidate ids, or the tail, which needs them blocked by
// R = ceil(K/64); when R < RB they are re-laid out through top[].
template <int RB>
__device__ __forceinline__ void wave_finish(const Params& p, uint64_t (&v)[RB], uint64_t* top, int row,
                            const RowCtl& rc) {
  const int l = lane_id();
  const int K = p.K;
  if (p.ids != nullptr) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int e = l * RB + i;
      if (e < K) p.ids[(size_t)row * K + e] = (int64_t)unpack_id(v[i]);
    }
    return;
  }
  if (p.words != nullptr) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int e = l * RB + i;
      if (e < K) p.words[(size_t)row * K + e] = global_word(v[i], p.id_offset);
    }
    return;
  }
  advance_offset(p);
  const int R = RB == 1 ? 1 : (rc.k + 63) >> 6;  // rc.k <= p.K <= 64 when RB = 1
  if (R != RB) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int e = l * RB + i;
      if (e < K) top[e] = v[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int e = l * R + j;
      v[j] = (j < R && e < rc.k) ? top[e] : 0ull;
    }
  }
  sample_tail<RB, false>(p, v, top, rc, row);
}

// ---- the kernel ----------------------------------------------------------------------------

// Opaque to the optimiser: the keys are "redefined" here, so per-chunk values derived from
// them in an earlier pass (masks) are recomputed instead of being kept live across passes.
template <int CH>
__device__ __forceinline__ void pass_barrier(uint32_t (&kv)[CH][4]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(kv[c][q]));
  }
}

// bit j set when element j (0..7) of the chunk has key >= L (L >= 1): per word, a saturating
// packed subtract of L-1 leaves a nonzero half exactly where key >= L, a packed min with 1
// turns the halves into 0/1, and the low-half bits (2q) and high-half bits (16 + 2q) of the
// four words are folded into bits 2q and 2q+1.
__device__ __forceinline__ uint32_t ge_mask(const uint32_t (&k)[4], uint32_t L) {
  const u16x2 lm1 = (u16x2)((unsigned short)(L - 1u));
  const u16x2 one = (u16x2)((unsigned short)1);
  uint32_t acc = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const u16x2 d = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, k[q]), lm1);
    acc |= __builtin_bit_cast(uint32_t, __builtin_elementwise_min(d, one)) << (2 * q);
  }
  return (acc | (acc >> 15)) & 0xFFu;
}

// bit j set when element j of the chunk has key == T
__device__ __forceinline__ uint32_t eq_mask(const uint32_t (&k)[4], uint32_t T) {
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    m |= (uint32_t)((k[q] & 0xFFFFu) == T) << (2 * q);
    m |= (uint32_t)((k[q] >> 16) == T) << (2 * q + 1);
  }
  return m;
}

// element j (0..7) of a chunk, j runtime: a select chain, never a dynamic register index
__device__ __forceinline__ uint32_t key_at(const uint32_t (&k)[4], int j) {
  const int q = j >> 1;
  const uint32_t w = q == 0 ? k[0] : (q == 1 ? k[1] : (q == 2 ? k[2] : k[3]));
  return (j & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// element j (0..15) of a chunk pair given as its eight words, j runtime: a select tree on the
// bits of j / 2, then the half (values, so the select never becomes an address into kv[])
__device__ __forceinline__ uint32_t key_of16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                             uint32_t w4, uint32_t w5, uint32_t w6, uint32_t w7,
                                             int j) {
  const int q = j >> 1;
  const bool b0 = (q & 1) != 0, b1 = (q & 2) != 0, b2 = (q & 4) != 0;
  const uint32_t x01 = b0 ? w1 : w0, x23 = b0 ? w3 : w2, x45 = b0 ? w5 : w4, x67 = b0 ? w7 : w6;
  const uint32_t y0 = b1 ? x23 : x01, y1 = b1 ? x67 : x45;
  const uint32_t w = b2 ? y1 : y0;
  return (j & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// Phase timestamps for tuning: thread 0 of each workgroup records the shader clock at fixed
// points into trace[workgroup * 16 + i] when the caller passes a trace buffer.
#define FSAMP_TRACE(i)                                                                       \
  do {                                                                                       \
    if (p.trace != nullptr && threadIdx.x == 0)                                              \
      p.trace[(size_t)blockIdx.x * 32 + (i)] = (int64_t)__builtin_amdgcn_s_memtime();        \
  } while (0)
// lane 0 of wave w (w < 14) records the shader clock once `dep` (a value computed from all
// of the wave's loads) exists into slot 18 + w; the empty asm consuming it keeps the clock
// read from being hoisted above that computation
#define FSAMP_WTRACE(dep)                                                                    \
  do {                                                                                       \
    if (p.trace != nullptr && lane_id() == 0 && (threadIdx.x >> 6) < 14) {                   \
      asm volatile("" ::"v"(dep));                                                           \
      p.trace[(size_t)blockIdx.x * 32 + 18 + (threadIdx.x >> 6)] =                           \
          (int64_t)__builtin_amdgcn_s_memtime();                                             \
    }                                                                                        \
  } while (0)
// the constant-rate (100 MHz) clock into slot 16 + i, to convert shader clocks to time
#define FSAMP_RTRACE(i)                                                                      \
  do {                                                                                       \
    if (p.trace != nullptr && threadIdx.x == 0)                                              \
      p.trace[(size_t)blockIdx.x * 32 + 16 + (i)] =                                          \
          (int64_t)__builtin_amdgcn_s_memrealtime();                                         \
  } while (0)

// Wave 0 after the gather.  The slice's top keff words, sorted, go to v[] blocked by RB
// (element l*RB + i in lane l, zeros past keff): candidates in per-wave regions of top[] or
// contiguous in cand[] are sorted in registers; sorted_in_lds means top[] already holds them.
// With S > 1 the list is handed to the row's last workgroup, which merges the S lists; the
// owner of the row's top K finishes (ids or the sampling tail).
template <int RB, int NT>
__device__ __forceinline__ void wave_back_wide(const Params& p, Smem<NT>& sm, int keff, int ncand,
                                               bool sorted_in_lds, bool regions, int row,
                                               int split, const RowCtl& rc, int S,
                                               const float* wpre);

template <int RB, int NT>
__device__ __forceinline__ void wave_tail_regs(const Params& p, Smem<NT>& sm, uint64_t (&v)[RB],
                                               int keff, int row, int split, const RowCtl& rc,
                                               int S);

// 64-bit value of lane `src` (per-lane source), as two 32-bit lane shuffles
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src, 64);
  const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Sorts up to 64 candidate words >= L descending, one per lane.  When every candidate key
// lies in [L, L + 2^14) (L >= 0xC000: the slice's bound sits in the top quarter of the key
// range, as for any row whose top values are positive) and ids fit in 18 bits, each word is
// (key - L) << 18 | (2^18 - 1 - id): the same order in 32 bits, which halves the network's
// work.  Zero words (padding) stay zero and sort last either way.
__device__ __forceinline__ uint64_t wave_sort64_words(uint64_t v, uint32_t L, int V) {
  if (L >= 0xC000u && V < (1 << 18)) {
    uint32_t w = 0u;
    if (v != 0ull) w = (((uint32_t)(v >> 32) - L) << 18) | ((uint32_t)(0x3FFFF - unpack_id(v)));
    w = wave_sort_desc<uint32_t>(w);
    return w != 0u ? pack((w >> 18) + L, 0x3FFFFu - (w & 0x3FFFFu)) : 0ull;
  }
  uint64_t a[1] = {v};
  wave_sort_desc_n<1>(a);
  return a[0];
}

// The descending top 64 of up to 128 candidate words >= L (a: candidate l, b: candidate 64 + l,
// zeros past the end), one per lane.  With every key in [L, L + 2^14) and ids below 2^18 the
// words are compared as 32-bit (key - L) << 18 | (2^18 - 1 - id), as in wave_sort64_words.
__device__ __forceinline__ uint64_t wave_top64_of128(uint64_t a, uint64_t b, uint32_t L, int V) {
  if (L >= 0xC000u && V < (1 << 18)) {
    auto to32 = [&](uint64_t v) -> uint32_t {
      return v != 0ull ? ((((uint32_t)(v >> 32) - L) << 18) | (0x3FFFFu - unpack_id(v))) : 0u;
    };
    const uint32_t w = wave_top64_of_two<uint32_t>(to32(a), to32(b));
    return w != 0u ? pack((w >> 18) + L, 0x3FFFFu - (w & 0x3FFFFu)) : 0ull;
  }
  return wave_top64_of_two<uint64_t>(a, b);
}

template <int RB, int NT>
__device__ __forceinline__ void wave_back(const Params& p, Smem<NT>& sm, int keff, int ncand, bool sorted_in_lds,
                          bool regions, int row, int split, const RowCtl& rc, uint32_t L,
                          uint64_t pre, int S, const float* wpre = nullptr) {
  if constexpr (RB > 4) {
    wave_back_wide<RB, NT>(p, sm, keff, ncand, sorted_in_lds, regions, row, split, rc, S, wpre);
    return;
  }
  const int l = lane_id();
  uint64_t v[RB];
  if (keff > 0 && !sorted_in_lds) {
    // candidates are contiguous: in top[] from the gather, in cand[] from the radix select
    const uint64_t* base = regions ? sm.top : sm.g.cand;
    auto load = [&](int e) -> uint64_t { return base[e]; };
    if (RB == 1 && regions && ncand <= 64) {
      // top[0..64) was read right after the gather barrier
      FSAMP_TRACE(14);
      v[0] = wave_sort64_words(l < ncand ? pre : 0ull, L, p.V);
      if (l >= keff) v[0] = 0ull;
    } else if (ncand <= 64 * RB) {
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int e = l * RB + i;
        v[i] = e < ncand ? load(e) : 0ull;
      }
      FSAMP_TRACE(14);
      wave_sort_desc_n<RB>(v);
#pragma unroll
      for (int i = 0; i < RB; ++i)
        if (l * RB + i >= keff) v[i] = 0ull;
    } else {
      wave_sort_topk(load, ncand, keff, sm.top);
      sorted_in_lds = true;
    }
  }
  if (keff > 0 && sorted_in_lds) {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int e = l * RB + i;
      v[i] = e < keff ? sm.top[e] : 0ull;
    }
  }
  if (keff <= 0) {
#pragma unroll
    for (int i = 0; i < RB; ++i) v[i] = 0ull;
  }
  wave_tail_regs<RB, NT>(p, sm, v, keff, row, split, rc, S);
}

// Wave 0 with the slice's sorted top keff in v[] (blocked by RB, zeros past keff): probe stop,
// split hand-off and row merge when S > 1, then the ids or the sampling tail.
template <int RB, int NT>
__device__ __forceinline__ void wave_tail_regs(const Params& p, Smem<NT>& sm, uint64_t (&v)[RB],
                                               int keff, int row, int split, const RowCtl& rc,
                                               int S) {
  const int l = lane_id();
  FSAMP_TRACE(5);
  if (p.stop == 4) {
    if (l == 0 && split == 0) p.out[row] = keff > 0 ? (int64_t)unpack_id(v[0]) : -1;
    return;
  }

  if (S > 1) {
    // 5. hand the slice's sorted top-K to the row's last workgroup.  The words are written
    //    with agent-scope atomic stores, s_waitcnt(0) holds the wave until every one of them is
    //    acknowledged, and the row's ticket is taken with an acquire-release agent-scope
    //    fetch_add, which orders the stores before the increment and the last arriver's reads
    //    of the other lists (agent-scope atomic loads) after it.  On MI355X the acquire-release
    //    ticket measured the same as a relaxed one here (10.05 against 10.07 us at B=1, six
    //    splits); a full __threadfence costs ~1.5 us more per hand-off.
    uint64_t* dst = p.partials + ((size_t)row * S + split) * p.K;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int e = l * RB + i;
      if (e < p.K) __hip_atomic_store(&dst[e], v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    unsigned prev = 0;
    if (l == 0)
      prev = __hip_atomic_fetch_add(&p.tickets[row * TICKET_STRIDE], 1u, __ATOMIC_ACQ_REL,
                                    __HIP_MEMORY_SCOPE_AGENT);
    prev = read_lane_u32(prev, 0);
    FSAMP_TRACE(6);
    if (prev != (unsigned)(S - 1)) return;
    if (l == 0)
      __hip_atomic_store(&p.tickets[row * TICKET_STRIDE], 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (p.stop == 5) {
      if (l == 0) p.out[row] = (int64_t)unpack_id(v[0]);
      return;
    }
    // 6. merge the S sorted lists of the row: stage them in LDS (every load in flight at
    //    once), then fold them in registers
    const int n = S * p.K;
    const uint64_t* src = p.partials + (size_t)row * S * p.K;
    load_lists(src, n, sm.g.cand);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    FSAMP_TRACE(7);
    wave_merge_lists<RB>(sm.g.cand, S, p.K, v);
    FSAMP_TRACE(8);
  }
  if (p.stop == 5 || p.stop == 6) {
    if (l == 0) p.out[row] = (int64_t)unpack_id(v[0]);
    return;
  }
  // 7. candidate ids, or the sampling tail
  wave_finish<RB>(p, v, sm.top, row, rc);
  FSAMP_TRACE(9);
  FSAMP_RTRACE(1);
}

// Wave 0 for K > 256: the same steps with the sorted words kept in top[] (LDS) between them,
// so that only the merge holds the wide lists in registers.
template <int RB, int NT>
__device__ __forceinline__ void wave_back_wide(const Params& p, Smem<NT>& sm, int keff, int ncand,
                                               bool sorted_in_lds, bool regions, int row,
                                               int split, const RowCtl& rc, int S,
                                               const float* wpre) {
  const int l = lane_id();
  if (keff > 0 && !sorted_in_lds) {
    const uint64_t* base = regions ? sm.top : sm.g.cand;
    auto load = [&](int e) -> uint64_t { return base[e]; };
    wave_sort_topk(load, ncand, keff, sm.top);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  FSAMP_TRACE(5);
  if (p.stop == 4) {
    if (l == 0 && split == 0) p.out[row] = keff > 0 ? (int64_t)unpack_id(sm.top[0]) : -1;
    return;
  }
  if (S > 1) {
    // hand-off and merge as in wave_back, through top[]
    uint64_t* dst = p.partials + ((size_t)row * S + split) * p.K;
    for (int i = l; i < p.K; i += 64)
      __hip_atomic_store(&dst[i], i < keff ? sm.top[i] : 0ull, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    unsigned prev = 0;
    if (l == 0)
      prev = __hip_atomic_fetch_add(&p.tickets[row * TICKET_STRIDE], 1u, __ATOMIC_ACQ_REL,
                                    __HIP_MEMORY_SCOPE_AGENT);
    prev = read_lane_u32(prev, 0);
    FSAMP_TRACE(6);
    if (prev != (unsigned)(S - 1)) return;
    if (l == 0)
      __hip_atomic_store(&p.tickets[row * TICKET_STRIDE], 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (p.stop == 5) {
      if (l == 0) p.out[row] = (int64_t)unpack_id(sm.top[0]);
      return;
    }
    const int n = S * p.K;
    const uint64_t* src = p.partials + (size_t)row * S * p.K;
    load_lists(src, n, sm.g.cand);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    FSAMP_TRACE(7);
    wave_merge_lists_dst<RB>(sm.g.cand, S, p.K, sm.top);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    FSAMP_TRACE(8);
  }
  if (p.stop == 5 || p.stop == 6) {
    if (l == 0) p.out[row] = (int64_t)unpack_id(sm.top[0]);
    return;
  }
  if (p.ids != nullptr) {
    for (int i = l; i < p.K; i += 64) p.ids[(size_t)row * p.K + i] = (int64_t)unpack_id(sm.top[i]);
    return;
  }
  if (p.words != nullptr) {
    for (int i = l; i < p.K; i += 64)
      p.words[(size_t)row * p.K + i] = global_word(sm.top[i], p.id_offset);
    return;
  }
  advance_offset(p);
  const uint64_t none[RB] = {};
  sample_tail<RB, true>(p, none, sm.top, rc, row, wpre);
  FSAMP_TRACE(9);
  FSAMP_RTRACE(1);
}

// lo + t*8 made opaque to the optimiser at each use site: element ids of chunk c are this plus
// the constant c*NT*8, computed where they are needed, so that per-chunk ids are not hoisted
// and kept live (one VGPR per chunk) across the phases that still hold the slice.
__device__ __forceinline__ uint32_t opaque_base(int lo, int t) {
  uint32_t b = (uint32_t)(lo + t * 8);
  asm volatile("" : "+v"(b));
  return b;
}

// Zero words that absent per-row inputs are read from instead (never written).
__device__ uint64_t g_zero_words[2];

// 0 in a VGPR, opaque to the optimiser (a per-lane value as far as it can tell)
__device__ __forceinline__ int opaque_vzero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// compile-time integer for the pair ranges of the gather
template <int N>
struct IC {
  static constexpr int value = N;
};

// f(IC<I>{}) for I = I0 .. I1-1 in order: loop bodies whose register indexes must be
// compile-time constants, however large the unrolled body grows
template <int I0, int I1, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I0 < I1) {
    f(IC<I0>{});
    static_for<I0 + 1, I1>(f);
  }
}

template <int NT, int CH, bool VEC, bool MERGE>
__global__ __launch_bounds__(NT) void fsamp_kernel(Params p) {
  static_assert(NT < 512 || sizeof(Smem<NT>::g) >= 2 * CAND_CAP * sizeof(uint64_t),
                "the wide merge keeps the lists and their binned copy in g");
  static_assert(sizeof(Smem<NT>::u) >= FSAMP_K_MAX * sizeof(float),
                "the wide tail's weights fit in u");
  constexpr int W = NT / 64;                 // waves per workgroup
  constexpr int NP = (CH + 1) / 2;           // chunk pairs
  __shared__ Smem<NT> sm;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wid = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform, known to the compiler
  const int row = blockIdx.x / p.S;
  const int split = blockIdx.x - row * p.S;
  const uint16_t* xr = p.logits + (size_t)row * (size_t)p.ld;
  const int lo = split * p.slice;
  const int hi = min(lo + p.slice, p.V);
  const int count = max(hi - lo, 0);
  const int keff = min(p.K, count);
  FSAMP_TRACE(0);
  FSAMP_RTRACE(0);
  // The row's uniform, offset and controls are fetched early, so that their latency hides
  // under the slice loads, and only read at the tail (row_ctl): a value consumed at once would
  // make the wave wait for its load before issuing the slice loads.  Tilings that load the
  // whole slice at once fetch them at kernel start; the pipelined (streaming) tilings fetch them
  // right after their last slice load is issued, so that the eight VGPRs they occupy are not
  // held while the slice fills the register file, and they land with the slice's last bytes.
  // Every one is loaded unconditionally, an absent one from a zero word, so that no branch
  // joins registers with loads pending on one side (which also makes the wave wait), and the
  // index carries a zero the compiler cannot see through, so that the values stay in VGPRs (a
  // load from a uniform address would be moved to SGPRs right where it is issued, which waits
  // for it).
  const int vz = opaque_vzero();
  const uint64_t* zw = g_zero_words;
  float u_ld, topp_ld, temp_ld;
  int32_t topk_ld;
  uint64_t off_ld, seed_ld;
  auto issue_ctl = [&]() {
    u_ld = (p.u != nullptr ? p.u + row : reinterpret_cast<const float*>(zw))[vz];
    off_ld = __hip_atomic_load((p.offset_src != nullptr ? p.offset_src : zw) + vz,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    seed_ld = (p.seed_src != nullptr ? p.seed_src : zw)[vz];
    topk_ld = (p.topk_row != nullptr ? p.topk_row + row : reinterpret_cast<const int32_t*>(zw))[vz];
    topp_ld = (p.topp_row != nullptr ? p.topp_row + row : reinterpret_cast<const float*>(zw))[vz];
    temp_ld = (p.temp_row != nullptr ? p.temp_row + row : reinterpret_cast<const float*>(zw))[vz];
  };
  constexpr bool CTL_LATE = pipe_depth<NT, CH, VEC>() > 0;
  if constexpr (!CTL_LATE) issue_ctl();
  auto row_ctl = [&]() -> RowCtl {
    // (made opaque here, so that no arithmetic on them is hoisted next to their loads)
    float u_v = u_ld, topp_v = topp_ld, temp_v = temp_ld;
    int32_t topk_v = topk_ld;
    uint64_t off_v = off_ld, seed_v = seed_ld;
    asm volatile("" : "+v"(u_v), "+v"(topp_v), "+v"(temp_v), "+v"(topk_v), "+v"(off_v),
                 "+v"(seed_v));
    RowCtl rc;
    if (p.u != nullptr) {
      rc.u = u_v;
    } else {
      // the (seed, offset) pair as at::cuda::philox::unpack gives it: device values when the
      // sources are set (a captured graph's seed and base offset), plus the call's offset
      const uint64_t seed = p.seed_src != nullptr ? seed_v : p.seed;
      const uint64_t off = (p.offset_src != nullptr ? off_v : 0ull) + p.offset;
      rc.u = rng_uniform(seed, off, (uint32_t)row);
    }
    rc.k = p.K;
    rc.top_p = p.top_p_f;
    rc.keep_all = p.keep_all;
    rc.inv_t = 1.0f;
    if (p.topk_row != nullptr) rc.k = min(max(topk_v, 1), p.K);
    if (p.topp_row != nullptr) {
      rc.top_p = topp_v;
      rc.keep_all = rc.top_p >= 1.0f ? 1 : 0;
    }
    if (p.temp_row != nullptr) {
      if (temp_v > 0.0f) rc.inv_t = 1.0f / temp_v;
      else rc.k = 1;  // temperature <= 0 (or NaN): greedy
    }
    return rc;
  };
  if (t == 0) sm.misc[M_CNT] = 0;
  if (t < 64) sm.top[t] = 0ull;  // the first 64 candidate slots, read whole after the gather

  // 1. load the slice into registers as packed keys (padding = key 0).  With VEC, V and the
  //    split bounds are multiples of 8, so a chunk is all in or all out; chunks past the slice
  //    load its last vector (a valid address) and are masked, so every load is unconditional
  //    and the key work on chunk c waits only for chunk c's load.
  uint32_t kv[CH][4];
  auto load_slice = [&]() {
    if (count > 0) {
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int e0 = lo + (c * NT + t) * 8;
        if constexpr (VEC) {
          const uint4 v = load_stream16(xr + min(e0, hi - 8));
          kv[c][0] = v.x;
          kv[c][1] = v.y;
          kv[c][2] = v.z;
          kv[c][3] = v.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int e = e0 + 2 * q;
            const uint32_t a = (e < hi) ? (uint32_t)xr[e] : 0u;
            const uint32_t b = (e + 1 < hi) ? (uint32_t)xr[e + 1] : 0u;
            kv[c][q] = a | (b << 16);
          }
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < CH; ++c) kv[c][0] = kv[c][1] = kv[c][2] = kv[c][3] = 0u;
    }
  };
  // one vector chunk (VEC only), c a compile-time index after unrolling
  auto load_chunk = [&](int c) {
    const int e0 = lo + (c * NT + t) * 8;
    const uint4 v = load_stream16(xr + min(e0, hi - 8));
    kv[c][0] = v.x;
    kv[c][1] = v.y;
    kv[c][2] = v.z;
    kv[c][3] = v.w;
  };
  // Streaming selection of the large tilings (SP): loads kept PD deep, the lower bound taken
  // from the first PB chunks, then PX more loads issued at once to cover the bound, and every
  // later chunk's candidates gathered as it lands (see the streaming block below).
  constexpr int PD = pipe_depth<NT, CH, VEC>();  // loads in flight (0: every load issued at once)
  constexpr bool SP = PD > 0;
  constexpr int PX = SP ? stream_extra_loads<CH>() : 0;
  constexpr int PB = SP ? (stream_bound_chunks<CH>() < ((CH - PD - PX) & ~1)
                               ? stream_bound_chunks<CH>()
                               : ((CH - PD - PX) & ~1))
                        : CH;
  static_assert(!SP || (PB >= 2 && PB % 2 == 0 && PB + PD + PX <= CH), "streaming plan");
  if constexpr (!SP) load_slice();
  // pm[i]: packed 16-bit maxima over the two chunks of pair i (even halves, odd halves); a
  // pair holds an element >= X iff pkmax(pm[i], (X-1) in both halves) differs from the latter
  uint32_t pm[NP];
  // vector chunks of this thread inside the slice are those with c*NT < nv_left (one register
  // and a compare with a constant per chunk, instead of a per-chunk address kept live)
  const int nv_left = (count >> 3) - t;
  auto convert = [&](int c) {
    const int e0 = lo + (c * NT + t) * 8;
    const bool in_slice = c * NT < nv_left;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t k = keys2(kv[c][q]);
      if constexpr (VEC) {
        if (!in_slice) k = 0u;
      } else {
        const int e = e0 + 2 * q;
        if (e >= hi) k &= 0xFFFF0000u;
        if (e + 1 >= hi) k &= 0x0000FFFFu;
      }
      kv[c][q] = k;
    }
    const uint32_t m2 = pkmax(pkmax(kv[c][0], kv[c][1]), pkmax(kv[c][2], kv[c][3]));
    pm[c >> 1] = (c & 1) ? pkmax(pm[c >> 1], m2) : m2;
  };
  auto tmax_of = [&](auto i0c, auto i1c) -> uint32_t {
    constexpr int I0 = decltype(i0c)::value, I1 = decltype(i1c)::value;
    uint32_t m = 0;
#pragma unroll
    for (int i = I0; i < I1; ++i) m = pkmax(m, pm[i]);
    return max(m & 0xFFFFu, m >> 16);
  };
  // pair of chunk c holds an element >= X (X >= 1)
  auto pair_ge = [&](int c, uint32_t X) -> bool {
    const uint32_t xm1 = (X - 1u) * 0x10001u;
    return pkmax(pm[c >> 1], xm1) != xm1;
  };

  // Lower bound for keff > 256 (wide k): the keff-th largest of the 8-element group maxima --
  // the two 16-bit halves of every pair maximum pm[i] (even and odd positions of the pair's two
  // chunks), 2 * NP per thread -- found exactly by a two-round radix select over LDS histograms
  // of those maxima only.  The groups are disjoint, so at least keff distinct elements are >= it.
  // On the C4 k=1024 rows this admits ~1.1k candidates per split, where the minimum of the
  // thread maxima admits ~7k.  With fewer than keff non-empty groups every element qualifies.
  auto group_bound = [&]() -> uint32_t {
    const int sub = wid & (NSUB - 1);
    zero_hist<NT>(sm.u.rx.hist);
    __syncthreads();
    FSAMP_TRACE(2);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const uint32_t g0 = pm[i] & 0xFFFFu, g1 = pm[i] >> 16;
      wave_add(sm.u.rx.hist + sub * 256, g0 >> 8, g0 != 0u);
      wave_add(sm.u.rx.hist + sub * 256, g1 >> 8, g1 != 0u);
    }
    __syncthreads();
    fold_hist<NT>(sm.u.rx.hist);
    __syncthreads();
    suffix256(sm.u.rx.hist, sm.u.rx.suf);
    __syncthreads();
    const int groups = __builtin_amdgcn_readfirstlane((int)sm.u.rx.suf[0]);
    if (groups < keff) return 1u;  // uniform: every thread read the same total
    find_bucket<NT>(sm.u.rx.suf, keff, 0, &sm.misc[M_HB], &sm.misc[M_ABOVE]);
    __syncthreads();
    const uint32_t hb = (uint32_t)__builtin_amdgcn_readfirstlane(sm.misc[M_HB]);
    const int above = __builtin_amdgcn_readfirstlane(sm.misc[M_ABOVE]);
    zero_hist<NT>(sm.u.rx.hist);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const uint32_t g0 = pm[i] & 0xFFFFu, g1 = pm[i] >> 16;
      wave_add(sm.u.rx.hist + sub * 256, g0 & 255u, g0 != 0u && (g0 >> 8) == hb);
      wave_add(sm.u.rx.hist + sub * 256, g1 & 255u, g1 != 0u && (g1 >> 8) == hb);
    }
    __syncthreads();
    fold_hist<NT>(sm.u.rx.hist);
    __syncthreads();
    suffix256(sm.u.rx.hist, sm.u.rx.suf);
    __syncthreads();
    find_bucket<NT>(sm.u.rx.suf, keff - above, above, &sm.misc[M_LB], &sm.misc[M_GT]);
    __syncthreads();
    FSAMP_TRACE(3);
    const uint32_t lb = (uint32_t)__builtin_amdgcn_readfirstlane(sm.misc[M_LB]);
    return max((hb << 8) | lb, 1u);
  };

  // 2. lower bound L of the keff-th largest key among the given thread maxima (keff <= NT by
  //    plan): the keff-th largest of the union of every wave's top-m thread maxima,
  //    m = max(ceil(keff/W), 64/W), doubled for keff <= 64 when that leaves fewer than 8
  //    published words beyond the keff-th: with no slack the bound is the smallest published
  //    maximum, which one wave holding fewer than its share of the top maxima pulls far down,
  //    and the streaming selection's rows then pass its 256-candidate sort (k=64 at B=256: 32.5
  //    against 19.9 us; for k > 64 the larger kth sort costs more than the tighter bound saves,
  //    k=65 at B=256: 21.5 against 20.2 us).  Maxima are made unique by the thread index in the
  //    low bits.  Each wave sorts its 64 maxima with the DPP network and publishes the top m;
  //    after one barrier every wave sorts the W*m published words itself (no second barrier).
  //    Past 256 published words (keff > 256) the group bound above is used instead, which
  //    keeps the register sort of more than 256 words out of the phase that holds the slice.
  auto lower_bound = [&](uint32_t tm) -> uint32_t {
    int m = min(64, max((keff + W - 1) / W, 64 / W));
    if (keff <= 64 && W * m - keff < 8 && 2 * W * m <= WSORT_MAX) m *= 2;
    const int n = W * m;
    if (n > WSORT_MAX) return group_bound();
    const uint32_t srt = wave_sort_desc<uint32_t>((tm << 10) | (uint32_t)t);
    if (lane < m) sm.u.lb[wid * m + lane] = srt;
    __syncthreads();
    FSAMP_TRACE(2);
    uint32_t kth;
    if (n <= 64) {
      kth = wave_kth_u32<1>(sm.u.lb, n, keff);
    } else if (n <= 128) {
      kth = wave_kth_u32<2>(sm.u.lb, n, keff);
    } else {
      kth = wave_kth_u32<4>(sm.u.lb, n, keff);
    }
    FSAMP_TRACE(3);
    return max(kth >> 10, 1u);
  };

  // 3. gather the elements >= L of pairs [I0, I1) into region_base[0, rw): each wave takes
  //    its slots with one LDS atomic on the counter *wc (slots past rw are counted, not
  //    written; more than WSORT_MAX sends the slice to the radix path).  Only threads with a
  //    pair >= L hold any, typically one pair each, so one pass over the pair maxima stages up
  //    to STAGE_SLOTS qualifying pairs per thread in LDS (two compares per pair, the pair
  //    stored under an exec mask), and the candidates are then extracted from the staged
  //    copies, where a runtime element index is an address instead of a select chain over the
  //    register array.  A thread with more qualifying pairs than slots gathers from its
  //    registers instead (per-chunk branches).
  auto stage = [&](auto i0c, auto i1c, uint32_t L, int& nst) {
    constexpr int I0 = decltype(i0c)::value, I1 = decltype(i1c)::value;
    const uint32_t lm1 = (L - 1u) * 0x10001u;
#pragma unroll
    for (int i = I0; i < I1; ++i) {
      const bool hit = pkmax(pm[i], lm1) != lm1;
      // most pairs hold no qualifying lane in the whole wave: one scalar branch skips them
      if (__ballot(hit) != 0ull) {
        if (hit && nst < STAGE_SLOTS) {
          sm.g.st.a[nst][t] = make_uint4(kv[2 * i][0], kv[2 * i][1], kv[2 * i][2], kv[2 * i][3]);
          if (2 * i + 1 < CH)
            sm.g.st.b[nst][t] = make_uint4(kv[2 * i + 1][0], kv[2 * i + 1][1], kv[2 * i + 1][2],
                                           kv[2 * i + 1][3]);
          else
            sm.g.st.b[nst][t] = make_uint4(0u, 0u, 0u, 0u);
          sm.meta[nst][t] = (uint8_t)i;
        }
        nst += hit ? 1 : 0;
      }
    }
  };
  // wc != nullptr: each wave takes its slots of region_base with one LDS atomic on *wc;
  // wc == nullptr: region_base is the wave's own region and wcnt its wave-uniform count
  auto extract = [&](auto c0c, auto c1c, uint32_t L, int nst, uint64_t* region_base, int rw,
                     int32_t* wc, int& wcnt) {
    constexpr int C0 = decltype(c0c)::value, C1 = decltype(c1c)::value;
    FSAMP_TRACE(13);
    const bool from_regs = nst > STAGE_SLOTS;
    auto staged_mask = [&](int s) -> uint32_t {
      const uint4 a = sm.g.st.a[s][t], b = sm.g.st.b[s][t];
      const uint32_t ka[4] = {a.x, a.y, a.z, a.w}, kb[4] = {b.x, b.y, b.z, b.w};
      return ge_mask(ka, L) | (ge_mask(kb, L) << 8);
    };
    int mine = 0;
    // the staged slots' masks, kept for the write pass: the LDS atomic between the two passes
    // would otherwise make the compiler read the staged copies again
    uint32_t smask[STAGE_SLOTS];
    if (from_regs) {
#pragma unroll
      for (int c = C0; c < C1; ++c)
        if (pair_ge(c, L)) mine += __popc(ge_mask(kv[c], L));
    } else {
#pragma unroll
      for (int s = 0; s < STAGE_SLOTS; ++s) {
        smask[s] = s < nst ? staged_mask(s) : 0u;
        mine += __popc(smask[s]);
      }
    }
    FSAMP_TRACE(10);
    if (__ballot(mine > 0) != 0ull) {
      const uint32_t incl = wave_incl_scan_u32((uint32_t)mine);
      int slot;
      if (wc != nullptr) {
        int base = 0;
        if (lane == 63) base = atomicAdd(wc, (int)incl);
        slot = __builtin_amdgcn_readlane(base, 63) + (int)incl - mine;
      } else {
        slot = wcnt + (int)incl - mine;
        wcnt += __builtin_amdgcn_readlane((int)incl, 63);
      }
      uint64_t* region = region_base;
      FSAMP_TRACE(11);
      if (from_regs) {
        const uint32_t idb = opaque_base(lo, t);
#pragma unroll
        for (int c = C0; c < C1; ++c) {
          if (pair_ge(c, L)) {
            uint32_t m = ge_mask(kv[c], L);
            const uint32_t id0 = idb + (uint32_t)(c * NT * 8);
            while (m != 0u) {
              const int j = __ffs(m) - 1;
              m &= m - 1u;
              if (slot < rw) region[slot] = pack(key_at(kv[c], j), id0 + (uint32_t)j);
              ++slot;
            }
          }
        }
      } else {
        const uint32_t idb = opaque_base(lo, t);
#pragma unroll
        for (int s = 0; s < STAGE_SLOTS; ++s) {
          uint32_t m = smask[s];
          if (m == 0u) continue;
          const int c0 = 2 * (int)sm.meta[s][t];
          const uint16_t* ka = reinterpret_cast<const uint16_t*>(&sm.g.st.a[s][t]);
          const uint16_t* kb = reinterpret_cast<const uint16_t*>(&sm.g.st.b[s][t]);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            const uint32_t key = j < 8 ? ka[j] : kb[j - 8];
            const uint32_t id = idb + (uint32_t)(((c0 + (j >> 3)) * NT) * 8 + (j & 7));
            if (slot < rw) region[slot] = pack(key, id);
            ++slot;
          }
        }
      }
    }
    FSAMP_TRACE(12);
  };

  // The streaming path's extraction of the staged pairs, transposed: the wave lists its staged
  // (lane, slot) entries in LDS, then takes them four at a time, sixteen lanes per entry and one
  // of the pair's sixteen elements per lane, so that a pass costs the same few instructions
  // whatever the lanes hold (a lane-per-pair extraction runs its per-element loop for the lane
  // with the most).  Elements >= L are appended to top[] at slots from one LDS atomic per group
  // on *cnt.  A lane that staged more pairs than slots sends the wave to extract().
  auto extract_t = [&](auto c0c, auto c1c, uint32_t L, int nst, int32_t* cnt) {
    if (__ballot(nst > STAGE_SLOTS) != 0ull) {
      int unused = 0;
      extract(c0c, c1c, L, nst, sm.top, FSAMP_K_MAX, cnt, unused);
      return;
    }
    uint8_t* ent = sm.ent[wid];
    int E = 0;  // wave-uniform
#pragma unroll
    for (int s = 0; s < STAGE_SLOTS; ++s) {
      const uint64_t bs = __ballot(s < nst);
      if (bs == 0ull) break;
      if (s < nst) {
        const int pos = E + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bs >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)bs, 0u));
        ent[pos] = (uint8_t)((lane << 2) | s);
      }
      E += (int)__popcll(bs);
    }
    if (E == 0) return;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const int j = lane & 15;   // element of the pair: chunk j >> 3, position j & 7
    const int eo = lane >> 4;  // entry within a group of four
    for (int e0 = 0; e0 < E; e0 += 4) {
      const int e = e0 + eo;
      bool ok = false;
      uint64_t word = 0ull;
      if (e < E) {
        const uint32_t en = ent[e];
        const int ts = wid * 64 + (int)(en >> 2);  // the thread that staged the pair
        const int sl = (int)(en & 3u);
        const uint16_t* src = j < 8 ? reinterpret_cast<const uint16_t*>(&sm.g.st.a[sl][ts])
                                    : reinterpret_cast<const uint16_t*>(&sm.g.st.b[sl][ts]);
        const uint32_t key = src[j & 7];
        const int c = 2 * (int)sm.meta[sl][ts] + (j >> 3);
        ok = key >= L;
        word = pack(key, (uint32_t)(lo + (c * NT + ts) * 8 + (j & 7)));
      }
      const uint64_t b = __ballot(ok);
      if (b == 0ull) continue;
      int base = 0;
      if (lane == 0) base = atomicAdd(cnt, (int)__popcll(b));
      base = __builtin_amdgcn_readlane(base, 0);
      if (ok) {
        const int slot = base + (int)__builtin_amdgcn_mbcnt_hi(
                                    (uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        if (slot < FSAMP_K_MAX) sm.top[slot] = word;
      }
    }
  };

  // candidates >= L of chunk pair i appended to top[] (capacity FSAMP_K_MAX; more are counted,
  // not written) at slots from one LDS atomic per wave on *cnt; used for the last pair of the
  // streaming path, whose data lands last (one compare and one scalar branch when the wave has
  // no candidate)
  auto gather_pair = [&](auto ic, uint32_t L, int32_t* cnt) {
    constexpr int i = decltype(ic)::value;
    constexpr int c0 = 2 * i, c1 = 2 * i + 1;
    const uint32_t lm1 = (L - 1u) * 0x10001u;
    const bool hit = pkmax(pm[i], lm1) != lm1;
    if (__ballot(hit) == 0ull) return;
    uint32_t m = 0u;
    if (hit) {
      m = ge_mask(kv[c0], L);
      if constexpr (c1 < CH) m |= ge_mask(kv[c1], L) << 8;
    }
    const uint32_t mine = (uint32_t)__popc(m);
    const uint32_t incl = wave_incl_scan_u32(mine);
    int base = 0;
    if (lane == 63) base = atomicAdd(cnt, (int)incl);
    int slot = __builtin_amdgcn_readlane(base, 63) + (int)(incl - mine);
    const uint32_t idb = opaque_base(lo, t);
    // (a wave-uniform loop around a guarded body: with a per-lane loop the select tree below
    // is folded into an address into the chunk pair, which moves the pair to scratch memory
    // for the whole kernel -- as key_at's chain does)
    for (;;) {
      if (__ballot(m != 0u) == 0ull) break;
      if (m != 0u) {
        const int j = __ffs(m) - 1;
        m &= m - 1u;
        uint32_t key;
        if constexpr (c1 < CH)
          key = key_of16(kv[c0][0], kv[c0][1], kv[c0][2], kv[c0][3], kv[c1][0], kv[c1][1],
                         kv[c1][2], kv[c1][3], j);
        else
          key = key_of16(kv[c0][0], kv[c0][1], kv[c0][2], kv[c0][3], 0u, 0u, 0u, 0u, j);
        const uint32_t id = idb + (uint32_t)((c0 + (j >> 3)) * NT * 8 + (j & 7));
        if (slot < FSAMP_K_MAX) sm.top[slot] = pack(key, id);
        ++slot;
      }
    }
  };

  // Load order of the streaming tilings: PD loads, then one more after each conversion up to
  // chunk PB-1; PX more at once before the bound; then load c + PD + PX after converting c.
  auto stream_loads_head = [&]() {
    static_for<0, PD>([&](auto cc) { load_chunk(decltype(cc)::value); });
    static_for<0, PB>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      __builtin_amdgcn_sched_barrier(0);
      convert(c);
      __builtin_amdgcn_sched_barrier(0);
      load_chunk(c + PD);
    });
    static_for<PB + PD, PB + PD + PX>([&](auto cc) { load_chunk(decltype(cc)::value); });
    if constexpr (PB + PD + PX >= CH) issue_ctl();  // the slice's last load is issued
    __builtin_amdgcn_sched_barrier(0);
  };
  // load c + PD + PX after chunk c is converted; the row controls after the slice's last load
  auto stream_next_load = [&](auto cc) {
    constexpr int c = decltype(cc)::value;
    if constexpr (c + PD + PX < CH) load_chunk(c + PD + PX);
    if constexpr (c + PD + PX == CH - 1) issue_ctl();
  };
  // the rest of the slice without a gather (ablation stops, wide k, fallback)
  auto stream_loads_tail = [&]() {
    static_for<PB, CH>([&](auto cc) {
      constexpr int c = decltype(cc)::value;
      __builtin_amdgcn_sched_barrier(0);
      convert(c);
      __builtin_amdgcn_sched_barrier(0);
      stream_next_load(cc);
    });
    FSAMP_WTRACE(pm[NP - 1]);
  };

  if constexpr (SP) {
    if (count > 0) {
      stream_loads_head();
    } else {
      issue_ctl();
#pragma unroll
      for (int c = 0; c < CH; ++c) kv[c][0] = kv[c][1] = kv[c][2] = kv[c][3] = 0u;
#pragma unroll
      for (int c = 0; c < PB; ++c) convert(c);
    }
    // Streaming selection for k <= 64 (every condition is uniform over the workgroup):
    //   L = the lower bound from the maxima of chunks 0..PB-1 (valid for the whole slice: the
    //   prefix alone holds keff distinct elements >= L); the prefix's candidates are staged and
    //   gathered while the last loads are in flight, the rest once it has landed; wave 0 then
    //   takes the top 64 of the (on C5, 70 to 124) candidates in registers.  More than 256
    //   falls back to the general selection below with the bound of the whole slice.
    if (count > 0 && keff <= 64 && p.stop >= 2) {
      const uint32_t L = lower_bound(tmax_of(IC<0>{}, IC<PB / 2>{}));
      if (p.stop == 2) {
        stream_loads_tail();
        if (t == 0 && split == 0) p.out[row] = (int64_t)L;
        return;
      }
      // Candidates are appended to top[] at slots from an LDS atomic on the candidate counter
      // (zeroed at kernel start), one per wave and gather: the prefix's, staged through LDS
      // while the last loads are in flight; the middle pairs' (staged one by one as each
      // lands, gathered while the last pair is still in flight); then the last pair's straight
      // from registers, the only gather after the last byte.  After the barrier the candidates
      // are top[0, total): wave 0 reads them without compacting per-wave lists.
      int32_t* cnt = &sm.misc[M_CNT];
      int nst = 0;
      stage(IC<0>{}, IC<PB / 2>{}, L, nst);
      extract_t(IC<0>{}, IC<PB>{}, L, nst, cnt);
      constexpr int LASTP = NP - 1;  // the last pair (chunk 2*LASTP, and 2*LASTP + 1 if < CH)
      int nst2 = 0;
      static_for<PB, CH>([&](auto cc) {
        constexpr int c = decltype(cc)::value;
        __builtin_amdgcn_sched_barrier(0);
        convert(c);
        __builtin_amdgcn_sched_barrier(0);
        stream_next_load(cc);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (((c & 1) == 1 || c == CH - 1) && c / 2 < LASTP)
          stage(IC<c / 2>{}, IC<c / 2 + 1>{}, L, nst2);
        if constexpr (c == 2 * LASTP - 1)  // every middle pair staged: gather them
          extract_t(IC<PB>{}, IC<2 * LASTP>{}, L, nst2, cnt);
      });
      FSAMP_WTRACE(pm[NP - 1]);
      gather_pair(IC<LASTP>{}, L, cnt);
      __syncthreads();
      FSAMP_TRACE(4);
      const int total = __builtin_amdgcn_readfirstlane(sm.misc[M_CNT]);
      if (p.stop == 3) {
        if (t == 0 && split == 0) p.out[row] = total;
        return;
      }
      if (total <= 256) {
        if (wid != 0) return;
        FSAMP_TRACE(14);
        auto cand = [&](int e) -> uint64_t { return e < total ? sm.top[e] : 0ull; };
        uint64_t v[1];
        if (total <= 64) {
          v[0] = wave_sort64_words(cand(lane), L, p.V);
        } else if (total <= 128) {
          v[0] = wave_top64_of128(cand(lane), cand(64 + lane), L, p.V);
        } else {
          // 129 to 256 (a tail of noisy rows, or ties at the bound): the top 64 of each half,
          // then of the two
          const uint64_t lo = wave_top64_of128(cand(lane), cand(64 + lane), L, p.V);
          const uint64_t hi = wave_top64_of128(cand(128 + lane), cand(192 + lane), L, p.V);
          v[0] = wave_top64_of128(lo, hi, L, p.V);
        }
        if (lane >= keff) v[0] = 0ull;
        const RowCtl rc = row_ctl();
        wave_tail_regs<1, NT>(p, sm, v, keff, row, split, rc, p.S);
        return;
      }
      // Too many candidates for the register sorts (heavy ties near the bound): the general
      // selection with the bound of the whole slice, on the slice read again from memory.  The
      // reload keeps the streamed chunks dead once gathered, so the registers they held are
      // free for the sort and the tail of the common case.  Every wave has read the total
      // before the counter is cleared for the general gather.
      __syncthreads();
      if (t == 0) sm.misc[M_CNT] = 0;
      load_slice();
#pragma unroll
      for (int c = 0; c < CH; ++c) convert(c);
    } else {
      if (count > 0) stream_loads_tail();
      else
        static_for<PB, CH>([&](auto cc) { convert(decltype(cc)::value); });
    }
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c) convert(c);
  }
  const uint32_t tmax = tmax_of(IC<0>{}, IC<NP>{});
  if constexpr (!SP) FSAMP_WTRACE(tmax);

  if (p.stop == 1) {
    const uint32_t wmax = wave_max_u32(tmax);
    if (t == 0) sm.misc[M_RED] = 0;
    __syncthreads();
    if (lane == 0) atomicMax(&sm.misc[M_RED], (int)wmax);
    __syncthreads();
    if (t == 0 && split == 0) p.out[row] = sm.misc[M_RED];
    return;
  }

  // Wide selection (k > WIDE_MIN, split rows, the MERGE instantiations of 512 threads and up):
  // the slice's top keff sorted into top[] by counting instead of comparison networks.
  //   a. M = the slice maximum; histogram of the 8-element group maxima (the halves of the
  //      pair maxima pm[]) over bins d = M - g < WIDE_BINS;
  //   b. L = M - d*, d* the first bin where the running count reaches keff: at least keff
  //      groups, so at least keff elements, are >= L (a valid lower bound, ~1.1k candidates
  //      at k = 1024 on the C4 rows);
  //   c. gather the elements >= L as (key, ~id) words (one register pass, wave slots from one
  //      LDS atomic), counting them per bin; bin starts by one block scan;
  //   d. scatter the words into their bins (an LDS atomic per word);
  //   e. rank each word inside its bin (the bin's other words above it) -- its rank in the
  //      slice -- and write ranks < keff to top[].
  // Nine barriers, one register pass after the bound and O(1) LDS work per candidate, where
  // the general path runs radix passes over the registers and a bitonic sort.  Returns false
  // (uniform) when the bound is farther than WIDE_BINS keys below M, the candidates overflow
  // CAND_CAP, or a bin exceeds WIDE_BIN_MAX: the general path then runs from the start (the
  // candidate counter is cleared again; nothing else it reads has been changed).
  auto wide_select = [&](uint32_t tm) -> bool {
    uint32_t* hist = sm.u.wb.hist;
    uint32_t* fill = sm.u.wb.fill;
    uint64_t* cbuf = sm.g.cand;
    for (int i = t; i < WIDE_BINS; i += NT) {
      hist[i] = 0u;
      fill[i] = 0u;
    }
    const uint32_t wm = wave_max_u32(tm);
    if (lane == 0) sm.wsum[0][wid] = (int)wm;
    __syncthreads();
    uint32_t M = 0;
#pragma unroll
    for (int w = 0; w < W; ++w) M = max(M, (uint32_t)sm.wsum[0][w]);
    M = __builtin_amdgcn_readfirstlane(M);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const uint32_t g0 = pm[i] & 0xFFFFu, g1 = pm[i] >> 16;
      if (g0 != 0u && M - g0 < (uint32_t)WIDE_BINS) atomicAdd(&hist[M - g0], 1u);
      if (g1 != 0u && M - g1 < (uint32_t)WIDE_BINS) atomicAdd(&hist[M - g1], 1u);
    }
    __syncthreads();
    FSAMP_TRACE(2);
    const int dstar = block_first_reach<NT, WIDE_BINS>(hist, (uint32_t)keff, sm.wsum[1],
                                                       &sm.misc[M_LB]);
    if (dstar < 0) return false;
    const uint32_t L = M - (uint32_t)dstar;
    // one pass over the registers: the words >= L into comp[] (slots per wave from one LDS
    // atomic, the lanes' offsets from a DPP scan of their counts), counted per bin
    uint64_t* comp = reinterpret_cast<uint64_t*>(&sm.g) + CAND_CAP;
    uint32_t mine = 0;
#pragma unroll
    for (int c = 0; c < CH; ++c)
      if (pair_ge(c, L)) mine += (uint32_t)__popc(ge_mask(kv[c], L));
    const uint32_t incl = wave_incl_scan_u32(mine);
    int wbase = 0;
    if (lane == 63) wbase = atomicAdd(&sm.misc[M_CNT], (int)incl);
    int slot = __builtin_amdgcn_readlane(wbase, 63) + (int)(incl - mine);
    const uint32_t idb = opaque_base(lo, t);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (pair_ge(c, L)) {
        uint32_t m = ge_mask(kv[c], L);
        const uint32_t id0 = idb + (uint32_t)(c * NT * 8);
        while (m != 0u) {
          const int j = __ffs(m) - 1;
          m &= m - 1u;
          const uint32_t key = key_at(kv[c], j);
          atomicAdd(&fill[M - key], 1u);
          if (slot < CAND_CAP) comp[slot] = pack(key, id0 + (uint32_t)j);
          ++slot;
        }
      }
    }
    __syncthreads();
    FSAMP_TRACE(3);
    const int n = __builtin_amdgcn_readfirstlane(sm.misc[M_CNT]);
    bool big = false;
    block_bin_starts<NT, WIDE_BINS>(fill, hist, (uint32_t)WIDE_BIN_MAX, sm.wsum[0], &big);
    if (big || n > CAND_CAP) {
      // every thread read the count before the bin scan's barriers: clear it for the general
      // selection's gather
      if (t == 0) sm.misc[M_CNT] = 0;
      return false;
    }
    // the words into their bins
    for (int i = t; i < n; i += NT) {
      const uint64_t w = comp[i];
      cbuf[atomicAdd(&hist[M - (uint32_t)(w >> 32)], 1u)] = w;
    }
    __syncthreads();
    FSAMP_TRACE(4);
    block_rank_bins<NT>(cbuf, n, M, hist, fill, keff, sm.top);
    __syncthreads();
    return true;
  };

  // Single-phase selection: L from every thread maximum, one gather, and the exact radix
  // select when the candidates overflow.
  int ncand = 0;
  uint64_t pre = 0ull;
  uint32_t L_sel = 1u;
  bool sorted_in_lds = false;
  bool regions = true;  // candidates in per-wave regions of top[] (else contiguous in cand[])
  bool wide_done = false;
  if constexpr (MERGE && NT >= 512) {
    if (keff > WIDE_MIN && p.S > 1 && p.stop >= 4) wide_done = wide_select(tmax);
  }
  if (wide_done) {
    ncand = keff;
    sorted_in_lds = true;
    regions = false;
  } else if (keff > 0) {
    const uint32_t L = lower_bound(tmax);
    if (p.stop == 2) {
      if (t == 0 && split == 0) p.out[row] = (int64_t)L;
      return;
    }
    int nst = 0;
    stage(IC<0>{}, IC<NP>{}, L, nst);
    int unused = 0;
    extract(IC<0>{}, IC<CH>{}, L, nst, sm.top, FSAMP_K_MAX, &sm.misc[M_CNT], unused);
    __syncthreads();
    pre = sm.top[lane];  // issued with the count read below: one LDS round trip for both
    L_sel = L;
    FSAMP_TRACE(4);
    // LDS loads count as divergent to the compiler; the total is uniform by construction
    const int total = __builtin_amdgcn_readfirstlane(sm.misc[M_CNT]);
    const bool wave_over = false;
    if (p.stop == 3) {
      if (t == 0 && split == 0) p.out[row] = total;
      return;
    }

    // 4. the slice's top-keff, sorted: up to WSORT_MAX candidates go straight to wave 0's
    //    register sort below; up to K_MAX (all of them in top[]) the workgroup sorts them in
    //    LDS; beyond that an exact radix select over the registers first reduces them to
    //    exactly keff.
    ncand = total;
    if (total > WSORT_MAX && total <= FSAMP_K_MAX && !wave_over) {
      // more candidates than wave 0 sorts in registers (heavy ties, wide k), but every one of
      // them was gathered into top[]: the workgroup sorts them where they are
      int P = 1;
      while (P < total) P <<= 1;
      for (int i = total + t; i < P; i += NT) sm.top[i] = 0ull;
      __syncthreads();
      if (keff <= 64) block_top_desc<NT, 1>(sm.top, P);
      else if (keff <= 128) block_top_desc<NT, 2>(sm.top, P);
      else if (keff <= 256) block_top_desc<NT, 4>(sm.top, P);
      else block_bitonic_sort_desc<NT>(sm.top, P);
      sorted_in_lds = true;
    } else if (total > WSORT_MAX || wave_over) {
      // candidates past the top[] buffer: exact radix select over the registers -- threshold
      // T, keys > T, and the lowest-id keys == T in id order -- into cand[0..keff), then sort
      pass_barrier<CH>(kv);
      const int sub = wid & (NSUB - 1);
      zero_hist<NT>(sm.u.rx.hist);
      __syncthreads();
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (pair_ge(c, L)) {
          uint32_t m = ge_mask(kv[c], L);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            wave_add(sm.u.rx.hist + sub * 256, key_at(kv[c], j) >> 8, true);
          }
        }
      }
      __syncthreads();
      fold_hist<NT>(sm.u.rx.hist);
      __syncthreads();
      suffix256(sm.u.rx.hist, sm.u.rx.suf);
      __syncthreads();
      find_bucket<NT>(sm.u.rx.suf, keff, 0, &sm.misc[M_HB], &sm.misc[M_ABOVE]);
      FSAMP_TRACE(1);
      zero_hist<NT>(sm.u.rx.hist);
      __syncthreads();
      const uint32_t hb = (uint32_t)sm.misc[M_HB];
      const int above = sm.misc[M_ABOVE];
      pass_barrier<CH>(kv);
      // keys with high byte hb are exactly the keys in [hb<<8, (hb<<8) + 255]
      const uint32_t band_lo = max(hb << 8, L);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (pair_ge(c, band_lo)) {
          uint32_t m = ge_mask(kv[c], band_lo);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            const uint32_t k = key_at(kv[c], j);
            wave_add(sm.u.rx.hist + sub * 256, k & 255u, (k >> 8) == hb);
          }
        }
      }
      __syncthreads();
      fold_hist<NT>(sm.u.rx.hist);
      __syncthreads();
      suffix256(sm.u.rx.hist, sm.u.rx.suf);
      __syncthreads();
      find_bucket<NT>(sm.u.rx.suf, keff - above, above, &sm.misc[M_LB], &sm.misc[M_GT]);
      if (t == 0) sm.misc[M_CNT] = 0;
      __syncthreads();
      const uint32_t T = (hb << 8) | (uint32_t)sm.misc[M_LB];
      const int n_gt = sm.misc[M_GT];
      const int need = keff - n_gt;
      pass_barrier<CH>(kv);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (pair_ge(c, T + 1u)) {
          uint32_t m = ge_mask(kv[c], T + 1u);
          const uint32_t id0 = opaque_base(lo, t) + (uint32_t)(c * NT * 8);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            sm.g.cand[atomicAdd(&sm.misc[M_CNT], 1)] = pack(key_at(kv[c], j), id0 + (uint32_t)j);
          }
        }
      }
      FSAMP_TRACE(14);
      pass_barrier<CH>(kv);
      // chunk c of every thread precedes chunk c+1 in id order, and within a chunk thread t
      // precedes t+1, so a block scan per chunk ranks the tied keys by id.  `taken` is
      // uniform, so the guard keeps every barrier uniform; the loop stays fully unrolled so
      // kv[] is never indexed dynamically.
      int taken = 0;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (taken < need) {
          uint32_t tiemask = eq_mask(kv[c], T);
          int chunk_total = 0;
          int rank = taken + block_excl_scan<NT>(__popc(tiemask), &chunk_total, sm.wsum[c & 1]);
          const uint32_t id0 = opaque_base(lo, t) + (uint32_t)(c * NT * 8);
          while (tiemask != 0u && rank < need) {
            const int j = __ffs(tiemask) - 1;
            tiemask &= tiemask - 1u;
            sm.g.cand[n_gt + rank] = pack(T, id0 + (uint32_t)j);
            ++rank;
          }
          taken += chunk_total;
        }
      }
      __syncthreads();
      FSAMP_TRACE(15);
      ncand = keff;
      regions = false;
      if (keff > WSORT_MAX) {
        // exactly keff (<= K_MAX) words in cand[]: pad to a power of two and sort in place
        int P = 1;
        while (P < keff) P <<= 1;
        for (int i = keff + t; i < P; i += NT) sm.g.cand[i] = 0ull;
        __syncthreads();
        block_bitonic_sort_desc<NT>(sm.g.cand, P);
        for (int i = t; i < keff; i += NT) sm.top[i] = sm.g.cand[i];
        sorted_in_lds = true;
      }
      __syncthreads();
    }
  }

  // 5-6'. Rows split over several workgroups with k > 128: the whole workgroup hands the
  //    slice's sorted list over and, in the row's last workgroup, reads the S lists back and
  //    folds them (workgroup bitonic merges), where one wave would take S-1 wide merges and
  //    S*K serial loads.  The words are agent-scope atomic stores, each wave waits for its
  //    own (s_waitcnt 0) before the workgroup barrier, and one relaxed agent-scope ticket
  //    follows.  This relies on a gfx950 property the HIP memory model does not state: an
  //    agent-scope atomic store is written through to the device-coherent level (sc1) and is
  //    visible to every agent-scope atomic load once s_waitcnt has seen it acknowledged.  An
  //    acquire-release ticket here measured 0.7 us slower (C4-like k=256: 22.67 against
  //    21.93 us), so the relaxed form stays; the wave-0 hand-off, where it is free, uses it.
  //    Compiled only into the MERGE instantiations, which the host launches for exactly those
  //    calls: the code would otherwise cost the common path (k <= 128) ~0.1-0.2 us.
  bool merged = false;
  if (MERGE && p.K > 128 && p.S > 1 && p.stop != 1 && p.stop != 2 && p.stop != 3) {
    if (keff > 0 && !sorted_in_lds) {
      if (wid == 0) {
        const uint64_t* base = regions ? sm.top : sm.g.cand;
        auto load = [&](int e) -> uint64_t { return base[e]; };
        wave_sort_topk(load, ncand, keff, sm.top);
      }
      __syncthreads();
    }
    FSAMP_TRACE(5);
    if (p.stop == 4) {
      if (t == 0 && split == 0) p.out[row] = keff > 0 ? (int64_t)unpack_id(sm.top[0]) : -1;
      return;
    }
    uint64_t* dst = p.partials + ((size_t)row * p.S + split) * p.K;
    for (int i = t; i < p.K; i += NT)
      __hip_atomic_store(&dst[i], i < keff ? sm.top[i] : 0ull, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0)
      sm.misc[M_RED] = (int)__hip_atomic_fetch_add(&p.tickets[row * TICKET_STRIDE], 1u,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int prev = __builtin_amdgcn_readfirstlane(sm.misc[M_RED]);
    FSAMP_TRACE(6);
    if (prev != p.S - 1) return;
    if (t == 0)
      __hip_atomic_store(&p.tickets[row * TICKET_STRIDE], 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (p.stop == 5) {
      if (t == 0) p.out[row] = (int64_t)unpack_id(sm.top[0]);
      return;
    }
    // the S lists into cand[], four agent-scope loads in flight per thread
    const int n = p.S * p.K;
    const uint64_t* src = p.partials + (size_t)row * p.S * p.K;
    constexpr bool WIDE_MERGE = NT >= 512;
    for (int i0 = 0; i0 < n; i0 += 4 * NT) {
      uint64_t w4[4];
  #pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = i0 + q * NT + t;
        w4[q] = i < n ? __hip_atomic_load(&src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : 0ull;
      }
  #pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = i0 + q * NT + t;
        if (i < n) sm.g.cand[i] = w4[q];
      }
    }
    __syncthreads();
    FSAMP_TRACE(7);
    // Wide lists: pairwise merges of the sorted lists, each output word placed by its
    // merge-path split (a binary search over the pair's diagonal), in ceil(log2 S) rounds with
    // a barrier each; the last round writes top[].  Lists ping-pong between cand[] and the
    // second half of g.
    bool ranked = false;
    if constexpr (WIDE_MERGE) {
      if (p.K > WIDE_MIN) {
        const int K = p.K;
        uint64_t* gw = reinterpret_cast<uint64_t*>(&sm.g);  // cand[] is its first CAND_CAP words
        int nl = p.S, cur = 0;
        while (nl > 1) {
          const int np = nl >> 1;
          const uint64_t* src = gw + cur * CAND_CAP;
          uint64_t* dst = nl == 2 ? sm.top : gw + (cur ^ 1) * CAND_CAP;
          for (int q = 0; q < np; ++q) {
            const uint64_t* a = src + (size_t)(2 * q) * K;
            const uint64_t* b = a + K;
            for (int r = t; r < K; r += NT) dst[q * K + r] = merge_path_at(a, b, K, r);
          }
          if (nl & 1)
            for (int r = t; r < K; r += NT) dst[np * K + r] = src[(nl - 1) * K + r];
          __syncthreads();
          nl = np + (nl & 1);
          cur ^= 1;
        }
        ranked = true;
      }
    }
    if (!ranked) {
      // top[0..P) runs the merged list (zeros past it); each further list, reversed, is
      // folded in by an elementwise maximum (a bitonic sequence holding the top P of both)
      // and a merge
      int P = 64;
      while (P < p.K) P <<= 1;
      for (int i = t; i < P; i += NT) sm.top[i] = i < p.K ? sm.g.cand[i] : 0ull;
      __syncthreads();
      for (int sl = 1; sl < p.S; ++sl) {
        for (int i = t; i < P; i += NT) {
          const int e = P - 1 - i;
          const uint64_t b = e < p.K ? sm.g.cand[sl * p.K + e] : 0ull;
          const uint64_t a = sm.top[i];
          sm.top[i] = a > b ? a : b;
        }
        __syncthreads();
        block_bitonic_merge_desc<NT>(sm.top, P);
      }
    }
    FSAMP_TRACE(8);
    merged = true;
  }

  // Wide sampling tails after the workgroup merge: the whole workgroup computes every rank's
  // unnormalised weight exp((x_i - m) * inv_t) into LDS (the operations wave 0's tail would
  // run, 16 per lane at k = 1024), so that wave 0 keeps only the serial sums, scans and draw.
  const float* wpre = nullptr;
  if constexpr (MERGE) {
    if (merged && p.K > 256 && p.ids == nullptr && p.words == nullptr && p.stop == 7) {
      const RowCtl rc0 = row_ctl();
      float* wl = reinterpret_cast<float*>(&sm.u);  // K <= 1024 floats; u is free by now
      const float m = key_to_float((uint32_t)(sm.top[0] >> 32), p.is_bf16);
      for (int i = t; i < rc0.k; i += NT)
        wl[i] = exp_nonpos((key_to_float((uint32_t)(sm.top[i] >> 32), p.is_bf16) - m) *
                           rc0.inv_t);
      __syncthreads();
      wpre = wl;
    }
  }

  // From here on wave 0 carries the workgroup alone: no more workgroup barriers.
  if (wid != 0) return;
  const RowCtl rc = row_ctl();
  // after the workgroup merge: the row's sorted top K in top[], nothing left to hand over
  int keff_b = keff, s_b = p.S;
  if (merged) {
    s_b = 1;
    keff_b = p.K;
    ncand = p.K;
    sorted_in_lds = true;
  }
  auto back = [&](auto rbc) {
    constexpr int RB = decltype(rbc)::value;
    wave_back<RB, NT>(p, sm, keff_b, ncand, sorted_in_lds, regions, row, split, rc, L_sel, pre,
                      s_b, wpre);
  };
  if (p.K <= 64) back(IC<1>{});
  else if (p.K <= 128) back(IC<2>{});
  else if (p.K <= 256) back(IC<4>{});
  else if (p.K <= 512) back(IC<8>{});
  else back(IC<16>{});
}

// ---- merge of N sorted candidate lists per row (fsamp_merge_sample) ----------------------------

// One wave per row: words[row] holds n_lists descending lists of p.K words (zero words past a
// short list).  The lists pass through LDS in batches of CAND_CAP / K (at least 4): each batch
// is staged with every load of it in flight, then folded into the running top K in registers
// with the bitonic top-merges of the split hand-off.  Every read of a list is an LDS read of
// the __shared__ array itself, never through a pointer that may address either LDS or global
// memory (such a pointer compiles to FLAT accesses, whose folded immediate offsets can leave
// the base address outside the LDS aperture).  The row finishes like the sampler's own: ids of
// the merged top K, or the fp32 tail.  RB = ceil(K / 64) rounded up to 1, 2, 4, 8 or 16.
template <int RB>
__global__ __launch_bounds__(64) void fsamp_merge_kernel(Params p, const uint64_t* words,
                                                         int n_lists) {
  __shared__ uint64_t lists[CAND_CAP];
  __shared__ uint64_t top[FSAMP_K_MAX];
  const int row = blockIdx.x;
  const int l = lane_id();
  const int K = p.K;
  const uint64_t* src = words + (size_t)row * (size_t)n_lists * (size_t)K;
  RowCtl rc;
  rc.u = p.u != nullptr ? p.u[row] : rng_uniform(p.seed, p.offset, (uint32_t)row);
  rc.k = K;
  rc.top_p = p.top_p_f;
  rc.keep_all = p.keep_all;
  rc.inv_t = 1.0f;
  const int per = CAND_CAP / K;  // lists per LDS batch
  uint64_t a[RB], b[RB];
  for (int s0 = 0; s0 < n_lists; s0 += per) {
    const int nb = min(per, n_lists - s0);
    const int n = nb * K;
    const uint64_t* bsrc = src + (size_t)s0 * (size_t)K;
    // the previous batch has been read (into registers) before it is overwritten
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    for (int i0 = 0; i0 < n; i0 += 8 * 64) {
      uint64_t w[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = i0 + q * 64 + l;
        w[q] = i < n ? bsrc[i] : 0ull;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = i0 + q * 64 + l;
        if (i < n) lists[i] = w[q];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    int s = 0;
    if (s0 == 0) {
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int f = l * RB + i;
        a[i] = f < K ? lists[f] : 0ull;
      }
      s = 1;
    }
    for (; s < nb; ++s) {
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int e = 64 * RB - 1 - (l * RB + i);
        b[i] = e < K ? lists[s * K + e] : 0ull;
      }
      wave_merge_top<RB>(a, b);
    }
  }
  if constexpr (RB <= 4) {
    wave_finish<RB>(p, a, top, row, rc);
  } else {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int e = l * RB + i;
      if (e < K) top[e] = a[i];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (p.ids != nullptr) {
      for (int i = l; i < K; i += 64) p.ids[(size_t)row * K + i] = (int64_t)unpack_id(top[i]);
      return;
    }
    const uint64_t none[RB] = {};
    sample_tail<RB, true>(p, none, top, rc, row);
  }
}

// ---- instantiation table -----------------------------------------------------------------------
//
// The instantiations are compiled in eight parts, in parallel: this file built with
// -DFSAMP_PART=n (n = 0..7) instantiates one group of tilings, common (n even) or MERGE (n odd;
// part 7 also holds the list-merge kernels), and the build without FSAMP_PART holds only the
// host-side table, which takes the addresses of
// every instantiation (their host stubs come from the parts at link time).

#define FSAMP_COMMON_VEC(NT_, CH_) template __global__ void fsamp_kernel<NT_, CH_, true, false>(Params);
#define FSAMP_COMMON_SCALAR(NT_, CH_) \
  template __global__ void fsamp_kernel<NT_, CH_, false, false>(Params);
#define FSAMP_MERGE_VEC(NT_, CH_) template __global__ void fsamp_kernel<NT_, CH_, true, true>(Params);
#define FSAMP_MERGE_SCALAR(NT_, CH_) \
  template __global__ void fsamp_kernel<NT_, CH_, false, true>(Params);

#if defined(FSAMP_PART)

#if FSAMP_PART == 0
FSAMP_KERNEL_LIST_VEC_256(FSAMP_COMMON_VEC)
#elif FSAMP_PART == 1
FSAMP_KERNEL_LIST_VEC_256(FSAMP_MERGE_VEC)
#elif FSAMP_PART == 2
FSAMP_KERNEL_LIST_VEC_512(FSAMP_COMMON_VEC)
#elif FSAMP_PART == 3
FSAMP_KERNEL_LIST_VEC_512(FSAMP_MERGE_VEC)
#elif FSAMP_PART == 4
FSAMP_KERNEL_LIST_VEC_1024(FSAMP_COMMON_VEC)
#elif FSAMP_PART == 5
FSAMP_KERNEL_LIST_VEC_1024(FSAMP_MERGE_VEC)
#elif FSAMP_PART == 6
FSAMP_KERNEL_LIST_SCALAR(FSAMP_COMMON_SCALAR)
#elif FSAMP_PART == 7
FSAMP_KERNEL_LIST_SCALAR(FSAMP_MERGE_SCALAR)
template __global__ void fsamp_merge_kernel<1>(Params, const uint64_t*, int);
template __global__ void fsamp_merge_kernel<2>(Params, const uint64_t*, int);
template __global__ void fsamp_merge_kernel<4>(Params, const uint64_t*, int);
template __global__ void fsamp_merge_kernel<8>(Params, const uint64_t*, int);
template __global__ void fsamp_merge_kernel<16>(Params, const uint64_t*, int);
#else
#error "FSAMP_PART must be in [0, 7]"
#endif

#else  // the table

#define FSAMP_EXTERN_COMMON_VEC(NT_, CH_) extern FSAMP_COMMON_VEC(NT_, CH_)
#define FSAMP_EXTERN_COMMON_SCALAR(NT_, CH_) extern FSAMP_COMMON_SCALAR(NT_, CH_)
#define FSAMP_EXTERN_MERGE_VEC(NT_, CH_) extern FSAMP_MERGE_VEC(NT_, CH_)
#define FSAMP_EXTERN_MERGE_SCALAR(NT_, CH_) extern FSAMP_MERGE_SCALAR(NT_, CH_)
FSAMP_KERNEL_LIST_VEC(FSAMP_EXTERN_COMMON_VEC)
FSAMP_KERNEL_LIST_SCALAR(FSAMP_EXTERN_COMMON_SCALAR)
FSAMP_KERNEL_LIST_VEC(FSAMP_EXTERN_MERGE_VEC)
FSAMP_KERNEL_LIST_SCALAR(FSAMP_EXTERN_MERGE_SCALAR)

#define FSAMP_INST_VEC(NT_, CH_)                                                   \
  {NT_, CH_, 1, (const void*)fsamp_kernel<NT_, CH_, true, false>,                  \
   (const void*)fsamp_kernel<NT_, CH_, true, true>, "fsamp_kernel<" #NT_ "," #CH_ ",vec>"},
#define FSAMP_INST_SCALAR(NT_, CH_)                                                \
  {NT_, CH_, 0, (const void*)fsamp_kernel<NT_, CH_, false, false>,                 \
   (const void*)fsamp_kernel<NT_, CH_, false, true>, "fsamp_kernel<" #NT_ "," #CH_ ",elem>"},

// host pass only: the device code of this unit holds no instantiation
#ifndef __HIP_DEVICE_COMPILE__
const KernelEntry kKernels[] = {FSAMP_KERNEL_LIST_VEC(FSAMP_INST_VEC)
                                    FSAMP_KERNEL_LIST_SCALAR(FSAMP_INST_SCALAR)};
const int kNumKernels = (int)(sizeof(kKernels) / sizeof(kKernels[0]));
#endif

extern template __global__ void fsamp_merge_kernel<1>(Params, const uint64_t*, int);
extern template __global__ void fsamp_merge_kernel<2>(Params, const uint64_t*, int);
extern template __global__ void fsamp_merge_kernel<4>(Params, const uint64_t*, int);
extern template __global__ void fsamp_merge_kernel<8>(Params, const uint64_t*, int);
extern template __global__ void fsamp_merge_kernel<16>(Params, const uint64_t*, int);
#ifndef __HIP_DEVICE_COMPILE__
const void* const kMergeKernels[5] = {
    (const void*)fsamp_merge_kernel<1>, (const void*)fsamp_merge_kernel<2>,
    (const void*)fsamp_merge_kernel<4>, (const void*)fsamp_merge_kernel<8>,
    (const void*)fsamp_merge_kernel<16>};
#endif

#endif  // FSAMP_PART

}  // namespace fsamp
