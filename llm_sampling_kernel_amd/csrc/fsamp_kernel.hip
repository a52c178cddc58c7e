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
// Selection, MI355X-first:
//   1. every thread issues all of its dwordx4 loads at once (CH chunks of 8 elements, chunk c
//      of thread t at uint4 index c*NT + t: coalesced), converts them to packed u16 keys with
//      16-bit packed integer ops and keeps a running packed max (v_pk_max_u16);
//   2. L = the k-th largest of the NT per-thread maxima is a lower bound of the slice's k-th
//      largest key (k threads each own an element >= L), found with two 8-bit LDS histograms
//      over NT values only;
//   3. elements >= L (typically ~1.5k of them, never the bulk of the slice) are compacted into
//      LDS as u64 (key << 32 | ~id) words, which are unique, so sorting them orders by value
//      and then by ascending id: the tie rule needs no extra pass;
//   4. if more than CAND_CAP elements are >= L (heavy ties), an exact radix select runs over
//      the register-resident keys instead: two 8-bit LDS histograms (restricted to keys >= L),
//      a gather of keys above the threshold and an id-ordered block scan of the tied keys that
//      takes the lowest `need` ids.
// No pass re-reads HBM.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "fsamp.h"
#include "fsamp_internal.h"

namespace fsamp {

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

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

// key -> fp32 value (the exact bf16/fp16 value; the -0 key decodes to +0)
__device__ __forceinline__ float key_to_float(uint32_t key, int is_bf16) {
  const uint32_t b = (key & 0x8000u) ? (key & 0x7FFFu) : ((0x10000u - key) & 0xFFFFu);
  if (is_bf16) return __uint_as_float(b << 16);
  return (float)__builtin_bit_cast(_Float16, (unsigned short)b);
}

// ---- fp32 tail helpers -------------------------------------------------------------------

// e^x for x <= 0: Cody-Waite split by ln2 (16-bit head, tail), degree-7 Taylor polynomial for
// |r| <= ln2/2 by Horner with fma, scale by 2^n from exponent bits; x < -86 gives 0.
// Bit-identical to the CPU oracle's exp, which evaluates the same operations in the same order.
__device__ __forceinline__ float exp_nonpos(float x) {
  if (!(x >= -86.0f)) return 0.0f;
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
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
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

struct Smem {
  uint64_t cand[CAND_CAP];   // candidate (key, ~id) words
  uint32_t hist[NSUB * 256]; // radix histograms (NSUB sub-histograms to spread LDS atomics)
  uint32_t suf[256];         // suffix sums of the folded histogram
  int32_t wsum[2][16];       // per-wave partials for block scans (double-buffered)
  int32_t misc[16];
};

enum { M_HB = 0, M_ABOVE, M_LB, M_GT, M_CNT, M_LAST, M_RED, M_TOTAL };

// ---- block primitives ----------------------------------------------------------------------

// inclusive prefix over the first W lanes of the wave (W a power of two <= 64)
template <int W = 64>
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < W; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Exclusive prefix of v over the workgroup in thread order; *total gets the sum.  Each wave
// scans the per-wave totals itself, so no more than two extra values stay live.
template <int NT>
__device__ __forceinline__ int block_excl_scan(int v, int* total, int32_t* wsum) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int incl = wave_incl_scan(v);
  if (lane == 63) wsum[wid] = incl;
  __syncthreads();
  const int ws = lane < NW ? wsum[lane] : 0;
  const int wincl = wave_incl_scan<NW>(ws);
  *total = __shfl(wincl, NW - 1, 64);
  return __shfl(wincl - ws, wid, 64) + incl - v;
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
    uint32_t incl = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = __shfl_up(incl, d, 64);
      if (l >= d) incl += o;
    }
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

// The want-th largest of one 16-bit value per thread (want <= NT), by two 8-bit histograms.
template <int NT>
__device__ uint32_t block_kth_of_one(uint32_t v, int want, Smem& sm) {
  zero_hist<NT>(sm.hist);
  __syncthreads();
  atomicAdd(&sm.hist[v >> 8], 1u);
  __syncthreads();
  suffix256(sm.hist, sm.suf);
  __syncthreads();
  find_bucket<NT>(sm.suf, want, 0, &sm.misc[M_HB], &sm.misc[M_ABOVE]);
  zero_hist<NT>(sm.hist);
  __syncthreads();
  const int hb = sm.misc[M_HB];
  const int above = sm.misc[M_ABOVE];
  if ((int)(v >> 8) == hb) atomicAdd(&sm.hist[v & 255u], 1u);
  __syncthreads();
  suffix256(sm.hist, sm.suf);
  __syncthreads();
  find_bucket<NT>(sm.suf, want - above, above, &sm.misc[M_LB], &sm.misc[M_GT]);
  __syncthreads();
  return ((uint32_t)hb << 8) | (uint32_t)sm.misc[M_LB];
}

// Descending bitonic sort of cand[0..n) in LDS (n <= CAND_CAP), padded with zeros to a
// power of two; zero is below every real (key >= 1) word.
template <int NT>
__device__ void block_sort_desc(uint64_t* cand, int n) {
  int P = 1;
  while (P < n) P <<= 1;
  for (int i = n + threadIdx.x; i < P; i += NT) cand[i] = 0ull;
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int q = threadIdx.x; q < (P >> 1); q += NT) {
        const int i = ((q & ~(j - 1)) << 1) | (q & (j - 1));
        const int ixj = i + j;
        const uint64_t a = cand[i], b = cand[ixj];
        const bool desc = (i & k) == 0;
        if (desc ? (a < b) : (a > b)) {
          cand[i] = b;
          cand[ixj] = a;
        }
      }
      __syncthreads();
    }
  }
}

// ---- the fp32 tail (one wave) ----------------------------------------------------------------

// Runs on wave 0 with the row's top K words sorted descending in cand[0..K).  The reduction
// and scan orders are fixed functions of K (R = ceil(K/64) ranks per lane, butterfly and
// Kogge-Stone over lane distances 1..32) and are mirrored by the CPU oracle.
__device__ void sample_tail(const Params& p, const uint64_t* cand, int K, int row) {
  const int l = threadIdx.x;  // 0..63
  const int R = (K + 63) >> 6;
  const int base = l * R;
  float w[RMAX], pr[RMAX], c[RMAX];
  const float m = key_to_float((uint32_t)(cand[0] >> 32), p.is_bf16);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    w[j] = 0.0f;
    if (j < R && base + j < K) {
      const float x = key_to_float((uint32_t)(cand[base + j] >> 32), p.is_bf16);
      w[j] = exp_nonpos(x - m);
      s = s + w[j];
    }
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) s = s + __shfl_xor(s, d, 64);
  const float z = s;
  float t = 0.0f;
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    pr[j] = 0.0f;
    if (j < R && base + j < K) {
      pr[j] = w[j] / z;
      t = t + pr[j];
    }
  }
  float incl = t;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float o = __shfl_up(incl, d, 64);
    if (l >= d) incl = o + incl;
  }
  float acc = __shfl_up(incl, 1, 64);
  if (l == 0) acc = 0.0f;
  int first_drop = K;
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    c[j] = 0.0f;
    if (j < R && base + j < K) {
      acc = acc + pr[j];
      c[j] = acc;
      const int idx = base + j;
      if (idx >= 1 && first_drop == K && !((c[j] - pr[j]) < p.top_p_f)) first_drop = idx;
    }
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) first_drop = min(first_drop, __shfl_xor(first_drop, d, 64));
  const int r = (p.keep_all || first_drop == K) ? K - 1 : first_drop - 1;
  // Z_p = c_r from the lane that owns rank r
  float mine_c = 0.0f;
#pragma unroll
  for (int j = 0; j < RMAX; ++j)
    if (j == r - base) mine_c = c[j];
  const float zp = __shfl(mine_c, r / R, 64);
  const float u = p.u ? p.u[row] : rng_uniform(p.seed, p.offset, (uint32_t)row);
  const float target = u * zp;
  int pick = K;
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    const int idx = base + j;
    if (j < R && idx <= r && pick == K && c[j] >= target) pick = idx;
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) pick = min(pick, __shfl_xor(pick, d, 64));
  if (pick == K) pick = r;
  if (l == 0) p.out[row] = (int64_t)unpack_id(cand[pick]);
  if (p.keep != nullptr) {
#pragma unroll
    for (int j = 0; j < RMAX; ++j) {
      const int idx = base + j;
      if (j < R && idx < K) {
        p.keep[(size_t)row * K + idx] = (uint8_t)(idx <= r);
        p.renormed[(size_t)row * K + idx] = idx <= r ? pr[j] / zp : 0.0f;
      }
    }
  }
}

// ---- the kernel ----------------------------------------------------------------------------

// Opaque to the optimiser: the keys are "redefined" here, so per-chunk values derived from
// them in an earlier pass (chunk maxima, masks) are recomputed instead of being kept live
// across the pass boundary -- at 19 chunks per thread those would cost ~40 VGPRs.
template <int CH>
__device__ __forceinline__ void pass_barrier(uint32_t (&kv)[CH][4]) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int q = 0; q < 4; ++q) asm volatile("" : "+v"(kv[c][q]));
  }
}

// bit j set when element j (0..7) of the chunk has key >= L
__device__ __forceinline__ uint32_t ge_mask(const uint32_t (&k)[4], uint32_t L) {
  uint32_t m = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    m |= (uint32_t)((k[q] & 0xFFFFu) >= L) << (2 * q);
    m |= (uint32_t)((k[q] >> 16) >= L) << (2 * q + 1);
  }
  return m;
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

// max key of one 8-element chunk (two packed dwords per pk_max step)
__device__ __forceinline__ uint32_t chunk_max(const uint32_t (&k)[4]) {
  const uint32_t m2 = pkmax(pkmax(k[0], k[1]), pkmax(k[2], k[3]));
  return max(m2 & 0xFFFFu, m2 >> 16);
}

template <int NT, int CH, bool VEC>
__global__ __launch_bounds__(NT) void fsamp_kernel(Params p) {
  __shared__ Smem sm;
  const int t = threadIdx.x;
  const int row = blockIdx.x / p.S;
  const int split = blockIdx.x - row * p.S;
  const uint16_t* xr = p.logits + (size_t)row * (size_t)p.V;
  const int lo = split * p.slice;
  const int hi = min(lo + p.slice, p.V);
  const int count = max(hi - lo, 0);
  const int keff = min(p.K, count);

  // 1. load the slice into registers as packed keys (padding = key 0); thread maximum.
  //    With VEC, V and the split bounds are multiples of 8, so a chunk is all in or all out.
  uint32_t kv[CH][4];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int e0 = lo + (c * NT + t) * 8;
    if constexpr (VEC) {
      if (e0 < hi) {
        const uint4 v = *reinterpret_cast<const uint4*>(xr + e0);
        kv[c][0] = v.x;
        kv[c][1] = v.y;
        kv[c][2] = v.z;
        kv[c][3] = v.w;
      } else {
        kv[c][0] = kv[c][1] = kv[c][2] = kv[c][3] = 0u;
      }
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
  uint32_t tmax2 = 0;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int e0 = lo + (c * NT + t) * 8;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t k = keys2(kv[c][q]);
      if constexpr (VEC) {
        if (e0 >= hi) k = 0u;
      } else {
        const int e = e0 + 2 * q;
        if (e >= hi) k &= 0xFFFF0000u;
        if (e + 1 >= hi) k &= 0x0000FFFFu;
      }
      kv[c][q] = k;
      tmax2 = pkmax(tmax2, k);
    }
  }
  const uint32_t tmax = max(tmax2 & 0xFFFFu, tmax2 >> 16);

  if (p.stop == 1) {
    if (t == 0) sm.misc[M_RED] = 0;
    __syncthreads();
    atomicMax(&sm.misc[M_RED], (int)tmax);
    __syncthreads();
    if (t == 0 && split == 0) p.out[row] = sm.misc[M_RED];
    return;
  }

  int ncand = 0;
  if (keff > 0) {
    // 2. lower bound L of the slice's keff-th largest key
    uint32_t L = 1u;
    if (keff <= NT) L = max(block_kth_of_one<NT>(tmax, keff, sm), 1u);
    if (p.stop == 2) {
      if (t == 0 && split == 0) p.out[row] = (int64_t)L;
      return;
    }

    // 3. count elements >= L, compact them if they fit.  Per chunk an 8-bit mask of the
    //    qualifying elements; the rare hits are visited with ffs so that nothing beyond the
    //    slice's own registers stays live.
    int mine = 0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (chunk_max(kv[c]) >= L) mine += __popc(ge_mask(kv[c], L));
    }
    int total = 0;
    const int off = block_excl_scan<NT>(mine, &total, sm.wsum[0]);
    pass_barrier<CH>(kv);
    if (total <= CAND_CAP) {
      int pos = off;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (chunk_max(kv[c]) >= L) {
          uint32_t m = ge_mask(kv[c], L);
          const uint32_t id0 = (uint32_t)(lo + (c * NT + t) * 8);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            sm.cand[pos++] = pack(key_at(kv[c], j), id0 + (uint32_t)j);
          }
        }
      }
      ncand = total;
    } else {
      // 4. exact radix select over the registers (heavy ties): threshold T, keys > T, and the
      //    lowest-id keys == T in id order
      const int sub = (t >> 6) & (NSUB - 1);
      zero_hist<NT>(sm.hist);
      __syncthreads();
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (chunk_max(kv[c]) >= L) {
          uint32_t m = ge_mask(kv[c], L);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            atomicAdd(&sm.hist[sub * 256 + (key_at(kv[c], j) >> 8)], 1u);
          }
        }
      }
      __syncthreads();
      fold_hist<NT>(sm.hist);
      __syncthreads();
      suffix256(sm.hist, sm.suf);
      __syncthreads();
      find_bucket<NT>(sm.suf, keff, 0, &sm.misc[M_HB], &sm.misc[M_ABOVE]);
      zero_hist<NT>(sm.hist);
      __syncthreads();
      const uint32_t hb = (uint32_t)sm.misc[M_HB];
      const int above = sm.misc[M_ABOVE];
      pass_barrier<CH>(kv);
      // keys with high byte hb are exactly the keys in [hb<<8, (hb<<8) + 255]
      const uint32_t band_lo = max(hb << 8, L);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (chunk_max(kv[c]) >= band_lo) {
          uint32_t m = ge_mask(kv[c], band_lo);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            const uint32_t k = key_at(kv[c], j);
            if ((k >> 8) == hb) atomicAdd(&sm.hist[sub * 256 + (k & 255u)], 1u);
          }
        }
      }
      __syncthreads();
      fold_hist<NT>(sm.hist);
      __syncthreads();
      suffix256(sm.hist, sm.suf);
      __syncthreads();
      find_bucket<NT>(sm.suf, keff - above, above, &sm.misc[M_LB], &sm.misc[M_GT]);
      if (t == 0) sm.misc[M_CNT] = 0;
      __syncthreads();
      const uint32_t T = (hb << 8) | (uint32_t)sm.misc[M_LB];
      const int n_gt = sm.misc[M_GT];
      const int need = keff - n_gt;
      pass_barrier<CH>(kv);
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        if (chunk_max(kv[c]) > T) {
          uint32_t m = ge_mask(kv[c], T + 1u);
          const uint32_t id0 = (uint32_t)(lo + (c * NT + t) * 8);
          while (m != 0u) {
            const int j = __ffs(m) - 1;
            m &= m - 1u;
            sm.cand[atomicAdd(&sm.misc[M_CNT], 1)] = pack(key_at(kv[c], j), id0 + (uint32_t)j);
          }
        }
      }
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
          const uint32_t id0 = (uint32_t)(lo + (c * NT + t) * 8);
          while (tiemask != 0u && rank < need) {
            const int j = __ffs(tiemask) - 1;
            tiemask &= tiemask - 1u;
            sm.cand[n_gt + rank] = pack(T, id0 + (uint32_t)j);
            ++rank;
          }
          taken += chunk_total;
        }
      }
      ncand = keff;
    }
    __syncthreads();
    if (p.stop == 3) {
      if (t == 0 && split == 0) p.out[row] = ncand;
      return;
    }
    block_sort_desc<NT>(sm.cand, ncand);
  }
  if (p.stop == 4) {
    if (t == 0 && split == 0) p.out[row] = keff > 0 ? (int64_t)unpack_id(sm.cand[0]) : -1;
    return;
  }

  if (p.S > 1) {
    // 5. hand the slice's top-K to the row's last workgroup
    uint64_t* dst = p.partials + ((size_t)row * p.S + split) * p.K;
    for (int i = t; i < p.K; i += NT) dst[i] = (i < keff) ? sm.cand[i] : 0ull;
    __threadfence();
    __syncthreads();
    if (t == 0) {
      const unsigned prev = atomicAdd(&p.tickets[row], 1u);
      sm.misc[M_LAST] = (prev == (unsigned)(p.S - 1)) ? 1 : 0;
    }
    __syncthreads();
    if (sm.misc[M_LAST] == 0) return;
    __threadfence();
    if (t == 0) atomicExch(&p.tickets[row], 0u);
    if (p.stop == 5) {
      if (t == 0) p.out[row] = (int64_t)unpack_id(sm.cand[0]);
      return;
    }
    // 6. merge: the S sorted lists of the row
    const int n = p.S * p.K;
    const uint64_t* src = p.partials + (size_t)row * p.S * p.K;
    for (int i = t; i < n; i += NT) sm.cand[i] = src[i];
    __syncthreads();
    block_sort_desc<NT>(sm.cand, n);
  }
  if (p.stop == 5 || p.stop == 6) {
    if (t == 0) p.out[row] = (int64_t)unpack_id(sm.cand[0]);
    return;
  }

  // 7. sampling tail, or the candidate ids
  if (p.ids != nullptr) {
    for (int i = t; i < p.K; i += NT) p.ids[(size_t)row * p.K + i] = (int64_t)unpack_id(sm.cand[i]);
    return;
  }
  if (t < 64) sample_tail(p, sm.cand, p.K, row);
}

// ---- instantiation table -----------------------------------------------------------------------

#define FSAMP_INST_VEC(NT_, CH_) \
  {NT_, CH_, 1, (const void*)fsamp_kernel<NT_, CH_, true>, "fsamp_kernel<" #NT_ "," #CH_ ",vec>"},
#define FSAMP_INST_SCALAR(NT_, CH_) \
  {NT_, CH_, 0, (const void*)fsamp_kernel<NT_, CH_, false>, "fsamp_kernel<" #NT_ "," #CH_ ",elem>"},

const KernelEntry kKernels[] = {FSAMP_KERNEL_LIST_VEC(FSAMP_INST_VEC)
                                    FSAMP_KERNEL_LIST_SCALAR(FSAMP_INST_SCALAR)};
const int kNumKernels = (int)(sizeof(kKernels) / sizeof(kKernels[0]));

#undef FSAMP_INST_VEC
#undef FSAMP_INST_SCALAR

}  // namespace fsamp
