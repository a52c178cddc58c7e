/*
 * fsamp_oracle.c -- CPU restatement of the reference sampler's semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and the product
 * path (llm_sampling_kernel_amd) never calls it.  It is a from-scratch restatement of
 *
 *   benchmarks/reference.py:29-81   sample_eager: stable descending sort -> [:k] -> softmax
 *                                    -> cumsum -> keep=(cumsum-probs)<top_p (all if top_p>=1)
 *                                    -> renorm -> draw
 *   benchmarks/reference.py:20-26   validate_logits (NaN / +inf / all -inf row)
 *   benchmarks/SEMANTICS.md:143-241 stage order, lowest-id tie rule, exclusive-prefix cut,
 *                                    top_p>=1 keeps all, inverse-CDF draw equivalence
 *   csrc/fused_sampling.cu:276-309  normalize-then-prefix cut, Z_p = c_r, draw u*Z_p
 *   csrc/fused_sampling.cuh:65-71   splitmix64 uniform for the (seed, offset, row) API
 *
 * with the draw made explicit: instead of torch.multinomial (reference.py:67) the caller
 * passes one uniform u in [0,1) per row and the token is the first kept rank i with
 * c_i >= u * Z_p (SEMANTICS.md:228-236 states that this is the same distribution).
 *
 * Floating point.  reference.py leaves the fp32 rounding of softmax and cumsum to torch,
 * whose summation order is unspecified.  This restatement fixes one order so that the GPU
 * kernel can be compared with it bit for bit:
 *   - exp is oracle_expf() below: Cody-Waite reduction by ln2 plus a degree-7 Taylor polynomial,
 *     evaluated with fmaf; inputs below -86 give exactly 0 (e^-86 < 2^-124);
 *   - the K survivors are dealt to 64 "lanes" in blocks of R = ceil(K/64); per-lane sums are
 *     serial; the 64 lane values are combined by one fixed inclusive scan (lane_scan below:
 *     Kogge-Stone over distances 1,2,4,8 inside 16-lane rows, then rows 1 and 3 add the last
 *     lane of the row below, then rows 2 and 3 add lane 31); z is the scan total of the w
 *     sums, the prefix c is the exclusive scan offset of the p sums followed by per-lane
 *     serial accumulation.
 * Against the torch fp32 computation this differs only by rounding; tests pin it against an
 * fp64 restatement (oracle_stages_f64) and the reference's closed-form cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { OR_F16 = 0, OR_BF16 = 1, OR_F32 = 2 };
enum { OR_OK = 0, OR_NAN = 1, OR_POSINF = 2, OR_ALLNEGINF = 3, OR_BADARG = 4, OR_NOMEM = 5 };

#define OR_LANES 64

/* ---- element decoding ------------------------------------------------------------------ */

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t man = h & 0x3FFu;
  float f;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in fp32 */
    f = ldexpf((float)man, -24);
    if (sign) f = -f;
    return f;
  }
  uint32_t u;
  if (exp == 0x1F) {
    u = sign | 0x7F800000u | (man << 13);
  } else {
    u = sign | ((exp + 112u) << 23) | (man << 13);
  }
  memcpy(&f, &u, 4);
  return f;
}

float oracle_to_float(uint16_t b, int dtype) {
  return dtype == OR_BF16 ? bf16_to_f32(b) : f16_to_f32(b);
}

/* Order key of a 16-bit float: descending value <=> descending key, -0 and +0 share a key,
 * so that equal values (reference.py:53 sorts values, and -0 == +0 there) tie and the tie is
 * decided by the token id alone.  Keys of real values are >= 1. */
uint32_t oracle_key16(uint16_t b) {
  return (b & 0x8000u) ? ((0x10000u - b) & 0xFFFFu) : (uint32_t)(b | 0x8000u);
}

/* ---- exp ------------------------------------------------------------------------------- */

/* e^x for x <= 0 (the only range the sampler needs: x = logit - max).
 * Cody-Waite: x = n*ln2 + r with n = rint(x*log2(e)), |r| <= ln2/2, ln2 split in a 16-bit
 * head (n*head is exact) and a tail; e^r by its Taylor series to r^7/7! (truncation error
 * < 4e-9 relative); the result is scaled by 2^n built from exponent bits. */
float oracle_expf(float x) {
  if (!(x >= -86.0f)) return 0.0f; /* also -inf and NaN */
  const float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.42860682030941723e-6f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n; /* in [-124, 0] */
  const uint32_t sb = (uint32_t)(ni + 127) << 23;
  float s;
  memcpy(&s, &sb, 4);
  return p * s;
}

/* ---- splitmix64 uniform (csrc/fused_sampling.cuh:65-71) -------------------------------- */

/* splitmix64's finalizer (Steele, Lea, Flood 2014; constants as published) applied to
 * seed + offset*golden64 + row*C, top 24 bits as a uniform in [0, 1). */
float oracle_rng_uniform(uint64_t seed, uint64_t offset, uint32_t row) {
  uint64_t z = seed + offset * 0x9E3779B97F4A7C15ull + (uint64_t)row * 0xD1B54A32D192ED03ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z = z ^ (z >> 31);
  return (float)((z >> 40) & 0xFFFFFFull) * (1.0f / 16777216.0f);
}

/* plain splitmix64 next(), used by the tests to check the mixing constants against the
 * generator's published output sequence */
uint64_t oracle_splitmix64_next(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* ---- validation (reference.py:20-26) --------------------------------------------------- */

int oracle_validate(const void* logits, int dtype, int64_t B, int64_t V) {
  if (B < 0 || V < 1 || (dtype != OR_F16 && dtype != OR_BF16 && dtype != OR_F32)) return OR_BADARG;
  int saw_posinf = 0, saw_allneg = 0;
  for (int64_t b = 0; b < B; ++b) {
    int64_t n_neginf = 0;
    for (int64_t i = 0; i < V; ++i) {
      float f = dtype == OR_F32 ? ((const float*)logits)[b * V + i]
                                : oracle_to_float(((const uint16_t*)logits)[b * V + i], dtype);
      if (isnan(f)) return OR_NAN;
      if (isinf(f)) {
        if (f > 0) saw_posinf = 1;
        else ++n_neginf;
      }
    }
    if (n_neginf == V) saw_allneg = 1;
  }
  if (saw_posinf) return OR_POSINF;
  if (saw_allneg) return OR_ALLNEGINF;
  return OR_OK;
}

/* ---- stable descending sort (reference.py:50-54) --------------------------------------- */

/* Full stable descending order of a 16-bit row: a counting sort on the order key, scanning
 * ids in ascending order so equal values keep ascending ids (torch.sort(stable=True)). */
static void stable_desc_order16(const uint16_t* row, int64_t V, uint32_t* counts /*65536*/,
                                int32_t* order) {
  memset(counts, 0, 65536 * sizeof(uint32_t));
  for (int64_t i = 0; i < V; ++i) counts[oracle_key16(row[i])]++;
  uint32_t acc = 0;
  for (int k = 65535; k >= 0; --k) {
    const uint32_t c = counts[k];
    counts[k] = acc;
    acc += c;
  }
  for (int64_t i = 0; i < V; ++i) order[counts[oracle_key16(row[i])]++] = (int32_t)i;
}

typedef struct {
  float v;
  int32_t id;
} vid_t;

static int cmp_vid_desc(const void* a, const void* b) {
  const vid_t* x = (const vid_t*)a;
  const vid_t* y = (const vid_t*)b;
  if (x->v > y->v) return -1;
  if (x->v < y->v) return 1;
  return (x->id > y->id) - (x->id < y->id);
}

/* fp32 rows (the reference tests' own closed-form cases use fp32 logits) */
static void stable_desc_order32(const float* row, int64_t V, vid_t* tmp, int32_t* order) {
  for (int64_t i = 0; i < V; ++i) {
    tmp[i].v = row[i];
    tmp[i].id = (int32_t)i;
  }
  qsort(tmp, (size_t)V, sizeof(vid_t), cmp_vid_desc);
  for (int64_t i = 0; i < V; ++i) order[i] = tmp[i].id;
}

/* The reference's own form of the selection, reference.py:48-54: the row converted to fp32
 * (x.to(float32)) and fully sorted, descending, by a stable sort -- here a bottom-up merge
 * sort of (value, id) pairs, O(V log V).  Runs are merged taking the left element while it is
 * not smaller, so equal values (and -0 == +0, as fp32 compares them) keep ascending ids.  Used
 * for the CPU baseline in the reference's form and to cross-check the counting sort above. */
static void stable_desc_order_merge(vid_t* a, vid_t* b, int64_t V, int32_t* order) {
  vid_t* src = a;
  vid_t* dst = b;
  for (int64_t w = 1; w < V; w <<= 1) {
    for (int64_t lo = 0; lo < V; lo += 2 * w) {
      const int64_t mid = lo + w < V ? lo + w : V;
      const int64_t hi = lo + 2 * w < V ? lo + 2 * w : V;
      int64_t i = lo, j = mid, o = lo;
      while (i < mid && j < hi) dst[o++] = (src[i].v >= src[j].v) ? src[i++] : src[j++];
      while (i < mid) dst[o++] = src[i++];
      while (j < hi) dst[o++] = src[j++];
    }
    vid_t* t = src;
    src = dst;
    dst = t;
  }
  for (int64_t i = 0; i < V; ++i) order[i] = src[i].id;
}

/* ---- fp32 tail in the fixed lane order --------------------------------------------------- */

typedef struct {
  int64_t pick;  /* rank of the drawn candidate */
  int64_t r;     /* last kept rank */
} tail_out_t;

/* Inclusive prefix of 64 lane values in the sampler's association: Kogge-Stone inside each
 * 16-lane row (lane i of a row adds lane i-d for d = 1, 2, 4, 8 when i >= d), then rows 1 and
 * 3 add the last lane of the row below, then rows 2 and 3 add lane 31.  Each step reads the
 * values of the previous step; every add is (source lane) + (own lane). */
static void lane_scan(float* v) {
  float nxt[OR_LANES];
  for (int d = 1; d < 16; d <<= 1) {
    for (int l = 0; l < OR_LANES; ++l) nxt[l] = ((l & 15) >= d) ? v[l - d] + v[l] : v[l];
    memcpy(v, nxt, sizeof(nxt));
  }
  for (int l = 0; l < OR_LANES; ++l) {
    const int row = l >> 4;
    nxt[l] = (row == 1 || row == 3) ? v[16 * row - 1] + v[l] : v[l];
  }
  memcpy(v, nxt, sizeof(nxt));
  for (int l = 0; l < OR_LANES; ++l) nxt[l] = (l >= 32) ? v[31] + v[l] : v[l];
  memcpy(v, nxt, sizeof(nxt));
}

/* x: K candidate values, descending.  Writes w (scratch), p, c; returns r and pick.
 * inv_t scales the shifted logits before exp, (x_j - m) * inv_t in fp32 (1 / temperature;
 * exactly 1 without a temperature, which leaves x_j - m unchanged). */
static tail_out_t tail_f32(const float* x, int K, double top_p, float u, float inv_t, float* w,
                           float* p, float* c) {
  const int R = (K + OR_LANES - 1) / OR_LANES;
  float lane_s[OR_LANES];
  const float m = x[0];
  for (int j = 0; j < K; ++j) w[j] = oracle_expf((x[j] - m) * inv_t);

  /* z: per-lane serial sums, combined by the lane scan; z is its last lane */
  for (int l = 0; l < OR_LANES; ++l) {
    float s = 0.0f;
    for (int j = l * R; j < l * R + R && j < K; ++j) s = s + w[j];
    lane_s[l] = s;
  }
  lane_scan(lane_s);
  const float z = lane_s[OR_LANES - 1];
  for (int j = 0; j < K; ++j) p[j] = w[j] / z;

  /* prefix: per-lane serial totals, lane scan, exclusive offsets, serial accumulation */
  for (int l = 0; l < OR_LANES; ++l) {
    float s = 0.0f;
    for (int j = l * R; j < l * R + R && j < K; ++j) s = s + p[j];
    lane_s[l] = s;
  }
  lane_scan(lane_s);
  for (int l = 0; l < OR_LANES; ++l) {
    float acc = (l == 0) ? 0.0f : lane_s[l - 1];
    for (int j = l * R; j < l * R + R && j < K; ++j) {
      acc = acc + p[j];
      c[j] = acc;
    }
  }

  /* cut on the exclusive prefix (reference.py:58-62): keep i iff c_i - p_i < top_p; the
   * kept set is the prefix up to the first dropped rank (rank 0 is always kept) */
  tail_out_t o;
  o.r = K - 1;
  if (top_p < 1.0) {
    const float pf = (float)top_p;
    for (int j = 1; j < K; ++j) {
      if (!((c[j] - p[j]) < pf)) {
        o.r = j - 1;
        break;
      }
    }
  }
  /* inverse-CDF draw against u * Z_p with Z_p = c_r (fused_sampling.cu:294-309) */
  const float target = u * c[o.r];
  o.pick = o.r;
  for (int j = 0; j <= o.r; ++j) {
    if (c[j] >= target) {
      o.pick = j;
      break;
    }
  }
  return o;
}

/* ---- public entry points ------------------------------------------------------------------ */

/*
 * oracle_sample: the whole sampler for B rows.
 *   logits   [B,V] fp16/bf16 bit patterns (uint16) or fp32
 *   u        [B] uniforms in [0,1)
 *   token_ids[B] (required)
 * Optional per-rank stage outputs, each [B,K] with K = min(top_k, V) (NULL to skip):
 *   topk_ids (int64), topk_vals (f32), probs (f32), cumsum (f32), keep (u8), renormed (f32);
 *   cutoff [B] int32 = number of kept ranks.
 * Returns OR_OK or OR_BADARG / OR_NOMEM.  Does not validate values (see oracle_validate).
 */
/*
 * oracle_sample_rows: oracle_sample with per-row controls (each array NULL or [B]), the
 * semantics of fsamp_sample_ex (include/fsamp.h):
 *   topk_row[b]  row b uses the first min(max(topk_row[b], 1), K) ranks of the top-K
 *   topp_row[b]  row b's threshold (fp32); >= 1 keeps every rank of the row
 *   temp_row[b]  inv_t = 1.0f / temp_row[b] scales (x - max) before exp; <= 0 or NaN: greedy
 * Stage outputs stay [B, K] with K = min(top_k, V); ranks past a row's own k are 0, and
 * probs / cumsum there are 0 as well.
 */
static int sample_rows_impl(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                            double top_p, const float* u, const int32_t* topk_row,
                            const float* topp_row, const float* temp_row, int64_t* token_ids,
                            int64_t* topk_ids, float* topk_vals, float* probs, float* cumsum,
                            uint8_t* keep, float* renormed, int32_t* cutoff, int nthreads,
                            int full_sort) {
  if (B < 0 || V < 1 || top_k < 1 || !(top_p > 0.0 && top_p <= 1.0) || u == NULL ||
      token_ids == NULL || (dtype != OR_F16 && dtype != OR_BF16 && dtype != OR_F32))
    return OR_BADARG;
  const int64_t K = top_k < V ? top_k : V;
  int status = OR_OK;
#ifdef _OPENMP
  if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
#endif
  for (int64_t b = 0; b < B; ++b) {
    int32_t* order = (int32_t*)malloc((size_t)V * sizeof(int32_t));
    const int use_counts = dtype != OR_F32 && !full_sort;
    uint32_t* counts = use_counts ? (uint32_t*)malloc(65536 * sizeof(uint32_t)) : NULL;
    vid_t* tmp = use_counts ? NULL : (vid_t*)malloc((size_t)V * 2 * sizeof(vid_t));
    float* x = (float*)malloc((size_t)K * 4 * sizeof(float));
    if (!order || (use_counts && !counts) || (!use_counts && !tmp) || !x) {
      status = OR_NOMEM;
    } else {
      if (full_sort) {
        for (int64_t i = 0; i < V; ++i) {
          tmp[i].v = dtype == OR_F32 ? ((const float*)logits)[b * V + i]
                                     : oracle_to_float(((const uint16_t*)logits)[b * V + i], dtype);
          tmp[i].id = (int32_t)i;
        }
        stable_desc_order_merge(tmp, tmp + V, V, order);
        for (int64_t j = 0; j < K; ++j)
          x[j] = dtype == OR_F32 ? ((const float*)logits)[b * V + order[j]]
                                 : oracle_to_float(((const uint16_t*)logits)[b * V + order[j]], dtype);
      } else if (dtype == OR_F32) {
        const float* row = (const float*)logits + b * V;
        stable_desc_order32(row, V, tmp, order);
        for (int64_t j = 0; j < K; ++j) x[j] = row[order[j]];
      } else {
        const uint16_t* row = (const uint16_t*)logits + b * V;
        stable_desc_order16(row, V, counts, order);
        for (int64_t j = 0; j < K; ++j) x[j] = oracle_to_float(row[order[j]], dtype);
      }
      float* w = x + K;
      float* p = x + 2 * K;
      float* c = x + 3 * K;
      int64_t kr = K;
      double pr = top_p;
      float inv_t = 1.0f;
      if (topk_row) kr = topk_row[b] < 1 ? 1 : (topk_row[b] > K ? K : topk_row[b]);
      if (topp_row) pr = (double)topp_row[b];
      if (temp_row) {
        if (temp_row[b] > 0.0f) inv_t = 1.0f / temp_row[b];
        else kr = 1;
      }
      const tail_out_t o = tail_f32(x, (int)kr, pr, u[b], inv_t, w, p, c);
      token_ids[b] = order[o.pick];
      const float zp = c[o.r];
      for (int64_t j = 0; j < K; ++j) {
        const int64_t at = b * K + j;
        const int in = j < kr;
        if (topk_ids) topk_ids[at] = order[j];
        if (topk_vals) topk_vals[at] = x[j];
        if (probs) probs[at] = in ? p[j] : 0.0f;
        if (cumsum) cumsum[at] = in ? c[j] : 0.0f;
        if (keep) keep[at] = (uint8_t)(in && j <= o.r);
        if (renormed) renormed[at] = in && j <= o.r ? p[j] / zp : 0.0f;
      }
      if (cutoff) cutoff[b] = (int32_t)(o.r + 1);
    }
    free(order);
    free(counts);
    free(tmp);
    free(x);
  }
  return status;
}

int oracle_sample_rows(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                       double top_p, const float* u, const int32_t* topk_row,
                       const float* topp_row, const float* temp_row, int64_t* token_ids,
                       int64_t* topk_ids, float* topk_vals, float* probs, float* cumsum,
                       uint8_t* keep, float* renormed, int32_t* cutoff, int nthreads) {
  return sample_rows_impl(logits, dtype, B, V, top_k, top_p, u, topk_row, topp_row, temp_row,
                          token_ids, topk_ids, topk_vals, probs, cumsum, keep, renormed, cutoff,
                          nthreads, 0);
}

/*
 * oracle_sample_fullsort: oracle_sample with the selection in the reference's own form
 * (reference.py:48-54): each row converted to fp32 and fully sorted by a stable merge sort
 * (stable_desc_order_merge), then the same fp32 tail.  Same outputs as oracle_sample; this is
 * the O(V log V) path the CPU baseline times.
 */
int oracle_sample_fullsort(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                           double top_p, const float* u, int64_t* token_ids, int64_t* topk_ids,
                           int nthreads) {
  return sample_rows_impl(logits, dtype, B, V, top_k, top_p, u, NULL, NULL, NULL, token_ids,
                          topk_ids, NULL, NULL, NULL, NULL, NULL, NULL, nthreads, 1);
}

int oracle_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                  double top_p, const float* u, int64_t* token_ids, int64_t* topk_ids,
                  float* topk_vals, float* probs, float* cumsum, uint8_t* keep,
                  float* renormed, int32_t* cutoff, int nthreads) {
  return oracle_sample_rows(logits, dtype, B, V, top_k, top_p, u, NULL, NULL, NULL, token_ids,
                            topk_ids, topk_vals, probs, cumsum, keep, renormed, cutoff, nthreads);
}

/*
 * oracle_stages_f64: the same pipeline in double precision (softmax, cumsum, cut, renorm),
 * the yardstick the fp32 restatement and the GPU are held to.  topk selection is shared with
 * oracle_sample (integer work, no rounding).  Outputs [B,K] doubles; cutoff [B].
 */
int oracle_stages_f64_t(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                        double top_p, double temperature, double* probs, double* cumsum,
                        double* renormed, int32_t* cutoff) {
  if (B < 0 || V < 1 || top_k < 1 || !(top_p > 0.0 && top_p <= 1.0) ||
      (dtype != OR_F16 && dtype != OR_BF16 && dtype != OR_F32))
    return OR_BADARG;
  const int64_t K = top_k < V ? top_k : V;
  int32_t* order = (int32_t*)malloc((size_t)V * sizeof(int32_t));
  uint32_t* counts = (uint32_t*)malloc(65536 * sizeof(uint32_t));
  vid_t* tmp = (vid_t*)malloc((size_t)V * sizeof(vid_t));
  double* x = (double*)malloc((size_t)K * sizeof(double));
  if (!order || !counts || !tmp || !x) {
    free(order);
    free(counts);
    free(tmp);
    free(x);
    return OR_NOMEM;
  }
  for (int64_t b = 0; b < B; ++b) {
    if (dtype == OR_F32) {
      const float* row = (const float*)logits + b * V;
      stable_desc_order32(row, V, tmp, order);
      for (int64_t j = 0; j < K; ++j) x[j] = row[order[j]];
    } else {
      const uint16_t* row = (const uint16_t*)logits + b * V;
      stable_desc_order16(row, V, counts, order);
      for (int64_t j = 0; j < K; ++j) x[j] = oracle_to_float(row[order[j]], dtype);
    }
    double* p = probs + b * K;
    double* c = cumsum + b * K;
    double z = 0.0;
    for (int64_t j = 0; j < K; ++j) {
      p[j] = exp((x[j] - x[0]) / temperature);
      z += p[j];
    }
    double acc = 0.0;
    for (int64_t j = 0; j < K; ++j) {
      p[j] /= z;
      acc += p[j];
      c[j] = acc;
    }
    int64_t r = K - 1;
    if (top_p < 1.0) {
      for (int64_t j = 1; j < K; ++j) {
        if (!(c[j - 1] < top_p)) {
          r = j - 1;
          break;
        }
      }
    }
    for (int64_t j = 0; j < K; ++j) renormed[b * K + j] = j <= r ? p[j] / c[r] : 0.0;
    cutoff[b] = (int32_t)(r + 1);
  }
  free(order);
  free(counts);
  free(tmp);
  free(x);
  return OR_OK;
}

int oracle_stages_f64(const void* logits, int dtype, int64_t B, int64_t V, int64_t top_k,
                      double top_p, double* probs, double* cumsum, double* renormed,
                      int32_t* cutoff) {
  return oracle_stages_f64_t(logits, dtype, B, V, top_k, top_p, 1.0, probs, cumsum, renormed,
                             cutoff);
}

/* ---- array helpers for the tests ---------------------------------------------------------- */

void oracle_expf_array(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_expf(x[i]);
}

void oracle_key16_array(const uint16_t* b, uint32_t* k, int64_t n) {
  for (int64_t i = 0; i < n; ++i) k[i] = oracle_key16(b[i]);
}

void oracle_rng_uniform_rows(uint64_t seed, uint64_t offset, int64_t B, float* u) {
  for (int64_t b = 0; b < B; ++b) u[b] = oracle_rng_uniform(seed, offset, (uint32_t)b);
}
