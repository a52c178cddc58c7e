// fsamp_probes.hip -- floor probes that bound the sampler from below on the same instrument
// (csrc/probes.cu:6-125 in the reference): an empty launch, one full argmax pass with one
// workgroup per row, and a split-row argmax pass plus a per-row merge; plus a load-only pass in
// the sampler's B=256 launch shape (no counterpart in the reference).

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>

#include "fsamp.h"
#include "fsamp_wave.h"

namespace {

__device__ __forceinline__ uint32_t key16(uint32_t b) {
  return (b & 0x8000u) ? ((0x10000u - b) & 0xFFFFu) : (b | 0x8000u);
}

__device__ __forceinline__ uint64_t pack(uint32_t key, uint32_t id) {
  return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - id);
}

__global__ void noop_kernel(int64_t* __restrict__ out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = 0;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// One 16-byte load with the nontemporal hint, as the sampler loads its logits.
__device__ __forceinline__ uint4 load_stream16(const uint4* a) {
  const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a));
  return make_uint4(r.x, r.y, r.z, r.w);
}

// Vector loads a thread issues before it reduces any of them: a full row of 151,936 16-bit
// logits is 18,992 vectors, so a 1024-thread workgroup covers it in one batch.
constexpr int SCAN_BATCH = 19;

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Two 16-bit floats -> two order keys (the map of key16, per half, with packed 16-bit ops):
// a negative half b becomes 0x10000 - b = (b ^ 0xFFFF) + 1, which never carries out of its
// half; a non-negative one becomes b | 0x8000.
__device__ __forceinline__ uint32_t keys2(uint32_t w) {
  const s16x2 v = __builtin_bit_cast(s16x2, w);
  const uint32_t su = __builtin_bit_cast(uint32_t, v >> (s16x2)(15));
  return (w ^ (su | 0x80008000u)) + (su & 0x00010001u);
}

__device__ __forceinline__ uint32_t pkmax(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a),
                                                                __builtin_bit_cast(u16x2, b)));
}

// max of (key, ~id) over [lo, hi) of one row, one thread's share.  The vector path keeps a
// batch of vectors as packed keys and takes their maximum with packed 16-bit maxima (about two
// operations per element, overlapped with the loads still in flight); only a batch that
// raises the thread's maximum is searched for the lowest index holding it.  Later batches
// hold higher indices, so an equal maximum there never wins.
__device__ __forceinline__ uint64_t scan_range(const uint16_t* __restrict__ row, int lo, int hi,
                                               int vec) {
  uint64_t best = 0;
  if (vec) {
    const int vlo = lo >> 3, vhi = hi >> 3;  // lo, hi multiples of 8 except the row end
    const uint4* rv = reinterpret_cast<const uint4*>(row);
    const int step = (int)blockDim.x;
    uint32_t best_key = 0, best_id = 0;  // key 0: nothing seen (every real value has key >= 1)
    for (int i0 = vlo + (int)threadIdx.x; i0 < vhi; i0 += SCAN_BATCH * step) {
      uint32_t k[SCAN_BATCH][4];
#pragma unroll
      for (int b = 0; b < SCAN_BATCH; ++b) {
        const int i = i0 + b * step;
        const uint4 v = i < vhi ? load_stream16(rv + i) : make_uint4(0u, 0u, 0u, 0u);
        k[b][0] = v.x;
        k[b][1] = v.y;
        k[b][2] = v.z;
        k[b][3] = v.w;
      }
      uint32_t mb[SCAN_BATCH];
      uint32_t bmax = 0;
#pragma unroll
      for (int b = 0; b < SCAN_BATCH; ++b) {
        const bool in = i0 + b * step < vhi;  // vectors past the row stay key 0
#pragma unroll
        for (int q = 0; q < 4; ++q) k[b][q] = in ? keys2(k[b][q]) : 0u;
        const uint32_t m2 = pkmax(pkmax(k[b][0], k[b][1]), pkmax(k[b][2], k[b][3]));
        mb[b] = max(m2 & 0xFFFFu, m2 >> 16);
        bmax = max(bmax, mb[b]);
      }
      if (bmax > best_key) {
        // the first vector of the batch that holds bmax (scanning down leaves the first),
        // then the first of its eight elements that does
        int fb = 0;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int b = SCAN_BATCH - 1; b >= 0; --b) {
          if (mb[b] == bmax) {
            fb = b;
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = k[b][q];
          }
        }
        int j = 0;
#pragma unroll
        for (int e = 7; e >= 0; --e) {
          const uint32_t key = (e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu);
          if (key == bmax) j = e;
        }
        best_key = bmax;
        best_id = (uint32_t)((i0 + fb * step) * 8 + j);
      }
    }
    if (best_key != 0u) best = pack(best_key, best_id);
    for (int i = vhi * 8 + (int)threadIdx.x; i < hi; i += blockDim.x) {
      const uint64_t a = pack(key16(row[i]), (uint32_t)i);
      best = a > best ? a : best;
    }
  } else {
    for (int i = lo + (int)threadIdx.x; i < hi; i += blockDim.x) {
      const uint64_t a = pack(key16(row[i]), (uint32_t)i);
      best = a > best ? a : best;
    }
  }
  return best;
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t* smem) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) {
    const uint64_t o = __shfl_xor(v, d, 64);
    v = o > v ? o : v;
  }
  if (lane == 0) smem[wid] = v;
  __syncthreads();
  if (wid == 0) {
    uint64_t x = lane < nw ? smem[lane] : 0ull;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
      const uint64_t o = __shfl_xor(x, d, 64);
      x = o > x ? o : x;
    }
    if (lane == 0) smem[0] = x;
  }
  __syncthreads();
  return smem[0];
}

__global__ __launch_bounds__(1024) void scan_rowblock_kernel(const uint16_t* __restrict__ x,
                                                             int64_t* __restrict__ out, int V,
                                                             int vec) {
  __shared__ uint64_t smem[16];
  const uint16_t* row = x + (size_t)blockIdx.x * V;
  const uint64_t best = block_max_u64(scan_range(row, 0, V, vec), smem);
  if (threadIdx.x == 0) out[blockIdx.x] = (int64_t)(0xFFFFFFFFu - (uint32_t)best);
}

__global__ __launch_bounds__(256) void scan_split_kernel(const uint16_t* __restrict__ x,
                                                         uint64_t* __restrict__ partial, int V,
                                                         int S, int slice, int vec) {
  __shared__ uint64_t smem[16];
  const int s = blockIdx.x % S, r = blockIdx.x / S;
  const uint16_t* row = x + (size_t)r * V;
  const int lo = std::min(s * slice, V), hi = std::min(lo + slice, V);
  const uint64_t best = block_max_u64(scan_range(row, lo, hi, vec), smem);
  if (threadIdx.x == 0) partial[(size_t)r * S + s] = best;
}

__global__ __launch_bounds__(64) void merge_partial_kernel(const uint64_t* __restrict__ partial,
                                                           int64_t* __restrict__ out, int S) {
  __shared__ uint64_t smem[16];
  uint64_t best = 0;
  for (int i = threadIdx.x; i < S; i += blockDim.x) {
    const uint64_t v = partial[(size_t)blockIdx.x * S + i];
    best = v > best ? v : best;
  }
  best = block_max_u64(best, smem);
  if (threadIdx.x == 0) out[blockIdx.x] = (int64_t)(0xFFFFFFFFu - (uint32_t)best);
}

// Pure streaming read of a whole batch, the read floor of the memory system with no row shape:
// workgroup g of STREAM_NT threads reads the STREAM_NT * STREAM_U vectors from
// g * STREAM_NT * STREAM_U on (thread t: vectors + u * STREAM_NT + t, all loads at once,
// nontemporal), turns them into order keys and writes each wave's largest key to
// wave_max[g * (STREAM_NT / 64) + w].  Thousands of short workgroups let the dispatcher hand
// the next block to whichever CU is free, so no CU waits on a late share of the batch.  On
// MI355X 256 x 4 measured best of the block sizes tried (256 or 1024 threads, 4 to 32 loads).
constexpr int STREAM_NT = 256, STREAM_U = 4;

__global__ __launch_bounds__(STREAM_NT) void stream_read_kernel(const uint4* __restrict__ x,
                                                                int64_t nvec,
                                                                uint32_t* __restrict__ wave_max) {
  const int64_t base = (int64_t)blockIdx.x * (STREAM_NT * STREAM_U) + threadIdx.x;
  uint4 v[STREAM_U];
#pragma unroll
  for (int u = 0; u < STREAM_U; ++u) v[u] = load_stream16(x + min(base + (int64_t)u * STREAM_NT, nvec - 1));
  uint32_t m = 0;
#pragma unroll
  for (int u = 0; u < STREAM_U; ++u)
    m = pkmax(m, pkmax(pkmax(keys2(v[u].x), keys2(v[u].y)), pkmax(keys2(v[u].z), keys2(v[u].w))));
  // the wave's maximum by DPP / permlane exchanges (no LDS round trip in a short workgroup)
  uint32_t mk = max(m & 0xFFFFu, m >> 16);
  mk = max(mk, fsamp::xor_lane<1>(mk));
  mk = max(mk, fsamp::xor_lane<2>(mk));
  mk = max(mk, fsamp::xor_lane<4>(mk));
  mk = max(mk, fsamp::xor_lane<8>(mk));
  mk = max(mk, fsamp::xor_lane<16>(mk));
  mk = max(mk, fsamp::xor_lane<32>(mk));
  if ((threadIdx.x & 63) == 0)
    wave_max[(size_t)blockIdx.x * (STREAM_NT / 64) + (threadIdx.x >> 6)] = mk;
}

// Load-only floor of the sampler's B=256 launch shape: one 512-thread workgroup per row, every
// thread reads its LOAD_CH nontemporal dwordx4 chunks (chunk c of thread t at vector c*512 + t,
// as the sampler lays its slice out) the way the sampler issues them -- LOAD_DEPTH loads in
// flight, chunk c converted to packed order keys before load c + LOAD_DEPTH is issued -- and
// keeps every converted chunk in registers to the end, as the sampler does; each wave then writes
// the maximum key of its share (no barrier, no LDS), so the kernel's time is the row read itself
// plus the launch.
constexpr int LOAD_NT = 512, LOAD_CH = 38, LOAD_DEPTH = 6;

__global__ __launch_bounds__(LOAD_NT) void load_rows_kernel(const uint16_t* __restrict__ x,
                                                            uint32_t* __restrict__ wave_max,
                                                            int V) {
  const uint4* rv = reinterpret_cast<const uint4*>(x + (size_t)blockIdx.x * V);
  const int nvec = V >> 3;
  const int t = threadIdx.x;
  uint32_t k[LOAD_CH][4];
  auto load = [&](int c) {
    const uint4 v = load_stream16(rv + min(c * LOAD_NT + t, nvec - 1));
    k[c][0] = v.x;
    k[c][1] = v.y;
    k[c][2] = v.z;
    k[c][3] = v.w;
  };
#pragma unroll
  for (int c = 0; c < LOAD_DEPTH; ++c) load(c);
  uint32_t m = 0;
#pragma unroll
  for (int c = 0; c < LOAD_CH; ++c) {
    __builtin_amdgcn_sched_barrier(0);
    const bool in = c * LOAD_NT + t < nvec;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      k[c][q] = in ? keys2(k[c][q]) : 0u;
      m = pkmax(m, k[c][q]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (c + LOAD_DEPTH < LOAD_CH) load(c + LOAD_DEPTH);
  }
  // every converted key stays live to here, as the sampler keeps its slice
  uint32_t live = 0;
#pragma unroll
  for (int c = 0; c < LOAD_CH; ++c) live ^= k[c][0] ^ k[c][1] ^ k[c][2] ^ k[c][3];
  asm volatile("" ::"v"(live));
  uint32_t mk = max(m & 0xFFFFu, m >> 16);
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) mk = max(mk, (uint32_t)__shfl_xor((int)mk, d, 64));
  if ((t & 63) == 0) wave_max[(size_t)blockIdx.x * (LOAD_NT / 64) + (t >> 6)] = mk;
}

int check(int dtype, int64_t B, int64_t V) {
  if (dtype != FSAMP_DTYPE_F16 && dtype != FSAMP_DTYPE_BF16) return FSAMP_ERR_DTYPE;
  if (B < 1 || V < 1 || V > (int64_t)0x7FFFFFF0 || B > (int64_t)0x7FFFFFFF) return FSAMP_ERR_SHAPE;
  return FSAMP_OK;
}

}  // namespace

extern "C" {

int fsamp_probe_noop(int64_t B, int64_t* out, hipStream_t stream) {
  if (B < 1) return FSAMP_ERR_SHAPE;
  if (out == nullptr) return FSAMP_ERR_NULL;
  hipLaunchKernelGGL(noop_kernel, dim3((unsigned)((B + 31) / 32)), dim3(32), 0, stream, out, (int)B);
  return hipGetLastError() == hipSuccess ? FSAMP_OK : FSAMP_ERR_LAUNCH;
}

int fsamp_probe_scan_rowblock(const void* logits, int dtype, int64_t B, int64_t V,
                              int64_t* out, hipStream_t stream) {
  const int rc = check(dtype, B, V);
  if (rc != FSAMP_OK) return rc;
  if (logits == nullptr || out == nullptr) return FSAMP_ERR_NULL;
  const int vec = ((uintptr_t)logits % 16 == 0) && (V % 8 == 0);
  hipLaunchKernelGGL(scan_rowblock_kernel, dim3((unsigned)B), dim3(1024), 0, stream,
                     static_cast<const uint16_t*>(logits), out, (int)V, vec);
  return hipGetLastError() == hipSuccess ? FSAMP_OK : FSAMP_ERR_LAUNCH;
}

int fsamp_probe_load(const void* logits, int dtype, int64_t B, int64_t V, uint32_t* wave_max,
                     hipStream_t stream) {
  const int rc = check(dtype, B, V);
  if (rc != FSAMP_OK) return rc;
  if (logits == nullptr || wave_max == nullptr) return FSAMP_ERR_NULL;
  if ((uintptr_t)logits % 16 != 0 || V % 8 != 0 || V > (int64_t)LOAD_NT * LOAD_CH * 8)
    return FSAMP_ERR_VOCAB;
  hipLaunchKernelGGL(load_rows_kernel, dim3((unsigned)B), dim3(LOAD_NT), 0, stream,
                     static_cast<const uint16_t*>(logits), wave_max, (int)V);
  return hipGetLastError() == hipSuccess ? FSAMP_OK : FSAMP_ERR_LAUNCH;
}

int64_t fsamp_probe_stream_words(int64_t B, int64_t V) {
  if (B < 1 || V < 1) return 0;
  const int64_t nvec = B * V / 8;
  return (nvec + STREAM_NT * STREAM_U - 1) / (STREAM_NT * STREAM_U) * (STREAM_NT / 64);
}

int fsamp_probe_stream(const void* logits, int dtype, int64_t B, int64_t V, uint32_t* wave_max,
                       int64_t n_words, hipStream_t stream) {
  const int rc = check(dtype, B, V);
  if (rc != FSAMP_OK) return rc;
  if (logits == nullptr || wave_max == nullptr) return FSAMP_ERR_NULL;
  if ((uintptr_t)logits % 16 != 0 || V % 8 != 0) return FSAMP_ERR_VOCAB;
  if (n_words < fsamp_probe_stream_words(B, V)) return FSAMP_ERR_WORKSPACE;
  const int64_t nvec = B * V / 8;
  const int64_t grid = (nvec + STREAM_NT * STREAM_U - 1) / (STREAM_NT * STREAM_U);
  if (grid > 0x7FFFFFFF) return FSAMP_ERR_SHAPE;
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(STREAM_NT), 0, stream,
                     static_cast<const uint4*>(logits), nvec, wave_max);
  return hipGetLastError() == hipSuccess ? FSAMP_OK : FSAMP_ERR_LAUNCH;
}

int fsamp_probe_scan_split(const void* logits, int dtype, int64_t B, int64_t V, int64_t splits,
                           int64_t* out, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int rc = check(dtype, B, V);
  if (rc != FSAMP_OK) return rc;
  if (splits < 1) return FSAMP_ERR_SPLITS;
  if (logits == nullptr || out == nullptr) return FSAMP_ERR_NULL;
  const int vec = ((uintptr_t)logits % 16 == 0) && (V % 8 == 0);
  const int units = (int)((V + 7) / 8);
  const int S = (int)std::min<int64_t>(splits, units);
  const int slice = ((units + S - 1) / S) * 8;
  if (ws == nullptr || ws_bytes < (size_t)B * (size_t)S * 8u) return FSAMP_ERR_WORKSPACE;
  uint64_t* partial = static_cast<uint64_t*>(ws);
  hipLaunchKernelGGL(scan_split_kernel, dim3((unsigned)(B * S)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(logits), partial, (int)V, S, slice, vec);
  if (hipGetLastError() != hipSuccess) return FSAMP_ERR_LAUNCH;
  hipLaunchKernelGGL(merge_partial_kernel, dim3((unsigned)B), dim3(64), 0, stream, partial, out, S);
  return hipGetLastError() == hipSuccess ? FSAMP_OK : FSAMP_ERR_LAUNCH;
}

}  // extern "C"
