// fsamp_probes.hip -- floor probes that bound the sampler from below on the same instrument
// (csrc/probes.cu:6-125 in the reference): an empty launch, one full argmax pass with one
// workgroup per row, and a split-row argmax pass plus a per-row merge.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>

#include "fsamp.h"

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

// max of (key, ~id) over [lo, hi) of one row, one thread's share
__device__ __forceinline__ uint64_t scan_range(const uint16_t* __restrict__ row, int lo, int hi,
                                               int vec) {
  uint64_t best = 0;
  if (vec) {
    const int vlo = lo >> 3, vhi = hi >> 3;  // lo, hi multiples of 8 except the row end
    const uint4* rv = reinterpret_cast<const uint4*>(row);
    for (int i = vlo + (int)threadIdx.x; i < vhi; i += blockDim.x) {
      const uint4 v = rv[i];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t a = pack(key16(w[q] & 0xFFFFu), (uint32_t)(i * 8 + 2 * q));
        const uint64_t b = pack(key16(w[q] >> 16), (uint32_t)(i * 8 + 2 * q + 1));
        best = a > best ? a : best;
        best = b > best ? b : best;
      }
    }
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
