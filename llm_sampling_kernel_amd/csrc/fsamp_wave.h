// fsamp_wave.h -- wave64 cross-lane primitives for gfx950 built on DPP, ds_swizzle and
// ds_bpermute, shared by the sampler kernel and its lane-layout tests.
//
// DPP moves (__builtin_amdgcn_update_dpp) are VALU operations with a few cycles of latency;
// ds_swizzle and ds_bpermute (what __shfl_* compiles to) round-trip through the LDS crossbar.
// The sorting networks and scans here sit on the critical path of a call, so each lane
// distance uses the cheapest form gfx950 has, all of them VALU:
//   xor 1, 2   quad_perm                      xor 8   row_ror:8 (a 16-lane row rotated by 8)
//   xor 4      row_shl:4 / row_shr:4 + select xor 16  v_permlane16_swap + select
//   xor 32     v_permlane32_swap + select
// and the inclusive scan uses row_shr:1,2,4,8 inside 16-lane rows, then row_bcast:15 and
// row_bcast:31 across rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fsamp {

// DPP control words (GFX9 encoding)
constexpr int DPP_QUAD_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int DPP_ROW_SHL4 = 0x104;
constexpr int DPP_ROW_SHR1 = 0x111;
constexpr int DPP_ROW_SHR2 = 0x112;
constexpr int DPP_ROW_SHR4 = 0x114;
constexpr int DPP_ROW_SHR8 = 0x118;
constexpr int DPP_ROW_ROR8 = 0x128;
constexpr int DPP_WAVE_SHR1 = 0x138;
constexpr int DPP_ROW_BCAST15 = 0x142;
constexpr int DPP_ROW_BCAST31 = 0x143;

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }

// value of lane (l ^ J) for J in {1, 2, 4, 8, 16, 32}.  The DPP moves leave no lane without
// a source (quad permutes and row rotates), or only lanes whose result the select below
// discards (row_shl:4 / row_shr:4), so they need no defined "old" value (mov_dpp).
template <int J>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  const int x = (int)v;
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(x, DPP_QUAD_XOR1, 0xF, 0xF, false);
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(x, DPP_QUAD_XOR2, 0xF, 0xF, false);
  } else if constexpr (J == 4) {
    const int up = __builtin_amdgcn_mov_dpp(x, DPP_ROW_SHL4, 0xF, 0xF, false);
    const int dn = __builtin_amdgcn_mov_dpp(x, DPP_ROW_SHR4, 0xF, 0xF, false);
    return (uint32_t)((lane_id() & 4) ? dn : up);
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp(x, DPP_ROW_ROR8, 0xF, 0xF, false);
  } else if constexpr (J == 16) {
    // swap(v, v): result[0] (vdst) has the even 16-lane rows' values in the odd rows,
    // result[1] (vsrc) the odd rows' values in the even rows
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane_id() & 16) ? r[0] : r[1];
  } else {
    static_assert(J == 32, "lane distance");
    // the same with the two 32-lane halves
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane_id() & 32) ? r[0] : r[1];
  }
}

template <int J>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
  const uint32_t lo = xor_lane<J>((uint32_t)v);
  const uint32_t hi = xor_lane<J>((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// One compare-exchange stage of a descending bitonic network over 64 lanes: block size K,
// partner distance J.  Within a K-block the direction alternates so that the final K=64
// merge leaves lane 0 with the largest value.  A lane keeps the larger of (own, partner)
// when it is the lower lane of a descending block or the upper lane of an ascending one.
//   For 32-bit values max and min are single VALU ops and the lane-constant select follows
// (no scalar step in the dependency chain); for 64-bit values one compare, xor-ed with the
// lane-constant predicate, picks the partner or not.
template <int K, int J, typename T, bool ASC = false>
__device__ __forceinline__ T bitonic_step(T v) {
  const int l = lane_id();
  const bool keep_hi = (((l & J) == 0) == ((l & K) == 0)) != ASC;
  if constexpr (sizeof(T) == 8) {
    const T o = (T)xor_lane64<J>((uint64_t)v);
    return ((o > v) == keep_hi) ? o : v;
  } else {
    const T o = (T)xor_lane<J>((uint32_t)v);
    const T hi = v > o ? v : o, lo = v > o ? o : v;
    return keep_hi ? hi : lo;
  }
}

template <int K, int J, typename T, bool ASC = false>
__device__ __forceinline__ T bitonic_merge_stages(T v) {
  v = bitonic_step<K, J, T, ASC>(v);
  if constexpr (J > 1) v = bitonic_merge_stages<K, J / 2, T, ASC>(v);
  return v;
}

template <int K, typename T, bool ASC = false>
__device__ __forceinline__ T bitonic_levels(T v) {
  if constexpr (K > 2) v = bitonic_levels<K / 2, T, ASC>(v);
  return bitonic_merge_stages<K, K / 2, T, ASC>(v);
}

// Full descending sort of one value per lane (64 values): lane 0 gets the largest.
template <typename T>
__device__ __forceinline__ T wave_sort_desc(T v) {
  return bitonic_levels<64, T>(v);
}

// Full ascending sort of one value per lane (every comparator mirrored): lane 0 the smallest.
template <typename T>
__device__ __forceinline__ T wave_sort_asc(T v) {
  return bitonic_levels<64, T, true>(v);
}

// The descending top 64 of two lists of 64 values, one of each per lane: a sorted descending,
// b ascending, the elementwise maximum is a bitonic sequence holding exactly the 64 largest of
// both, and the six half-cleaner stages of the last bitonic level sort it.
template <typename T>
__device__ __forceinline__ T wave_top64_of_two(T a, T b) {
  a = wave_sort_desc<T>(a);
  b = wave_sort_asc<T>(b);
  const T m = a > b ? a : b;
  return bitonic_merge_stages<64, 32, T>(m);
}

// Inclusive prefix sum over the 64 lanes in a fixed association: Kogge-Stone inside each
// 16-lane row (distances 1, 2, 4, 8; lane i of a row adds lane i-d when i >= d), then row 1
// and row 3 add the last lane of the row below (row_bcast:15), then rows 2 and 3 add lane 31
// (row_bcast:31).  Every add is x_{src} + x_{own} with the source read before the step.
__device__ __forceinline__ float wave_incl_scan_f32(float v) {
  int x = __float_as_int(v);
  x = __float_as_int(__int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR1, 0xF, 0xF, true)) + __int_as_float(x));
  x = __float_as_int(__int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR2, 0xF, 0xF, true)) + __int_as_float(x));
  x = __float_as_int(__int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR4, 0xF, 0xF, true)) + __int_as_float(x));
  x = __float_as_int(__int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR8, 0xF, 0xF, true)) + __int_as_float(x));
  x = __float_as_int(__int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_ROW_BCAST15, 0xA, 0xF, false)) + __int_as_float(x));
  x = __float_as_int(__int_as_float(__builtin_amdgcn_update_dpp(0, x, DPP_ROW_BCAST31, 0xC, 0xF, false)) + __int_as_float(x));
  return __int_as_float(x);
}

// Value of lane l-1 (0 for lane 0).
__device__ __forceinline__ float wave_shr1_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_WAVE_SHR1, 0xF, 0xF, true));
}

// Uniform value of lane `l` (l uniform).
__device__ __forceinline__ float read_lane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__device__ __forceinline__ uint32_t read_lane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}

}  // namespace fsamp

namespace fsamp {

// Inclusive prefix sum of unsigned integers over the 64 lanes (same DPP structure as the fp32
// scan; integer adds, so the association does not matter).
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  int x = (int)v;
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR1, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR2, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR4, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_SHR8, 0xF, 0xF, true);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_BCAST15, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, DPP_ROW_BCAST31, 0xC, 0xF, false);
  return (uint32_t)x;
}

// ---- register sorting networks over 64*R u64 words, blocked layout ------------------------
// Lane l holds elements e = l*R + i, i < R.  A stage compares e with e ^ J; within a block of
// K elements the direction is descending when (e & K) == 0, so a full network leaves element 0
// (lane 0, i = 0) with the largest word.  Distances J < R stay inside a lane; larger ones pair
// lane l with lane l ^ (J / R).

template <int R, int K, int J, bool ASC = false>
__device__ __forceinline__ void net_stage(uint64_t (&v)[R]) {
  const int l = lane_id();
  if constexpr (J < R) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if ((i & J) == 0) {
        const bool desc = (((l * R + i) & K) == 0) != ASC;
        const uint64_t a = v[i], b = v[i + J];
        if ((a < b) == desc) {
          v[i] = b;
          v[i + J] = a;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint64_t o = xor_lane64<J / R>(v[i]);
      const int e = l * R + i;
      const bool keep_hi = ((e & J) == 0) == (((e & K) == 0) != ASC);
      v[i] = ((o > v[i]) == keep_hi) ? o : v[i];
    }
  }
}

template <int R, int K, int J, bool ASC = false>
__device__ __forceinline__ void net_merge(uint64_t (&v)[R]) {
  net_stage<R, K, J, ASC>(v);
  if constexpr (J > 1) net_merge<R, K, J / 2, ASC>(v);
}

template <int R, int K, bool ASC = false>
__device__ __forceinline__ void net_sort_levels(uint64_t (&v)[R]) {
  if constexpr (K > 2) net_sort_levels<R, K / 2, ASC>(v);
  net_merge<R, K, K / 2, ASC>(v);
}

// Full descending sort of the 64*R words.
template <int R>
__device__ __forceinline__ void wave_sort_desc_n(uint64_t (&v)[R]) {
  net_sort_levels<R, 64 * R>(v);
}

// Full ascending sort of the 64*R words (every comparator mirrored): element 0 is the
// smallest, which is the reversed layout wave_merge_top takes for its second list.
template <int R>
__device__ __forceinline__ void wave_sort_asc_n(uint64_t (&v)[R]) {
  net_sort_levels<R, 64 * R, true>(v);
}

// v holds a descending list A; b_rev holds a descending list B with element e stored at
// position 64R-1-e.  Leaves v with the descending top 64R of A and B: the elementwise maximum
// of A and reversed B is a bitonic sequence holding exactly those words; half-cleaners sort it.
template <int R>
__device__ __forceinline__ void wave_merge_top(uint64_t (&v)[R], const uint64_t (&b_rev)[R]) {
#pragma unroll
  for (int i = 0; i < R; ++i) v[i] = v[i] > b_rev[i] ? v[i] : b_rev[i];
  net_merge<R, 64 * R, 32 * R>(v);
}

}  // namespace fsamp
