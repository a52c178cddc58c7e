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
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, DPP_QUAD_XOR1, 0xF, 0xF, true);
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, DPP_QUAD_XOR2, 0xF, 0xF, true);
  } else if constexpr (J == 4) {
    const int up = __builtin_amdgcn_mov_dpp(x, DPP_ROW_SHL4, 0xF, 0xF, false);
    const int dn = __builtin_amdgcn_mov_dpp(x, DPP_ROW_SHR4, 0xF, 0xF, false);
    return (uint32_t)((lane_id() & 4) ? dn : up);
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, DPP_ROW_ROR8, 0xF, 0xF, true);
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

// ---- 32-bit networks in the flip form, one compare-exchange stage per asm block -------------
//
// Every block of a level is sorted the same way (descending: the lower lane keeps the larger
// word, or ascending), so the lanes that keep the larger word of a stage are the lanes whose
// bit b is clear, b the stage's bit: the first stage of level K pairs lane l with l ^ (K-1)
// (b = log2(K/2)), the later ones with l ^ J (b = log2 J).  Partners come from DPP moves
// folded into v_max/v_min (quad_perm, row_half_mirror, row_mirror, row_shl/shr:4, row_ror:8)
// or from v_permlane16/32_swap.  For b >= 2 the keep-max lanes are whole 4-lane banks (b = 2,
// 3) or 16-lane rows (b = 4, 5): v_max writes those lanes and v_min the others through the DPP
// bank/row write masks, so the stage is two independent instructions and no select.  For
// b < 2 a v_cndmask with a constant lane mask picks max or min.  Each block starts with the
// two wait states a DPP read of a VGPR written by the previous VALU instruction needs.

namespace flipnet {

// keep-max lane masks for b = 0, 1 (lanes with bit b clear)
constexpr uint64_t KEEP_B0 = 0x5555555555555555ull;
constexpr uint64_t KEEP_B1 = 0x3333333333333333ull;

// partner by quad_perm, keep-max lanes given by a 64-bit mask
#define FSAMP_QSTAGE(QP)                                                                        \
  template <bool ASC>                                                                           \
  __device__ __forceinline__ uint32_t qstage_##QP(uint32_t v, uint64_t keep_max) {              \
    uint32_t mx, mn, r;                                                                         \
    asm("s_nop 1\n\t"                                                                  \
                 "v_max_u32_dpp %1, %3, %3 " QPSTR_##QP " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_min_u32_dpp %2, %3, %3 " QPSTR_##QP " row_mask:0xf bank_mask:0xf\n\t"        \
                 "v_cndmask_b32_e64 %0, %2, %1, %4"                                             \
                 : "=v"(r), "=&v"(mx), "=&v"(mn)                                                \
                 : "v"(v), "s"(ASC ? ~keep_max : keep_max));                                    \
    return r;                                                                                   \
  }
#define QPSTR_x1 "quad_perm:[1,0,3,2]"
#define QPSTR_x2 "quad_perm:[2,3,0,1]"
#define QPSTR_x3 "quad_perm:[3,2,1,0]"
FSAMP_QSTAGE(x1)
FSAMP_QSTAGE(x2)
FSAMP_QSTAGE(x3)
#undef FSAMP_QSTAGE

// partner by one DPP pattern for every lane; MAXBANKS / MINBANKS are the bank write masks
#define FSAMP_BSTAGE(NAME, CTL, MAXB, MINB)                                                     \
  template <bool ASC>                                                                           \
  __device__ __forceinline__ uint32_t NAME(uint32_t v) {                                        \
    uint32_t r;                                                                                 \
    if constexpr (!ASC)                                                                         \
      asm("s_nop 1\n\t"                                                                \
                   "v_max_u32_dpp %0, %1, %1 " CTL " row_mask:0xf bank_mask:" MAXB "\n\t"       \
                   "v_min_u32_dpp %0, %1, %1 " CTL " row_mask:0xf bank_mask:" MINB              \
                   : "=&v"(r) : "v"(v));                                                        \
    else                                                                                        \
      asm("s_nop 1\n\t"                                                                \
                   "v_min_u32_dpp %0, %1, %1 " CTL " row_mask:0xf bank_mask:" MAXB "\n\t"       \
                   "v_max_u32_dpp %0, %1, %1 " CTL " row_mask:0xf bank_mask:" MINB              \
                   : "=&v"(r) : "v"(v));                                                        \
    return r;                                                                                   \
  }
FSAMP_BSTAGE(flip8, "row_half_mirror", "0x5", "0xa")  // l ^ 7,  b = 2
FSAMP_BSTAGE(flip16, "row_mirror", "0x3", "0xc")      // l ^ 15, b = 3
FSAMP_BSTAGE(ror8, "row_ror:8", "0x3", "0xc")         // l ^ 8,  b = 3
#undef FSAMP_BSTAGE

// l ^ 4, b = 2: banks 0 and 2 take lane l + 4 (row_shl:4), banks 1 and 3 lane l - 4 (row_shr:4)
template <bool ASC>
__device__ __forceinline__ uint32_t x4(uint32_t v) {
  uint32_t r;
  if constexpr (!ASC)
    asm("s_nop 1\n\t"
                 "v_max_u32_dpp %0, %1, %1 row_shl:4 row_mask:0xf bank_mask:0x5\n\t"
                 "v_min_u32_dpp %0, %1, %1 row_shr:4 row_mask:0xf bank_mask:0xa"
                 : "=&v"(r) : "v"(v));
  else
    asm("s_nop 1\n\t"
                 "v_min_u32_dpp %0, %1, %1 row_shl:4 row_mask:0xf bank_mask:0x5\n\t"
                 "v_max_u32_dpp %0, %1, %1 row_shr:4 row_mask:0xf bank_mask:0xa"
                 : "=&v"(r) : "v"(v));
  return r;
}

// Partner words of a row-level stage (b = 4 or 5) in two registers, then the masked max/min:
// `even` holds the partner of the rows in MAXROWS' pattern, `odd` of the others.
#define FSAMP_ROWPAIR(MAXR, MINR)                                                               \
  if constexpr (!ASC)                                                                           \
    asm("s_nop 1\n\t"                                                                  \
                 "v_max_u32_dpp %0, %1, %3 quad_perm:[0,1,2,3] row_mask:" MAXR " bank_mask:0xf\n\t" \
                 "v_min_u32_dpp %0, %2, %3 quad_perm:[0,1,2,3] row_mask:" MINR " bank_mask:0xf"   \
                 : "=&v"(r) : "v"(pa), "v"(pb), "v"(v));                                        \
  else                                                                                          \
    asm("s_nop 1\n\t"                                                                  \
                 "v_min_u32_dpp %0, %1, %3 quad_perm:[0,1,2,3] row_mask:" MAXR " bank_mask:0xf\n\t" \
                 "v_max_u32_dpp %0, %2, %3 quad_perm:[0,1,2,3] row_mask:" MINR " bank_mask:0xf"   \
                 : "=&v"(r) : "v"(pa), "v"(pb), "v"(v));

// l ^ 16, b = 4: after v_permlane16_swap of two copies, the second holds the odd rows' words in
// the even rows (the partners of rows 0 and 2, which keep the max) and the first the even rows'
// words in the odd rows
template <bool ASC>
__device__ __forceinline__ uint32_t x16(uint32_t v) {
  uint32_t a = v, b = v, r;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  const uint32_t pa = b, pb = a;
  FSAMP_ROWPAIR("0x5", "0xa")
  return r;
}

// l ^ 31, b = 4: row_mirror, then the l ^ 16 exchange of the mirrored words
template <bool ASC>
__device__ __forceinline__ uint32_t flip32(uint32_t v) {
  uint32_t a, b, r;
  asm("s_nop 1\n\t"
               "v_mov_b32_dpp %0, %2 row_mirror row_mask:0xf bank_mask:0xf\n\t"
               "v_mov_b32_dpp %1, %2 row_mirror row_mask:0xf bank_mask:0xf\n\t"
               "s_nop 1\n\t"
               "v_permlane16_swap_b32 %0, %1\n\t"
               "s_nop 1"
               : "=&v"(a), "=&v"(b) : "v"(v));
  const uint32_t pa = b, pb = a;
  FSAMP_ROWPAIR("0x5", "0xa")
  return r;
}

// l ^ 32, b = 5: after v_permlane32_swap of two copies, the second holds the upper half's words
// in the lower half (partners of rows 0 and 1, which keep the max), the first the lower half's
// words in the upper half
template <bool ASC>
__device__ __forceinline__ uint32_t x32(uint32_t v) {
  uint32_t a = v, b = v, r;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  const uint32_t pa = b, pb = a;
  FSAMP_ROWPAIR("0x3", "0xc")
  return r;
}

// l ^ 63, b = 5: t = row_mirror(v); v_permlane32_swap of two copies of t gives rows
// (t0, t1, t0, t1) and (t2, t3, t2, t3); s = (t2, t3, t0, t1) by row-masked moves; after
// v_permlane16_swap of two copies of s they hold (t2, t2, t0, t0) and (t3, t3, t1, t1), so
// rows 0 and 2 find their partner in the second, rows 1 and 3 in the first.
template <bool ASC>
__device__ __forceinline__ uint32_t flip64(uint32_t v) {
  uint32_t x, y, s0, s1, r;
  asm("s_nop 1\n\t"
               "v_mov_b32_dpp %0, %4 row_mirror row_mask:0xf bank_mask:0xf\n\t"
               "v_mov_b32_dpp %1, %4 row_mirror row_mask:0xf bank_mask:0xf\n\t"
               "s_nop 1\n\t"
               "v_permlane32_swap_b32 %0, %1\n\t"
               "s_nop 1\n\t"
               "v_mov_b32_dpp %2, %1 quad_perm:[0,1,2,3] row_mask:0x3 bank_mask:0xf\n\t"
               "v_mov_b32_dpp %2, %0 quad_perm:[0,1,2,3] row_mask:0xc bank_mask:0xf\n\t"
               "v_mov_b32_e32 %3, %2\n\t"
               "s_nop 1\n\t"
               "v_permlane16_swap_b32 %2, %3\n\t"
               "s_nop 1"
               : "=&v"(x), "=&v"(y), "=&v"(s0), "=&v"(s1) : "v"(v));
  if constexpr (!ASC)
    asm("v_max_u32_dpp %0, %2, %3 quad_perm:[0,1,2,3] row_mask:0x1 bank_mask:0xf\n\t"
                 "v_max_u32_dpp %0, %1, %3 quad_perm:[0,1,2,3] row_mask:0x2 bank_mask:0xf\n\t"
                 "v_min_u32_dpp %0, %2, %3 quad_perm:[0,1,2,3] row_mask:0x4 bank_mask:0xf\n\t"
                 "v_min_u32_dpp %0, %1, %3 quad_perm:[0,1,2,3] row_mask:0x8 bank_mask:0xf"
                 : "=&v"(r) : "v"(s0), "v"(s1), "v"(v));
  else
    asm("v_min_u32_dpp %0, %2, %3 quad_perm:[0,1,2,3] row_mask:0x1 bank_mask:0xf\n\t"
                 "v_min_u32_dpp %0, %1, %3 quad_perm:[0,1,2,3] row_mask:0x2 bank_mask:0xf\n\t"
                 "v_max_u32_dpp %0, %2, %3 quad_perm:[0,1,2,3] row_mask:0x4 bank_mask:0xf\n\t"
                 "v_max_u32_dpp %0, %1, %3 quad_perm:[0,1,2,3] row_mask:0x8 bank_mask:0xf"
                 : "=&v"(r) : "v"(s0), "v"(s1), "v"(v));
  return r;
}
#undef FSAMP_ROWPAIR

// half-cleaner stages J, J/2, ..., 1 of one level
template <int J, bool ASC>
__device__ __forceinline__ uint32_t clean(uint32_t v) {
  if constexpr (J == 32) v = x32<ASC>(v);
  if constexpr (J >= 16) v = x16<ASC>(v);
  if constexpr (J >= 8) v = ror8<ASC>(v);
  if constexpr (J >= 4) v = x4<ASC>(v);
  if constexpr (J >= 2) v = qstage_x2<ASC>(v, KEEP_B1);
  if constexpr (J >= 1) v = qstage_x1<ASC>(v, KEEP_B0);
  return v;
}

// the full 64-lane sort: levels 2 .. 64, each a flip stage and the half-cleaners below it
template <bool ASC>
__device__ __forceinline__ uint32_t sort64(uint32_t v) {
  v = qstage_x1<ASC>(v, KEEP_B0);                 // level 2 (the flip is l ^ 1)
  v = qstage_x3<ASC>(v, KEEP_B1);                 // level 4
  v = clean<1, ASC>(v);
  v = flip8<ASC>(v);                              // level 8
  v = clean<2, ASC>(v);
  v = flip16<ASC>(v);                             // level 16
  v = clean<4, ASC>(v);
  v = flip32<ASC>(v);                             // level 32
  v = clean<8, ASC>(v);
  v = flip64<ASC>(v);                             // level 64
  return clean<16, ASC>(v);
}


// ---- the two sorts of wave_top64_of_two in one chain of blocks: a descending and b ascending,
// stage by stage, so that each block carries two independent compare-exchanges (the second
// sort's comparators are the first's mirrored: where a keeps the max, b keeps the min)

#define FSAMP_DQSTAGE(QP)                                                                        \
  __device__ __forceinline__ void dq_##QP(uint32_t& a, uint32_t& b, uint64_t keep_max) {        \
    uint32_t a1, a2, b1, b2, ra, rb;                                                             \
    asm("s_nop 1\n\t"                                                                            \
        "v_max_u32_dpp %2, %6, %6 " QPSTR_##QP " row_mask:0xf bank_mask:0xf\n\t"                  \
        "v_min_u32_dpp %3, %6, %6 " QPSTR_##QP " row_mask:0xf bank_mask:0xf\n\t"                  \
        "v_max_u32_dpp %4, %7, %7 " QPSTR_##QP " row_mask:0xf bank_mask:0xf\n\t"                  \
        "v_min_u32_dpp %5, %7, %7 " QPSTR_##QP " row_mask:0xf bank_mask:0xf\n\t"                  \
        "v_cndmask_b32_e64 %0, %3, %2, %8\n\t"                                                   \
        "v_cndmask_b32_e64 %1, %4, %5, %8"                                                       \
        : "=v"(ra), "=v"(rb), "=&v"(a1), "=&v"(a2), "=&v"(b1), "=&v"(b2)                         \
        : "v"(a), "v"(b), "s"(keep_max));                                                        \
    a = ra;                                                                                      \
    b = rb;                                                                                      \
  }
FSAMP_DQSTAGE(x1)
FSAMP_DQSTAGE(x2)
FSAMP_DQSTAGE(x3)
#undef FSAMP_DQSTAGE

#define FSAMP_DBSTAGE(NAME, CTLMAX, CTLMIN, MAXB, MINB)                                          \
  __device__ __forceinline__ void NAME(uint32_t& a, uint32_t& b) {                              \
    uint32_t ra, rb;                                                                             \
    asm("s_nop 1\n\t"                                                                            \
        "v_max_u32_dpp %0, %2, %2 " CTLMAX " row_mask:0xf bank_mask:" MAXB "\n\t"                \
        "v_min_u32_dpp %0, %2, %2 " CTLMIN " row_mask:0xf bank_mask:" MINB "\n\t"                \
        "v_min_u32_dpp %1, %3, %3 " CTLMAX " row_mask:0xf bank_mask:" MAXB "\n\t"                \
        "v_max_u32_dpp %1, %3, %3 " CTLMIN " row_mask:0xf bank_mask:" MINB                       \
        : "=&v"(ra), "=&v"(rb) : "v"(a), "v"(b));                                                \
    a = ra;                                                                                      \
    b = rb;                                                                                      \
  }
FSAMP_DBSTAGE(d_flip8, "row_half_mirror", "row_half_mirror", "0x5", "0xa")
FSAMP_DBSTAGE(d_flip16, "row_mirror", "row_mirror", "0x3", "0xc")
FSAMP_DBSTAGE(d_ror8, "row_ror:8", "row_ror:8", "0x3", "0xc")
FSAMP_DBSTAGE(d_x4, "row_shl:4", "row_shr:4", "0x5", "0xa")
#undef FSAMP_DBSTAGE

// row-level stages: partners of a in (pa for the keep-max rows, pb for the others), of b in
// (qa, qb); a keeps the max in rows MAXR, b the min
#define FSAMP_DROWPAIR(MAXR, MINR)                                                               \
  asm("s_nop 1\n\t"                                                                              \
      "v_max_u32_dpp %0, %2, %6 quad_perm:[0,1,2,3] row_mask:" MAXR " bank_mask:0xf\n\t"          \
      "v_min_u32_dpp %0, %3, %6 quad_perm:[0,1,2,3] row_mask:" MINR " bank_mask:0xf\n\t"          \
      "v_min_u32_dpp %1, %4, %7 quad_perm:[0,1,2,3] row_mask:" MAXR " bank_mask:0xf\n\t"          \
      "v_max_u32_dpp %1, %5, %7 quad_perm:[0,1,2,3] row_mask:" MINR " bank_mask:0xf"              \
      : "=&v"(ra), "=&v"(rb) : "v"(pa), "v"(pb), "v"(qa), "v"(qb), "v"(a), "v"(b));

__device__ __forceinline__ void d_x16(uint32_t& a, uint32_t& b) {
  uint32_t a0 = a, a1 = a, b0 = b, b1 = b, ra, rb;
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_permlane16_swap_b32 %2, %3\n\ts_nop 1"
      : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1));
  const uint32_t pa = a1, pb = a0, qa = b1, qb = b0;
  FSAMP_DROWPAIR("0x5", "0xa")
  a = ra;
  b = rb;
}

__device__ __forceinline__ void d_x32(uint32_t& a, uint32_t& b) {
  uint32_t a0 = a, a1 = a, b0 = b, b1 = b, ra, rb;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\tv_permlane32_swap_b32 %2, %3\n\ts_nop 1"
      : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1));
  const uint32_t pa = a1, pb = a0, qa = b1, qb = b0;
  FSAMP_DROWPAIR("0x3", "0xc")
  a = ra;
  b = rb;
}

__device__ __forceinline__ void d_flip32(uint32_t& a, uint32_t& b) {
  uint32_t a0, a1, b0, b1, ra, rb;
  asm("s_nop 1\n\t"
      "v_mov_b32_dpp %0, %4 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "v_mov_b32_dpp %1, %4 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "v_mov_b32_dpp %2, %5 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "v_mov_b32_dpp %3, %5 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_permlane16_swap_b32 %0, %1\n\t"
      "v_permlane16_swap_b32 %2, %3\n\t"
      "s_nop 1"
      : "=&v"(a0), "=&v"(a1), "=&v"(b0), "=&v"(b1) : "v"(a), "v"(b));
  const uint32_t pa = a1, pb = a0, qa = b1, qb = b0;
  FSAMP_DROWPAIR("0x5", "0xa")
  a = ra;
  b = rb;
}
#undef FSAMP_DROWPAIR

// partner l ^ 63 of both (see flip64): rows 0 and 2 of the second register, rows 1 and 3 of
// the first
__device__ __forceinline__ void d_flip64(uint32_t& a, uint32_t& b) {
  uint32_t x, y, s0, s1, u, w, t0, t1, ra, rb;
  asm("s_nop 1\n\t"
      "v_mov_b32_dpp %0, %8 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "v_mov_b32_dpp %1, %8 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "v_mov_b32_dpp %4, %9 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "v_mov_b32_dpp %5, %9 row_mirror row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "v_permlane32_swap_b32 %4, %5\n\t"
      "s_nop 1\n\t"
      "v_mov_b32_dpp %2, %1 quad_perm:[0,1,2,3] row_mask:0x3 bank_mask:0xf\n\t"
      "v_mov_b32_dpp %2, %0 quad_perm:[0,1,2,3] row_mask:0xc bank_mask:0xf\n\t"
      "v_mov_b32_dpp %6, %5 quad_perm:[0,1,2,3] row_mask:0x3 bank_mask:0xf\n\t"
      "v_mov_b32_dpp %6, %4 quad_perm:[0,1,2,3] row_mask:0xc bank_mask:0xf\n\t"
      "v_mov_b32_e32 %3, %2\n\t"
      "v_mov_b32_e32 %7, %6\n\t"
      "s_nop 1\n\t"
      "v_permlane16_swap_b32 %2, %3\n\t"
      "v_permlane16_swap_b32 %6, %7\n\t"
      "s_nop 1"
      : "=&v"(x), "=&v"(y), "=&v"(s0), "=&v"(s1), "=&v"(u), "=&v"(w), "=&v"(t0), "=&v"(t1)
      : "v"(a), "v"(b));
  asm("v_max_u32_dpp %0, %3, %6 quad_perm:[0,1,2,3] row_mask:0x1 bank_mask:0xf\n\t"
      "v_max_u32_dpp %0, %2, %6 quad_perm:[0,1,2,3] row_mask:0x2 bank_mask:0xf\n\t"
      "v_min_u32_dpp %0, %3, %6 quad_perm:[0,1,2,3] row_mask:0x4 bank_mask:0xf\n\t"
      "v_min_u32_dpp %0, %2, %6 quad_perm:[0,1,2,3] row_mask:0x8 bank_mask:0xf\n\t"
      "v_min_u32_dpp %1, %5, %7 quad_perm:[0,1,2,3] row_mask:0x1 bank_mask:0xf\n\t"
      "v_min_u32_dpp %1, %4, %7 quad_perm:[0,1,2,3] row_mask:0x2 bank_mask:0xf\n\t"
      "v_max_u32_dpp %1, %5, %7 quad_perm:[0,1,2,3] row_mask:0x4 bank_mask:0xf\n\t"
      "v_max_u32_dpp %1, %4, %7 quad_perm:[0,1,2,3] row_mask:0x8 bank_mask:0xf"
      : "=&v"(ra), "=&v"(rb) : "v"(s0), "v"(s1), "v"(t0), "v"(t1), "v"(a), "v"(b));
  a = ra;
  b = rb;
}

template <int J>
__device__ __forceinline__ void dclean(uint32_t& a, uint32_t& b) {
  if constexpr (J == 32) d_x32(a, b);
  if constexpr (J >= 16) d_x16(a, b);
  if constexpr (J >= 8) d_ror8(a, b);
  if constexpr (J >= 4) d_x4(a, b);
  if constexpr (J >= 2) dq_x2(a, b, KEEP_B1);
  if constexpr (J >= 1) dq_x1(a, b, KEEP_B0);
}

// a sorted descending and b ascending, in one chain
__device__ __forceinline__ void sort64_pair(uint32_t& a, uint32_t& b) {
  dq_x1(a, b, KEEP_B0);
  dq_x3(a, b, KEEP_B1);
  dclean<1>(a, b);
  d_flip8(a, b);
  dclean<2>(a, b);
  d_flip16(a, b);
  dclean<4>(a, b);
  d_flip32(a, b);
  dclean<8>(a, b);
  d_flip64(a, b);
  dclean<16>(a, b);
}

}  // namespace flipnet

// Full descending sort of one value per lane (64 values): lane 0 gets the largest.
template <typename T>
__device__ __forceinline__ T wave_sort_desc(T v) {
  if constexpr (sizeof(T) == 4) return (T)flipnet::sort64<false>((uint32_t)v);
  else return bitonic_levels<64, T>(v);
}

// Full ascending sort of one value per lane (every comparator mirrored): lane 0 the smallest.
template <typename T>
__device__ __forceinline__ T wave_sort_asc(T v) {
  if constexpr (sizeof(T) == 4) return (T)flipnet::sort64<true>((uint32_t)v);
  else return bitonic_levels<64, T, true>(v);
}

// The descending top 64 of two lists of 64 values, one of each per lane: a sorted descending,
// b ascending, the elementwise maximum is a bitonic sequence holding exactly the 64 largest of
// both, and the six half-cleaner stages of the last bitonic level sort it.
template <typename T>
__device__ __forceinline__ T wave_top64_of_two(T a, T b) {
  if constexpr (sizeof(T) == 4) {
    uint32_t x = (uint32_t)a, y = (uint32_t)b;
    flipnet::sort64_pair(x, y);
    return (T)flipnet::clean<32, false>(x > y ? x : y);
  } else {
    a = wave_sort_desc<T>(a);
    b = wave_sort_asc<T>(b);
    const T m = a > b ? a : b;
    return bitonic_merge_stages<64, 32, T>(m);
  }
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
