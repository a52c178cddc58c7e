// fsamp_selftest.hip -- lane-layout self-test of the wave primitives in fsamp_wave.h.
// One wave of one workgroup writes, per lane, what each primitive returns for a known input;
// the host compares with the layouts the sampler assumes.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "fsamp.h"
#include "fsamp_wave.h"

namespace {

// out layout (uint32 words, 64 per row): 0..5 xor_lane<1,2,4,8,16,32>(lane); 6 wave sort of a
// permutation (lane*37 mod 64); 7 bitcast of the inclusive scan of (lane+1); 8 wave_shr1 of
// (lane+1); 9 scan of 1.0 per lane; 10 wave sort of u64 keys (high halves); 11 low halves.
__global__ __launch_bounds__(64) void wave_selftest_kernel(uint32_t* out) {
  using namespace fsamp;
  const uint32_t l = (uint32_t)lane_id();
  out[0 * 64 + l] = xor_lane<1>(l);
  out[1 * 64 + l] = xor_lane<2>(l);
  out[2 * 64 + l] = xor_lane<4>(l);
  out[3 * 64 + l] = xor_lane<8>(l);
  out[4 * 64 + l] = xor_lane<16>(l);
  out[5 * 64 + l] = xor_lane<32>(l);
  out[6 * 64 + l] = wave_sort_desc<uint32_t>((l * 37u) & 63u);
  out[7 * 64 + l] = __float_as_uint(wave_incl_scan_f32((float)(l + 1)));
  out[8 * 64 + l] = __float_as_uint(wave_shr1_f32((float)(l + 1)));
  out[9 * 64 + l] = __float_as_uint(wave_incl_scan_f32(1.0f));
  const uint64_t k = ((uint64_t)((l * 21u) & 63u) << 32) | (0xFFFFFFFFu - l);
  const uint64_t s = wave_sort_desc<uint64_t>(k);
  out[10 * 64 + l] = (uint32_t)(s >> 32);
  out[11 * 64 + l] = (uint32_t)s;
}

}  // namespace

extern "C" int fsamp_debug_wave_selftest(uint32_t* out, hipStream_t stream) {
  if (out == nullptr) return FSAMP_ERR_NULL;
  hipLaunchKernelGGL(wave_selftest_kernel, dim3(1), dim3(64), 0, stream, out);
  return hipGetLastError() == hipSuccess ? FSAMP_OK : FSAMP_ERR_LAUNCH;
}
