// The hardware OCP e4m3 conversion (v_cvt_pk_fp8_f32, round to nearest even) against the software encoder
// e4m3_encode (hn_common.h), for the checks that allow the kernels to use the hardware form: not part of the
// product library (built into hy_nomas/libhynomas_probes.so).
//
//   hnp_e4m3_mismatches  for every fp32 bit pattern u in [lo, hi), with both signs, converts (x, -x) into the
//                        low half-word and (-x, x) into the high half-word of one register, so both byte
//                        positions, both half-words and both signs are covered, and counts the codes that
//                        differ from e4m3_encode.  Each thread writes its count and the lowest differing
//                        pattern (0xFFFFFFFF if none) to its own slot: no atomics.
#include "../hn_common.h"

namespace {

__global__ __launch_bounds__(256) void e4m3_check(uint32_t lo, uint32_t hi, uint32_t* count, uint32_t* first) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t stride = gridDim.x * blockDim.x;
  uint32_t bad = 0, low = 0xffffffffu;
  for (uint64_t u = (uint64_t)lo + tid; u < hi; u += stride) {
    const float x = __uint_as_float((uint32_t)u);
    const float nx = __uint_as_float((uint32_t)u ^ 0x80000000u);
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, nx, 0, false);
    w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(nx, x, (int)w, true);
    const uint32_t sx = hn::e4m3_encode(x), snx = hn::e4m3_encode(nx);
    const uint32_t want = sx | (snx << 8) | (snx << 16) | (sx << 24);
    if (w != want) {
      bad++;
      low = (uint32_t)u < low ? (uint32_t)u : low;
    }
  }
  count[tid] = bad;
  first[tid] = low;
}

}  // namespace

// count / first: blocks * 256 slots each (device memory).  Returns 0, or 1 for bad arguments.
extern "C" int hnp_e4m3_mismatches(uint32_t lo, uint32_t hi, int blocks, void* count, void* first, void* stream) {
  if (!count || !first || blocks <= 0 || hi < lo) return 1;
  hipLaunchKernelGGL(e4m3_check, dim3(blocks), dim3(256), 0, (hipStream_t)stream, lo, hi, (uint32_t*)count,
                     (uint32_t*)first);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
