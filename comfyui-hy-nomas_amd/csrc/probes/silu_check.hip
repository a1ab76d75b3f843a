// silu_bf16 and its pair form silu_bf16x2 (hn_common.h: the hardware exponential and reciprocal, with the
// library form near bf16 rounding midpoints) against rbf16(silu_f32(g)) for every bf16 value g: not part of
// the product library (built into hy_nomas/libhynomas_probes.so).
//
//   hnp_silu_mismatches  thread t < 65536 evaluates silu_bf16 and the reference form for the bf16 bit
//                        pattern t, and silu_bf16x2 on the pair (t, t * 40503 mod 2^16) (an odd multiplier
//                        permutes the patterns, so every value also takes the second slot once).  It writes
//                        silu_bf16's fp32 bits to value[t], and to bad[t] a bit mask: 1 if silu_bf16 differs
//                        from the reference, 2 / 4 if the pair's first / second result does; no atomics.
#include "../hn_common.h"

namespace {

__global__ __launch_bounds__(256) void silu_check(uint32_t* value, uint32_t* bad) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 65536u) return;
  const float g = __uint_as_float(t << 16);
  const float fast = hn::silu_bf16(g), ref = hn::rbf16(hn::silu_f32(g));
  const uint32_t t2 = (t * 40503u) & 0xffffu;
  const float g2 = __uint_as_float(t2 << 16), ref2 = hn::rbf16(hn::silu_f32(g2));
  float s0, s1;
  hn::silu_bf16x2(g, g2, s0, s1);
  value[t] = __float_as_uint(fast);
  bad[t] = (__float_as_uint(fast) != __float_as_uint(ref) ? 1u : 0u) |
           (__float_as_uint(s0) != __float_as_uint(ref) ? 2u : 0u) |
           (__float_as_uint(s1) != __float_as_uint(ref2) ? 4u : 0u);
}

}  // namespace

// value, bad: 65536 slots each (device memory).  Returns 0, or 1 for a null pointer.
extern "C" int hnp_silu_mismatches(void* value, void* bad, void* stream) {
  if (!value || !bad) return 1;
  hipLaunchKernelGGL(silu_check, dim3(256), dim3(256), 0, (hipStream_t)stream, (uint32_t*)value, (uint32_t*)bad);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
