// silu_bf16 (hn_common.h: the hardware exponential and reciprocal, with the library form near bf16
// rounding midpoints) against rbf16(silu_f32(g)) for every bf16 value g: not part of the product library
// (built into hy_nomas/libhynomas_probes.so).
//
//   hnp_silu_mismatches  thread t < 65536 evaluates both forms for the bf16 bit pattern t, writes the fast
//                        form's fp32 bits to value[t] and 1 to bad[t] if the two differ, else 0: no atomics.
#include "../hn_common.h"

namespace {

__global__ __launch_bounds__(256) void silu_check(uint32_t* value, uint32_t* bad) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= 65536u) return;
  const float g = __uint_as_float(t << 16);
  const float fast = hn::silu_bf16(g), ref = hn::rbf16(hn::silu_f32(g));
  value[t] = __float_as_uint(fast);
  bad[t] = __float_as_uint(fast) != __float_as_uint(ref) ? 1u : 0u;
}

}  // namespace

// value, bad: 65536 slots each (device memory).  Returns 0, or 1 for a null pointer.
extern "C" int hnp_silu_mismatches(void* value, void* bad, void* stream) {
  if (!value || !bad) return 1;
  hipLaunchKernelGGL(silu_check, dim3(256), dim3(256), 0, (hipStream_t)stream, (uint32_t*)value, (uint32_t*)bad);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
