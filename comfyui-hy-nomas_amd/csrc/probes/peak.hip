// Peak-rate probes for the benchmark's roofline denominators (bench.py --peaks): not part of the product
// library.  Built into hy_nomas/libhynomas_probes.so by build.py.
//
//   hnp_mfma_loop  every wave holds kFrags weight-like and activation-like operand fragments (read once from
//                  global memory, so the matrix cores see real data: the chip's power limit, and with it the
//                  clock, depends on how the operand bits toggle) and issues back-to-back MFMAs on kChains
//                  independent accumulators.  Two waves per SIMD.  Reports the shader-clock cycles and the
//                  100 MHz reference-clock ticks of the first wave, so the effective clock is known.
//   hnp_copy       a 16-byte-per-lane streaming copy with non-temporal loads and stores.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kFrags = 4;
constexpr int kChains = 4;
constexpr int kPatterns = 64;   // distinct operand sets; wave w uses set w % kPatterns
constexpr int kWaves = 4;       // per workgroup

__device__ __forceinline__ uint64_t memrealtime() { return __builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ uint64_t memtime() { return __builtin_amdgcn_s_memtime(); }

__global__ __launch_bounds__(kWaves * 64) void mfma_i8_loop(const v4i* a, const v4i* b, int iters, int* out,
                                                            uint64_t* clocks) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int set = wave % kPatterns;
  v4i fa[kFrags], fb[kFrags];
#pragma unroll
  for (int f = 0; f < kFrags; f++) {
    fa[f] = a[(set * kFrags + f) * 64 + lane];
    fb[f] = b[(set * kFrags + f) * 64 + lane];
  }
  v16i acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[c][r] = 0;
  const uint64_t t0 = memtime(), r0 = memrealtime();
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int f = 0; f < kFrags; f++)
#pragma unroll
      for (int c = 0; c < kChains; c++)
        acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[f], fb[(f + c) % kFrags], acc[c], 0, 0, 0);
  }
  const uint64_t t1 = memtime(), r1 = memrealtime();
  int s = 0;
#pragma unroll
  for (int c = 0; c < kChains; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) s += acc[c][r];
  out[(int64_t)wave * 64 + lane] = s;
  if (wave == 0 && lane == 0) {
    clocks[0] = t1 - t0;
    clocks[1] = r1 - r0;
  }
}

__global__ __launch_bounds__(kWaves * 64) void mfma_fp8_loop(const v8i* a, const v8i* b, int iters, int* out,
                                                             uint64_t* clocks) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int set = wave % kPatterns;
  v8i fa[kFrags], fb[kFrags];
#pragma unroll
  for (int f = 0; f < kFrags; f++) {
    fa[f] = a[(set * kFrags + f) * 64 + lane];
    fb[f] = b[(set * kFrags + f) * 64 + lane];
  }
  v16f acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[c][r] = 0.0f;
  const uint64_t t0 = memtime(), r0 = memrealtime();
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int f = 0; f < kFrags; f++)
#pragma unroll
      for (int c = 0; c < kChains; c++)
        acc[c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[f], fb[(f + c) % kFrags], acc[c], 0, 0, 0, 0, 0, 0);
  }
  const uint64_t t1 = memtime(), r1 = memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < kChains; c++)
#pragma unroll
    for (int r = 0; r < 16; r++) s += acc[c][r];
  out[(int64_t)wave * 64 + lane] = __float_as_int(s);
  if (wave == 0 && lane == 0) {
    clocks[0] = t1 - t0;
    clocks[1] = r1 - r0;
  }
}

// One 16-byte chunk per thread, one pass of the grid (the caller launches ceil(n / 256) workgroups).
__global__ __launch_bounds__(256) void copy16(const v4i* __restrict__ src, v4i* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

// Operand buffers: kPatterns * kFrags * 64 fragments of 16 bytes (int8) or 32 bytes (fp8) each, for a and b.
extern "C" int64_t hnp_operand_bytes(int kind) { return (int64_t)kPatterns * kFrags * 64 * (kind == 0 ? 16 : 32); }

// MFMAs per wave per iteration, and the operations of one MFMA (2 * 32 * 32 * K).
extern "C" int hnp_mfma_per_iter(void) { return kFrags * kChains; }
extern "C" int64_t hnp_ops_per_mfma(int kind) { return kind == 0 ? 2LL * 32 * 32 * 32 : 2LL * 32 * 32 * 64; }
extern "C" int hnp_waves_per_block(void) { return kWaves; }

// kind 0: int8 (v_mfma_i32_32x32x32_i8), 1: fp8 e4m3 (v_mfma_f32_32x32x64_f8f6f4).  out: blocks * kWaves * 64
// ints; clocks: 2 uint64 (shader-clock cycles, 100 MHz ticks of wave 0's loop).  Returns 0, or 1 for bad
// arguments, 2 for a launch error.
extern "C" int hnp_mfma_loop(int kind, const void* a, const void* b, int iters, int blocks, int* out,
                             uint64_t* clocks, void* stream) {
  if (!a || !b || !out || !clocks || iters <= 0 || blocks <= 0 || (kind != 0 && kind != 1)) return 1;
  hipStream_t st = (hipStream_t)stream;
  if (kind == 0)
    hipLaunchKernelGGL(mfma_i8_loop, dim3(blocks), dim3(kWaves * 64), 0, st, (const v4i*)a, (const v4i*)b, iters, out,
                       clocks);
  else
    hipLaunchKernelGGL(mfma_fp8_loop, dim3(blocks), dim3(kWaves * 64), 0, st, (const v8i*)a, (const v8i*)b, iters,
                       out, clocks);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// dst[0:bytes) = src[0:bytes); bytes % 16 == 0, both 16-byte aligned.  (`blocks` is unused: one thread per chunk.)
extern "C" int hnp_copy(const void* src, void* dst, int64_t bytes, int blocks, void* stream) {
  (void)blocks;
  if (!src || !dst || bytes <= 0 || bytes % 16 || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15)) return 1;
  const int64_t n = bytes / 16, grid = (n + 255) / 256;
  if (grid > 0x7fffffff) return 1;
  hipLaunchKernelGGL(copy16, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const v4i*)src, (v4i*)dst, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
