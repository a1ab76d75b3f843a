// Shared device helpers for the gfx950 kernels of the quantized DiT linear path.
//
// Numerics follow the reference's Triton kernels (hy_nomas/kernels.py, hy_nomas/fused.py):
//   * bf16 rounding on the bits, ties to even (kernels.py:67-71);
//   * int8 codes: IEEE fp32 x / scale, then round half away from zero, clamp +-127 (kernels.py:33-36);
//   * fp8 codes: x / scale cast to OCP e4m3fn with round to nearest even (kernels.py:39-41).
// All kernels are compiled with -ffp-contract=off; every fused multiply-add is spelled out.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hynomas.h"

namespace hn {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// ----------------------------------------------------------------------------------------------
// scalar conversions

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN becomes the quiet NaN 0x7FC0 (torch's rule).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// fp32 -> the nearest bf16 value, kept in fp32 (kernels.py:67-71, no NaN special case).
__device__ __forceinline__ float rbf16(float x) {
  uint32_t b = __float_as_uint(x);
  b = (b + (((b >> 16) & 1u) + 0x7fffu)) & 0xffff0000u;
  return __uint_as_float(b);
}

// fp16 bits <-> fp32 through the hardware conversion (exact widening; RNE narrowing).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// OCP e4m3fn encoding, round to nearest even; values that round past 448 give the NaN code 0x7F.
__device__ __forceinline__ uint32_t e4m3_encode(float f) {
  uint32_t sign = (__float_as_uint(f) >> 24) & 0x80u;
  float a = __builtin_fabsf(f);
  uint32_t code;
  if (a < 0x1p-6f) {
    code = (uint32_t)__builtin_rintf(a * 512.0f);  // subnormal grid 2^-9; 8 encodes 2^-6
  } else {
    uint32_t b = __float_as_uint(a);
    b += 0x7ffffu + ((b >> 20) & 1u);               // round the fp32 mantissa to 3 bits, ties to even
    uint32_t e = (b >> 23) - 120u;                  // rebias 127 -> 7
    code = (e << 3) | ((b >> 20) & 7u);
    code = (b >> 23) >= 136u ? 0x7fu : code;        // 2^9 and above (incl. inf / NaN)
    code = code > 0x7eu ? 0x7fu : code;
  }
  return sign | code;
}

// ----------------------------------------------------------------------------------------------
// quantization arithmetic

// Group scales (kernels.py:33, kernels.py:39).
__device__ __forceinline__ float int8_scale(float peak) { return peak > 0.0f ? peak / 127.0f : 1.0f; }
__device__ __forceinline__ float fp8_scale(float peak) { return (peak > 1e-12f ? peak : 1e-12f) / 448.0f; }

// IEEE x / s for bf16-valued x and a scale derived from a bf16 absmax, in three VALU ops instead of a
// full division: q0 = x * r, e = fma(-q0, s, x), q = fma(e, r, q0), r = 1 / s (correctly rounded).
// Checked exhaustively on the CPU for every bf16 absmax and every bf16 |x| <= absmax (int8: same fp32
// bits; fp8: same e4m3 code) when r is finite and x == 0 or |x| >= 2^-100; other lanes divide.
struct FastDiv {
  float s, r;
  bool ok;
  __device__ __forceinline__ explicit FastDiv(float scale) : s(scale) {
    r = 1.0f / scale;
    ok = __builtin_isfinite(r);
  }
  __device__ __forceinline__ float operator()(float x) const {
    float q0 = x * r;
    float e = __builtin_fmaf(-q0, s, x);
    float q = __builtin_copysignf(__builtin_fmaf(e, r, q0), x);
    float ax = __builtin_fabsf(x);
    if (__builtin_expect(!ok || (ax != 0.0f && ax < 0x1p-100f), 0)) q = x / s;
    return q;
  }
};

// Round half away from zero (kernels.py:35: floor(y + 0.5) / ceil(y - 0.5), each sum rounded in fp32),
// clamp to +-127.  trunc(y + copysign(0.5, y)) equals that rule bit for bit: floor and trunc agree on
// the non-negative branch, ceil and trunc on the negative one.
__device__ __forceinline__ int round_half_away_i8(float y) {
  float t = y + __builtin_copysignf(0.5f, y);
  t = __builtin_fminf(__builtin_fmaxf(t, -127.0f), 127.0f);
  return (int)t;  // truncates toward zero; NaN gives 0
}

__device__ __forceinline__ int round_half_even_i8(float y) {
  float t = __builtin_rintf(y);
  t = __builtin_fminf(__builtin_fmaxf(t, -127.0f), 127.0f);
  return (int)t;
}

template <int ROUND>
__device__ __forceinline__ int round_i8(float y) {
  if constexpr (ROUND == HN_ROUND_HALF_EVEN) return round_half_even_i8(y);
  else return round_half_away_i8(y);
}

// Pack four int8 codes (low byte first).
__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// ----------------------------------------------------------------------------------------------
// cross-lane reductions (wave64)

__device__ __forceinline__ float shfl_xor_f(float v, int mask, int width = 64) { return __shfl_xor(v, mask, width); }

// max over the 16 lanes of each DPP row
__device__ __forceinline__ float row16_max(float v) {
  v = __builtin_fmaxf(v, shfl_xor_f(v, 1, 16));
  v = __builtin_fmaxf(v, shfl_xor_f(v, 2, 16));
  v = __builtin_fmaxf(v, shfl_xor_f(v, 4, 16));
  v = __builtin_fmaxf(v, shfl_xor_f(v, 8, 16));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  v = __builtin_fmaxf(v, shfl_xor_f(v, 16));
  v = __builtin_fmaxf(v, shfl_xor_f(v, 32));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += shfl_xor_f(v, m);
  return v;
}

// ----------------------------------------------------------------------------------------------
// 16-byte vector loads of 8 two-byte values, widened to fp32

template <int DT>
struct In;

template <>
struct In<HN_DTYPE_BF16> {
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static void widen8(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

template <>
struct In<HN_DTYPE_F16> {
  static constexpr int kBytes = 2;
  __device__ __forceinline__ static void widen8(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      f[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
      f[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
};

template <int DT>
__device__ __forceinline__ uint32_t pack2_out(float a, float b) {
  if constexpr (DT == HN_DTYPE_BF16) return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
  else return f32_to_f16_bits(a) | (f32_to_f16_bits(b) << 16);
}

}  // namespace hn

// ----------------------------------------------------------------------------------------------
// host-side error plumbing shared by every entry point

namespace hn {
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);
}  // namespace hn

#define HN_REQUIRE(cond, ...)            \
  do {                                   \
    if (!(cond)) {                       \
      ::hn::set_error(__VA_ARGS__);      \
      return HN_ERR_ARG;                 \
    }                                    \
  } while (0)

#define HN_LAUNCH_CHECK(what) ::hn::hip_status(hipGetLastError(), what)
