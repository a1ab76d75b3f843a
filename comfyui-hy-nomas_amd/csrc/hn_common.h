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

// torch's silu of a bf16 value, computed in fp32 as x / (1 + exp(-x)) (the reference's F.silu,
// hy_nomas/pixelumm.py:322, on a bf16 tensor).
__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

// rbf16(silu_f32(g)) for a g that is a bf16 value, from the hardware base-2 exponential and reciprocal
// (v_exp_f32, v_rcp_f32).  For g >= -16 that value is within about 20 fp32 ulps of silu_f32(g) (the
// exponential's input carries |g| log2(e) 2^-24 of relative error), so both round to the same bf16 value
// unless it lies within 32 ulps of a rounding midpoint; such lanes, g < -16 and non-finite g take silu_f32.
// Exhaustively equal to rbf16(silu_f32(g)) for all 65536 bf16 g (libhynomas_probes.so: hnp_silu_mismatches).
__device__ __forceinline__ float silu_bf16(float g) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  const float f = g * __builtin_amdgcn_rcpf(1.0f + e);
  const uint32_t low = __float_as_uint(f) & 0xffffu;
  if (__builtin_expect((low - 0x7fe0u) < 0x40u || !(g >= -16.0f), 0)) return rbf16(silu_f32(g));
  return rbf16(f);
}

// silu_bf16 of two values, the fast path's rounding by the hardware pair conversion (its values are finite,
// where the pack equals rbf16); lanes that take the slow path (as in silu_bf16) round in software.
__device__ __forceinline__ uint32_t bf16x2_finite(float a, float b);
__device__ __forceinline__ void silu_bf16x2(float g0, float g1, float& s0, float& s1) {
  const float e0 = __builtin_amdgcn_exp2f(g0 * -1.4426950408889634f);
  const float e1 = __builtin_amdgcn_exp2f(g1 * -1.4426950408889634f);
  const float f0 = g0 * __builtin_amdgcn_rcpf(1.0f + e0);
  const float f1 = g1 * __builtin_amdgcn_rcpf(1.0f + e1);
  const uint32_t p = bf16x2_finite(f0, f1);
  s0 = __uint_as_float(p << 16);
  s1 = __uint_as_float(p & 0xffff0000u);
  const uint32_t l0 = __float_as_uint(f0) & 0xffffu, l1 = __float_as_uint(f1) & 0xffffu;
  if (__builtin_expect((l0 - 0x7fe0u) < 0x40u || !(g0 >= -16.0f), 0)) s0 = rbf16(silu_f32(g0));
  if (__builtin_expect((l1 - 0x7fe0u) < 0x40u || !(g1 >= -16.0f), 0)) s1 = rbf16(silu_f32(g1));
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

// Four e4m3 codes, low byte first, by the hardware conversion (v_cvt_pk_fp8_f32: OCP e4m3fn, round to nearest
// even).  It equals e4m3_encode for every finite |x| < 2^9 of either sign (an exhaustive check on the GPU over
// all such fp32 values, both byte positions and both half-words); the kernels use it only for the finite
// quotients x / scale of a fast group, which lie within 448 (1 + 2^-22).
__device__ __forceinline__ uint32_t e4m3_pack4_hw(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// ----------------------------------------------------------------------------------------------
// quantization arithmetic

// Group scales (kernels.py:33, kernels.py:39).
__device__ __forceinline__ float int8_scale(float peak) { return peak > 0.0f ? peak / 127.0f : 1.0f; }
__device__ __forceinline__ float fp8_scale(float peak) { return (peak > 1e-12f ? peak : 1e-12f) / 448.0f; }

// The same scales for a peak with fast_group(peak): the quotient by the constant from its correctly
// rounded reciprocal and one FMA correction, equal to the IEEE quotient for every bf16 peak >= 2^-80
// (checked exhaustively on the CPU).
__device__ __forceinline__ float div_by_const(float d, float c, float rc) {
  const float q0 = d * rc;
  const float e = __builtin_fmaf(-q0, c, d);
  return __builtin_fmaf(e, rc, q0);
}
// 1/sqrt(v) from the hardware reciprocal square root (1 ulp) and one Newton step, for row statistics
// (where the reductions' own order already moves the last bits).  v = +inf gives 0, v = 0 gives +inf and a
// NaN stays NaN, as 1/sqrt(v).
__device__ __forceinline__ float rsqrt_refined(float v) {
  const float r0 = __builtin_amdgcn_rsqf(v);
  const float h = __builtin_fmaf(-0.5f * v * r0, r0, 0.5f);  // (1 - v r0^2) / 2
  return __builtin_isfinite(h) ? __builtin_fmaf(r0, h, r0) : r0;
}
__device__ __forceinline__ float int8_scale_fast(float peak) { return div_by_const(peak, 127.0f, 1.0f / 127.0f); }
__device__ __forceinline__ float fp8_scale_fast(float peak) {
  return div_by_const(peak > 1e-12f ? peak : 1e-12f, 448.0f, 1.0f / 448.0f);
}

// IEEE x / s for bf16-valued x and a scale derived from a bf16 absmax, in three VALU ops per value instead
// of a full division: q0 = x * r, e = fma(-q0, s, x), q = fma(e, r, q0), r = 1 / s (correctly rounded).
// Checked exhaustively on the CPU for every bf16 absmax and every bf16 |x| <= absmax (int8: same fp32
// bits; fp8: same e4m3 code) when r is finite and x == 0 or |x| >= 2^-100.  Callers use it for a whole
// group when `fast_group(peak)` holds: then r is finite, and any 0 < |x| < 2^-100 gives |x / s| < 2^-11
// on both paths, which is code 0 for int8 and for e4m3 (half its smallest subnormal is 2^-10).  Groups
// with a smaller peak, and inputs that are not bf16 values, divide.  KEEP_SIGN restores the sign of a
// zero quotient (-0 / s = -0 matters for the e4m3 sign bit, not for int8 codes).
template <bool KEEP_SIGN>
struct FastDiv {
  float s, r;
  // r = RN(1 / scale): the hardware reciprocal (1 ulp) refined by one Newton step, which lands exactly on
  // the correctly rounded reciprocal from anywhere within 2 ulp of it for every scale of a fast group
  // (checked exhaustively on the CPU).
  __device__ __forceinline__ explicit FastDiv(float scale) : s(scale) {
    const float r0 = __builtin_amdgcn_rcpf(scale);
    r = __builtin_fmaf(__builtin_fmaf(-r0, scale, 1.0f), r0, r0);
  }
  __device__ __forceinline__ float operator()(float x) const {
    const float q0 = x * r;
    const float e = __builtin_fmaf(-q0, s, x);
    const float q = __builtin_fmaf(e, r, q0);
    return KEEP_SIGN ? __builtin_copysignf(q, x) : q;
  }
};

__device__ __forceinline__ bool fast_group(float peak) { return peak >= 0x1p-80f; }

// int8 quotients in two VALU ops per value: with r = RN(1 / s) as above and its remainder
// rl = RN(fma(-s, r, 1) * r), q = fma(x, r, x * rl).  For every bf16 absmax 2^-80 <= peak < 2^100 and every
// bf16 |x| <= peak, both signs, q gives the same int8 code as IEEE x / s for both roundings (exhaustive CPU
// check).  From 2^100 up, rl falls into the subnormals and loses the bits it carries, so those groups
// divide.  (x * r alone is not enough: it changes codes next to exact .5 ties, e.g. x = peak / 2.)
struct FastDivI8 {
  float r, rl;
  __device__ __forceinline__ explicit FastDivI8(float scale) {
    const float r0 = __builtin_amdgcn_rcpf(scale);
    r = __builtin_fmaf(__builtin_fmaf(-r0, scale, 1.0f), r0, r0);
    rl = __builtin_fmaf(-scale, r, 1.0f) * r;
  }
  __device__ __forceinline__ float operator()(float x) const { return __builtin_fmaf(x, r, x * rl); }
};

__device__ __forceinline__ bool fast_group_i8(float peak) { return peak >= 0x1p-80f && peak < 0x1p100f; }

// The fast quotient and its group condition for each code kind: two ops for int8, three for e4m3.
template <int KIND>
struct FastQuot {
  using Div = FastDivI8;
  __device__ __forceinline__ static bool ok(float peak) { return fast_group_i8(peak); }
};
template <>
struct FastQuot<HN_KIND_FP8> {
  using Div = FastDiv<true>;
  __device__ __forceinline__ static bool ok(float peak) { return fast_group(peak); }
};

// Code of y = x / scale with |x| <= the group's peak (so |y| <= 127 * (1 + 2^-22) and no clamp is needed):
// round half away from zero as trunc(y + copysign(0.5, y)); NaN gives 0.
__device__ __forceinline__ int round_half_away_i8_inrange(float y) {
  return (int)(y + __builtin_copysignf(0.5f, y));
}

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

// The half-even int8 code of y, for |y| <= 127 (1 + 2^-22), as the low byte of the result: adding 1.5 * 2^23
// rounds y to an integer n, ties to even (the sum's fp32 spacing is 1 and 1.5 * 2^23 is even), leaving the
// bits 0x4B400000 + n, whose low byte is n's two's-complement byte.  One op instead of rint and a conversion;
// only the low byte is meaningful, which is all pack4_i8 reads.
__device__ __forceinline__ int rne_code_bits(float y) { return (int)__float_as_uint(y + 12582912.0f); }

// Pack four int8 codes (low byte first).
__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
  const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);  // [a.b0, b.b0, 0, 0]
  const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
  return __builtin_amdgcn_perm(cd, ab, 0x05040100u);                                // [ab.b0, ab.b1, cd.b0, cd.b1]
}

// Streamed accesses (each byte read or written once per launch): non-temporal, so the stream does not
// displace cached data that is reused (per-batch factors, tables).  A 16-byte copy over 1 GiB buffers
// runs at ~6.5 TB/s this way against ~6.2 TB/s with plain loads and stores.
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
  return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
__device__ __forceinline__ uint2 ld_nt8(const void* p) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  const v2i v = __builtin_nontemporal_load(reinterpret_cast<const v2i*>(p));
  return make_uint2((uint32_t)v[0], (uint32_t)v[1]);
}
__device__ __forceinline__ void st_nt16(void* p, uint4 v) {
  __builtin_nontemporal_store(v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w}, reinterpret_cast<v4i*>(p));
}
__device__ __forceinline__ void st_nt8(void* p, uint2 v) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(v2i{(int)v.x, (int)v.y}, reinterpret_cast<v2i*>(p));
}

// fp32 pair -> packed bf16 pair, round to nearest even, with the hardware conversion (v_cvt_pk_bf16_f32).
// It equals f32_to_bf16_bits for every non-NaN input; NaNs keep their sign and payload bits (quieted)
// instead of becoming 0x7FC0, so callers use it where the values are known to be finite.
__device__ __forceinline__ uint32_t bf16x2_finite(float a, float b) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
}

// ----------------------------------------------------------------------------------------------
// direct-to-LDS loads (gfx950)

typedef __attribute__((address_space(3))) void* lds_ptr;

// Wave-wide direct-to-LDS loads: lane i's 16 (or 4) bytes from g land at lds_wave_base + i * 16 (or 4).
__device__ __forceinline__ void g2lds16(const void* g, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr)lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void g2lds4(const void* g, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr)lds_wave_base, 4, 0, 0);
}

// The same through a raw buffer descriptor: lane i's bytes at base + soffset + voffset_i (voffset in a
// VGPR, soffset in an SGPR), so a stage's loads need no per-lane 64-bit address arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  // no stride, every 32-bit offset in range, gfx9 raw-buffer format word
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
}
__device__ __forceinline__ void b2lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, char* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds_wave_base, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void b2lds4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, char* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds_wave_base, 4, voff, soff, 0, 0);
}

// ----------------------------------------------------------------------------------------------
// cross-lane reductions (wave64)

__device__ __forceinline__ float shfl_xor_f(float v, int mask, int width = 64) { return __shfl_xor(v, mask, width); }

// DPP lane moves (VALU, no LDS round trip).  Controls: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140, row_bcast15 = 0x142, row_bcast31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Lane n of each DPP row of 16, read by every lane of the row (row_newbcast); n must fold to a constant.
__device__ __forceinline__ float row_bcast(float v, int n) {
  switch (n) {
    case 0: return dpp_f<0x150>(v);
    case 1: return dpp_f<0x151>(v);
    case 2: return dpp_f<0x152>(v);
    case 3: return dpp_f<0x153>(v);
    case 4: return dpp_f<0x154>(v);
    case 5: return dpp_f<0x155>(v);
    case 6: return dpp_f<0x156>(v);
    case 7: return dpp_f<0x157>(v);
    case 8: return dpp_f<0x158>(v);
    case 9: return dpp_f<0x159>(v);
    case 10: return dpp_f<0x15A>(v);
    case 11: return dpp_f<0x15B>(v);
    case 12: return dpp_f<0x15C>(v);
    case 13: return dpp_f<0x15D>(v);
    case 14: return dpp_f<0x15E>(v);
    default: return dpp_f<0x15F>(v);
  }
}

// Max over the 16 lanes of each DPP row of non-negative values (compared as integers: the order of
// non-negative floats, NaN above +inf).  Every lane of the row gets the result.
__device__ __forceinline__ float row16_max_nonneg(float v) {
  uint32_t u = __float_as_uint(v);
  u = max(u, dpp_u<0xB1>(u));
  u = max(u, dpp_u<0x4E>(u));
  u = max(u, dpp_u<0x141>(u));
  u = max(u, dpp_u<0x140>(u));
  return __uint_as_float(u);
}

// Sum over the 64 lanes: butterflies within each row of 16, then rows 0..3 folded into lane 63 with row
// broadcasts; the total is read from lane 63 (wave-uniform).
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  v += dpp_f<0x142, 0xa>(v);  // rows 1, 3 += last lane of rows 0, 2
  v += dpp_f<0x143, 0xc>(v);  // rows 2, 3 += last lane of row 1
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Max over the 64 lanes of non-negative values (as row16_max_nonneg), wave-uniform.
__device__ __forceinline__ float wave_max_nonneg(float v) {
  uint32_t u = __float_as_uint(row16_max_nonneg(v));
  u = max(u, dpp_u<0x142, 0xa>(u));
  u = max(u, dpp_u<0x143, 0xc>(u));
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)u, 63));
}

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

// The one-call linear (linear.hip): workspace size, argument checks, and quantize-then-GEMM into a
// workspace that holds the activation codes and scales.
int64_t linear_workspace_bytes(int64_t M, int64_t K, int64_t group);
int check_linear(const char* who, const void* x, int64_t M, int64_t N, int64_t K, int64_t group, int kind,
                 const void* qw, const float* sw, const void* out);
int run_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind, int rounding,
               const void* qw, int64_t ldw, const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias,
               int bias_dtype, int64_t N, void* out, int out_dtype, int64_t ldo, uint8_t* ws, void* stream);
}  // namespace hn

#define HN_REQUIRE(cond, ...)            \
  do {                                   \
    if (!(cond)) {                       \
      ::hn::set_error(__VA_ARGS__);      \
      return HN_ERR_ARG;                 \
    }                                    \
  } while (0)

#define HN_LAUNCH_CHECK(what) ::hn::hip_status(hipGetLastError(), what)
