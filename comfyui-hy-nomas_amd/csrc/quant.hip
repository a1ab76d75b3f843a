// Dynamic activation quantization (hy_nomas/kernels.py:22-54, _quantize_kernel / quantize_activations).
//
// Two layouts of scales:
//   group 128 -- the reference: one scale per token and 128 channels.  Sixteen lanes own one group
//                (16 x 16-byte loads = 128 bf16); the group absmax is a 16-lane DPP-row reduction.
//   group K   -- one scale per token.  One wavefront owns one row and keeps it in registers between
//                the absmax pass and the code pass, so x is read from HBM once.
// Both are single-pass HBM-bound kernels: 16-byte loads, 8-byte code stores, fp32 math.
#include "hn_common.h"

namespace hn {

// 8 consecutive input values of one lane, loaded as 16 (2-byte types) or 32 (fp32) bytes.
template <int DT>
struct Chunk8 {
  uint4 v[DT == HN_DTYPE_F32 ? 2 : 1];
  __device__ __forceinline__ void load(const char* p) {
    v[0] = ld_nt16(p);
    if constexpr (DT == HN_DTYPE_F32) v[1] = ld_nt16(p + 16);
  }
  __device__ __forceinline__ void widen(float* f) const {
    if constexpr (DT == HN_DTYPE_F32) {
      f[0] = __uint_as_float(v[0].x); f[1] = __uint_as_float(v[0].y);
      f[2] = __uint_as_float(v[0].z); f[3] = __uint_as_float(v[0].w);
      f[4] = __uint_as_float(v[1].x); f[5] = __uint_as_float(v[1].y);
      f[6] = __uint_as_float(v[1].z); f[7] = __uint_as_float(v[1].w);
    } else {
      In<DT>::widen8(v[0], f);
    }
  }
  static constexpr int kElemBytes = DT == HN_DTYPE_F32 ? 4 : 2;
};

// Codes of 8 values with one scale; returns them packed in 8 bytes.  FAST: bf16-valued inputs in a group
// with FastQuot<KIND>::ok(peak) -- the exact fast quotient, and (int8) no clamp since |x| <= peak.  Otherwise an
// IEEE division and the clamped rounding.
template <int KIND, int ROUND, bool FAST>
__device__ __forceinline__ uint2 encode8(const float* f, float scale) {
  int c[8];
  if constexpr (FAST && KIND == HN_KIND_FP8) {
    const typename FastQuot<KIND>::Div div(scale);
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = div(f[i]);
    return make_uint2(e4m3_pack4_hw(y[0], y[1], y[2], y[3]), e4m3_pack4_hw(y[4], y[5], y[6], y[7]));
  } else if constexpr (FAST) {
    const typename FastQuot<KIND>::Div div(scale);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float y = div(f[i]);
      if constexpr (ROUND == HN_ROUND_HALF_EVEN) c[i] = rne_code_bits(y);  // low byte only: packed below
      else c[i] = round_half_away_i8_inrange(y);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float y = f[i] / scale;
      if constexpr (KIND == HN_KIND_FP8) c[i] = (int)e4m3_encode(y);
      else c[i] = round_i8<ROUND>(y);
    }
  }
  return make_uint2(pack4_i8(c[0], c[1], c[2], c[3]), pack4_i8(c[4], c[5], c[6], c[7]));
}

// Scale and codes of one group from its absmax `peak` (non-negative, NaN-free).  bf16 inputs in a group
// with FastQuot<KIND>::ok(peak) use the fast exact quotients (hn_common.h); other groups and inputs divide.
template <int DT, int KIND, int ROUND>
__device__ __forceinline__ uint2 encode8_group(const float* f, float peak, float& scale) {
  if constexpr (DT == HN_DTYPE_BF16) {
    if (__builtin_expect(FastQuot<KIND>::ok(peak), 1)) {
      scale = KIND == HN_KIND_INT8 ? int8_scale_fast(peak) : fp8_scale_fast(peak);
      return encode8<KIND, ROUND, true>(f, scale);
    }
  }
  scale = KIND == HN_KIND_INT8 ? int8_scale(peak) : fp8_scale(peak);
  return encode8<KIND, ROUND, false>(f, scale);
}

// ---------------------------------------------------------------------------------------------
// group = 128: 16 lanes per group, UNROLL groups per lane-slot in flight.
constexpr int kG128Threads = 256;
constexpr int kG128Unroll = 4;

template <int DT, int KIND, int ROUND>
__global__ __launch_bounds__(kG128Threads) void quant_g128_kernel(const char* __restrict__ x, int64_t ldx_bytes,
                                                                  uint8_t* __restrict__ q, int64_t ldq,
                                                                  float* __restrict__ s, int64_t lds,
                                                                  int64_t groups_per_row, int64_t n_groups) {
  using C = Chunk8<DT>;
  const int lane16 = threadIdx.x & 15;
  const int slot = threadIdx.x >> 4;  // 16 group slots per block
  const int64_t base = (int64_t)blockIdx.x * (16 * kG128Unroll);
  C chunk[kG128Unroll];
  int64_t row[kG128Unroll], grp[kG128Unroll];
  bool live[kG128Unroll];
#pragma unroll
  for (int u = 0; u < kG128Unroll; u++) {
    int64_t gi = base + u * 16 + slot;
    live[u] = gi < n_groups;
    gi = live[u] ? gi : 0;
    row[u] = gi / groups_per_row;
    grp[u] = gi - row[u] * groups_per_row;
    chunk[u].load(x + row[u] * ldx_bytes + (grp[u] * 128 + lane16 * 8) * C::kElemBytes);
  }
#pragma unroll
  for (int u = 0; u < kG128Unroll; u++) {
    float f[8];
    chunk[u].widen(f);
    float peak = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) peak = __builtin_fmaxf(peak, __builtin_fabsf(f[i]));
    peak = row16_max_nonneg(peak);  // per-lane maxima are NaN-free and >= 0
    float sc;
    const uint2 codes = encode8_group<DT, KIND, ROUND>(f, peak, sc);
    if (live[u]) {
      st_nt8(q + row[u] * ldq + grp[u] * 128 + lane16 * 8, codes);
      if (lane16 == 0) s[row[u] * lds + grp[u]] = sc;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// group = K: one wave per row, CPL chunks of 8 values per lane held in registers.
constexpr int kRowThreads = 256;

template <int DT, int KIND, int ROUND, int CPL>
__global__ __launch_bounds__(kRowThreads) void quant_row_kernel(const char* __restrict__ x, int64_t ldx_bytes,
                                                                uint8_t* __restrict__ q, int64_t ldq,
                                                                float* __restrict__ s, int64_t lds, int64_t M,
                                                                int64_t K) {
  using C = Chunk8<DT>;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (r >= M) return;  // whole wave exits together
  const int64_t nchunk = K / 8;
  const char* xr = x + r * ldx_bytes;
  C chunk[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    int64_t c = lane + 64 * i;
    if (c < nchunk) chunk[i].load(xr + c * 8 * C::kElemBytes);
  }
  float peak = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    int64_t c = lane + 64 * i;
    if (c < nchunk) {
      float f[8];
      chunk[i].widen(f);
#pragma unroll
      for (int j = 0; j < 8; j++) peak = __builtin_fmaxf(peak, __builtin_fabsf(f[j]));
    }
  }
  peak = wave_max_nonneg(peak);  // per-lane maxima are NaN-free and >= 0
  float sc = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    int64_t c = lane + 64 * i;
    if (c < nchunk) {
      float f[8];
      chunk[i].widen(f);
      st_nt8(q + r * ldq + c * 8, encode8_group<DT, KIND, ROUND>(f, peak, sc));
    }
  }
  if (lane == 0) s[r * lds] = sc;  // lane 0 always owns chunk 0 (K >= 128)
}

template <int DT, int KIND, int ROUND>
static int launch_quant(const void* x, int64_t ldx, int64_t M, int64_t K, int64_t group, void* q, int64_t ldq,
                        float* s, int64_t lds, hipStream_t st) {
  const int eb = DT == HN_DTYPE_F32 ? 4 : 2;
  if (group == 128) {
    const int64_t gpr = K / 128, n = M * gpr;
    const int64_t blocks = (n + 16 * kG128Unroll - 1) / (16 * kG128Unroll);
    hipLaunchKernelGGL((quant_g128_kernel<DT, KIND, ROUND>), dim3((unsigned)blocks), dim3(kG128Threads), 0, st,
                       (const char*)x, ldx * eb, (uint8_t*)q, ldq, s, lds, gpr, n);
    return HN_LAUNCH_CHECK("quant_g128_kernel");
  }
  // one scale per row (group == K)
  const int64_t cpl = (K / 8 + 63) / 64;
  const unsigned blocks = (unsigned)((M + 3) / 4);
#define HN_ROW_CASE(N)                                                                                       \
  if (cpl <= N) {                                                                                            \
    hipLaunchKernelGGL((quant_row_kernel<DT, KIND, ROUND, N>), dim3(blocks), dim3(kRowThreads), 0, st,       \
                       (const char*)x, ldx * eb, (uint8_t*)q, ldq, s, lds, M, K);                            \
    return HN_LAUNCH_CHECK("quant_row_kernel");                                                              \
  }
  HN_ROW_CASE(1) HN_ROW_CASE(2) HN_ROW_CASE(3) HN_ROW_CASE(4) HN_ROW_CASE(6) HN_ROW_CASE(8) HN_ROW_CASE(12)
  HN_ROW_CASE(16) HN_ROW_CASE(24) HN_ROW_CASE(32)
#undef HN_ROW_CASE
  set_error("hn_quantize_act: per-token quantization supports K <= 16384 (got K=%lld)", (long long)K);
  return HN_ERR_UNSUPPORTED;
}

template <int DT>
static int dispatch_quant(const void* x, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind, int rounding,
                          void* q, int64_t ldq, float* s, int64_t lds, hipStream_t st) {
  if (kind == HN_KIND_FP8) return launch_quant<DT, HN_KIND_FP8, HN_ROUND_HALF_AWAY>(x, ldx, M, K, group, q, ldq, s, lds, st);
  if (rounding == HN_ROUND_HALF_EVEN)
    return launch_quant<DT, HN_KIND_INT8, HN_ROUND_HALF_EVEN>(x, ldx, M, K, group, q, ldq, s, lds, st);
  return launch_quant<DT, HN_KIND_INT8, HN_ROUND_HALF_AWAY>(x, ldx, M, K, group, q, ldq, s, lds, st);
}

}  // namespace hn

extern "C" int hn_quantize_act(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind,
                               int rounding, void* q, int64_t ldq, float* s, int64_t lds, void* stream) {
  using namespace hn;
  HN_REQUIRE(M >= 0 && K > 0, "hn_quantize_act: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  HN_REQUIRE(K % 128 == 0, "hn_quantize_act: K=%lld is not a multiple of 128", (long long)K);
  HN_REQUIRE(group == 128 || group == K, "hn_quantize_act: group must be 128 or K (got %lld)", (long long)group);
  HN_REQUIRE(kind == HN_KIND_INT8 || kind == HN_KIND_FP8, "hn_quantize_act: bad kind %d", kind);
  HN_REQUIRE(rounding == HN_ROUND_HALF_AWAY || rounding == HN_ROUND_HALF_EVEN, "hn_quantize_act: bad rounding %d",
             rounding);
  HN_REQUIRE(ldx >= K && ldq >= K && lds >= K / group, "hn_quantize_act: row strides smaller than the rows");
  HN_REQUIRE(ldx % 8 == 0 && ldq % 8 == 0, "hn_quantize_act: row strides must be multiples of 8 elements");
  HN_REQUIRE(x && q && s, "hn_quantize_act: null pointer");
  HN_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0, "hn_quantize_act: x must be 16-byte and q 8-byte aligned");
  if (M == 0) return HN_OK;
  hipStream_t st = (hipStream_t)stream;
  switch (x_dtype) {
    case HN_DTYPE_BF16: return dispatch_quant<HN_DTYPE_BF16>(x, ldx, M, K, group, kind, rounding, q, ldq, s, lds, st);
    case HN_DTYPE_F16: return dispatch_quant<HN_DTYPE_F16>(x, ldx, M, K, group, kind, rounding, q, ldq, s, lds, st);
    case HN_DTYPE_F32: return dispatch_quant<HN_DTYPE_F32>(x, ldx, M, K, group, kind, rounding, q, ldq, s, lds, st);
    default: break;
  }
  set_error("hn_quantize_act: unsupported x dtype %d", x_dtype);
  return HN_ERR_UNSUPPORTED;
}
