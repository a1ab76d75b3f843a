// Fused DiT elementwise kernels (hy_nomas/fused.py, hy_nomas/kernels.py:173-207).
//
// Row kernels (adaLN, adaLN+quant): one wavefront per token row; the row is loaded once with 16-byte
// loads, kept in registers for the mean / variance / output passes, and the statistics are wave
// reductions.  Head kernels (QK norm + RoPE): D/8 lanes per (token, head), 16 bytes per lane.
// The gated residual streams rows with 16-byte accesses.  All are single-pass and HBM-bound.
#include "hn_common.h"

namespace hn {

template <int DT>
__device__ __forceinline__ void widen8(const uint4& v, float* f) {
  In<DT>::widen8(v, f);
}

template <int DT>
__device__ __forceinline__ uint4 narrow8(const float* f) {
  return make_uint4(pack2_out<DT>(f[0], f[1]), pack2_out<DT>(f[2], f[3]), pack2_out<DT>(f[4], f[5]),
                    pack2_out<DT>(f[6], f[7]));
}

// ---------------------------------------------------------------------------------------------
// value rounding to the tensor dtype, kept in fp32
template <int DT>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (DT == HN_DTYPE_BF16) return rbf16(v);
  else return f16_bits_to_f32(f32_to_f16_bits(v));
}

// 8 fp32 values -> 8 packed 2-byte values.  FINITE: the values are known not to be NaN, so the hardware
// bf16 conversion (equal to the torch rule on every non-NaN value) is used.
// fp16: the fp32 values are materialized first; the compiler would otherwise fuse a producing fma with the
// conversion into one mixed-precision fma rounding once to fp16, where the reference rounds to fp32 first.
template <int DT, bool FINITE>
__device__ __forceinline__ uint4 narrow8x(const float* f) {
  if constexpr (DT == HN_DTYPE_BF16 && FINITE) {
    return make_uint4(bf16x2_finite(f[0], f[1]), bf16x2_finite(f[2], f[3]), bf16x2_finite(f[4], f[5]),
                      bf16x2_finite(f[6], f[7]));
  } else if constexpr (DT == HN_DTYPE_F16) {
    float g[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      g[k] = f[k];
      asm volatile("" : "+v"(g[k]));
    }
    return narrow8<DT>(g);
  } else {
    return narrow8<DT>(f);
  }
}

// ---------------------------------------------------------------------------------------------
// adaLN: y = norm(x) * rbf16(1 + scale[b]) + shift[b]          (fused.py:37-52)
// adaLN + quant: y = rbf16(...), then int8 per 128 channels      (kernels.py:173-195)
//
// One wavefront per token row, 8 rows per block, all rows of a block in one batch b.  Each wave issues its
// row's loads first; meanwhile the block stages b's modulation factors g = rbf16(1 + scale[b]) and
// h = shift[b] as fp32 in LDS, in four planes of D/8 float4 (g[0:4], g[4:8], h[0:4], h[4:8] of each
// 8-channel chunk) so a wave's reads are consecutive 16-byte slots.  Rows whose statistics are not
// finite (NaN / inf inputs) take the exact software rounding.
constexpr int kRowWaves = 8;
constexpr int kRowThreads = kRowWaves * 64;

template <int DT, int NORM, bool QUANT, int ROUND, int CPL, bool FULL, bool PT>
__global__ __launch_bounds__(kRowThreads) void adaln_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ shift,
                                                            const uint16_t* __restrict__ scale, int64_t L,
                                                            int64_t D, float rd, float eps, int blocks_per_batch,
                                                            uint16_t* __restrict__ y, int8_t* __restrict__ q,
                                                            float* __restrict__ s) {
  extern __shared__ float4 fac[];
  const int nchunk = (int)(D / 8);
  const int64_t b = blockIdx.x / blocks_per_batch;
  const int jb = blockIdx.x % blocks_per_batch;
  // quantizing rows: the wave index is made uniform, so the row index and the code and scale output bases
  // stay in scalar registers (the plain adaLN rows measured faster without it)
  const int lane = threadIdx.x & 63;
  const int wave = QUANT ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : (int)(threadIdx.x >> 6);
  const int64_t l = (int64_t)jb * kRowWaves + wave;
  const bool live = l < L;  // whole wave
  const int64_t r = b * L + (live ? l : L - 1);
  auto has = [&](int i) { return FULL || lane + 64 * i < nchunk; };
  uint4 xv[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++)
    if (has(i)) xv[i] = ld_nt16(x + r * D + (lane + 64 * i) * 8);
  // the row's outputs: chunk i of this lane at a fixed offset from one per-row base (512 codes / 1 KB of
  // 2-byte outputs / 4 group scales further per chunk), so the stores take immediate offsets
  uint16_t* const yrow = QUANT ? nullptr : y + r * D + lane * 8;
  int8_t* const qrow = QUANT ? q + r * D + lane * 8 : nullptr;
  float* const srow = QUANT && !PT ? s + r * (D / 128) + (lane >> 4) : nullptr;

  int fin = 1;
  for (int c = threadIdx.x; c < nchunk; c += kRowThreads) {
    float sc[8], sh[8], g[8];
    widen8<DT>(*reinterpret_cast<const uint4*>(scale + b * D + c * 8), sc);
    widen8<DT>(*reinterpret_cast<const uint4*>(shift + b * D + c * 8), sh);
    // g = rbf16(1 + scale) is finite exactly when scale is (1 + the largest bf16 rounds back to it)
    bool f = true;
#pragma unroll
    for (int j = 0; j < 8; j++) f = f && __builtin_isfinite(sc[j]) && __builtin_isfinite(sh[j]);
    if (f) {  // no NaN: the hardware conversion is the software rounding
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const uint32_t w = bf16x2_finite(1.0f + sc[j], 1.0f + sc[j + 1]);
        g[j] = __uint_as_float(w << 16);
        g[j + 1] = __uint_as_float(w & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) g[j] = rbf16(1.0f + sc[j]);
    }
    fin &= f;
    fac[c] = make_float4(g[0], g[1], g[2], g[3]);
    fac[nchunk + c] = make_float4(g[4], g[5], g[6], g[7]);
    fac[2 * nchunk + c] = make_float4(sh[0], sh[1], sh[2], sh[3]);
    fac[3 * nchunk + c] = make_float4(sh[4], sh[5], sh[6], sh[7]);
  }
  // Block-wide AND of the staging threads' finiteness: each wave's vote goes to one byte past the factor
  // planes, so a single barrier publishes both the planes and the votes.
  uint8_t* votes = reinterpret_cast<uint8_t*>(fac + 4 * nchunk);
  const bool wave_fin = __builtin_amdgcn_ballot_w64(!fin) == 0;
  if (lane == 0) votes[threadIdx.x >> 6] = wave_fin;
  __syncthreads();
  static_assert(kRowWaves == 8, "eight votes are read as one 8-byte word");
  const bool fac_finite = *reinterpret_cast<const uint64_t*>(votes) == 0x0101010101010101ull;
  if (!live) return;

  // Rows of up to 4096 channels are widened once into fp32 registers; wider rows stay packed and are
  // widened in each pass.
  constexpr bool KEEP = CPL <= 8;
  float f[KEEP ? CPL : 1][8];
  if constexpr (KEEP) {
#pragma unroll
    for (int i = 0; i < CPL; i++)
      if (has(i)) widen8<DT>(xv[i], f[i]);
  }
  // value j of chunk i of the row
  auto val = [&](int i, int j) -> float {
    if constexpr (KEEP) {
      return f[i][j];
    } else {
      const uint32_t w = (&xv[i].x)[j >> 1];
      if constexpr (DT == HN_DTYPE_BF16) return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
      else return f16_bits_to_f32((j & 1) ? (w >> 16) : (w & 0xffffu));
    }
  };
  // statistics in fp32: per-lane sums, then a wave reduction (two passes, as the reference); the fp32
  // copies are centred in place by the second pass
  float mean = 0.0f;
  if constexpr (NORM == HN_NORM_LAYER) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; i++)
      if (has(i))
#pragma unroll
        for (int j = 0; j < 8; j++) acc += val(i, j);
    mean = div_by_const(wave_sum_dpp(acc), (float)D, rd);
  }
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; i++)
    if (has(i))
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float c = val(i, j) - mean;
        if constexpr (KEEP) f[i][j] = c;
        sq = __builtin_fmaf(c, c, sq);
      }
  const float var = div_by_const(wave_sum_dpp(sq), (float)D, rd);
  const float rstd = rsqrt_refined(var + eps);
  const bool finite = fac_finite && __builtin_isfinite(mean) && __builtin_isfinite(rstd);
  if constexpr (QUANT && PT) {
    // one scale per token: y = rbf16(modulated norm) for the whole row, the row absmax, then the codes
    static_assert(!QUANT || !PT || KEEP, "per-token adaLN quantization keeps the row in registers (D <= 4096)");
    float peak = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const int c = lane + 64 * i;
      if (has(i)) {
        const float4 g0 = fac[c], g1 = fac[nchunk + c], h0 = fac[2 * nchunk + c], h1 = fac[3 * nchunk + c];
        const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const float h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        if (__builtin_expect(finite, 1) && DT == HN_DTYPE_BF16) {
          // finite statistics and factors: no NaN reaches the rounding, so the hardware conversion applies
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            const uint32_t w = bf16x2_finite(__builtin_fmaf(f[i][j] * rstd, g[j], h[j]),
                                             __builtin_fmaf(f[i][j + 1] * rstd, g[j + 1], h[j + 1]));
            f[i][j] = __uint_as_float(w << 16);
            f[i][j + 1] = __uint_as_float(w & 0xffff0000u);
            peak = __builtin_fmaxf(peak, __builtin_fabsf(f[i][j]));
            peak = __builtin_fmaxf(peak, __builtin_fabsf(f[i][j + 1]));
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float o = __builtin_fmaf(f[i][j] * rstd, g[j], h[j]);
            f[i][j] = rbf16(o);
            peak = __builtin_fmaxf(peak, __builtin_fabsf(f[i][j]));  // NaN-free, >= 0
          }
        }
      }
    }
    peak = wave_max_nonneg(peak);
    const bool fast = fast_group_i8(peak);
    const float gs = fast ? int8_scale_fast(peak) : int8_scale(peak);
    const FastDivI8 div(gs);
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const int c = lane + 64 * i;
      if (has(i)) {
        int cd[8];
        if (__builtin_expect(fast, 1)) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float v = div(f[i][j]);
            cd[j] = ROUND == HN_ROUND_HALF_EVEN ? rne_code_bits(v) : round_half_away_i8_inrange(v);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; j++) cd[j] = round_i8<ROUND>(f[i][j] / gs);
        }
        st_nt8(qrow + 512 * i, make_uint2(pack4_i8(cd[0], cd[1], cd[2], cd[3]), pack4_i8(cd[4], cd[5], cd[6], cd[7])));
      }
    }
    if (lane == 0) s[r] = gs;
    return;
  }
  if constexpr (QUANT && !PT && KEEP && FULL && DT == HN_DTYPE_BF16) {
    // g128 codes of a finite row whose groups all take the fast quotient (the usual case): every chunk is
    // modulated and rounded first, the group peaks reduced together, and one wave vote replaces the
    // per-group branches; codes and scales are those of the general loop below.
    if (__builtin_expect(finite, 1)) {
      float pk[CPL];
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const int c = lane + 64 * i;
        const float4 g0 = fac[c], g1 = fac[nchunk + c], h0 = fac[2 * nchunk + c], h1 = fac[3 * nchunk + c];
        const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const float h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        float peak = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          const uint32_t w = bf16x2_finite(__builtin_fmaf(f[i][j] * rstd, g[j], h[j]),
                                           __builtin_fmaf(f[i][j + 1] * rstd, g[j + 1], h[j + 1]));
          f[i][j] = __uint_as_float(w << 16);
          f[i][j + 1] = __uint_as_float(w & 0xffff0000u);
          peak = __builtin_fmaxf(peak, __builtin_fabsf(f[i][j]));
          peak = __builtin_fmaxf(peak, __builtin_fabsf(f[i][j + 1]));
        }
        pk[i] = peak;
      }
#pragma unroll
      for (int i = 0; i < CPL; i++) pk[i] = row16_max_nonneg(pk[i]);  // D % 128 == 0: a DPP row holds one group
      // Each group's scale and quotient constants are formed once, in lane k < CPL of its 16-lane row (lane k
      // takes chunk k's group, channels 128 (4k + row) on), and chunk i reads them from lane i of the row with
      // a DPP broadcast, instead of every lane forming them for each of its chunks; one store then writes the
      // row's group scales.  The lanes k >= CPL keep chunk 0's group, so the vote covers exactly the groups.
      static_assert(CPL <= 16, "one lane of the row per chunk");
      const int k = lane & 15;
      float pkk = pk[0];
#pragma unroll
      for (int i = 1; i < CPL; i++) pkk = k == i ? pk[i] : pkk;
      if (__builtin_expect(__all(fast_group_i8(pkk)), 1)) {
        const float gs = int8_scale_fast(pkk);
        const FastDivI8 div_k(gs);
#pragma unroll
        for (int i = 0; i < CPL; i++) {
          FastDivI8 div = div_k;
          div.r = row_bcast(div_k.r, i);
          div.rl = row_bcast(div_k.rl, i);
          int cd[8];
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float v = div(f[i][j]);
            cd[j] = ROUND == HN_ROUND_HALF_EVEN ? rne_code_bits(v) : round_half_away_i8_inrange(v);
          }
          st_nt8(qrow + 512 * i, make_uint2(pack4_i8(cd[0], cd[1], cd[2], cd[3]), pack4_i8(cd[4], cd[5], cd[6], cd[7])));
        }
        if (k < CPL) srow[4 * k] = gs;  // srow[4 k] is group 4 k + row
      } else {
#pragma unroll
        for (int i = 0; i < CPL; i++) {
          const float gs = fast_group_i8(pk[i]) ? int8_scale_fast(pk[i]) : int8_scale(pk[i]);
          int cd[8];
          if (fast_group_i8(pk[i])) {
            const FastDivI8 div(gs);
#pragma unroll
            for (int j = 0; j < 8; j++) {
              const float v = div(f[i][j]);
              cd[j] = ROUND == HN_ROUND_HALF_EVEN ? rne_code_bits(v) : round_half_away_i8_inrange(v);
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; j++) cd[j] = round_i8<ROUND>(f[i][j] / gs);
          }
          st_nt8(qrow + 512 * i, make_uint2(pack4_i8(cd[0], cd[1], cd[2], cd[3]), pack4_i8(cd[4], cd[5], cd[6], cd[7])));
          srow[4 * i] = gs;
        }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const int c = lane + 64 * i;
    if (has(i)) {
      const float4 g0 = fac[c], g1 = fac[nchunk + c], h0 = fac[2 * nchunk + c], h1 = fac[3 * nchunk + c];
      const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
      const float h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float n = (KEEP ? val(i, j) : val(i, j) - mean) * rstd;
        o[j] = __builtin_fmaf(n, g[j], h[j]);  // n * rbf16(1 + scale) + shift, contracted as Triton does
      }
      if constexpr (!QUANT) {
        const uint4 packed = finite ? narrow8x<DT, true>(o) : narrow8x<DT, false>(o);
        st_nt16(yrow + 512 * i, packed);
      } else {
        float peak = 0.0f;
        if (__builtin_expect(finite, 1) && DT == HN_DTYPE_BF16) {
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            const uint32_t w = bf16x2_finite(o[j], o[j + 1]);
            o[j] = __uint_as_float(w << 16);
            o[j + 1] = __uint_as_float(w & 0xffff0000u);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; j++) o[j] = rbf16(o[j]);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) peak = __builtin_fmaxf(peak, __builtin_fabsf(o[j]));  // NaN-free, >= 0
        // D % 128 == 0: the 16 lanes of a DPP row hold exactly one 128-channel group
        peak = row16_max_nonneg(peak);
        float gs;
        int cd[8];
        if (__builtin_expect(fast_group_i8(peak), 1)) {
          gs = int8_scale_fast(peak);
          const FastDivI8 div(gs);
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float v = div(o[j]);
            cd[j] = ROUND == HN_ROUND_HALF_EVEN ? rne_code_bits(v) : round_half_away_i8_inrange(v);
          }
        } else {
          gs = int8_scale(peak);
#pragma unroll
          for (int j = 0; j < 8; j++) cd[j] = round_i8<ROUND>(o[j] / gs);
        }
        st_nt8(qrow + 512 * i, make_uint2(pack4_i8(cd[0], cd[1], cd[2], cd[3]), pack4_i8(cd[4], cd[5], cd[6], cd[7])));
        // all 16 lanes of the group store the same scale to the same address (no divergent branch)
        srow[4 * i] = gs;
      }
    }
  }
}

template <int DT, int NORM, bool QUANT, int ROUND, bool PT>
static int launch_adaln(const void* x, const void* shift, const void* scale, int64_t B, int64_t L, int64_t D,
                        float eps, void* y, int8_t* q, float* s, hipStream_t st) {
  const int64_t cpl = (D / 8 + 63) / 64;
  const int64_t per_batch = (L + kRowWaves - 1) / kRowWaves;
  if (B * per_batch > 0x7fffffff) {
    set_error("adaln: too many rows (B=%lld, L=%lld)", (long long)B, (long long)L);
    return HN_ERR_UNSUPPORTED;
  }
  const unsigned blocks = (unsigned)(B * per_batch);
  const size_t lds = (size_t)D * 8 + 16;  // four planes of D/8 float4, then the waves' finiteness votes
  const float rd = 1.0f / (float)D;  // correctly rounded: the kernels divide by D with one correction step
#define HN_CASE(N)                                                                                              \
  if (cpl <= N) {                                                                                               \
    if (D == 512 * N)                                                                                           \
      hipLaunchKernelGGL((adaln_kernel<DT, NORM, QUANT, ROUND, N, true, PT>), dim3(blocks), dim3(kRowThreads), lds, \
                         st, (const uint16_t*)x, (const uint16_t*)shift, (const uint16_t*)scale, L, D, rd, eps, \
                         (int)per_batch, (uint16_t*)y, q, s);                                                   \
    else                                                                                                        \
      hipLaunchKernelGGL((adaln_kernel<DT, NORM, QUANT, ROUND, N, false, PT>), dim3(blocks), dim3(kRowThreads), lds,\
                         st, (const uint16_t*)x, (const uint16_t*)shift, (const uint16_t*)scale, L, D, rd, eps, \
                         (int)per_batch, (uint16_t*)y, q, s);                                                   \
    return HN_LAUNCH_CHECK("adaln_kernel");                                                                     \
  }
  HN_CASE(1) HN_CASE(2) HN_CASE(3) HN_CASE(4) HN_CASE(5) HN_CASE(6) HN_CASE(8)
  if constexpr (!PT) {
    HN_CASE(12) HN_CASE(16) HN_CASE(24) HN_CASE(32)
  }
#undef HN_CASE
  if (PT) set_error("adaln_quant: per-token scales support D <= 4096 (got %lld)", (long long)D);
  else set_error("adaln: D=%lld exceeds the supported 16384", (long long)D);
  return HN_ERR_UNSUPPORTED;
}

template <int DT, bool QUANT, int ROUND, bool PT = false>
static int adaln_norm(int norm, const void* x, const void* shift, const void* scale, int64_t B, int64_t L,
                      int64_t D, float eps, void* y, int8_t* q, float* s, hipStream_t st) {
  if (norm == HN_NORM_RMS)
    return launch_adaln<DT, HN_NORM_RMS, QUANT, ROUND, PT>(x, shift, scale, B, L, D, eps, y, q, s, st);
  return launch_adaln<DT, HN_NORM_LAYER, QUANT, ROUND, PT>(x, shift, scale, B, L, D, eps, y, q, s, st);
}

// ---------------------------------------------------------------------------------------------
// gated residual: out = x + round(y * gate[b])                   (fused.py:108-118)
// A copy-shaped stream: block (64, 4) covers 64 chunks of 8 channels x 4 rows, one 16-byte chunk of x, y
// and out per thread and row (the gate chunk is an L2 hit); blockIdx.y strides over row groups.  No
// integer division per element; the batch of a row is computed once per wave.
constexpr int kGrRows = 4;

// FRAMES: the camera module's per-frame output is then added (hy_nomas/model.py:518-520): token r of
// [B, T * P] tokens belongs to frame row r / P of frame [B, T, D]; the sum is rounded to the dtype before
// the add, as the reference's two tensor operations do.
template <int DT, bool FRAMES>
__global__ __launch_bounds__(256) void gated_residual_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ yv,
                                                             const uint16_t* __restrict__ gate,
                                                             const uint16_t* __restrict__ frame, int64_t P,
                                                             uint16_t* __restrict__ out, int64_t rows, int64_t L,
                                                             int cpr) {
  const int c = blockIdx.x * 64 + threadIdx.x;
  if (c >= cpr) return;
  const int64_t D = (int64_t)cpr * 8;
  for (int64_t r = (int64_t)blockIdx.y * kGrRows + threadIdx.y; r < rows; r += (int64_t)gridDim.y * kGrRows) {
    const int64_t b = L == rows ? 0 : r / L;  // one batch: no division
    const uint4 xv = ld_nt16(x + r * D + c * 8);
    const uint4 yy = ld_nt16(yv + r * D + c * 8);
    const uint4 gv = *reinterpret_cast<const uint4*>(gate + b * D + c * 8);
    float a[8], bb[8], g[8], o[8], fr[8];
    widen8<DT>(xv, a);
    widen8<DT>(yy, bb);
    widen8<DT>(gv, g);
    if constexpr (FRAMES) widen8<DT>(*reinterpret_cast<const uint4*>(frame + (r / P) * D + c * 8), fr);
    bool nan = false;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      o[j] = a[j] + round_to<DT>(bb[j] * g[j]);
      if constexpr (FRAMES) {
        float s = round_to<DT>(o[j]);
        asm volatile("" : "+v"(s));  // rounded on its own, never fused into the add below
        o[j] = s + fr[j];
      }
      nan |= o[j] != o[j];
    }
    uint4 packed;
    if (__builtin_expect(nan, 0)) packed = narrow8x<DT, false>(o);
    else packed = narrow8x<DT, true>(o);
    st_nt16(out + r * D + c * 8, packed);
  }
}

template <int DT, bool FRAMES = false>
static int launch_gated_residual(const void* x, const void* y, const void* gate, int64_t rows, int64_t L, int64_t D,
                                 void* out, hipStream_t st, const void* frame = nullptr, int64_t P = 1) {
  const int64_t cpr = D / 8;
  if (cpr > 0x7fffffff) {
    set_error("hn_gated_residual: D too large");
    return HN_ERR_UNSUPPORTED;
  }
  const int64_t gx = (cpr + 63) / 64;
  int64_t gy = (rows + kGrRows - 1) / kGrRows;
  gy = gy > 65535 ? 65535 : gy;
  hipLaunchKernelGGL((gated_residual_kernel<DT, FRAMES>), dim3((unsigned)gx, (unsigned)gy), dim3(64, kGrRows), 0,
                     st, (const uint16_t*)x, (const uint16_t*)y, (const uint16_t*)gate, (const uint16_t*)frame, P,
                     (uint16_t*)out, rows, L, (int)cpr);
  return HN_LAUNCH_CHECK("gated_residual_kernel");
}

// ---------------------------------------------------------------------------------------------
// Row-scaled int8 dequantization: out[r, :] = dtype(float(q[r, :]) * s[r])      (world.py:93-94)
// One thread per 8 codes: an 8-byte load and, for 2-byte outputs, one 16-byte store, so each store
// instruction writes 1 KB of consecutive output and the stream can bypass the caches.  A code b (as an
// unsigned byte after flipping its sign bit) is q = b - 128, so q * s = fma(b, s, -128 s) with -128 s
// exact: the one rounding of the product, from the single-instruction unsigned byte conversion.
template <int DT, bool WIDE>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const int8_t* __restrict__ q, int64_t ldq,
                                                           const float* __restrict__ s, int64_t lds,
                                                           int64_t rows, int cpr, void* __restrict__ out,
                                                           int64_t ldo) {
  int64_t r;
  int c;
  if constexpr (WIDE) {  // more than 2^32 chunks
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= rows * cpr) return;
    r = t / cpr;
    c = (int)(t - r * cpr);
  } else {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= (uint32_t)(rows * cpr)) return;
    const uint32_t r32 = t / (uint32_t)cpr;
    r = r32;
    c = (int)(t - r32 * (uint32_t)cpr);
  }
  const uint2 v = ld_nt8(q + r * ldq + c * 8);
  const float sc = s[r * lds];
  const float off = -128.0f * sc;
  const uint32_t w[2] = {v.x ^ 0x80808080u, v.y ^ 0x80808080u};
  float f[8];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    f[4 * k + 0] = __builtin_fmaf((float)(w[k] & 0xffu), sc, off);  // v_cvt_f32_ubyte0..3
    f[4 * k + 1] = __builtin_fmaf((float)((w[k] >> 8) & 0xffu), sc, off);
    f[4 * k + 2] = __builtin_fmaf((float)((w[k] >> 16) & 0xffu), sc, off);
    f[4 * k + 3] = __builtin_fmaf((float)(w[k] >> 24), sc, off);
  }
  if constexpr (DT == HN_DTYPE_F32) {
    float4* o = reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + r * ldo + c * 8);
    o[0] = make_float4(f[0], f[1], f[2], f[3]);
    o[1] = make_float4(f[4], f[5], f[6], f[7]);
  } else {
    uint16_t* o = reinterpret_cast<uint16_t*>(out) + r * ldo + c * 8;
    if (__builtin_expect(sc == sc, 1)) st_nt16(o, narrow8x<DT, true>(f));
    else st_nt16(o, narrow8x<DT, false>(f));  // a NaN scale takes the software rounding (torch's NaN code)
  }
}

// ---------------------------------------------------------------------------------------------
// QK RMSNorm + interleaved RoPE                                  (fused.py:65-91)

// Sum over aligned groups of W lanes (W = 8, 16 or 32), every lane of a group getting the total, in the
// butterfly order of xor shuffles with masks 1, 2, 4, ...  Inside a DPP row the steps are quad_perm and
// mirror moves: after the two quad steps every lane of a quad holds the same value, so the half-row
// mirror delivers the xor-4 partner's value and the row mirror the xor-8 partner's.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W == 8 || W == 16 || W == 32, "group of 8, 16 or 32 lanes");
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  if constexpr (W >= 16) v += dpp_f<0x140>(v);
  if constexpr (W == 32) v += shfl_xor_f(v, 16, 32);
  return v;
}

// One lane's 8 dims of a normalized (and rotated) head row: bf16(bf16(x * r) * w), then the interleaved
// rotation.  HW: the roundings use the hardware conversion, equal to rbf16 on every non-NaN input.
template <bool ROPE, bool HW>
__device__ __forceinline__ void qk_rows8(const float* f, float r, const float* wv, const float* cv, const float* sv,
                                         float* o) {
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float ne, no;
    if constexpr (HW) {
      const uint32_t a = bf16x2_finite(f[i] * r, f[i + 1] * r);
      const uint32_t b = bf16x2_finite(__uint_as_float(a << 16) * wv[i], __uint_as_float(a & 0xffff0000u) * wv[i + 1]);
      ne = __uint_as_float(b << 16);
      no = __uint_as_float(b & 0xffff0000u);
    } else {
      ne = rbf16(rbf16(f[i] * r) * wv[i]);
      no = rbf16(rbf16(f[i + 1] * r) * wv[i + 1]);
    }
    if constexpr (ROPE) {
      o[i] = ne * cv[i] - no * sv[i];
      o[i + 1] = no * cv[i + 1] + ne * sv[i + 1];
    } else {
      o[i] = ne;
      o[i + 1] = no;
    }
  }
}

// W = D / 8 lanes per head, lane j holding dims [8j, 8j + 8).  Each W-lane group normalizes G heads of
// one token (G = 6, 4, 2 or 1, the largest that divides the head count): the weight and the token's
// rotary rows are loaded once per group, and the group's G head rows are all in flight before the
// first is reduced.
template <int W, bool ROPE, int G>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ cs,
                                                           const float* __restrict__ sn, int64_t n_groups,
                                                           int64_t H, int64_t L, float eps,
                                                           uint16_t* __restrict__ y) {
  constexpr int D = W * 8;
  const int64_t grp = ((int64_t)blockIdx.x * 256 + threadIdx.x) / W;  // (batch * token, head group) index
  const int j = threadIdx.x & (W - 1);
  const bool live = grp < n_groups;
  const int64_t gg = live ? grp : 0;
  const int64_t per_tok = H / G;
  const int64_t bl = gg / per_tok, h0 = (gg - bl * per_tok) * G;
  const int64_t token = bl % L;
  float wv[8], cv[8], sv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) wv[i] = w[j * 8 + i];
  if constexpr (ROPE) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      cv[i] = cs[token * D + j * 8 + i];
      sv[i] = sn[token * D + j * 8 + i];
    }
  }
  uint4 xr[G];
#pragma unroll
  for (int g = 0; g < G; g++) xr[g] = ld_nt16(x + bl * ldx + (h0 + g) * D + j * 8);
#pragma unroll
  for (int g = 0; g < G; g++) {
    float f[8];
    widen8<HN_DTYPE_BF16>(xr[g], f);
    float se = 0.0f, so = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      se = __builtin_fmaf(f[i], f[i], se);
      so = __builtin_fmaf(f[i + 1], f[i + 1], so);
    }
    se = group_sum<W>(se);
    so = group_sum<W>(so);
    const float r = 1.0f / __builtin_sqrtf((se + so) / (float)D + eps);
    // A NaN reaching any rounding propagates into the outputs it feeds, so outputs free of NaN mean the
    // hardware roundings saw no NaN and equal the software ones; a lane with a NaN output recomputes its
    // dims with the software rounding and torch's NaN code.
    float o[8];
    qk_rows8<ROPE, true>(f, r, wv, cv, sv, o);
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 8; i += 2) nan |= __builtin_isunordered(o[i], o[i + 1]);
    uint4 packed;
    if (__builtin_expect(nan, 0)) {
      qk_rows8<ROPE, false>(f, r, wv, cv, sv, o);
      packed = narrow8x<HN_DTYPE_BF16, false>(o);
    } else {
      packed = narrow8x<HN_DTYPE_BF16, true>(o);
    }
    if (live) st_nt16(y + (bl * H + h0 + g) * D + j * 8, packed);
  }
}

// ---------------------------------------------------------------------------------------------
// PixelUMM split-half RMSNorm + sectioned rotate-half MRoPE, head_dim 128 (fused.py:131-175).
// 16 lanes per head, lane j holding dims [8j, 8j + 8), and G heads of one token per 16-lane group as in
// qk_norm_rope_kernel.  T section = lanes 0-7 (rotate-half
// partner 4 lanes away), H section = lanes 8-11, W section = lanes 12-15 (partner 2 lanes away).
template <int G>
__global__ __launch_bounds__(256) void pixelumm_qk_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          const float* __restrict__ wt,
                                                          const float* __restrict__ whw,
                                                          const float* __restrict__ cs,
                                                          const float* __restrict__ sn, int64_t n_groups, int64_t H,
                                                          float eps, uint16_t* __restrict__ y) {
  constexpr int D = 128;
  const int64_t grp = ((int64_t)blockIdx.x * 256 + threadIdx.x) / 16;
  const int j = threadIdx.x & 15;
  const bool live = grp < n_groups;
  const int64_t gg = live ? grp : 0;
  const int64_t per_tok = H / G;
  const int64_t t = gg / per_tok, h0 = (gg - t * per_tok) * G;
  const float* wp = j < 8 ? wt + j * 8 : whw + (j - 8) * 8;
  float wv[8], cv[8], sv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    wv[i] = wp[i];
    cv[i] = cs[t * D + j * 8 + i];
    sv[i] = sn[t * D + j * 8 + i];
  }
  const int partner_xor = j < 8 ? 4 : 2;
  const bool first = j < 8 ? (j < 4) : ((j & 3) < 2);
  uint4 xr[G];
#pragma unroll
  for (int g = 0; g < G; g++) xr[g] = ld_nt16(x + t * ldx + (h0 + g) * D + j * 8);
#pragma unroll
  for (int g = 0; g < G; g++) {
    float f[8];
    widen8<HN_DTYPE_BF16>(xr[g], f);
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) sq = __builtin_fmaf(f[i], f[i], sq);
    // lanes 0-7 reduce the T half, lanes 8-15 the HW half
    sq = group_sum<8>(sq);
    const float rr = 1.0f / __builtin_sqrtf(sq / (float)(D / 2) + eps);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = f[i] * rr * wv[i];
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float p = __shfl(v[i], (threadIdx.x & 63) ^ partner_xor, 64);
      o[i] = first ? v[i] * cv[i] - p * sv[i] : v[i] * cv[i] + p * sv[i];
    }
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 8; i += 2) nan |= __builtin_isunordered(o[i], o[i + 1]);
    uint4 packed;
    if (__builtin_expect(nan, 0)) packed = narrow8x<HN_DTYPE_BF16, false>(o);
    else packed = narrow8x<HN_DTYPE_BF16, true>(o);
    if (live) st_nt16(y + (t * H + h0 + g) * D + j * 8, packed);
  }
}

}  // namespace hn

// =============================================================================================
// C ABI

using namespace hn;

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

extern "C" int hn_adaln(const void* x, const void* shift, const void* scale, int dtype, int64_t B, int64_t L,
                        int64_t D, float eps, int norm, void* y, void* stream) {
  HN_REQUIRE(B >= 0 && L >= 0 && D > 0, "hn_adaln: bad shape");
  HN_REQUIRE(D % 8 == 0, "hn_adaln: D=%lld must be a multiple of 8", (long long)D);
  HN_REQUIRE(norm == HN_NORM_LAYER || norm == HN_NORM_RMS, "hn_adaln: bad norm %d", norm);
  HN_REQUIRE(x && shift && scale && y, "hn_adaln: null pointer");
  HN_REQUIRE(aligned16(x) && aligned16(shift) && aligned16(scale) && aligned16(y), "hn_adaln: pointers must be 16-byte aligned");
  if (B * L == 0) return HN_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == HN_DTYPE_BF16)
    return adaln_norm<HN_DTYPE_BF16, false, HN_ROUND_HALF_AWAY>(norm, x, shift, scale, B, L, D, eps, y, nullptr, nullptr, st);
  if (dtype == HN_DTYPE_F16)
    return adaln_norm<HN_DTYPE_F16, false, HN_ROUND_HALF_AWAY>(norm, x, shift, scale, B, L, D, eps, y, nullptr, nullptr, st);
  set_error("hn_adaln: unsupported dtype %d", dtype);
  return HN_ERR_UNSUPPORTED;
}

extern "C" int hn_adaln_quant(const void* x, const void* shift, const void* scale, int dtype, int64_t B, int64_t L,
                              int64_t D, float eps, int norm, int rounding, int64_t group, int8_t* q, float* s,
                              void* stream) {
  HN_REQUIRE(B >= 0 && L >= 0 && D > 0, "hn_adaln_quant: bad shape");
  HN_REQUIRE(D % 128 == 0, "hn_adaln_quant: D=%lld must be a multiple of 128", (long long)D);
  HN_REQUIRE(group == 128 || group == D, "hn_adaln_quant: group must be 128 or D (got %lld)", (long long)group);
  HN_REQUIRE(norm == HN_NORM_LAYER || norm == HN_NORM_RMS, "hn_adaln_quant: bad norm %d", norm);
  HN_REQUIRE(rounding == HN_ROUND_HALF_AWAY || rounding == HN_ROUND_HALF_EVEN, "hn_adaln_quant: bad rounding");
  HN_REQUIRE(x && shift && scale && q && s, "hn_adaln_quant: null pointer");
  HN_REQUIRE(aligned16(x) && aligned16(shift) && aligned16(scale) && ((uintptr_t)q & 7) == 0,
             "hn_adaln_quant: misaligned pointer");
  if (B * L == 0) return HN_OK;
  hipStream_t st = (hipStream_t)stream;
  const bool pt = group == D && D != 128;  // one scale per token (a single group of 128 is the g128 layout)
#define HN_AQ(DT, RD)                                                                                      \
  return pt ? adaln_norm<DT, true, RD, true>(norm, x, shift, scale, B, L, D, eps, nullptr, q, s, st)      \
            : adaln_norm<DT, true, RD, false>(norm, x, shift, scale, B, L, D, eps, nullptr, q, s, st)
  if (dtype == HN_DTYPE_BF16) {
    if (rounding == HN_ROUND_HALF_EVEN) HN_AQ(HN_DTYPE_BF16, HN_ROUND_HALF_EVEN);
    HN_AQ(HN_DTYPE_BF16, HN_ROUND_HALF_AWAY);
  }
  if (dtype == HN_DTYPE_F16) {
    if (rounding == HN_ROUND_HALF_EVEN) HN_AQ(HN_DTYPE_F16, HN_ROUND_HALF_EVEN);
    HN_AQ(HN_DTYPE_F16, HN_ROUND_HALF_AWAY);
  }
#undef HN_AQ
  set_error("hn_adaln_quant: unsupported dtype %d", dtype);
  return HN_ERR_UNSUPPORTED;
}

extern "C" int hn_gated_residual(const void* x, const void* y, const void* gate, int dtype, int64_t B, int64_t L,
                                 int64_t D, void* out, void* stream) {
  HN_REQUIRE(B >= 0 && L >= 0 && D > 0, "hn_gated_residual: bad shape");
  HN_REQUIRE(D % 8 == 0, "hn_gated_residual: D=%lld must be a multiple of 8", (long long)D);
  HN_REQUIRE(x && y && gate && out, "hn_gated_residual: null pointer");
  HN_REQUIRE(aligned16(x) && aligned16(y) && aligned16(gate) && aligned16(out), "hn_gated_residual: pointers must be 16-byte aligned");
  if (B * L == 0) return HN_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == HN_DTYPE_BF16) return launch_gated_residual<HN_DTYPE_BF16>(x, y, gate, B * L, L, D, out, st);
  if (dtype == HN_DTYPE_F16) return launch_gated_residual<HN_DTYPE_F16>(x, y, gate, B * L, L, D, out, st);
  set_error("hn_gated_residual: unsupported dtype %d", dtype);
  return HN_ERR_UNSUPPORTED;
}

extern "C" int hn_gated_residual_frames(const void* x, const void* y, const void* gate, const void* frame, int dtype,
                                        int64_t B, int64_t T, int64_t P, int64_t D, void* out, void* stream) {
  HN_REQUIRE(B >= 0 && T >= 0 && P > 0 && D > 0, "hn_gated_residual_frames: bad shape");
  HN_REQUIRE(D % 8 == 0, "hn_gated_residual_frames: D=%lld must be a multiple of 8", (long long)D);
  HN_REQUIRE(x && y && gate && frame && out, "hn_gated_residual_frames: null pointer");
  HN_REQUIRE(aligned16(x) && aligned16(y) && aligned16(gate) && aligned16(frame) && aligned16(out),
             "hn_gated_residual_frames: pointers must be 16-byte aligned");
  if (B * T == 0) return HN_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == HN_DTYPE_BF16)
    return launch_gated_residual<HN_DTYPE_BF16, true>(x, y, gate, B * T * P, T * P, D, out, st, frame, P);
  if (dtype == HN_DTYPE_F16)
    return launch_gated_residual<HN_DTYPE_F16, true>(x, y, gate, B * T * P, T * P, D, out, st, frame, P);
  set_error("hn_gated_residual_frames: unsupported dtype %d", dtype);
  return HN_ERR_UNSUPPORTED;
}

extern "C" int hn_dequantize_rows(const int8_t* q, int64_t ldq, const float* s, int64_t lds, int64_t rows,
                                  int64_t D, void* out, int out_dtype, int64_t ldo, void* stream) {
  HN_REQUIRE(rows >= 0 && D > 0, "hn_dequantize_rows: bad shape");
  HN_REQUIRE(D % 16 == 0, "hn_dequantize_rows: D=%lld must be a multiple of 16", (long long)D);
  HN_REQUIRE(ldq >= D && ldq % 16 == 0 && ldo >= D && ldo % 16 == 0 && lds >= 0,
             "hn_dequantize_rows: row strides must cover the rows and be multiples of 16 elements");
  HN_REQUIRE(out_dtype >= HN_DTYPE_BF16 && out_dtype <= HN_DTYPE_F32, "hn_dequantize_rows: bad out dtype %d", out_dtype);
  HN_REQUIRE(q && s && out, "hn_dequantize_rows: null pointer");
  HN_REQUIRE(aligned16(q) && aligned16(out), "hn_dequantize_rows: codes and output must be 16-byte aligned");
  if (rows == 0) return HN_OK;
  const int64_t cpr = D / 8, n = rows * cpr;
  HN_REQUIRE(cpr <= 0x7fffffff && (n + 255) / 256 <= 0x7fffffff, "hn_dequantize_rows: too large");
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipStream_t st = (hipStream_t)stream;
#define HN_DQ(DT, WIDE)                                                                                          \
  hipLaunchKernelGGL((dequant_rows_kernel<DT, WIDE>), dim3(blocks), dim3(256), 0, st, q, ldq, s, lds, rows, (int)cpr, \
                     out, ldo)
  const bool wide = (int64_t)blocks * 256 > 0xffffffffLL;
  if (out_dtype == HN_DTYPE_BF16) { if (wide) HN_DQ(HN_DTYPE_BF16, true); else HN_DQ(HN_DTYPE_BF16, false); }
  else if (out_dtype == HN_DTYPE_F16) { if (wide) HN_DQ(HN_DTYPE_F16, true); else HN_DQ(HN_DTYPE_F16, false); }
  else { if (wide) HN_DQ(HN_DTYPE_F32, true); else HN_DQ(HN_DTYPE_F32, false); }
#undef HN_DQ
  return HN_LAUNCH_CHECK("dequant_rows_kernel");
}

template <int W, bool ROPE>
static void qk_norm_rope_launch_g(int g, dim3 grid, hipStream_t st, const uint16_t* x, int64_t ldx, const float* w,
                                  const float* cs, const float* sn, int64_t n_groups, int64_t H, int64_t L,
                                  float eps, uint16_t* y) {
  if (g == 6) hipLaunchKernelGGL((qk_norm_rope_kernel<W, ROPE, 6>), grid, dim3(256), 0, st, x, ldx, w, cs, sn, n_groups, H, L, eps, y);
  else if (g == 4) hipLaunchKernelGGL((qk_norm_rope_kernel<W, ROPE, 4>), grid, dim3(256), 0, st, x, ldx, w, cs, sn, n_groups, H, L, eps, y);
  else if (g == 2) hipLaunchKernelGGL((qk_norm_rope_kernel<W, ROPE, 2>), grid, dim3(256), 0, st, x, ldx, w, cs, sn, n_groups, H, L, eps, y);
  else hipLaunchKernelGGL((qk_norm_rope_kernel<W, ROPE, 1>), grid, dim3(256), 0, st, x, ldx, w, cs, sn, n_groups, H, L, eps, y);
}

static void qk_norm_rope_launch(int w, int g, bool rope, dim3 grid, hipStream_t st, const uint16_t* x, int64_t ldx,
                                const float* wt, const float* cs, const float* sn, int64_t n_groups, int64_t H,
                                int64_t L, float eps, uint16_t* y) {
  if (w == 8) {
    if (rope) qk_norm_rope_launch_g<8, true>(g, grid, st, x, ldx, wt, cs, sn, n_groups, H, L, eps, y);
    else qk_norm_rope_launch_g<8, false>(g, grid, st, x, ldx, wt, cs, sn, n_groups, H, L, eps, y);
  } else if (w == 16) {
    if (rope) qk_norm_rope_launch_g<16, true>(g, grid, st, x, ldx, wt, cs, sn, n_groups, H, L, eps, y);
    else qk_norm_rope_launch_g<16, false>(g, grid, st, x, ldx, wt, cs, sn, n_groups, H, L, eps, y);
  } else {
    if (rope) qk_norm_rope_launch_g<32, true>(g, grid, st, x, ldx, wt, cs, sn, n_groups, H, L, eps, y);
    else qk_norm_rope_launch_g<32, false>(g, grid, st, x, ldx, wt, cs, sn, n_groups, H, L, eps, y);
  }
}

extern "C" int hn_qk_norm_rope(const void* x, int64_t ldx, const float* weight, const float* cos_t, const float* sin_t,
                               int64_t B, int64_t L, int64_t H, int64_t D, float eps, void* y, void* stream) {
  HN_REQUIRE(B >= 0 && L >= 0 && H > 0, "hn_qk_norm_rope: bad shape");
  HN_REQUIRE(D == 64 || D == 128 || D == 256, "hn_qk_norm_rope: head dim %lld not in {64, 128, 256}", (long long)D);
  HN_REQUIRE(ldx >= H * D && ldx % 8 == 0, "hn_qk_norm_rope: bad token stride %lld", (long long)ldx);
  HN_REQUIRE(x && weight && y, "hn_qk_norm_rope: null pointer");
  HN_REQUIRE((cos_t == nullptr) == (sin_t == nullptr), "hn_qk_norm_rope: cos and sin must both be given or both NULL");
  HN_REQUIRE(aligned16(x) && aligned16(y), "hn_qk_norm_rope: x and y must be 16-byte aligned");
  const int64_t n_heads = B * L * H;
  if (n_heads == 0) return HN_OK;
  const int g = H % 6 == 0 ? 6 : H % 4 == 0 ? 4 : H % 2 == 0 ? 2 : 1;
  const int w = (int)(D / 8);
  const int64_t n_groups = n_heads / g;
  const unsigned blocks = (unsigned)((n_groups * w + 255) / 256);
  qk_norm_rope_launch(w, g, cos_t != nullptr, dim3(blocks), (hipStream_t)stream, (const uint16_t*)x, ldx, weight,
                      cos_t, sin_t, n_groups, H, L, eps, (uint16_t*)y);
  return HN_LAUNCH_CHECK("qk_norm_rope_kernel");
}

extern "C" int hn_pixelumm_qk(const void* x, int64_t ldx, const void* weight_t, const void* weight_hw,
                              const float* cos_t, const float* sin_t, int64_t N, int64_t H, int64_t D, float eps,
                              void* y, void* stream) {
  HN_REQUIRE(N >= 0 && H > 0, "hn_pixelumm_qk: bad shape");
  HN_REQUIRE(D == 128, "hn_pixelumm_qk: head dim %lld unsupported (128 only)", (long long)D);
  HN_REQUIRE(ldx >= H * D && ldx % 8 == 0, "hn_pixelumm_qk: bad token stride %lld", (long long)ldx);
  HN_REQUIRE(x && weight_t && weight_hw && cos_t && sin_t && y, "hn_pixelumm_qk: null pointer");
  HN_REQUIRE(aligned16(x) && aligned16(y), "hn_pixelumm_qk: x and y must be 16-byte aligned");
  const int64_t n_heads = N * H;
  if (n_heads == 0) return HN_OK;
  const int g = H % 6 == 0 ? 6 : H % 4 == 0 ? 4 : H % 2 == 0 ? 2 : 1;
  const int64_t n_groups = n_heads / g;
  const dim3 grid((unsigned)((n_groups * 16 + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  const float* wt = (const float*)weight_t;
  const float* whw = (const float*)weight_hw;
  const uint16_t* xx = (const uint16_t*)x;
  uint16_t* yy = (uint16_t*)y;
  if (g == 6) hipLaunchKernelGGL(pixelumm_qk_kernel<6>, grid, dim3(256), 0, st, xx, ldx, wt, whw, cos_t, sin_t, n_groups, H, eps, yy);
  else if (g == 4) hipLaunchKernelGGL(pixelumm_qk_kernel<4>, grid, dim3(256), 0, st, xx, ldx, wt, whw, cos_t, sin_t, n_groups, H, eps, yy);
  else if (g == 2) hipLaunchKernelGGL(pixelumm_qk_kernel<2>, grid, dim3(256), 0, st, xx, ldx, wt, whw, cos_t, sin_t, n_groups, H, eps, yy);
  else hipLaunchKernelGGL(pixelumm_qk_kernel<1>, grid, dim3(256), 0, st, xx, ldx, wt, whw, cos_t, sin_t, n_groups, H, eps, yy);
  return HN_LAUNCH_CHECK("pixelumm_qk_kernel");
}
