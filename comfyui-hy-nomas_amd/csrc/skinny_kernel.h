// Skinny int8 block GEMM: M <= 4 tokens (the per-sample linears of a DiT step, e.g. the modulation
// linear vec -> 6 x hidden of hy_nomas/model.py:306-314, run through kernels.block_linear with M = batch).
//
// At M <= 4 the weight stream is the whole cost (N x K bytes, each used M times), so the matrix cores
// are not needed: a wave owns 4 weight rows, reads 1 KB of each row per step (16 bytes per lane, row-
// contiguous), multiplies with v_dot4 against the same 16 bytes of every token's codes, and produces
// exact int32 dot products.  The numbers are those of block_gemm_kernel bit for bit:
//   * per-token scales: whole-K int32 sum (a 64-lane reduction), then fma(float(acc) * sa, sw, 0);
//   * g128: the 8 lanes of a 128-byte group reduce its exact int32 partial, and the group partials are
//     folded in group order, acc = fma(float(part) * sa[m, g], sw[n, g], acc) (block weight scales:
//     acc = fma(float(part), sa[m, g] * sw[n / 128, g], acc)), from the partials read lane by lane;
//   * + bias (absent: -0.0), optional GELU, the same output conversion.
#pragma once

#include "gemm_kernel.h"

namespace hn {

constexpr int kSkinnyRows = 4;     // weight rows per wave
constexpr int kSkinnyWaves = 4;    // waves per workgroup
constexpr int kSkinnyMaxM = 4;

// MODE 0: per-token x per-channel (whole-K int32); 1: g128 with one weight-scale row per channel;
// 2: g128 with one weight-scale row per 128 channels.
template <int MT, int MODE, int EPI, int OUT_DT>
__global__ __launch_bounds__(kSkinnyWaves * 64) void skinny_gemm_kernel(const GemmArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t n0 = ((int64_t)blockIdx.x * kSkinnyWaves + (threadIdx.x >> 6)) * kSkinnyRows;
  if (n0 >= a.N) return;  // whole wave (the kernel has no workgroup barrier)
  const int G = (int)(a.K / 128);
  const int steps = (G + 7) / 8;
  const int M = (int)a.M;

  const uint8_t* wrow[kSkinnyRows];
#pragma unroll
  for (int r = 0; r < kSkinnyRows; r++) wrow[r] = a.qw + (n0 + r < a.N ? n0 + r : a.N - 1) * a.ldw;
  const uint8_t* xrow[MT];
#pragma unroll
  for (int m = 0; m < MT; m++) xrow[m] = a.qa + (int64_t)(m < M ? m : M - 1) * a.lda;

  int32_t acc32[kSkinnyRows][MT];
  float facc[kSkinnyRows][MT];
#pragma unroll
  for (int r = 0; r < kSkinnyRows; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) { acc32[r][m] = 0; facc[r][m] = 0.0f; }

  // Step s covers bytes [1024 s, 1024 s + 1024) of every row: lane l holds group 8 s + l / 8, bytes
  // 16 (l % 8) .. of it.  Lanes past the last group load nothing and contribute 0.
  // g128: each lane also loads the scales of its group (weight rows r, tokens m), so the per-group
  // products of the fold are formed in every lane at once and read lane by lane (lane 8 j: group 8 s + j).
  const float* swrow[kSkinnyRows];
  const float* sarow[MT];
#pragma unroll
  for (int r = 0; r < kSkinnyRows; r++) {
    const int64_t n = n0 + r < a.N ? n0 + r : a.N - 1;
    swrow[r] = MODE == 2 ? a.sw + (n / 128) * a.ldsw : a.sw + n * a.ldsw;
  }
#pragma unroll
  for (int m = 0; m < MT; m++) sarow[m] = a.sa + (int64_t)(m < M ? m : M - 1) * a.ldsa;
  v4i wv[2][kSkinnyRows], xv[2][MT];
  float swl[2][kSkinnyRows], sal[2][MT];
  auto load = [&](int s, int buf) __attribute__((always_inline)) {
    const bool ok = 8 * s + (lane >> 3) < G;
    const uint32_t off = (uint32_t)s * 1024u + (uint32_t)lane * 16u;
#pragma unroll
    for (int r = 0; r < kSkinnyRows; r++)
      wv[buf][r] = ok ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wrow[r] + off)) : v4i{0, 0, 0, 0};
#pragma unroll
    for (int m = 0; m < MT; m++) xv[buf][m] = ok ? *reinterpret_cast<const v4i*>(xrow[m] + off) : v4i{0, 0, 0, 0};
    if constexpr (MODE != 0) {
      const int gl = min(8 * s + (lane >> 3), G - 1);
#pragma unroll
      for (int r = 0; r < kSkinnyRows; r++) swl[buf][r] = swrow[r][gl];
#pragma unroll
      for (int m = 0; m < MT; m++) sal[buf][m] = sarow[m][gl];
    }
  };
  auto compute = [&](int s, int buf) __attribute__((always_inline)) {
    float t[kSkinnyRows][MT], f[kSkinnyRows][MT];
#pragma unroll
    for (int r = 0; r < kSkinnyRows; r++) {
#pragma unroll
      for (int m = 0; m < MT; m++) {
        int d = 0;
        d = __builtin_amdgcn_sdot4(wv[buf][r].x, xv[buf][m].x, d, false);
        d = __builtin_amdgcn_sdot4(wv[buf][r].y, xv[buf][m].y, d, false);
        d = __builtin_amdgcn_sdot4(wv[buf][r].z, xv[buf][m].z, d, false);
        d = __builtin_amdgcn_sdot4(wv[buf][r].w, xv[buf][m].w, d, false);
        if constexpr (MODE == 0) {
          acc32[r][m] += d;
        } else {
          // the group's exact partial in all 8 of its lanes (|part| <= 128 * 127^2 < 2^31), with DPP
          // lane moves: xor 1, xor 2 inside each quad, then the mirrored quad of the half-row
          d += (int)dpp_u<0xB1>((uint32_t)d);
          d += (int)dpp_u<0x4E>((uint32_t)d);
          d += (int)dpp_u<0x141>((uint32_t)d);
          // per-channel scales: t = part * sa, then fma(t, sw, acc); block scales: fma(part, sa * sw, acc)
          if constexpr (MODE == 2) {
            t[r][m] = (float)d;
            f[r][m] = sal[buf][m] * swl[buf][r];
          } else {
            t[r][m] = (float)d * sal[buf][m];
          }
        }
      }
    }
    if constexpr (MODE != 0) {
      auto fold = [&](int j) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < kSkinnyRows; r++) {
          const float swj = MODE == 2 ? 0.0f : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(swl[buf][r]), 8 * j));
#pragma unroll
          for (int m = 0; m < MT; m++) {
            const float tj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t[r][m]), 8 * j));
            const float fj = MODE == 2 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f[r][m]), 8 * j)) : swj;
            facc[r][m] = __builtin_fmaf(tj, fj, facc[r][m]);
          }
        }
      };
      if (8 * s + 8 <= G) {
#pragma unroll
        for (int j = 0; j < 8; j++) fold(j);
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++)
          if (8 * s + j < G) fold(j);
      }
    }
  };
  load(0, 0);
  int s = 0;
  for (; s + 1 < steps; s += 2) {
    load(s + 1, 1);
    compute(s, 0);
    if (s + 2 < steps) load(s + 2, 0);
    compute(s + 1, 1);
  }
  if (s < steps) compute(s, 0);

  if constexpr (MODE == 0) {
#pragma unroll
    for (int r = 0; r < kSkinnyRows; r++)
#pragma unroll
      for (int m = 0; m < MT; m++) {
        int v = acc32[r][m];
        v += __shfl_xor(v, 1);
        v += __shfl_xor(v, 2);
        v += __shfl_xor(v, 4);
        v += __shfl_xor(v, 8);
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        const int64_t n = n0 + r < a.N ? n0 + r : a.N - 1;
        facc[r][m] = __builtin_fmaf((float)v * a.sa[(int64_t)(m < M ? m : M - 1) * a.ldsa], a.sw[n * a.ldsw], 0.0f);
      }
  }
  // every lane holds the same results; lane r * MT + m stores output (m, n0 + r)
#pragma unroll
  for (int r = 0; r < kSkinnyRows; r++)
#pragma unroll
    for (int m = 0; m < MT; m++) {
      const int64_t n = n0 + r;
      if (lane == r * MT + m && m < M && n < a.N) {
        float v = facc[r][m] + (a.bias ? load_bias(a.bias, a.bias_dtype, n) : -0.0f);
        if constexpr (EPI == HN_EPI_GELU) v = rbf16(gelu_tanh(rbf16(v)));
        if constexpr (OUT_DT == HN_DTYPE_F32) reinterpret_cast<float*>(a.out)[m * a.ldo + n] = v;
        else reinterpret_cast<uint16_t*>(a.out)[m * a.ldo + n] = (uint16_t)(cvt2_out<OUT_DT>(v, v) & 0xffffu);
      }
    }
}

}  // namespace hn
