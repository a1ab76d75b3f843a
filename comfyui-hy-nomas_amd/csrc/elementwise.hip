// Fused DiT elementwise kernels (hy_nomas/fused.py, hy_nomas/kernels.py:173-207).
//
// Row kernels (adaLN, adaLN+quant): one wavefront per token row; the row is loaded once with 16-byte
// loads, kept in registers for the mean / variance / output passes, and the statistics are wave
// reductions.  Head kernels (QK norm + RoPE): D/8 lanes per (token, head), 16 bytes per lane.
// The gated residual is a flat 16-byte streaming kernel.  All are single-pass and HBM-bound.
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
// adaLN: y = norm(x) * rbf16(1 + scale[b]) + shift[b]          (fused.py:37-52)
// adaLN + quant: y = rbf16(...), then int8 per 128 channels      (kernels.py:173-195)
constexpr int kRowThreads = 256;

template <int DT, int NORM, bool QUANT, int ROUND, int CPL>
__global__ __launch_bounds__(kRowThreads) void adaln_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ shift,
                                                            const uint16_t* __restrict__ scale, int64_t rows,
                                                            int64_t L, int64_t D, float eps,
                                                            uint16_t* __restrict__ y, int8_t* __restrict__ q,
                                                            float* __restrict__ s) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole wave exits together
  const int64_t b = r / L;
  const int64_t nchunk = D / 8;
  const uint16_t* xr = x + r * D;
  uint4 xv[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    int64_t c = lane + 64 * i;
    if (c < nchunk) xv[i] = *reinterpret_cast<const uint4*>(xr + c * 8);
  }
  // statistics in fp32: per-lane sums, then a wave reduction
  float mean = 0.0f;
  if constexpr (NORM == HN_NORM_LAYER) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      if (lane + 64 * i < nchunk) {
        float f[8];
        widen8<DT>(xv[i], f);
#pragma unroll
        for (int j = 0; j < 8; j++) acc += f[j];
      }
    }
    mean = wave_sum(acc) / (float)D;
  }
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    if (lane + 64 * i < nchunk) {
      float f[8];
      widen8<DT>(xv[i], f);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        float c = f[j] - mean;
        sq = __builtin_fmaf(c, c, sq);
      }
    }
  }
  const float var = wave_sum(sq) / (float)D;
  const float rstd = 1.0f / __builtin_sqrtf(var + eps);
  const uint16_t* shb = shift + b * D;
  const uint16_t* scb = scale + b * D;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const int64_t c = lane + 64 * i;
    if (c < nchunk) {
      float f[8], sh[8], sc[8], o[8];
      widen8<DT>(xv[i], f);
      widen8<DT>(*reinterpret_cast<const uint4*>(shb + c * 8), sh);
      widen8<DT>(*reinterpret_cast<const uint4*>(scb + c * 8), sc);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        float n = (f[j] - mean) * rstd;
        o[j] = n * rbf16(1.0f + sc[j]) + sh[j];
      }
      if constexpr (!QUANT) {
        *reinterpret_cast<uint4*>(y + r * D + c * 8) = narrow8<DT>(o);
      } else {
        float peak = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          o[j] = rbf16(o[j]);
          peak = __builtin_fmaxf(peak, __builtin_fabsf(o[j]));
        }
        // D % 128 == 0: the 16 lanes of a DPP row hold exactly one 128-channel group
        peak = row16_max(peak);
        const float gs = int8_scale(peak);
        FastDiv div(gs);
        int cd[8];
#pragma unroll
        for (int j = 0; j < 8; j++) cd[j] = round_i8<ROUND>(div(o[j]));
        *reinterpret_cast<uint2*>(q + r * D + c * 8) =
            make_uint2(pack4_i8(cd[0], cd[1], cd[2], cd[3]), pack4_i8(cd[4], cd[5], cd[6], cd[7]));
        if ((lane & 15) == 0) s[r * (D / 128) + c / 16] = gs;
      }
    }
  }
}

template <int DT, int NORM, bool QUANT, int ROUND>
static int launch_adaln(const void* x, const void* shift, const void* scale, int64_t B, int64_t L, int64_t D,
                        float eps, void* y, int8_t* q, float* s, hipStream_t st) {
  const int64_t rows = B * L;
  const int64_t cpl = (D / 8 + 63) / 64;
  const unsigned blocks = (unsigned)((rows + 3) / 4);
#define HN_CASE(N)                                                                                              \
  if (cpl <= N) {                                                                                               \
    hipLaunchKernelGGL((adaln_kernel<DT, NORM, QUANT, ROUND, N>), dim3(blocks), dim3(kRowThreads), 0, st,       \
                       (const uint16_t*)x, (const uint16_t*)shift, (const uint16_t*)scale, rows, L, D, eps,     \
                       (uint16_t*)y, q, s);                                                                     \
    return HN_LAUNCH_CHECK("adaln_kernel");                                                                     \
  }
  HN_CASE(1) HN_CASE(2) HN_CASE(3) HN_CASE(4) HN_CASE(5) HN_CASE(6) HN_CASE(8) HN_CASE(12) HN_CASE(16)
  HN_CASE(24) HN_CASE(32)
#undef HN_CASE
  set_error("adaln: D=%lld exceeds the supported 16384", (long long)D);
  return HN_ERR_UNSUPPORTED;
}

template <int DT, bool QUANT, int ROUND>
static int adaln_norm(int norm, const void* x, const void* shift, const void* scale, int64_t B, int64_t L,
                      int64_t D, float eps, void* y, int8_t* q, float* s, hipStream_t st) {
  if (norm == HN_NORM_RMS) return launch_adaln<DT, HN_NORM_RMS, QUANT, ROUND>(x, shift, scale, B, L, D, eps, y, q, s, st);
  return launch_adaln<DT, HN_NORM_LAYER, QUANT, ROUND>(x, shift, scale, B, L, D, eps, y, q, s, st);
}

// ---------------------------------------------------------------------------------------------
// gated residual: out = x + rbf16(y * gate[b])                   (fused.py:108-118)
constexpr int kFlatThreads = 256;
constexpr int kFlatUnroll = 4;

template <int DT>
__global__ __launch_bounds__(kFlatThreads) void gated_residual_kernel(const uint16_t* __restrict__ x,
                                                                      const uint16_t* __restrict__ yv,
                                                                      const uint16_t* __restrict__ gate,
                                                                      uint16_t* __restrict__ out, int64_t nchunk,
                                                                      int64_t chunks_per_row, int64_t L) {
  const int64_t base = (int64_t)blockIdx.x * (kFlatThreads * kFlatUnroll) + threadIdx.x;
  uint4 xv[kFlatUnroll], yvv[kFlatUnroll], gv[kFlatUnroll];
#pragma unroll
  for (int u = 0; u < kFlatUnroll; u++) {
    int64_t c = base + u * kFlatThreads;
    int64_t cc = c < nchunk ? c : 0;
    int64_t row = cc / chunks_per_row;
    int64_t col = cc - row * chunks_per_row;
    int64_t b = row / L;
    xv[u] = *reinterpret_cast<const uint4*>(x + cc * 8);
    yvv[u] = *reinterpret_cast<const uint4*>(yv + cc * 8);
    gv[u] = *reinterpret_cast<const uint4*>(gate + (b * chunks_per_row + col) * 8);
  }
#pragma unroll
  for (int u = 0; u < kFlatUnroll; u++) {
    int64_t c = base + u * kFlatThreads;
    float a[8], bb[8], g[8], o[8];
    widen8<DT>(xv[u], a);
    widen8<DT>(yvv[u], bb);
    widen8<DT>(gv[u], g);
#pragma unroll
    for (int j = 0; j < 8; j++) o[j] = a[j] + rbf16(bb[j] * g[j]);
    if (c < nchunk) *reinterpret_cast<uint4*>(out + c * 8) = narrow8<DT>(o);
  }
}

// ---------------------------------------------------------------------------------------------
// QK RMSNorm + interleaved RoPE                                  (fused.py:65-91)
// W = D / 8 lanes per (token, head); 64 / W heads per wavefront.
template <int W, bool ROPE>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ cs,
                                                           const float* __restrict__ sn, int64_t n_heads,
                                                           int64_t H, int64_t L, float eps,
                                                           uint16_t* __restrict__ y) {
  constexpr int D = W * 8;
  const int64_t hg = ((int64_t)blockIdx.x * 256 + threadIdx.x) / W;  // (batch * token, head) index
  const int j = threadIdx.x & (W - 1);
  const bool live = hg < n_heads;
  const int64_t hh = live ? hg : 0;
  const int64_t bl = hh / H, h = hh - bl * H;
  const int64_t token = bl % L;
  float f[8];
  widen8<HN_DTYPE_BF16>(*reinterpret_cast<const uint4*>(x + bl * ldx + h * D + j * 8), f);
  float se = 0.0f, so = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    se = __builtin_fmaf(f[i], f[i], se);
    so = __builtin_fmaf(f[i + 1], f[i + 1], so);
  }
#pragma unroll
  for (int m = 1; m < W; m <<= 1) {
    se += shfl_xor_f(se, m, W);
    so += shfl_xor_f(so, m, W);
  }
  const float r = 1.0f / __builtin_sqrtf((se + so) / (float)D + eps);
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const float ne = rbf16(rbf16(f[i] * r) * w[j * 8 + i]);
    const float no = rbf16(rbf16(f[i + 1] * r) * w[j * 8 + i + 1]);
    if constexpr (ROPE) {
      const float* c = cs + token * D + j * 8;
      const float* s = sn + token * D + j * 8;
      o[i] = ne * c[i] - no * s[i];
      o[i + 1] = no * c[i + 1] + ne * s[i + 1];
    } else {
      o[i] = ne;
      o[i + 1] = no;
    }
  }
  if (live) *reinterpret_cast<uint4*>(y + hh * D + j * 8) = narrow8<HN_DTYPE_BF16>(o);
}

// ---------------------------------------------------------------------------------------------
// PixelUMM split-half RMSNorm + sectioned rotate-half MRoPE, head_dim 128 (fused.py:131-175).
// 16 lanes per (token, head); lane j holds dims [8j, 8j + 8).  T section = lanes 0-7 (rotate-half
// partner 4 lanes away), H section = lanes 8-11, W section = lanes 12-15 (partner 2 lanes away).
__global__ __launch_bounds__(256) void pixelumm_qk_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          const float* __restrict__ wt,
                                                          const float* __restrict__ whw,
                                                          const float* __restrict__ cs,
                                                          const float* __restrict__ sn, int64_t n_heads, int64_t H,
                                                          float eps, uint16_t* __restrict__ y) {
  constexpr int D = 128;
  const int64_t hg = ((int64_t)blockIdx.x * 256 + threadIdx.x) / 16;
  const int j = threadIdx.x & 15;
  const bool live = hg < n_heads;
  const int64_t hh = live ? hg : 0;
  const int64_t t = hh / H, h = hh - t * H;
  float f[8];
  widen8<HN_DTYPE_BF16>(*reinterpret_cast<const uint4*>(x + t * ldx + h * D + j * 8), f);
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) sq = __builtin_fmaf(f[i], f[i], sq);
  // lanes 0-7 reduce the T half, lanes 8-15 the HW half
  sq += shfl_xor_f(sq, 1, 16);
  sq += shfl_xor_f(sq, 2, 16);
  sq += shfl_xor_f(sq, 4, 16);
  const float rr = 1.0f / __builtin_sqrtf(sq / (float)(D / 2) + eps);
  const float* wv = j < 8 ? wt + j * 8 : whw + (j - 8) * 8;
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = f[i] * rr * wv[i];
  const int partner_xor = j < 8 ? 4 : 2;
  const bool first = j < 8 ? (j < 4) : ((j & 3) < 2);
  const float* c = cs + t * D + j * 8;
  const float* s = sn + t * D + j * 8;
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float p = __shfl(v[i], (threadIdx.x & 63) ^ partner_xor, 64);
    o[i] = first ? v[i] * c[i] - p * s[i] : v[i] * c[i] + p * s[i];
  }
  if (live) *reinterpret_cast<uint4*>(y + hh * D + j * 8) = narrow8<HN_DTYPE_BF16>(o);
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
                              int64_t D, float eps, int norm, int rounding, int8_t* q, float* s, void* stream) {
  HN_REQUIRE(B >= 0 && L >= 0 && D > 0, "hn_adaln_quant: bad shape");
  HN_REQUIRE(D % 128 == 0, "hn_adaln_quant: D=%lld must be a multiple of 128", (long long)D);
  HN_REQUIRE(norm == HN_NORM_LAYER || norm == HN_NORM_RMS, "hn_adaln_quant: bad norm %d", norm);
  HN_REQUIRE(rounding == HN_ROUND_HALF_AWAY || rounding == HN_ROUND_HALF_EVEN, "hn_adaln_quant: bad rounding");
  HN_REQUIRE(x && shift && scale && q && s, "hn_adaln_quant: null pointer");
  HN_REQUIRE(aligned16(x) && aligned16(shift) && aligned16(scale) && ((uintptr_t)q & 7) == 0,
             "hn_adaln_quant: misaligned pointer");
  if (B * L == 0) return HN_OK;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == HN_DTYPE_BF16) {
    if (rounding == HN_ROUND_HALF_EVEN)
      return adaln_norm<HN_DTYPE_BF16, true, HN_ROUND_HALF_EVEN>(norm, x, shift, scale, B, L, D, eps, nullptr, q, s, st);
    return adaln_norm<HN_DTYPE_BF16, true, HN_ROUND_HALF_AWAY>(norm, x, shift, scale, B, L, D, eps, nullptr, q, s, st);
  }
  if (dtype == HN_DTYPE_F16) {
    if (rounding == HN_ROUND_HALF_EVEN)
      return adaln_norm<HN_DTYPE_F16, true, HN_ROUND_HALF_EVEN>(norm, x, shift, scale, B, L, D, eps, nullptr, q, s, st);
    return adaln_norm<HN_DTYPE_F16, true, HN_ROUND_HALF_AWAY>(norm, x, shift, scale, B, L, D, eps, nullptr, q, s, st);
  }
  set_error("hn_adaln_quant: unsupported dtype %d", dtype);
  return HN_ERR_UNSUPPORTED;
}

extern "C" int hn_gated_residual(const void* x, const void* y, const void* gate, int dtype, int64_t B, int64_t L,
                                 int64_t D, void* out, void* stream) {
  HN_REQUIRE(B >= 0 && L >= 0 && D > 0, "hn_gated_residual: bad shape");
  HN_REQUIRE(D % 8 == 0, "hn_gated_residual: D=%lld must be a multiple of 8", (long long)D);
  HN_REQUIRE(x && y && gate && out, "hn_gated_residual: null pointer");
  HN_REQUIRE(aligned16(x) && aligned16(y) && aligned16(gate) && aligned16(out), "hn_gated_residual: pointers must be 16-byte aligned");
  const int64_t nchunk = B * L * D / 8;
  if (nchunk == 0) return HN_OK;
  const int64_t per_block = kFlatThreads * kFlatUnroll;
  const unsigned blocks = (unsigned)((nchunk + per_block - 1) / per_block);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == HN_DTYPE_BF16) {
    hipLaunchKernelGGL(gated_residual_kernel<HN_DTYPE_BF16>, dim3(blocks), dim3(kFlatThreads), 0, st,
                       (const uint16_t*)x, (const uint16_t*)y, (const uint16_t*)gate, (uint16_t*)out, nchunk, D / 8, L);
    return HN_LAUNCH_CHECK("gated_residual_kernel");
  }
  if (dtype == HN_DTYPE_F16) {
    hipLaunchKernelGGL(gated_residual_kernel<HN_DTYPE_F16>, dim3(blocks), dim3(kFlatThreads), 0, st,
                       (const uint16_t*)x, (const uint16_t*)y, (const uint16_t*)gate, (uint16_t*)out, nchunk, D / 8, L);
    return HN_LAUNCH_CHECK("gated_residual_kernel");
  }
  set_error("hn_gated_residual: unsupported dtype %d", dtype);
  return HN_ERR_UNSUPPORTED;
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
  const int64_t w = D / 8;
  const unsigned blocks = (unsigned)((n_heads * w + 255) / 256);
  hipStream_t st = (hipStream_t)stream;
#define HN_QK(WW, R)                                                                                          \
  hipLaunchKernelGGL((qk_norm_rope_kernel<WW, R>), dim3(blocks), dim3(256), 0, st, (const uint16_t*)x, ldx,   \
                     weight, cos_t, sin_t, n_heads, H, L, eps, (uint16_t*)y)
  const bool rope = cos_t != nullptr;
  if (w == 8) { if (rope) HN_QK(8, true); else HN_QK(8, false); }
  else if (w == 16) { if (rope) HN_QK(16, true); else HN_QK(16, false); }
  else { if (rope) HN_QK(32, true); else HN_QK(32, false); }
#undef HN_QK
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
  const unsigned blocks = (unsigned)((n_heads * 16 + 255) / 256);
  hipLaunchKernelGGL(pixelumm_qk_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x, ldx,
                     (const float*)weight_t, (const float*)weight_hw, cos_t, sin_t, n_heads, H, eps, (uint16_t*)y);
  return HN_LAUNCH_CHECK("pixelumm_qk_kernel");
}
