/*
 * hynomas.h -- C ABI of the gfx950 (MI355X) kernels for Hy-Nomas' quantized DiT linear path.
 *
 * The reference (PedroMarinhoDev/ComfyUI-Hy-Nomas) exposes this path as Python functions backed by
 * Triton kernels; each entry point below replaces one of them and cites it (reference-tree file:line).
 * The Python modules hy_nomas/kernels.py, fused.py and ops.py of this package keep the reference's call
 * signatures and call these entry points through ctypes.
 *
 * Conventions shared by every entry point:
 *   - all tensor arguments are device pointers; sizes and strides are in elements;
 *   - the last dimension of every matrix is unit-stride; row strides are explicit;
 *   - `stream` is a hipStream_t (pass torch.cuda.current_stream().cuda_stream); the call only enqueues
 *     work, outputs are owned by the caller, nothing is allocated;
 *   - the return value is HN_OK or an error code; hn_last_error() describes the last failure of the
 *     calling thread.  Shapes are validated before any launch.
 */
#ifndef HYNOMAS_H
#define HYNOMAS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum hn_status { HN_OK = 0, HN_ERR_ARG = 1, HN_ERR_HIP = 2, HN_ERR_UNSUPPORTED = 3 };

/* element types of activation / output tensors */
enum hn_dtype { HN_DTYPE_BF16 = 0, HN_DTYPE_F16 = 1, HN_DTYPE_F32 = 2 };

/* code types of quantized operands: int8, or OCP float8 e4m3fn (torch.float8_e4m3fn) */
enum hn_kind { HN_KIND_INT8 = 0, HN_KIND_FP8 = 1 };

/* int8 rounding of x / scale: half away from zero (the reference's rule), or half to even */
enum hn_round { HN_ROUND_HALF_AWAY = 0, HN_ROUND_HALF_EVEN = 1 };

/* GEMM epilogues (kernels.py:149 EPILOGUES), a raw int32 accumulator output for testing, and the SwiGLU
 * product of the PixelUMM decoder MLP requantized for its down projection */
enum hn_epilogue { HN_EPI_NONE = 0, HN_EPI_GELU = 1, HN_EPI_GELU_QUANT = 2, HN_EPI_ACC32 = 3, HN_EPI_SWIGLU_QUANT = 4 };

/* row normalisation of the adaLN kernels: LayerNorm without affine (the reference), or RMSNorm */
enum hn_norm { HN_NORM_LAYER = 0, HN_NORM_RMS = 1 };

/* Library version (major * 10000 + minor * 100 + patch). */
int hn_version(void);

/* Text of the calling thread's last error ("" if none). */
const char* hn_last_error(void);

/*
 * Dynamic activation quantization.  Replaces kernels.quantize_activations / _quantize_kernel
 * (hy_nomas/kernels.py:22-54).
 *   x [M, K] (x_dtype, row stride ldx) -> q [M, K] int8 or e4m3 codes (row stride ldq),
 *   s [M, K / group] fp32 (row stride lds).
 * group = 128 reproduces the reference (one scale per token and 128 channels); group = K gives one scale
 * per token.  K % 128 == 0.  int8: scale = absmax / 127 (1 for an all-zero group); fp8: scale =
 * max(absmax, 1e-12) / 448.
 */
int hn_quantize_act(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind,
                    int rounding, void* q, int64_t ldq, float* s, int64_t lds, void* stream);

/*
 * Block-scaled 8-bit GEMM.  Replaces kernels.block_gemm / _gemm_body (hy_nomas/kernels.py:80-170).
 *   out[m, n] = sum_g (part_g[m, n] * sa[m, g]) * sw[n, g]  (+ bias[n]),  g over K / group groups,
 * part_g the exact int32 (int8) or fp32 (fp8) dot product of group g; the sum runs in group order as
 * acc = fma(part * sa, sw, acc).
 *   qa [M, K] codes (row stride lda), qw [N, K] codes (row stride ldw, K-major: the NT layout),
 *   sa [M, K / group] (row stride ldsa), sw [N / sw_rows, K / group] (row stride ldsw), fp32;
 *   bias [N] of bias_dtype or NULL.
 * sw_rows = 1: one weight-scale row per output channel (the reference's layout).  sw_rows = 128 (group
 * 128 only): one row per 128 output channels, sw [ceil(N / 128), K / 128] -- the 128 x 128 block scales
 * of the FP8 block-128 weight layout (hy_nomas/pixelumm.py:60-63, 77-82) without the repeat_interleave
 * its fp8 linear applies before block_linear (pixelumm.py:147-152); the fold is then
 * acc = fma(part, sa * sw, acc).
 * group = 128 (the reference's g128 layout) or K (per-token activations x per-channel weights); with int8
 * codes, group = K (and ACC32) needs K < 131072, so that the whole-K int32 sum cannot overflow.
 * epilogue NONE: out [M, N] of out_dtype.  GELU: out = bf16(gelu_tanh(bf16(acc))) (kernels.py:125-128).
 * GELU_QUANT: out int8 [M, N] codes of the GELU output, quantized per row and 128 columns, with scales
 * qs [M, N / 128] (kernels.py:129-137); N % 128 == 0.  ACC32: out int32 [M, N] = full-K integer dot
 * products (int8 only; a test hook, scales and bias are ignored).
 * SWIGLU_QUANT: the decoder MLP's down_proj input, down_proj(silu(gate_proj(x)) * up_proj(x))
 * (hy_nomas/pixelumm.py:314-323), from one GEMM over the gate and up weights.  qw [N, K] holds them
 * interleaved in 128-row blocks: rows 256 b .. 256 b + 127 are gate rows 128 b .., the next 128 rows the
 * up rows 128 b .. (sw, and bias if given, interleaved the same way).  With g = bf16(gate output) and
 * u = bf16(up output), h = bf16(bf16(g / (1 + exp(-g))) * u) (torch's bf16 silu and product) is quantized
 * per row and 128 columns like hn_quantize_act with this GEMM's kind: out [M, N / 2] codes (int8 or e4m3,
 * row stride ldo), qs [M, N / 256] fp32.  N % 256 == 0; per-token scales (group == K), or fp8 with
 * sw_rows == 128.
 * K % 128 == 0; M, N >= 1.
 */
int hn_block_gemm(const void* qa, int64_t lda, const float* sa, int64_t ldsa, const void* qw, int64_t ldw,
                  const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype, int64_t M, int64_t N, int64_t K,
                  int64_t group, int kind, int epilogue, void* out, int out_dtype, int64_t ldo, float* qs,
                  int64_t ldqs, void* stream);

/*
 * W8A8 linear in one call: dynamic activation quantization (as hn_quantize_act) followed by the block-scaled
 * GEMM (as hn_block_gemm, epilogue NONE).  Replaces kernels.block_linear (hy_nomas/kernels.py:210-222) for
 * K % 128 == 0 and M > 0; the reference's dequantize + F.linear fallback for other shapes stays with the
 * caller.
 *   x [M, K] (x_dtype, row stride ldx) is quantized per token and `group` channels (128: the reference;
 *   K: one scale per token) with `kind` codes and `rounding`; the codes and scales are written to
 *   `workspace` (256-byte aligned, at least hn_block_linear_workspace_bytes(M, K, group) bytes; its contents
 *   on entry do not matter and are overwritten) and multiplied with qw / sw / bias as hn_block_gemm does,
 *   into out [M, N] of out_dtype (row stride ldo).
 * With kind FP8 and sw_rows == 128 the weight scales must be positive and finite.
 */
int64_t hn_block_linear_workspace_bytes(int64_t M, int64_t K, int64_t group);

int hn_block_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind,
                    int rounding, const void* qw, int64_t ldw, const float* sw, int64_t ldsw, int64_t sw_rows,
                    const void* bias, int bias_dtype, int64_t N, void* out, int out_dtype, int64_t ldo,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * hn_block_linear without a workspace argument and without allocating: the activation codes and scales go
 * to a scratch array of HN_NOALLOC_SCRATCH_BYTES in device memory that the library holds on each GPU it
 * runs on until the process ends.  No counterpart in the reference: this entry point is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops that forbid hipMalloc).
 * Arguments and results are those of hn_block_linear; a problem needing more than
 * HN_NOALLOC_SCRATCH_BYTES (hn_block_linear_workspace_bytes(M, K, group)) is rejected with HN_ERR_ARG.
 * All calls on one GPU share its array: calls that overlap on one GPU (other streams or threads) race,
 * and must be serialized by the caller.  The first call on each device looks up the array's device address
 * (hipGetSymbolAddress); callers that capture the call into a HIP graph make one call on that device before
 * capturing.  The captured call records kernel launches only (no memset, copy or allocation).
 */
#define HN_NOALLOC_SCRATCH_BYTES (32LL << 20)

int hn_block_linear_noalloc(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind,
                            int rounding, const void* qw, int64_t ldw, const float* sw, int64_t ldsw, int64_t sw_rows,
                            const void* bias, int bias_dtype, int64_t N, void* out, int out_dtype, int64_t ldo,
                            void* stream);

/*
 * The QKV projection of a double-stream block with QK-norm and RoPE in its epilogue, written head-major
 * for attention.  Replaces the block_gemm of the three q/k/v linears plus the two fused.qk_norm_rope
 * calls of DoubleStreamBlock._qkv (hy_nomas/model.py:253-267, fused.py:65-105), and the [B, L, H, D] ->
 * [B, H, L, D] copies attention makes of q, k and v.
 *   qa [B * L, K] codes with scales sa, qw [3 * hidden, K] = the q, k and v weights stacked (scales sw
 *   [3 * hidden / sw_rows, K / group], bias [3 * hidden] or NULL), as hn_block_gemm;
 *   out bf16 [3, B, hidden / 128, L_total, 128]: part 0/1/2 = q/k/v, token l of batch b at row
 *   l_offset + l, so two streams (image, text) can fill one buffer at their own token offsets.
 * q and k: x = bf16(projection), r = 1 / sqrt(mean over the head's 128 channels of x^2 + eps),
 * n = bf16(bf16(x r) * w) with w = q_norm_w / k_norm_w ([128] fp32), then, if cos/sin ([L, 128] fp32) are
 * given, (n_2i c_2i - n_2i+1 s_2i, n_2i+1 c_2i+1 + n_2i s_2i+1) for the pairs (2i, 2i + 1).  v: bf16.
 * Head dim 128; hidden % 128 == 0.
 */
int hn_qkv_heads(const void* qa, int64_t lda, const float* sa, int64_t ldsa, const void* qw, int64_t ldw,
                 const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype, int64_t B,
                 int64_t L, int64_t hidden, int64_t K, int64_t group, int kind, const float* q_norm_w,
                 const float* k_norm_w, const float* cos_t, const float* sin_t, float eps, void* out,
                 int64_t L_total, int64_t l_offset, void* stream);

/*
 * hn_qkv_heads with v written straight into the V^T layout hn_attention reads (its `vt`, `svb`, `svh`, `svd`),
 * replacing the head-major v and the V^T copy the HIP attention backend would make of it (the V operand of
 * hy_nomas/model.py:145-150 `attention`): out then holds only q and k, [2, B, hidden / 128, L_total, 128];
 * token l of batch b lands at key l_offset + l of V^T rows b, h.  Needs L % 32 == 0, l_offset % 16 == 0, a
 * 16-byte aligned vt, strides that are multiples of 8 with svd >= l_offset + L, svh >= 128 svd and
 * svb >= (hidden / 128) svh.  Keys this call does not write (other streams, the padding up to a multiple of
 * 64) are left as they are.  Other arguments and results are those of hn_qkv_heads.
 */
int hn_qkv_heads_vt(const void* qa, int64_t lda, const float* sa, int64_t ldsa, const void* qw, int64_t ldw,
                    const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype, int64_t B,
                    int64_t L, int64_t hidden, int64_t K, int64_t group, int kind, const float* q_norm_w,
                    const float* k_norm_w, const float* cos_t, const float* sin_t, float eps, void* out,
                    int64_t L_total, int64_t l_offset, void* vt, int64_t svb, int64_t svh, int64_t svd,
                    void* stream);

/*
 * Softmax attention over all keys (no mask).  Replaces the scaled-dot-product attention of the double-stream
 * block (hy_nomas/model.py:145-150 `attention`, which hands q / k / v [B, L, H, D] to ComfyUI's backend),
 * and each query group's call in segment_attention (model.py:199-223) once the caller has gathered that
 * group's keys.
 *   out[b, i, h, :] = sum_j softmax_j(scale * q[b, i, h, :] . k[b, j, h, :]) v[b, j, h, :]
 * bf16 q, k, out with head dim D == 128 (contiguous), any element strides of batch / head / token;
 * V is given transposed with the keys of each 16-key group reordered: key j = 16 g + 8 a + 4 b + c
 * (a, b in {0, 1}, c in 0..3) of dim d at vt + b svb + h svh + d svd + 16 g + 8 b + 4 a + c (the order 0-3,
 * 8-11, 4-7, 12-15 in each group), and every V^T row must be readable up to ceil(Lk / 64) * 64 positions with
 * finite values at the positions of keys past Lk (svd >= that; zeros are the usual padding).
 * 0 < skj <= 2^23 and 0 < svd <= 2^22 elements.
 * fp32 scores and softmax, bf16 probabilities in the second product, bf16 out.  Lk >= 1.
 */
int hn_attention(const void* q, int64_t sqb, int64_t sqh, int64_t sqi, const void* k, int64_t skb, int64_t skh,
                 int64_t skj, const void* vt, int64_t svb, int64_t svh, int64_t svd, void* out, int64_t sob,
                 int64_t soh, int64_t soi, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, float scale,
                 void* stream);

/*
 * LayerNorm (or RMSNorm) + adaLN modulate.  Replaces fused.adaln / _adaln_kernel (hy_nomas/fused.py:37-62).
 *   x [B, L, D] contiguous (x_dtype bf16 or fp16), shift/scale [B, D] -> y [B, L, D] (same dtype):
 *   y = norm(x) * bf16(1 + scale[b]) + shift[b].
 */
int hn_adaln(const void* x, const void* shift, const void* scale, int dtype, int64_t B, int64_t L, int64_t D,
             float eps, int norm, void* y, void* stream);

/*
 * LayerNorm (or RMSNorm) + modulate + int8 quantization.  Replaces kernels.adaln_quant / _adaln_quant_kernel
 * (hy_nomas/kernels.py:173-207).  D % 128 == 0 (any multiple, e.g. 3072).
 *   q [B * L, D] int8 codes of bf16(norm(x) * bf16(1 + scale) + shift), scales s fp32:
 *   group = 128 (the reference): s [B * L, D / 128], one scale per token and 128 channels;
 *   group = D (per-token extension, D <= 4096): s [B * L, 1].
 */
int hn_adaln_quant(const void* x, const void* shift, const void* scale, int dtype, int64_t B, int64_t L,
                   int64_t D, float eps, int norm, int rounding, int64_t group, int8_t* q, float* s, void* stream);

/*
 * Gated residual.  Replaces fused.gated_residual / _gated_residual_kernel (hy_nomas/fused.py:108-128).
 *   out = x + bf16(y * gate[b]) rounded to the dtype; x, y, out [B, L, D] contiguous, gate [B, D].
 */
int hn_gated_residual(const void* x, const void* y, const void* gate, int dtype, int64_t B, int64_t L,
                      int64_t D, void* out, void* stream);

/*
 * Gated residual, then the camera module's per-frame output added to every token of its frame: the end
 * of a double-stream block's image side plus the broadcast add after it (hy_nomas/model.py:275-284 with
 * hy_nomas/model.py:518-520), in one pass.
 *   out = dtype(dtype(x + bf16(y * gate[b])) + frame[b, t]) for token p of frame t:
 *   x, y, out [B, T * P, D] contiguous, gate [B, D], frame [B, T, D] contiguous, all of dtype.
 */
int hn_gated_residual_frames(const void* x, const void* y, const void* gate, const void* frame, int dtype,
                             int64_t B, int64_t T, int64_t P, int64_t D, void* out, void* stream);

/*
 * Row-scaled int8 dequantization.  Replaces world.dequantize_kv (hy_nomas/world.py:93-94):
 *   out[r, :] = out_dtype(float(q[r, :]) * s[r * lds]), the fp32 product rounded once, then to out_dtype.
 *   q [rows, D] int8 (row stride ldq), s fp32 (lds = 1 for [rows, 1]), out [rows, D] (row stride ldo).
 *   D % 16 == 0; q, out 16-byte aligned; row strides multiples of 16 elements.  The matching quantizer
 *   (world.quantize_kv, world.py:83-90: absmax per token and head, half away from zero) is
 *   hn_quantize_act with group = D.
 */
int hn_dequantize_rows(const int8_t* q, int64_t ldq, const float* s, int64_t lds, int64_t rows, int64_t D,
                       void* out, int out_dtype, int64_t ldo, void* stream);

/*
 * Per-head RMSNorm + interleaved RoPE.  Replaces fused.qk_norm_rope / _qk_norm_rope_kernel
 * (hy_nomas/fused.py:65-105).
 *   x [B, L, H, D] bf16 with token stride ldx (heads contiguous, batch stride L * ldx), weight [D] fp32
 *   holding the bf16 weight's values, cos/sin [L, D] fp32 or both NULL (no rotation) -> y [B, L, H, D]
 *   bf16 contiguous.  D in {64, 128, 256}.
 */
int hn_qk_norm_rope(const void* x, int64_t ldx, const float* weight, const float* cos_t, const float* sin_t,
                    int64_t B, int64_t L, int64_t H, int64_t D, float eps, void* y, void* stream);

/*
 * PixelUMM split-half RMSNorm + sectioned MRoPE.  Replaces fused.pixelumm_qk / _pixelumm_qk_kernel
 * (hy_nomas/fused.py:131-186).
 *   x [N, H, D] bf16 with token stride ldx, weight_t / weight_hw [D / 2] fp32 (the weights' values),
 *   cos/sin [N, D] fp32 -> y [N, H, D] bf16.  D == 128 (PixelUMM's head_dim).
 */
int hn_pixelumm_qk(const void* x, int64_t ldx, const void* weight_t, const void* weight_hw, const float* cos_t,
                   const float* sin_t, int64_t N, int64_t H, int64_t D, float eps, void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HYNOMAS_H */
