/*
 * CPU restatement of Hy-Nomas' quantized DiT linear path (TEST INFRASTRUCTURE ONLY).
 *
 * This file is the parity oracle.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only to check results.  The
 * product path (comfyui-hy-nomas_amd/) never links or calls it.
 *
 * Every float operation is written out in the order the reference evaluates
 * it, compiled with -ffp-contract=off so the compiler cannot fuse a multiply
 * and an add behind our back; fused multiply-adds are spelled fmaf() where the
 * oracle defines one.
 *
 * Reference lines followed (file:line in the reference tree):
 *   hy_nomas/kernels.py:22-42   _quantize_kernel           -> hno_quantize
 *   hy_nomas/kernels.py:67-71   _rbf16                     -> rbf16
 *   hy_nomas/kernels.py:74-77   _gelu_tanh                 -> gelu_tanh
 *   hy_nomas/kernels.py:80-137  _gemm_body                 -> hno_block_gemm
 *   hy_nomas/kernels.py:173-195 _adaln_quant_kernel        -> hno_adaln (quant=1)
 *   hy_nomas/fused.py:37-52     _adaln_kernel              -> hno_adaln (quant=0)
 *   hy_nomas/fused.py:65-91     _qk_norm_rope_kernel       -> hno_qk_norm_rope
 *   hy_nomas/fused.py:108-118   _gated_residual_kernel     -> hno_gated_residual
 *   hy_nomas/fused.py:131-175   _pixelumm_qk_kernel        -> hno_pixelumm_qk
 *   hy_nomas/ops.py:41-62       quantize_g128/dequantize   -> hno_quantize (group 128)
 *   hy_nomas/pixelumm.py:322    MLP silu(gate) * up        -> hno_swiglu
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HNO_KIND_INT8 0
#define HNO_KIND_FP8 1
#define HNO_ROUND_HALF_AWAY 0
#define HNO_ROUND_HALF_EVEN 1
#define HNO_EPI_NONE 0
#define HNO_EPI_GELU 1
#define HNO_EPI_GELU_QUANT 2
#define HNO_NORM_LAYER 0
#define HNO_NORM_RMS 1

static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* kernels.py:67-71: round an fp32 to the nearest bf16 (ties to even), kept as fp32. */
static inline float rbf16(float x) {
    uint32_t b = bits_of(x);
    b = (b + (((b >> 16) & 1u) + 0x7FFFu)) & 0xFFFF0000u;
    return float_of(b);
}

/* torch's fp32 -> bf16 store conversion (round to nearest even, NaN kept quiet). */
float hno_bf16_round(float x) {
    if (isnan(x)) return float_of(0x7FC00000u);
    return rbf16(x);
}

/* OCP e4m3fn encoding with round-to-nearest-even.  Anything that rounds past
 * 448 lands on the single NaN code 0x7F (e4m3fn has no infinity); this is the
 * behaviour of torch's .to(torch.float8_e4m3fn) (kernels.py:41 stores
 * x / scale, which never exceeds 448 by more than one fp32 ulp). */
uint8_t hno_e4m3_encode(float f) {
    uint8_t sign = (uint8_t)((bits_of(f) >> 24) & 0x80u);
    float a = fabsf(f);
    if (isnan(a)) return (uint8_t)(0x7F | sign);
    if (a < 0x1p-6f) {                       /* subnormal range: multiples of 2^-9 */
        float m = rintf(a * 0x1p9f);         /* exact scaling, RNE rounding */
        return (uint8_t)(sign | (uint8_t)m); /* m == 8 encodes 2^-6, the first normal */
    }
    if (a >= 512.0f) return (uint8_t)(0x7F | sign);
    int e;
    frexpf(a, &e);
    e -= 1;                                  /* a = mant * 2^e with mant in [1, 2) */
    float mant = ldexpf(a, -e);
    int m = (int)rintf((mant - 1.0f) * 8.0f);
    if (m == 8) { m = 0; e += 1; }
    int code = ((e + 7) << 3) | m;
    if (code >= 0x7F) code = 0x7F;
    return (uint8_t)(sign | (uint8_t)code);
}

float hno_e4m3_decode(uint8_t c) {
    int sign = c & 0x80;
    int e = (c >> 3) & 0xF;
    int m = c & 7;
    float v;
    if (e == 0xF && m == 7) v = NAN;
    else if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sign ? -v : v;
}

/* kernels.py:35 (and ops.py:50, world.py:89): round half away from zero, computed
 * in fp32 exactly as written: y + 0.5 is itself an fp32 sum before floor. */
static inline float round_code(float y, int rounding) {
    if (rounding == HNO_ROUND_HALF_EVEN) return rintf(y);
    return y >= 0.0f ? floorf(y + 0.5f) : ceilf(y - 0.5f);
}

static inline float clamp127(float y) {
    if (y < -127.0f) y = -127.0f;
    if (y > 127.0f) y = 127.0f;
    return y;
}

/* int8 scale of a group (kernels.py:33): absmax / 127, or 1 for an all-zero group. */
static inline float int8_scale(float peak) { return peak > 0.0f ? peak / 127.0f : 1.0f; }
/* fp8 scale of a group (kernels.py:39): max(absmax, 1e-12) / 448. */
static inline float fp8_scale(float peak) { return (peak > 1e-12f ? peak : 1e-12f) / 448.0f; }

/* Quantize one run of n values with one scale; writes codes and returns the scale. */
static float quant_run(const float* x, int64_t n, int kind, int rounding, void* q) {
    float peak = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > peak) peak = a;
    }
    if (kind == HNO_KIND_INT8) {
        float s = int8_scale(peak);
        int8_t* qo = (int8_t*)q;
        for (int64_t i = 0; i < n; i++) qo[i] = (int8_t)clamp127(round_code(x[i] / s, rounding));
        return s;
    }
    float s = fp8_scale(peak);
    uint8_t* qo = (uint8_t*)q;
    for (int64_t i = 0; i < n; i++) qo[i] = hno_e4m3_encode(x[i] / s);
    return s;
}

/* kernels.py:22-54 (group 128) generalised to any group that divides K; group == K
 * is one scale per token.  x [M, ldx] fp32 (values of the bf16 input) ->
 * q [M, K] int8 / e4m3 codes, s [M, K / group]. */
void hno_quantize(const float* x, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind, int rounding,
                  void* q, float* s) {
    int64_t ng = K / group;
    for (int64_t m = 0; m < M; m++) {
        for (int64_t g = 0; g < ng; g++) {
            char* qrow = (char*)q + m * K + g * group;
            s[m * ng + g] = quant_run(x + m * ldx + g * group, group, kind, rounding, qrow);
        }
    }
}

/* kernels.py:74-77, evaluated in fp32 in the order written. */
static inline float gelu_tanh(float x) {
    float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    float sig = 1.0f / (1.0f + expf(-(2.0f * inner)));
    return 0.5f * x * (1.0f + (2.0f * sig - 1.0f));
}

float hno_gelu_tanh(float x) { return gelu_tanh(x); }

/* pixelumm.py:322, F.silu(gate) * up on bf16 tensors: silu in fp32 as x / (1 + exp(-x)), rounded to
 * bf16, then the bf16 product (exact in fp32) rounded to bf16. */
static inline float silu(float x) { return x / (1.0f + expf(-x)); }

float hno_silu(float x) { return silu(x); }

void hno_swiglu(const float* g, const float* u, int64_t n, float* h) {
    for (int64_t i = 0; i < n; i++) h[i] = rbf16(rbf16(silu(g[i])) * u[i]);
}

/* kernels.py:80-137.  For each output element, group by group in order:
 *     acc = fma(part_g * sa[m, g], sb[n, g], acc)
 * where part_g is the exact int32 dot product of the group (int8) or the fp32
 * product sum (fp8, summed in double here, rounded once), then acc += bias[n].
 * epilogue 0: out = acc (the caller rounds to the output dtype);
 * epilogue 1: out = rbf16(gelu(rbf16(acc)));
 * epilogue 2: as 1, then int8 per row and 128 output columns -> qout, qs.
 * acc32, if not NULL, receives the full-K int32 dot products (int8 only).
 * qa [M, K], qw [N, K] codes; sa [M, K/group], sb [N, K/group]. */
void hno_block_gemm(const void* qa, const float* sa, const void* qw, const float* sb, const float* bias,
                    int64_t M, int64_t N, int64_t K, int64_t group, int kind, int epilogue,
                    float* out, int8_t* qout, float* qs, int32_t* acc32) {
    int64_t ng = K / group;
    float* dec_a = NULL;
    float* dec_b = NULL;
    if (kind == HNO_KIND_FP8) {
        const uint8_t* a8 = (const uint8_t*)qa;
        const uint8_t* b8 = (const uint8_t*)qw;
        dec_a = (float*)malloc(sizeof(float) * M * K);
        dec_b = (float*)malloc(sizeof(float) * N * K);
        for (int64_t i = 0; i < M * K; i++) dec_a[i] = hno_e4m3_decode(a8[i]);
        for (int64_t i = 0; i < N * K; i++) dec_b[i] = hno_e4m3_decode(b8[i]);
    }
    #pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; m++) {
        for (int64_t n = 0; n < N; n++) {
            float acc = 0.0f;
            int64_t full = 0;
            for (int64_t g = 0; g < ng; g++) {
                float part;
                if (kind == HNO_KIND_INT8) {
                    const int8_t* a = (const int8_t*)qa + m * K + g * group;
                    const int8_t* b = (const int8_t*)qw + n * K + g * group;
                    int64_t p = 0;
                    for (int64_t k = 0; k < group; k++) p += (int64_t)a[k] * (int64_t)b[k];
                    full += p;
                    part = (float)p;
                } else {
                    const float* a = dec_a + m * K + g * group;
                    const float* b = dec_b + n * K + g * group;
                    double p = 0.0;
                    for (int64_t k = 0; k < group; k++) p += (double)a[k] * (double)b[k];
                    part = (float)p;
                }
                float t = part * sa[m * ng + g];
                acc = fmaf(t, sb[n * ng + g], acc);
            }
            if (acc32) acc32[m * N + n] = (int32_t)full;
            if (bias) acc = acc + bias[n];
            if (epilogue == HNO_EPI_NONE) out[m * N + n] = acc;
            else out[m * N + n] = rbf16(gelu_tanh(rbf16(acc)));
        }
        if (epilogue == HNO_EPI_GELU_QUANT) {
            for (int64_t t = 0; t < N / 128; t++) {
                qs[m * (N / 128) + t] = quant_run(out + m * N + t * 128, 128, HNO_KIND_INT8,
                                                  HNO_ROUND_HALF_AWAY, qout + m * N + t * 128);
            }
        }
    }
    free(dec_a);
    free(dec_b);
}

/* fused.py:37-52 (quant == 0) and kernels.py:173-195 (quant == 1), plus the
 * RMSNorm variant (norm == 1: n = x * rsqrt(mean(x^2) + eps), no centring).
 * Row statistics are accumulated in double (the exact value rounded once);
 * n = (x - mean) * rsqrt(var + eps) in fp32; y = n * rbf16(1 + scale) + shift.
 * quant == 0: y_out = y (caller rounds to bf16).
 * quant == 1: y = rbf16(y), then int8 per 128 channels into q, s. */
void hno_adaln(const float* x, const float* shift, const float* scale, int64_t B, int64_t L, int64_t D, float eps,
               int norm, int quant, int rounding, float* y_out, int8_t* q, float* s) {
    #pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < B * L; row++) {
        int64_t b = row / L;
        const float* xr = x + row * D;
        double sum = 0.0, sq = 0.0;
        float mean = 0.0f;
        if (norm == HNO_NORM_LAYER) {
            for (int64_t i = 0; i < D; i++) sum += xr[i];
            mean = (float)(sum / (double)D);
            for (int64_t i = 0; i < D; i++) {
                double c = (double)xr[i] - (double)mean;
                sq += c * c;
            }
        } else {
            for (int64_t i = 0; i < D; i++) sq += (double)xr[i] * (double)xr[i];
        }
        float var = (float)(sq / (double)D);
        float rstd = (float)(1.0 / sqrt((double)(var + eps)));
        float* yr = y_out + row * D;
        for (int64_t i = 0; i < D; i++) {
            float n = (xr[i] - mean) * rstd;
            float one_plus = rbf16(1.0f + scale[b * D + i]);
            float v = n * one_plus + shift[b * D + i];
            yr[i] = quant ? rbf16(v) : v;
        }
        if (quant) {
            for (int64_t g = 0; g < D / 128; g++)
                s[row * (D / 128) + g] = quant_run(yr + g * 128, 128, HNO_KIND_INT8, rounding, q + row * D + g * 128);
        }
    }
}

/* fused.py:108-118: out = x + rbf16(y * gate[b]); the caller rounds to bf16. */
void hno_gated_residual(const float* x, const float* y, const float* gate, int64_t B, int64_t L, int64_t D,
                        float* out) {
    for (int64_t row = 0; row < B * L; row++) {
        int64_t b = row / L;
        for (int64_t i = 0; i < D; i++) out[row * D + i] = x[row * D + i] + rbf16(y[row * D + i] * gate[b * D + i]);
    }
}

/* fused.py:65-91.  x rows of D values (one per batch, token, head) with token
 * stride ldx (in elements); output contiguous [B, L, H, D] before the bf16 cast.
 * r = rsqrt(mean(x^2) + eps) (sum in double); ne = rbf16(rbf16(xe * r) * we);
 * RoPE on interleaved pairs: oe = ne*c_e - no*s_e, oo = no*c_o + ne*s_o. */
void hno_qk_norm_rope(const float* x, int64_t ldx, const float* w, const float* cosv, const float* sinv,
                      int64_t B, int64_t L, int64_t H, int64_t D, float eps, int rope, float* out) {
    #pragma omp parallel for schedule(static)
    for (int64_t bl = 0; bl < B * L; bl++) {
        int64_t token = bl % L;
        for (int64_t h = 0; h < H; h++) {
            const float* xr = x + bl * ldx + h * D;
            double sq = 0.0;
            for (int64_t i = 0; i < D; i++) sq += (double)xr[i] * (double)xr[i];
            float r = (float)(1.0 / sqrt((double)((float)(sq / (double)D) + eps)));
            float* o = out + (bl * H + h) * D;
            for (int64_t i = 0; i < D; i += 2) {
                float ne = rbf16(rbf16(xr[i] * r) * w[i]);
                float no = rbf16(rbf16(xr[i + 1] * r) * w[i + 1]);
                if (rope) {
                    const float* c = cosv + token * D;
                    const float* sn = sinv + token * D;
                    o[i] = ne * c[i] - no * sn[i];
                    o[i + 1] = no * c[i + 1] + ne * sn[i + 1];
                } else {
                    o[i] = ne;
                    o[i + 1] = no;
                }
            }
        }
    }
}

/* fused.py:131-175: PixelUMM split-half RMSNorm + sectioned rotate-half MRoPE.
 * x [N, ldx] token rows holding H heads of D; wt, whw [D/2]; cos/sin [N, D];
 * out [N, H, D] before the bf16 cast. */
void hno_pixelumm_qk(const float* x, int64_t ldx, const float* wt, const float* whw, const float* cosv,
                     const float* sinv, int64_t N, int64_t H, int64_t D, float eps, float* out) {
    int64_t half = D / 2, quarter = D / 4, eighth = D / 8;
    for (int64_t t = 0; t < N; t++) {
        const float* c = cosv + t * D;
        const float* sn = sinv + t * D;
        for (int64_t h = 0; h < H; h++) {
            const float* xr = x + t * ldx + h * D;
            float* o = out + (t * H + h) * D;
            double st = 0.0, shw = 0.0;
            for (int64_t i = 0; i < half; i++) st += (double)xr[i] * (double)xr[i];
            for (int64_t i = half; i < D; i++) shw += (double)xr[i] * (double)xr[i];
            float rt = (float)(1.0 / sqrt((double)((float)(st / (double)half) + eps)));
            float rhw = (float)(1.0 / sqrt((double)((float)(shw / (double)half) + eps)));
            for (int64_t i = 0; i < quarter; i++) {
                float t0 = xr[i] * rt * wt[i];
                float t1 = xr[quarter + i] * rt * wt[quarter + i];
                o[i] = t0 * c[i] - t1 * sn[i];
                o[quarter + i] = t1 * c[quarter + i] + t0 * sn[quarter + i];
            }
            for (int64_t j = 0; j < eighth; j++) {
                float h0 = xr[half + j] * rhw * whw[j];
                float h1 = xr[half + eighth + j] * rhw * whw[eighth + j];
                float w0 = xr[half + quarter + j] * rhw * whw[quarter + j];
                float w1 = xr[half + quarter + eighth + j] * rhw * whw[quarter + eighth + j];
                o[half + j] = h0 * c[half + j] - h1 * sn[half + j];
                o[half + eighth + j] = h1 * c[half + eighth + j] + h0 * sn[half + eighth + j];
                o[half + quarter + j] = w0 * c[half + quarter + j] - w1 * sn[half + quarter + j];
                o[half + quarter + eighth + j] = w1 * c[half + quarter + eighth + j] + w0 * sn[half + quarter + eighth + j];
            }
        }
    }
}

/* Division lemma used by the device quantizers.  For a group whose bf16 absmax
 * `peak` is at least 2^-80 the device computes every quotient x / s (x a bf16
 * value, |x| <= peak) as q0 = x * rcp(s); e = fma(-q0, s, x); q1 = fma(e, rcp(s),
 * q0), and an int8 code as trunc(q1 + copysign(0.5, q1)) without a clamp (or
 * rint(q1) for half-to-even); smaller peaks divide.  This routine checks that
 * rule exhaustively over every positive finite bf16 peak >= 2^-80 and every bf16
 * |x| <= peak against the reference rule (IEEE x / s, then floor(q + .5) /
 * ceil(q - .5) clamped to +-127, or rint + clamp), comparing int8 codes for both
 * roundings (kind 0) or e4m3 codes (kind 1).  Returns the number of mismatches. */
static int ref_code_half_away(float q) {
    float t = q >= 0.0f ? floorf(q + 0.5f) : ceilf(q - 0.5f);
    t = fminf(fmaxf(t, -127.0f), 127.0f);
    return (int)t;
}
static int ref_code_half_even(float q) {
    float t = rintf(q);
    t = fminf(fmaxf(t, -127.0f), 127.0f);
    return (int)t;
}
int64_t hno_check_fast_division(int fp8, int64_t peak_begin, int64_t peak_end) {
    int64_t bad = 0;
    #pragma omp parallel for reduction(+:bad) schedule(dynamic, 64)
    for (int64_t pbi = peak_begin; pbi < peak_end; pbi++) {
        uint32_t pb = (uint32_t)pbi;
        float p = float_of(pb << 16);
        if (!(p >= 0x1p-80f)) continue;  /* the device divides these groups */
        float s = fp8 ? fp8_scale(p) : int8_scale(p);
        float r = 1.0f / s;
        if (!isfinite(r)) { bad++; continue; }
        for (uint32_t xb = 0; xb <= pb; xb++) {
            for (int sign = 0; sign < 2; sign++) {
                float x = float_of((xb << 16) | (sign ? 0x80000000u : 0u));
                float ref = x / s;
                float q0 = x * r;
                float e = fmaf(-q0, s, x);
                float got = fmaf(e, r, q0);
                if (fp8) {
                    got = copysignf(got, x);
                    if (hno_e4m3_encode(got) != hno_e4m3_encode(ref)) bad++;
                } else {
                    int fast_away = (int)(got + copysignf(0.5f, got));
                    int fast_even = (int)rintf(got);
                    if (fast_away != ref_code_half_away(ref) || fast_even != ref_code_half_even(ref)) bad++;
                }
            }
        }
    }
    return bad;
}

/* Two-operation form of the same int8 quotient: with r = RN(1 / s) and rl = RN(fma(-s, r, 1) * r),
 * q = fma(x, r, x * rl).  The device uses it for int8 groups whose bf16 absmax `peak` satisfies
 * 2^-80 <= peak < 2^100 (above that rl is subnormal and loses the bits it carries); other groups
 * divide.  Checks every such bf16 peak and every bf16 |x| <= peak, both signs, against the reference
 * rule (IEEE x / s, floor / ceil or rint, clamped) for both roundings.  Returns the mismatches.
 * `drop_rl` plants a mistake (rl = 0, i.e. q = x * r) so a test can see the check catch it. */
int64_t hno_check_fast_division2(int64_t peak_begin, int64_t peak_end, int drop_rl) {
    int64_t bad = 0;
    #pragma omp parallel for reduction(+:bad) schedule(dynamic, 64)
    for (int64_t pbi = peak_begin; pbi < peak_end; pbi++) {
        uint32_t pb = (uint32_t)pbi;
        float p = float_of(pb << 16);
        if (!(p >= 0x1p-80f && p < 0x1p100f)) continue;
        float s = int8_scale(p);
        float r = 1.0f / s;
        float rl = drop_rl ? 0.0f : fmaf(-s, r, 1.0f) * r;
        for (uint32_t xb = 0; xb <= pb; xb++) {
            for (int sign = 0; sign < 2; sign++) {
                float x = float_of((xb << 16) | (sign ? 0x80000000u : 0u));
                float ref = x / s;
                float got = fmaf(x, r, x * rl);
                int fast_away = (int)(got + copysignf(0.5f, got));
                int fast_even = (int)rintf(got);
                if (fast_away != ref_code_half_away(ref) || fast_even != ref_code_half_even(ref)) bad++;
            }
        }
    }
    return bad;
}

/* The device's reciprocal of a group scale s (peaks >= 2^-80): r0 = v_rcp_f32(s), accurate to 1 ulp,
 * refined by one Newton step r1 = fma(fma(-r0, s, 1), r0, r0).  For every bf16 peak >= 2^-80 and both
 * scale kinds, this checks that every r0 within +-2 ulp of RN(1 / s) refines to exactly RN(1 / s), so
 * the result does not depend on the hardware's approximation.  Returns the number of failures. */
int64_t hno_check_reciprocal_refinement(void) {
    int64_t bad = 0;
    #pragma omp parallel for reduction(+:bad) schedule(static)
    for (int64_t pbi = 1; pbi < 0x7F80; pbi++) {
        float p = float_of((uint32_t)pbi << 16);
        if (!(p >= 0x1p-80f)) continue;
        for (int fp8 = 0; fp8 < 2; fp8++) {
            float sc = fp8 ? fp8_scale(p) : int8_scale(p);
            float want = 1.0f / sc;
            uint32_t wb = bits_of(want);
            for (int d = -2; d <= 2; d++) {
                float r0 = float_of(wb + (uint32_t)d);
                float e = fmaf(-r0, sc, 1.0f);
                float r1 = fmaf(e, r0, r0);
                if (bits_of(r1) != wb) bad++;
            }
        }
    }
    return bad;
}

/* The device's group scales for peaks >= 2^-80: peak / 127 (int8) and max(peak, 1e-12) / 448 (fp8)
 * as q0 = d * rcp(c); e = fma(-q0, c, d); q1 = fma(e, rcp(c), q0) with rcp(c) the correctly rounded
 * reciprocal of the constant.  Checks every positive finite bf16 peak >= 2^-80 against IEEE
 * division; returns the number of mismatches. */
int64_t hno_check_scale_division(void) {
    int64_t bad = 0;
    for (uint32_t pb = 1; pb < 0x7F80u; pb++) {
        float p = float_of(pb << 16);
        if (!(p >= 0x1p-80f)) continue;
        for (int fp8 = 0; fp8 < 2; fp8++) {
            float c = fp8 ? 448.0f : 127.0f;
            float d = fp8 ? (p > 1e-12f ? p : 1e-12f) : p;
            float r = 1.0f / c;
            float q0 = d * r;
            float e = fmaf(-q0, c, d);
            float got = fmaf(e, r, q0);
            float ref = fp8 ? fp8_scale(p) : int8_scale(p);
            if (bits_of(got) != bits_of(ref)) bad++;
        }
    }
    return bad;
}

void hno_e4m3_encode_array(const float* a, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; i++) out[i] = hno_e4m3_encode(a[i]);
}
