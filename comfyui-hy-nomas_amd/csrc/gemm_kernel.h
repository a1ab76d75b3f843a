// Block-scaled 8-bit GEMM on the gfx950 matrix cores (hy_nomas/kernels.py:80-170, _gemm_body / block_gemm).
//
//   out[m, n] = sum_g fma-chain( part_g[m, n] * sa[m, g], sw[n, g] )  (+ bias[n]),  then an epilogue.
//
// Operand roles.  The weight tile is the MFMA "A" operand (rows = output channels n) and the activation
// tile the "B" operand (columns = tokens m), so each lane of a 32x32 accumulator holds one token and runs
// of four consecutive output channels: 8-byte bf16 stores along the contiguous N axis of out [M, N].
//
// Tiling.  A workgroup owns a BN x BM output tile (BN = WN*TN*32 channels, BM = WM*TM*32 tokens) and walks
// K in stages of 128 bytes (one g128 group).  Each stage stages the weight and activation tiles in LDS
// (double buffered; rows of 128 bytes, 16-byte chunks XOR-swizzled by row so that the ds_read_b128 of 8
// consecutive rows hit 8 distinct bank groups).  Global loads of stage k+1 are issued before the MFMAs
// of stage k and land in LDS after them, so one barrier per stage suffices.
//
// Group modes.  group == K (per-token activations x per-channel weights): one integer (int8) or fp32 (fp8)
// accumulator across the whole K, dequantized once in the epilogue.  group == 128 (the reference's g128
// layout): each stage produces the group partial, which is folded into an fp32 accumulator with
// acc = fma(float(part) * sa[m, g], sw[n, g], acc); the per-stage scales ride along in LDS.
//
// Workgroup order.  Consecutive workgroup ids are dealt round-robin to the 8 XCDs; the id is remapped so
// each XCD owns a contiguous range of tiles, which are then visited in column groups of 8 token tiles so
// that concurrently running tiles share weight and activation panels in that XCD's L2.
#pragma once

#include "hn_common.h"

namespace hn {

struct GemmArgs {
  const uint8_t* qa;
  int64_t lda;
  const float* sa;
  int64_t ldsa;
  const uint8_t* qw;
  int64_t ldw;
  const float* sw;
  int64_t ldsw;
  const void* bias;
  int bias_dtype;
  int64_t M, N, K;
  void* out;
  int64_t ldo;
  float* qs;
  int64_t ldqs;
  int tiles_m, tiles_n;
  int vec_store;    // out rows 8-byte aligned and N % 4 == 0
  int stage_store;  // 2-byte out with 16-byte aligned rows and N % 8 == 0: LDS-staged 16-byte stores
};

constexpr int kBK = 128;      // bytes of K per stage (= one g128 group)
constexpr int kGroupM = 8;    // token tiles per column group in the tile order
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_remap(int bid, int nb) {
  const int xcd = bid % kXcds, local = bid / kXcds;
  const int per = nb / kXcds, rem = nb % kXcds;
  return xcd * per + (xcd < rem ? xcd : rem) + local;
}

// Swizzled byte offset of 16-byte chunk c of tile row `row` (rows are 128 bytes).
__device__ __forceinline__ int swz(int row, int c) { return row * kBK + ((c ^ (row & 7)) << 4); }

__device__ __forceinline__ float load_bias(const void* bias, int dt, int64_t n) {
  if (dt == HN_DTYPE_BF16) return bf16_bits_to_f32(((const uint16_t*)bias)[n]);
  if (dt == HN_DTYPE_F16) return f16_bits_to_f32(((const uint16_t*)bias)[n]);
  return ((const float*)bias)[n];
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // kernels.py:74-77, fp32, evaluated in the order written
  float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  float sig = 1.0f / (1.0f + expf(-(2.0f * inner)));
  return 0.5f * x * (1.0f + (2.0f * sig - 1.0f));
}

template <int KIND>
struct Mfma;

// int8: v_mfma_i32_32x32x32_i8 -- 16 bytes of A and B per lane, 16 int32 accumulators.
template <>
struct Mfma<HN_KIND_INT8> {
  using Frag = v4i;
  using Acc = v16i;
  static constexpr int kSliceK = 32;  // K bytes per instruction
  __device__ __forceinline__ static Acc run(const Frag& a, const Frag& b, const Acc& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static Frag load(const char* tile, int row, int slice, int lane) {
    return *reinterpret_cast<const Frag*>(tile + swz(row, slice * 2 + (lane >> 5)));
  }
  __device__ __forceinline__ static float to_f32(int v) { return (float)v; }
  __device__ __forceinline__ static float get(const Acc& c, int r) { return __int_as_float(c[r]); }
  __device__ __forceinline__ static void put(Acc& c, int r, float v) { c[r] = __float_as_int(v); }
};

// fp8 e4m3: v_mfma_f32_32x32x64_f8f6f4 (format 0 = e4m3 for both operands, no block scales) --
// 32 bytes of A and B per lane, 16 fp32 accumulators.
template <>
struct Mfma<HN_KIND_FP8> {
  using Frag = v8i;
  using Acc = v16f;
  static constexpr int kSliceK = 64;
  __device__ __forceinline__ static Acc run(const Frag& a, const Frag& b, const Acc& c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
  __device__ __forceinline__ static Frag load(const char* tile, int row, int slice, int lane) {
    const int c0 = slice * 4 + (lane >> 5) * 2;
    v4i lo = *reinterpret_cast<const v4i*>(tile + swz(row, c0));
    v4i hi = *reinterpret_cast<const v4i*>(tile + swz(row, c0 + 1));
    Frag f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
  __device__ __forceinline__ static float to_f32(float v) { return v; }
  __device__ __forceinline__ static float get(const Acc& c, int r) { return c[r]; }
  __device__ __forceinline__ static void put(Acc& c, int r, float v) { c[r] = v; }
};

typedef __attribute__((address_space(3))) void* lds_ptr;

// Wave-wide direct-to-LDS loads: lane i's 16 (or 4) bytes from g land at lds_wave_base + i * 16 (or 4).
__device__ __forceinline__ void g2lds16(const void* g, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr)lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void g2lds4(const void* g, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr)lds_wave_base, 4, 0, 0);
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int KIND, int EPI, bool G128, int WN, int WM, int TN, int TM, int OUT_DT>
__global__ __launch_bounds__(WN* WM * 64) void block_gemm_kernel(const GemmArgs a) {
  using MF = Mfma<KIND>;
  using Acc = typename MF::Acc;
  using Frag = typename MF::Frag;
  constexpr int NW = WN * WM;
  constexpr int BN = WN * TN * 32, BM = WM * TM * 32;
  constexpr int A_BYTES = BN * kBK, B_BYTES = BM * kBK;
  constexpr int SC_BYTES = G128 ? (BN + BM) * 4 : 0;
  constexpr int STAGE = A_BYTES + B_BYTES + SC_BYTES;
  constexpr int A_KB = BN / 8 / NW, B_KB = BM / 8 / NW;  // 1 KB direct loads per wave per stage
  constexpr int SLICES = kBK / MF::kSliceK;
  static_assert(A_KB * NW * 8 == BN && B_KB * NW * 8 == BM, "tile rows not divisible among waves");
  static_assert(!G128 || (BN + BM) / 64 <= NW, "not enough waves to stage the scales");
  static_assert(EPI != HN_EPI_GELU_QUANT || TN * 32 == 128, "gelu_quant needs a 128-channel wave tile");
  // Epilogue staging of 2-byte outputs: each wave transposes its BMW x BNW sub-tile through LDS (token-major
  // rows padded by 16 bytes) so the stores are full 16-byte lanes along N; the per-channel scales and bias
  // sit after the staging area.
  constexpr bool STAGED = OUT_DT != HN_DTYPE_F32 && (EPI == HN_EPI_NONE || EPI == HN_EPI_GELU);
  constexpr int OPITCH = TN * 32 * 2 + 16;
  constexpr int EP_OFF = STAGED ? NW * TM * 32 * OPITCH : 0;
  constexpr int SMEM = EP_OFF + 2 * BN * 4 > 2 * STAGE ? EP_OFF + 2 * BN * 4 : 2 * STAGE;
  __shared__ __align__(16) char smem[SMEM];

  // ---- tile coordinates
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int group_size = kGroupM * a.tiles_n;
  const int first_m = (logical / group_size) * kGroupM;
  const int size_m = min(a.tiles_m - first_m, kGroupM);
  const int tm_idx = first_m + (logical % group_size) % size_m;
  const int tn_idx = (logical % group_size) / size_m;
  const int64_t m0 = (int64_t)tm_idx * BM, n0 = (int64_t)tn_idx * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave % WN, wm = wave / WN;

  // ---- direct-to-LDS load plan.  Wave w fills the 1 KB blocks q = w + NW * u of each tile; block q is
  // rows 8q .. 8q+7, and lane i lands in row 8q + i/8 at physical chunk i%8, which holds logical chunk
  // (i%8) ^ (i/8) under the row swizzle.
  const int lrow = lane >> 3, lchunk = (lane & 7) ^ (lane >> 3);
  const uint8_t* gw[A_KB];
  const uint8_t* ga[B_KB];
#pragma unroll
  for (int u = 0; u < A_KB; u++) {
    const int64_t n = min(n0 + (int64_t)(wave + NW * u) * 8 + lrow, a.N - 1);
    gw[u] = a.qw + n * a.ldw + lchunk * 16;
  }
#pragma unroll
  for (int u = 0; u < B_KB; u++) {
    const int64_t m = min(m0 + (int64_t)(wave + NW * u) * 8 + lrow, a.M - 1);
    ga[u] = a.qa + m * a.lda + lchunk * 16;
  }
  // g128: waves 0 .. BN/64-1 stage sw[n0 + 64 w + lane, g], the next BM/64 waves sa[m0 + ..., g]
  const float* gsc = nullptr;
  int sc_off = 0;
  if constexpr (G128) {
    if (wave < BN / 64) {
      gsc = a.sw + min(n0 + wave * 64 + lane, a.N - 1) * a.ldsw;
      sc_off = wave * 256;
    } else if (wave < (BN + BM) / 64) {
      gsc = a.sa + min(m0 + (wave - BN / 64) * 64 + lane, a.M - 1) * a.ldsa;
      sc_off = wave * 256;
    }
  }

  auto issue_stage = [&](int kt, int buf) {
    char* base = smem + buf * STAGE;
    const int64_t k0 = (int64_t)kt * kBK;
#pragma unroll
    for (int u = 0; u < A_KB; u++) g2lds16(gw[u] + k0, base + (wave + NW * u) * 1024);
#pragma unroll
    for (int u = 0; u < B_KB; u++) g2lds16(ga[u] + k0, base + A_BYTES + (wave + NW * u) * 1024);
    if constexpr (G128) {
      if (gsc) g2lds4(gsc + kt, base + A_BYTES + B_BYTES + sc_off);
    }
  };

  // ---- accumulators
  Acc acc[TN][TM];                            // MFMA accumulators (whole K, or one group in g128 mode)
  v16f facc[G128 ? TN : 1][G128 ? TM : 1];    // g128: fp32 running sum over groups
#pragma unroll
  for (int i = 0; i < TN; i++)
#pragma unroll
    for (int j = 0; j < TM; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
  if constexpr (G128) {
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
      for (int j = 0; j < TM; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) facc[i][j][r] = 0.0f;
  }

  const int nk = (int)(a.K / kBK);
  const int wrow_n = wn * TN * 32 + (lane & 31);  // this lane's A-fragment row within the weight tile
  const int wrow_m = wm * TM * 32 + (lane & 31);  // and B-fragment row within the activation tile

  issue_stage(0, 0);
  wait_vmem();
  __syncthreads();

  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) issue_stage(kt + 1, buf ^ 1);
    const char* As = smem + buf * STAGE;
    const char* Bs = As + A_BYTES;
    if constexpr (G128) {
#pragma unroll
      for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++)
#pragma unroll
          for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    }
#pragma unroll
    for (int s = 0; s < SLICES; s++) {
      Frag fa[TN], fb[TM];
#pragma unroll
      for (int i = 0; i < TN; i++) fa[i] = MF::load(As, wrow_n + i * 32, s, lane);
#pragma unroll
      for (int j = 0; j < TM; j++) fb[j] = MF::load(Bs, wrow_m + j * 32, s, lane);
#pragma unroll
      for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++) acc[i][j] = MF::run(fa[i], fb[j], acc[i][j]);
    }
    if constexpr (G128) {
      const float* sc = reinterpret_cast<const float*>(As + A_BYTES + B_BYTES);
#pragma unroll
      for (int j = 0; j < TM; j++) {
        const float sam = sc[BN + wrow_m + j * 32];
#pragma unroll
        for (int i = 0; i < TN; i++) {
#pragma unroll
          for (int rr = 0; rr < 4; rr++) {
            const float4 swv =
                *reinterpret_cast<const float4*>(sc + wn * TN * 32 + i * 32 + rr * 8 + (lane >> 5) * 4);
            facc[i][j][rr * 4 + 0] = __builtin_fmaf(MF::to_f32(acc[i][j][rr * 4 + 0]) * sam, swv.x, facc[i][j][rr * 4 + 0]);
            facc[i][j][rr * 4 + 1] = __builtin_fmaf(MF::to_f32(acc[i][j][rr * 4 + 1]) * sam, swv.y, facc[i][j][rr * 4 + 1]);
            facc[i][j][rr * 4 + 2] = __builtin_fmaf(MF::to_f32(acc[i][j][rr * 4 + 2]) * sam, swv.z, facc[i][j][rr * 4 + 2]);
            facc[i][j][rr * 4 + 3] = __builtin_fmaf(MF::to_f32(acc[i][j][rr * 4 + 3]) * sam, swv.w, facc[i][j][rr * 4 + 3]);
          }
        }
      }
    }
    wait_vmem();
    __syncthreads();
  }

  // ---- epilogue: lane holds token m = m0 + wrow_m + 32 j and channels n = n0 + wn*TN*32 + 32 i + 8 rr
  //      + 4 (lane >> 5) + q (q = 0..3) in register rr * 4 + q of tile (i, j).
  const int64_t nb = n0 + wn * TN * 32 + (lane >> 5) * 4;
  if constexpr (EPI == HN_EPI_ACC32) {
#pragma unroll
    for (int j = 0; j < TM; j++) {
      const int64_t m = m0 + wrow_m + j * 32;
      if (m < a.M) {
        int32_t* o = reinterpret_cast<int32_t*>(a.out) + m * a.ldo;
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int64_t n = nb + i * 32 + (r >> 2) * 8 + (r & 3);
            if (n < a.N) o[n] = (int32_t)acc[i][j][r];
          }
      }
    }
    return;
  } else {
    // Per-channel scale (per-token mode) and bias of the block's BN channels, staged in the idle LDS.
    float* ep = reinterpret_cast<float*>(smem + EP_OFF);
    for (int t = tid; t < BN; t += NW * 64) {
      const int64_t n = min(n0 + t, a.N - 1);
      ep[t] = G128 ? 0.0f : a.sw[n * a.ldsw];
      ep[BN + t] = a.bias ? load_bias(a.bias, a.bias_dtype, n) : 0.0f;
    }
    __syncthreads();
    const bool has_bias = a.bias != nullptr;
    const int nloc = wn * TN * 32 + (lane >> 5) * 4;
#pragma unroll
    for (int j = 0; j < TM; j++) {
      const int64_t m = m0 + wrow_m + j * 32;
      const bool m_ok = m < a.M;
      const float sam = G128 ? 0.0f : a.sa[(m_ok ? m : a.M - 1) * a.ldsa];
      // dequantize + bias (+ GELU) in place; the results overwrite the accumulator registers as fp32 bits
#pragma unroll
      for (int i = 0; i < TN; i++) {
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
          const float4 sw4 = *reinterpret_cast<const float4*>(ep + nloc + i * 32 + rr * 8);
          const float4 b4 = *reinterpret_cast<const float4*>(ep + BN + nloc + i * 32 + rr * 8);
          const float swq[4] = {sw4.x, sw4.y, sw4.z, sw4.w};
          const float bq[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const int r = rr * 4 + q;
            float v;
            if constexpr (G128) v = facc[i][j][r];
            else v = __builtin_fmaf(MF::to_f32(acc[i][j][r]) * sam, swq[q], 0.0f);
            if (has_bias) v = v + bq[q];
            if constexpr (EPI == HN_EPI_GELU || EPI == HN_EPI_GELU_QUANT) v = rbf16(gelu_tanh(rbf16(v)));
            MF::put(acc[i][j], r, v);
          }
        }
      }
      if constexpr (EPI == HN_EPI_GELU_QUANT) {
        // the wave's TN*32 = 128 channels are one group: lanes l and l^32 hold them for token m
        float peak = 0.0f;
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
          for (int r = 0; r < 16; r++) peak = __builtin_fmaxf(peak, __builtin_fabsf(MF::get(acc[i][j], r)));
        peak = __builtin_fmaxf(peak, shfl_xor_f(peak, 32));
        const float gs = int8_scale(peak);
        FastDiv div(gs);
        if (m_ok) {
          int8_t* o = reinterpret_cast<int8_t*>(a.out) + m * a.ldo;
#pragma unroll
          for (int i = 0; i < TN; i++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
              const int64_t n = nb + i * 32 + rr * 8;
              const uint32_t w = pack4_i8(round_half_away_i8(div(MF::get(acc[i][j], rr * 4 + 0))), round_half_away_i8(div(MF::get(acc[i][j], rr * 4 + 1))),
                                          round_half_away_i8(div(MF::get(acc[i][j], rr * 4 + 2))), round_half_away_i8(div(MF::get(acc[i][j], rr * 4 + 3))));
              if (n < a.N) *reinterpret_cast<uint32_t*>(o + n) = w;
            }
          // N % 128 == 0, so the group is either wholly inside N or wholly past it
          if (lane < 32 && n0 + wn * 128 < a.N) a.qs[m * a.ldqs + (n0 + wn * 128) / 128] = gs;
        }
      } else if (STAGED && a.stage_store) {
        // token row j*32 + (lane & 31) of this wave's staged sub-tile
        char* ob = smem + wave * TM * 32 * OPITCH + (j * 32 + (lane & 31)) * OPITCH;
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
          for (int rr = 0; rr < 4; rr++) {
            const int ocol = i * 32 + rr * 8 + (lane >> 5) * 4;
            *reinterpret_cast<uint2*>(ob + ocol * 2) =
                make_uint2(pack2_out<OUT_DT>(MF::get(acc[i][j], rr * 4 + 0), MF::get(acc[i][j], rr * 4 + 1)),
                           pack2_out<OUT_DT>(MF::get(acc[i][j], rr * 4 + 2), MF::get(acc[i][j], rr * 4 + 3)));
          }
      } else if (m_ok) {
#pragma unroll
        for (int i = 0; i < TN; i++)
#pragma unroll
          for (int rr = 0; rr < 4; rr++) {
            const int64_t n = nb + i * 32 + rr * 8;
            const float v0 = MF::get(acc[i][j], rr * 4 + 0), v1 = MF::get(acc[i][j], rr * 4 + 1), v2 = MF::get(acc[i][j], rr * 4 + 2), v3 = MF::get(acc[i][j], rr * 4 + 3);
            if constexpr (OUT_DT == HN_DTYPE_F32) {
              float* o = reinterpret_cast<float*>(a.out) + m * a.ldo + n;
              if (a.vec_store && n + 3 < a.N) {
                *reinterpret_cast<float4*>(o) = make_float4(v0, v1, v2, v3);
              } else {
                if (n < a.N) o[0] = v0;
                if (n + 1 < a.N) o[1] = v1;
                if (n + 2 < a.N) o[2] = v2;
                if (n + 3 < a.N) o[3] = v3;
              }
            } else {
              uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + m * a.ldo + n;
              const uint32_t lo = pack2_out<OUT_DT>(v0, v1), hi = pack2_out<OUT_DT>(v2, v3);
              if (a.vec_store && n + 3 < a.N) {
                *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
              } else {
                if (n < a.N) o[0] = (uint16_t)(lo & 0xffffu);
                if (n + 1 < a.N) o[1] = (uint16_t)(lo >> 16);
                if (n + 2 < a.N) o[2] = (uint16_t)(hi & 0xffffu);
                if (n + 3 < a.N) o[3] = (uint16_t)(hi >> 16);
              }
            }
          }
      }
    }
    if constexpr (STAGED) {
      if (a.stage_store) {
        // write-back: 16 bytes per lane along N, rows of TN*32 channels; non-temporal so the output stream
        // does not evict the operand panels other tiles are still reading from L2
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes have landed
        __builtin_amdgcn_wave_barrier();
        const char* ob = smem + wave * TM * 32 * OPITCH;
        constexpr int LPR = TN * 32 * 2 / 16, RPI = 64 / LPR;  // lanes per token row, rows per instruction
#pragma unroll
        for (int r0 = 0; r0 < TM * 32; r0 += RPI) {
          const int orow = r0 + lane / LPR, ocol = (lane % LPR) * 8;
          const v4i v = *reinterpret_cast<const v4i*>(ob + orow * OPITCH + ocol * 2);
          const int64_t m = m0 + wm * TM * 32 + orow, n = n0 + wn * TN * 32 + ocol;
          if (m < a.M && n < a.N)
            __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(a.out) + m * a.ldo + n));
        }
      }
    }
  }
}

}  // namespace hn
