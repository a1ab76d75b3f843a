// Block-scaled 8-bit GEMM on the gfx950 matrix cores (hy_nomas/kernels.py:80-170, _gemm_body / block_gemm).
//
//   out[m, n] = sum_g fma-chain( part_g[m, n] * sa[m, g], sw[n, g] )  (+ bias[n]),  then an epilogue.
//
// Operand roles.  The weight tile is the MFMA "A" operand (rows = output channels n) and the activation
// tile the "B" operand (columns = tokens m), so each lane of a 32x32 accumulator holds one token and runs
// of four consecutive output channels: 8-byte stores along the contiguous N axis of out [M, N].
//
// Tiling.  A workgroup owns a BN x BM output tile (BN = WN*TN*32 channels, BM = WM*TM*32 tokens) and walks
// K in stages of BK bytes.  Each stage's weight and activation rows are copied straight from global memory
// into LDS (gfx950 global_load_lds_dwordx4: no staging registers, no ds_write) into a ring of NS stage
// buffers, NS - 1 stages ahead of the stage being multiplied, so NS - 1 stages of loads are in flight
// while the matrix cores work.  One barrier per stage: it publishes stage kt to every wave and retires
// the buffer of stage kt - 1, which the loads of stage kt + NS - 1 then overwrite.
//
// LDS layout.  A stage row of BK bytes is BK / 16 chunks of 16 bytes, XOR-swizzled by row so that the 16
// lanes the LDS serves together (rows r .. r + 15 of one MFMA fragment read) hit 16 distinct bank
// groups: chunk c of row r sits at chunk c ^ ((r >> 2) & 3) for 64-byte rows and c ^ ((r >> 1) & 7) for
// 128-byte rows.  The direct loads write 1 KB per wave instruction in lane order, so the swizzle is
// applied on the global side: lane i fetches the logical chunk that belongs at its physical slot.
//
// Group modes.  group == K (per-token activations x per-channel weights): one integer (int8) or fp32 (fp8)
// accumulator across the whole K, dequantized once in the epilogue.  group == 128 (the reference's g128
// layout): the stages of one 128-byte group produce its partial, which is folded into an fp32 accumulator
// with acc = fma(float(part) * sa[m, g], sw[n, g], acc); the group's scales ride along in LDS.  With the
// fp8 128 x 128 block weight scales (one scale row per 128 channels) the fold is
// acc = fma(float(part), sa[m, g] * sw[block, g], acc): one VALU op per output and group.
//
// Workgroup order.  Consecutive workgroup ids are dealt round-robin to the 8 XCDs; the id is remapped so
// each XCD owns a contiguous range of tiles, which are then visited in column groups of 8 token tiles so
// that concurrently running tiles share weight and activation panels in that XCD's L2.
#pragma once

#include <type_traits>
#include <utility>

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
  int sw_rows;  // output channels per weight-scale row: 1, or 128 (fp8 128 x 128 block scales)
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
  // kEpiQkvHeads: the QKV projection of hidden = N / 3 channels, rows m = b * hm_L + l, written head-major
  // to out [3, hm_B, hidden / 128, hm_Ltot, 128] at token hm_loff + l; q and k RMS-normalized per head
  // with weights hm_wq / hm_wk ([128] fp32), then rotated by hm_cos / hm_sin ([hm_L, 128] fp32) if given
  int64_t hm_L, hm_Ltot, hm_loff, hm_hidden, hm_B;
  const float* hm_wq;
  const float* hm_wk;
  const float* hm_cos;
  const float* hm_sin;
  float hm_eps;
  // hm_vt: the v heads go to V^T instead (the attention kernel's layout): element (b, h, d, key p) at
  // hm_vt + b hm_svb + h hm_svh + d hm_svd + p, keys of each 16-key group in the order 0-3, 8-11, 4-7, 12-15,
  // token l at key hm_loff + l (hm_L % 32 == 0, hm_loff % 16 == 0)
  uint16_t* hm_vt;
  int64_t hm_svb, hm_svh, hm_svd;
};

// Internal epilogue id of the head-major QKV projection (entry point hn_qkv_heads).
constexpr int kEpiQkvHeads = 5;

constexpr int kGroupK = 128;  // bytes of K per scale group (the g128 layout)
constexpr int kGroupM = 8;    // token tiles per column group in the tile order
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_remap(int bid, int nb) {
  const int xcd = bid % kXcds, local = bid / kXcds;
  const int per = nb / kXcds, rem = nb % kXcds;
  return xcd * per + (xcd < rem ? xcd : rem) + local;
}

// Physical chunk of logical 16-byte chunk c in stage row `row` (rows of BK bytes).
template <int BK>
__device__ __forceinline__ int swz_chunk(int row, int c) {
  static_assert(BK == 64 || BK == 128, "stage rows are 64 or 128 bytes");
  if constexpr (BK == 64) return c ^ ((row >> 2) & 3);
  else return c ^ ((row >> 1) & 7);
}

__device__ __forceinline__ float load_bias(const void* bias, int dt, int64_t n) {
  if (dt == HN_DTYPE_BF16) return bf16_bits_to_f32(((const uint16_t*)bias)[n]);
  if (dt == HN_DTYPE_F16) return f16_bits_to_f32(((const uint16_t*)bias)[n]);
  return ((const float*)bias)[n];
}
// the same in two steps: the element's bits (no use of the loaded value, so no wait for it), then the value
__device__ __forceinline__ uint32_t load_bias_bits(const void* bias, int dt, int64_t n) {
  return dt == HN_DTYPE_F32 ? ((const uint32_t*)bias)[n] : (uint32_t)((const uint16_t*)bias)[n];
}
__device__ __forceinline__ float bias_from_bits(uint32_t b, int dt) {
  if (dt == HN_DTYPE_BF16) return bf16_bits_to_f32(b);
  if (dt == HN_DTYPE_F16) return f16_bits_to_f32(b);
  return __uint_as_float(b);
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // kernels.py:74-77 in fp32, in the order written, with sigmoid(2 inner) = 1 / (1 + exp(-2 inner)) taken
  // from the hardware base-2 exponential and reciprocal (v_exp_f32, v_rcp_f32: about 1 ulp each).  The
  // result carries a few fp32 ulps of error, which the bf16 rounding that follows hides for all but
  // about 1e-4 of the outputs (the reference's tolerance is 1e-3).  exp overflowing to inf gives
  // sigmoid 0, and underflowing to 0 gives 1, as the exact function.
  const float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(inner * -2.8853900817779268f);  // exp(-2 inner)
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  return 0.5f * x * (1.0f + (2.0f * sig - 1.0f));
}

template <int KIND>
struct Mfma;

// int8: v_mfma_i32_32x32x32_i8 -- 16 bytes of A and B per lane (logical chunk 2s + lane/32 of slice s),
// 16 int32 accumulators.
template <>
struct Mfma<HN_KIND_INT8> {
  using Frag = v4i;
  using Acc = v16i;
  static constexpr int kSliceK = 32;  // K bytes per instruction
  template <int BK>
  __device__ __forceinline__ static Frag load(const char* tile, int row, int slice, int lane) {
    return *reinterpret_cast<const Frag*>(tile + row * BK + (swz_chunk<BK>(row, slice * 2 + (lane >> 5)) << 4));
  }
  __device__ __forceinline__ static Acc run(const Frag& a, const Frag& b, const Acc& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static float to_f32(int v) { return (float)v; }
  __device__ __forceinline__ static float get(const Acc& c, int r) { return __int_as_float(c[r]); }
  __device__ __forceinline__ static void put(Acc& c, int r, float v) { c[r] = __float_as_int(v); }
};

// fp8 e4m3: v_mfma_f32_32x32x64_f8f6f4 (format 0 = e4m3 for both operands, no block scales) --
// 32 bytes of A and B per lane (logical chunks 4s + 2 (lane/32) and the next), 16 fp32 accumulators.
template <>
struct Mfma<HN_KIND_FP8> {
  using Frag = v8i;
  using Acc = v16f;
  static constexpr int kSliceK = 64;
  template <int BK>
  __device__ __forceinline__ static Frag load(const char* tile, int row, int slice, int lane) {
    const int c0 = slice * 4 + (lane >> 5) * 2;
    const v4i lo = *reinterpret_cast<const v4i*>(tile + row * BK + (swz_chunk<BK>(row, c0) << 4));
    const v4i hi = *reinterpret_cast<const v4i*>(tile + row * BK + (swz_chunk<BK>(row, c0 + 1) << 4));
    Frag f;
    f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
    f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
    return f;
  }
  __device__ __forceinline__ static Acc run(const Frag& a, const Frag& b, const Acc& c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
  __device__ __forceinline__ static float to_f32(float v) { return v; }
  __device__ __forceinline__ static float get(const Acc& c, int r) { return c[r]; }
  __device__ __forceinline__ static void put(Acc& c, int r, float v) { c[r] = v; }
};

// facc[r] = fma(float(part[r]) * sa, w, facc[r]) where w is lane (l & ~15) + r of `w16` (a DPP row
// broadcast of lane r of the caller's 16-lane row): one v_fmac_f32_dpp per output.  The fma is the
// same single rounding as __builtin_fmaf.
template <int R>
__device__ __forceinline__ float fmac_row_bcast(float acc, float w16, float t) {
  asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(w16), "v"(t), "n"(R));
  return acc;
}
template <typename Acc, int... R>
__device__ __forceinline__ void fold_row_bcast(v16f& facc, const Acc& part, float sa, float w16,
                                               std::integer_sequence<int, R...>) {
  ((facc[R] = fmac_row_bcast<R>(facc[R], w16, (float)part[R] * sa)), ...);
}
// registers R0 .. R0 + RN - 1 of the same fold
template <int R0, typename Acc, int... R>
__device__ __forceinline__ void fold_rows_bcast(v16f& facc, const Acc& part, float sa, float w16,
                                                std::integer_sequence<int, R...>) {
  ((facc[R0 + R] = fmac_row_bcast<R0 + R>(facc[R0 + R], w16, (float)part[R0 + R] * sa)), ...);
}

// f(std::integral_constant<int, I>()) for I = 0 .. N - 1, in order
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>()), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_seq(f, std::make_integer_sequence<int, N>());
}

// Wait until at most N of this wave's vector-memory loads are outstanding (they retire in issue order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  // gfx9 s_waitcnt: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]; others left at max
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without a memory fence: LDS data published by the barrier is either this kernel's
// direct loads, retired by wait_vmcnt first, or ds_writes retired by an lgkmcnt wait first.  The memory
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// 2-byte outputs are converted to bf16 / fp16 two at a time (round to nearest even).
template <int DT>
__device__ __forceinline__ uint32_t cvt2_out(float a, float b) {
  if constexpr (DT == HN_DTYPE_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
  } else {
    return pack2_out<DT>(a, b);
  }
}

// Persistent kernel: gridDim.x workgroups (at most one per CU) walk the tile list.  Workgroup b runs on
// XCD b % 8 (the dispatcher deals workgroups to XCDs round-robin); each XCD owns a contiguous range of the
// tile order, and its workgroups take every nw-th tile of that range, so the tiles in flight on one XCD
// at any time are consecutive (8 token tiles x 4 channel tiles share their panels in that XCD's L2).
// The first stage of the next tile is issued before the current tile's epilogue, so its load latency
// hides behind the epilogue and the epilogue's stores drain while it lands.
template <int KIND, int EPI, bool G128, int WN, int WM, int TN, int TM, int OUT_DT, int BK, int NS, bool WBLK,
          int WPE = WN * WM / 4>
__global__ __launch_bounds__(WN* WM * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void block_gemm_kernel(const GemmArgs a) {
  using MF = Mfma<KIND>;
  using Acc = typename MF::Acc;
  using Frag = typename MF::Frag;
  constexpr int NW = WN * WM;
  constexpr int BN = WN * TN * 32, BM = WM * TM * 32;
  constexpr int A_BYTES = BN * BK, B_BYTES = BM * BK;
  constexpr int SC_SLOTS = (BN + BM) / 64;                   // g128: 64-float scale slots per stage
  constexpr int SC_PER_WAVE = G128 ? (SC_SLOTS + NW - 1) / NW : 0;
  constexpr int SC_BYTES = SC_PER_WAVE * NW * 256;           // g128 scales of one stage
  constexpr int SCR = (NS + 1) * SC_BYTES;                   // the scales' ring, at offset 0
  constexpr int STAGE = A_BYTES + B_BYTES;                   // operand bytes of one stage buffer
  constexpr int ROWS_PER_KB = 1024 / BK, CHUNKS = BK / 16;
  constexpr int A_KB = A_BYTES / 1024 / NW, B_KB = B_BYTES / 1024 / NW;  // 1 KB direct loads per wave
  constexpr int LOADS = A_KB + B_KB + SC_PER_WAVE;                        // per wave per stage
  constexpr int SLICES = BK / MF::kSliceK;
  constexpr int STAGES_PER_GROUP = kGroupK / BK;
  static_assert(A_KB * NW * 1024 == A_BYTES && B_KB * NW * 1024 == B_BYTES, "tile rows not divisible among waves");
  static_assert(NS == 2, "two stage buffers: the next tile's first stage fills buffer 0 during the epilogue");
  static_assert(SLICES >= 2 && SLICES % 2 == 0, "fragment sets alternate per slice, starting each stage at set 0");
  static_assert(kGroupK % BK == 0, "stage size");
  static_assert(EPI != HN_EPI_GELU_QUANT || TN * 32 == 128, "gelu_quant needs a 128-channel wave tile");
  // swiglu_quant: wave wn = 0 holds gate rows and wn = 1 the up rows of the same 128 MLP channels (the
  // weight interleaves them in 128-row blocks), and each finishes half of the wave's tokens
  static_assert(EPI != HN_EPI_SWIGLU_QUANT || (WN == 2 && TN * 32 == 128 && TM % 2 == 0),
                "swiglu_quant needs two 128-channel waves per tile row and an even token split");
  // WBLK: one weight-scale row per 128 output channels (the fp8 128 x 128 block layout); a wave's TN * 32
  // channels then lie in one block, so the group fold multiplies by one scale product per token
  static_assert(!WBLK || (G128 && (TN * 32) % 128 == 0 && BN % 128 == 0), "block weight scales");
  // RESCALE (fp8 with block weight scales): no separate fp32 running sum.  The matrix core accumulates
  // every group straight into acc, kept in units of the current group's scale product: at each group
  // boundary acc *= ss_g / ss_{g+1} (one VALU op per output, issued block by block between the next
  // group's first products), and the epilogue multiplies by the last group's ss.
  // ss_g = sa[m, g] * sw[block, g] is positive (both quantizers floor their scales).
  constexpr bool RESCALE = G128 && WBLK && KIND == HN_KIND_FP8;
  // Epilogue staging of 2-byte outputs, one block of 32 tokens at a time: each wave transposes its
  // 32 x BNW sub-tile through LDS (token-major rows padded by 16 bytes) so the stores are full 16-byte
  // lanes along N.  The staging area lies past stage buffer 0 (which holds the next tile's first stage).
  // The tile's epilogue operands (per-channel scales and bias, per-token scales) are written at the tile
  // top, while stage buffer 1 fills, so they lie past both the staging area and the stage ring.
  constexpr bool STAGED =
      OUT_DT != HN_DTYPE_F32 && (EPI == HN_EPI_NONE || EPI == HN_EPI_GELU || EPI == kEpiQkvHeads);
  static_assert(EPI != kEpiQkvHeads || (TN * 32 == 128 && OUT_DT == HN_DTYPE_BF16),
                "head-major QKV: one 128-channel head per wave, bf16 out");
  constexpr int OPITCH = TN * 32 * 2 + 16;
  constexpr int STG_OFF = SCR + STAGE;
  constexpr int RING_END = SCR + NS * STAGE;
  // swiglu_quant hands half of each wave's bf16 outputs to its partner wave through the same area
  constexpr int XCH_WAVE = EPI == HN_EPI_SWIGLU_QUANT ? (TM / 2) * TN * 32 * 32 * 2 : 0;
  constexpr int STG_BYTES = STAGED ? NW * 32 * OPITCH : NW * XCH_WAVE;
  constexpr int STG_END = STG_OFF + STG_BYTES;
  constexpr int EP_OFF = STG_END > RING_END ? STG_END : RING_END;
  constexpr int EP_BYTES = EPI == HN_EPI_ACC32 ? 0 : (2 * BN + BM) * 4;  // sw | bias | sa of the tile
  // (two operand buffers when the next tile's are parked before this tile's epilogue)
  constexpr int EP_BUFS = STAGED && !G128 && (EPI == HN_EPI_NONE || EPI == HN_EPI_GELU) ? 2 : 1;
  constexpr int SMEM = EP_OFF + EP_BUFS * EP_BYTES > RING_END ? EP_OFF + EP_BUFS * EP_BYTES : RING_END;
  __shared__ __align__(16) char smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;

  // ---- this workgroup's tiles
  const int G = gridDim.x, b = blockIdx.x;
  const int xcd = b % kXcds, slot = b / kXcds;
  const int nwx = G / kXcds + (xcd < G % kXcds ? 1 : 0);
  const int before = xcd * (G / kXcds) + min(xcd, G % kXcds);
  const int tiles = a.tiles_m * a.tiles_n;
  const int t_end = (int)((int64_t)tiles * (before + nwx) / G);
  int t = (int)((int64_t)tiles * before / G) + slot;
  if (t >= t_end) return;  // whole workgroup

  auto tile_origin = [&](int tt, int64_t& m0, int64_t& n0) {
    const int group_size = kGroupM * a.tiles_n;
    const int first_m = (tt / group_size) * kGroupM;
    const int size_m = min(a.tiles_m - first_m, kGroupM);
    m0 = (int64_t)(first_m + (tt % group_size) % size_m) * BM;
    n0 = (int64_t)((tt % group_size) / size_m) * BN;
  };

  // ---- direct-to-LDS load plan.  Wave w fills the 1 KB blocks q = w + NW * u of each tile; block q is
  // rows q * ROWS_PER_KB + lane / CHUNKS, and lane i lands at physical chunk i % CHUNKS, so it fetches the
  // logical chunk swz_chunk(row, i % CHUNKS) (the swizzle is an involution).  Rows past M or N re-read
  // the last row; their products are never stored.
  // g128: scale slot q < BN/64 holds sw[n0 + 64 q + lane, g], the next BM/64 slots sa[m0 + ..., g]; wave w
  // fills slots w + NW * u.  Slots past SC_SLOTS load a scale nobody reads, so every wave issues LOADS
  // loads per stage.
  // Addresses are a wave-uniform tile base plus a 32-bit per-lane offset (the SGPR-base form of the load).
  const uint8_t* wbase;
  const uint8_t* abase;
  uint32_t woff[A_KB], aoff[B_KB];
  const float* scbase[SC_PER_WAVE > 0 ? SC_PER_WAVE : 1];
  uint32_t scoff[SC_PER_WAVE > 0 ? SC_PER_WAVE : 1];
  // buffer descriptors of the tile's operand panels and scale rows (the direct loads add a per-lane byte
  // offset and the stage's byte offset)
  __amdgpu_buffer_rsrc_t wrsrc, arsrc, screc[SC_PER_WAVE > 0 ? SC_PER_WAVE : 1];
  auto plan_loads = [&](int64_t m0, int64_t n0, int lane) {
    wbase = a.qw + n0 * a.ldw;
    abase = a.qa + m0 * a.lda;
    // last valid row of each operand tile (tiles past the edge re-read it)
    const int64_t nrem1 = a.N - 1 - n0, mrem1 = a.M - 1 - m0;
    const int nlim = nrem1 < BN - 1 ? (int)nrem1 : BN - 1, mlim = mrem1 < BM - 1 ? (int)mrem1 : BM - 1;
    const uint32_t ldw = (uint32_t)a.ldw, lda = (uint32_t)a.lda;
#pragma unroll
    for (int u = 0; u < A_KB; u++) {
      const int row = (wave + NW * u) * ROWS_PER_KB + lane / CHUNKS;
      woff[u] = (uint32_t)min(row, nlim) * ldw + (swz_chunk<BK>(row, lane % CHUNKS) << 4);
    }
#pragma unroll
    for (int u = 0; u < B_KB; u++) {
      const int row = (wave + NW * u) * ROWS_PER_KB + lane / CHUNKS;
      aoff[u] = (uint32_t)min(row, mlim) * lda + (swz_chunk<BK>(row, lane % CHUNKS) << 4);
    }
#pragma unroll
    for (int u = 0; u < SC_PER_WAVE; u++) {
      const int q = wave + NW * u;
      if (q < BN / 64) {
        if constexpr (WBLK) {  // the scale row of the channel's 128-block (n0 is a multiple of 128)
          scbase[u] = a.sw + (n0 / 128) * a.ldsw;
          scoff[u] = (uint32_t)(min(q * 64 + lane, nlim) / 128) * (uint32_t)a.ldsw;
        } else {
          scbase[u] = a.sw + n0 * a.ldsw;
          scoff[u] = (uint32_t)min(q * 64 + lane, nlim) * (uint32_t)a.ldsw;
        }
      } else if (q < SC_SLOTS) {
        scbase[u] = a.sa + m0 * a.ldsa;
        scoff[u] = (uint32_t)min((q - BN / 64) * 64 + lane, mlim) * (uint32_t)a.ldsa;
      } else {
        // weight-scale row 0: it exists in both scale layouts (with block scales, sw has only
        // ceil(N / 128) rows, so row n0 may lie past the end)
        scbase[u] = a.sw;
        scoff[u] = 0;
      }
    }
    wrsrc = buffer_rsrc(wbase);
    arsrc = buffer_rsrc(abase);
#pragma unroll
    for (int u = 0; u < SC_PER_WAVE; u++) screc[u] = buffer_rsrc(scbase[u]);
  };
  const int nk = (int)(a.K / BK);
  // int8 per-token tiles (whole-K int32 sums: the order of the stages does not change them) walk K backwards
  // on every other tile of the workgroup.  The tiles an XCD runs next share the activation panels of the
  // ones it just finished, and then start on the stages those read last, which are still in L2.  (fp8 sums
  // are fp32 and keep one order.)
  constexpr bool SERP = !G128 && KIND == HN_KIND_INT8;
  bool krev = false;
  // byte offset of stage kt within the K extent
  auto kofs = [&](int kt) __attribute__((always_inline)) {
    return (uint32_t)(SERP && krev ? nk - 1 - kt : kt) * BK;
  };
  // load q (0 <= q < LOADS) of stage kt: weight rows, then activation rows, then scales
  auto issue_load = [&](int kt, int buf, int q) __attribute__((always_inline)) {
    char* base = smem + SCR + buf * STAGE;
    if (q < A_KB) {
      b2lds16(wrsrc, woff[q], kofs(kt), base + (wave + NW * q) * 1024);
    } else if (q < A_KB + B_KB) {
      const int u = q - A_KB;
      b2lds16(arsrc, aoff[u], kofs(kt), base + A_BYTES + (wave + NW * u) * 1024);
    } else {
      const int u = q - A_KB - B_KB;
      b2lds4(screc[u], scoff[u] * 4u, (uint32_t)(kt / STAGES_PER_GROUP) * 4u,
             smem + (kt % (NS + 1)) * SC_BYTES + (wave + NW * u) * 256);
    }
  };
  auto issue_stage = [&](int kt, int buf) {
#pragma unroll
    for (int q = 0; q < LOADS; q++) issue_load(kt, buf, q);
  };


  const int wrow_n = wn * TN * 32 + (lane & 31);  // this lane's A-fragment row within the weight tile
  const int wrow_m = wm * TM * 32 + (lane & 31);  // and B-fragment row within the activation tile

  // Fragments are read one MFMA slice ahead of the slice being multiplied (two register sets); the
  // stage barrier sits between the last slice's reads and its MFMAs.
  Frag fa[2][TN], fb[2][TM];
  auto read_frags = [&](int set, const char* stage_base, int slice) {
#pragma unroll
    for (int i = 0; i < TN; i++) fa[set][i] = MF::template load<BK>(stage_base, wrow_n + i * 32, slice, lane);
#pragma unroll
    for (int j = 0; j < TM; j++) fb[set][j] = MF::template load<BK>(stage_base + A_BYTES, wrow_m + j * 32, slice, lane);
  };

  // Block-major g128 loop (BMAJ: a separate fp32 running sum, one group per stage).  A wave multiplies its
  // TN x TM 32x32 blocks one after another (channel block i outer, token block j inner), each through all the
  // stage's slices, so a block's group partial is complete after SLICES products.  Its fold is issued
  // between the products of the next block, which accumulate into the second of two partial register sets:
  // the matrix core works on one block while the VALU folds the previous one.  The stage's last block is
  // folded during the next stage's first block (and after the tile's last stage).  The activation fragments
  // of every token block and slice are read once per stage and stay in registers; the weight fragments of
  // channel block i + 1 replace those of block i slice by slice during block i's last token block.
  constexpr bool BMAJ = G128 && !RESCALE && !WBLK && STAGES_PER_GROUP == 1;
  static_assert(!BMAJ || TM >= 2, "the weight fragments of the next channel block are read during the last token block");
  Frag fbs[BMAJ ? TM : 1][BMAJ ? SLICES : 1], fas[BMAJ ? SLICES : 1];

  // The tile's epilogue operands (per-channel weight scale and bias, per-token activation scale), parked in
  // LDS for the epilogue.  Rows and channels past the edge take the last valid one; an absent bias reads as
  // -0.0, which leaves every sum (signed zeros included) unchanged.  Most epilogues fetch them at the tile
  // top, where their latency overlaps the wait for stage 0.  The plain staged per-token epilogues
  // (EARLY_EP) fetch the next tile's before the last stage of this one and park them in the other of two
  // operand buffers before this tile's epilogue, so no load into registers is pending when that epilogue's
  // stores are issued: the next tile top then waits for its first stage alone and leaves the stores (the
  // youngest vector-memory ops; the counter retires in issue order) in flight under its first products.
  constexpr int EP_PER = EPI == HN_EPI_ACC32 ? 0 : (BN + NW * 64 - 1) / (NW * 64);
  constexpr int EPM_PER = EPI == HN_EPI_ACC32 || G128 ? 0 : (BM + NW * 64 - 1) / (NW * 64);
  constexpr bool EARLY_EP = STAGED && !G128 && (EPI == HN_EPI_NONE || EPI == HN_EPI_GELU);
  constexpr int NST = TM * 32 / (64 / (TN * 32 * 2 / 16));  // the staged epilogue's stores per full tile
  static_assert(NST < 64, "vmcnt range");
  float ep_sw[EP_PER > 0 ? EP_PER : 1], ep_b[EP_PER > 0 ? EP_PER : 1], ep_sa[EPM_PER > 0 ? EPM_PER : 1];
  uint32_t ep_bb[EP_PER > 0 ? EP_PER : 1];  // EARLY_EP: the bias bits (-0.0 when absent), converted when parked
  auto fetch_ep = [&](int64_t tm0, int64_t tn0) __attribute__((always_inline)) {
    const int64_t nleft0 = a.N - tn0, mleft0 = a.M - tm0;
    const int nlast = nleft0 < BN ? (int)nleft0 - 1 : BN - 1, mlast = mleft0 < BM ? (int)mleft0 - 1 : BM - 1;
#pragma unroll
    for (int u = 0; u < EP_PER; u++) {
      const int tt = tid + u * NW * 64;
      const int64_t n = tn0 + (tt < nlast ? tt : nlast);
      ep_sw[u] = G128 ? 0.0f : a.sw[n * a.ldsw];
      if constexpr (EARLY_EP) ep_bb[u] = a.bias ? load_bias_bits(a.bias, a.bias_dtype, n) : 0x80000000u;
      else ep_b[u] = a.bias ? load_bias(a.bias, a.bias_dtype, n) : -0.0f;
    }
#pragma unroll
    for (int u = 0; u < EPM_PER; u++) {
      const int tt = tid + u * NW * 64;
      ep_sa[u] = a.sa[(tm0 + (tt < mlast ? tt : mlast)) * a.ldsa];
    }
  };
  auto write_ep = [&](int buf) __attribute__((always_inline)) {
    if constexpr (EPI != HN_EPI_ACC32) {
      float* ep = reinterpret_cast<float*>(smem + EP_OFF + buf * EP_BYTES);
#pragma unroll
      for (int u = 0; u < EP_PER; u++) {
        const int tt = tid + u * NW * 64;
        const float b = EARLY_EP ? (a.bias ? bias_from_bits(ep_bb[u], a.bias_dtype) : -0.0f) : ep_b[u];
        if (tt < BN) { ep[tt] = ep_sw[u]; ep[BN + tt] = b; }
      }
#pragma unroll
      for (int u = 0; u < EPM_PER; u++) {
        const int tt = tid + u * NW * 64;
        if (tt < BM) ep[2 * BN + tt] = ep_sa[u];
      }
    }
  };
  bool stores_full = false;  // EARLY_EP: the previous tile's epilogue issued all NST of its stores
  int epb = 0;               // EARLY_EP: the operand buffer of the current tile

  int64_t m0, n0;
  tile_origin(t, m0, n0);
  plan_loads(m0, n0, lane);
  if constexpr (EARLY_EP) {  // the first tile's operands (published by the first tile-top barrier)
    fetch_ep(m0, n0);
    write_ep(0);
  }
  issue_stage(0, 0);

  for (;;) {
    // A per-tile copy of the lane id that the compiler cannot see through: the lane-dependent index
    // math of the epilogue and of the next tile's load plan is recomputed per tile instead of being
    // hoisted out of the tile loop and kept live (which would spill).
    int tl = lane;
    asm volatile("" : "+v"(tl));
    // ---- main loop of tile (m0, n0); its stage 0 is in flight into buffer 0
    Acc acc[TN][TM];                            // MFMA accumulators (whole K, or one group in g128 mode)
    v16f facc[G128 && !RESCALE ? TN : 1][G128 && !RESCALE ? TM : 1];  // g128: fp32 running sum over groups
    float ss_last[TM];                          // RESCALE: the latest group's scale product per token
#pragma unroll
    for (int j = 0; j < TM; j++) ss_last[j] = 1.0f;
#pragma unroll
    for (int i = 0; i < TN; i++)
#pragma unroll
      for (int j = 0; j < TM; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    if constexpr (G128 && !RESCALE) {
#pragma unroll
      for (int i = 0; i < TN; i++)
#pragma unroll
        for (int j = 0; j < TM; j++)
#pragma unroll
          for (int r = 0; r < 16; r++) facc[i][j][r] = 0.0f;
    }
    if constexpr (!EARLY_EP) fetch_ep(m0, n0);
    // stage 0 (and the epilogue operands) have landed and every wave's staging and operand reads of the
    // previous epilogue are done, so buffer 1 and the operand area are free.  After a full tile of a plain
    // staged epilogue its NST stores are the youngest vector-memory ops and may still be in flight (the
    // counter retires in issue order); otherwise this also retires the previous tile's stores.
    if (EARLY_EP && stores_full) wait_vmcnt<NST>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    barrier();
    if constexpr (!EARLY_EP) write_ep(0);
    if (1 < nk) issue_stage(1, 1);
    if constexpr (BMAJ) {
#pragma unroll
      for (int j = 0; j < TM; j++)
#pragma unroll
        for (int s = 0; s < SLICES; s++) fbs[j][s] = MF::template load<BK>(smem + SCR + A_BYTES, wrow_m + j * 32, s, lane);
#pragma unroll
      for (int s = 0; s < SLICES; s++) fas[s] = MF::template load<BK>(smem + SCR, wrow_n, s, lane);
    } else {
      read_frags(0, smem + SCR, 0);
    }

    // products of weight fragments [i0, i1) with every activation fragment of register set `set`
    // rs (RESCALE, a stage's first slice): each accumulator block is moved to this group's scale product
    // just before its first product of the stage, 16 multiplies per block interleaved with the matrix core
    // fresh: the group's first products, which start the partial from zero (the inline constant 0 as the
    // accumulator operand) instead of adding to a zeroed set
    auto mfma_rows = [&](int set, int i0, int i1, const float* rs = nullptr, bool fresh = false)
        __attribute__((always_inline)) {
#pragma unroll
      for (int i = i0; i < i1; i++)
#pragma unroll
        for (int j = 0; j < TM; j++) {
          if (rs) {
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] *= rs[j];
          }
          if (fresh) acc[i][j] = MF::run(fa[set][i], fb[set][j], Acc{});
          else acc[i][j] = MF::run(fa[set][i], fb[set][j], acc[i][j]);
        }
      if (rs) {
#pragma unroll
        for (int i = i0; i < i1; i++)
#pragma unroll
          for (int j = 0; j < TM; j++) {
            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          }
      }
    };
    // One K stage (kt, in buffer `buf`).  The schedule is pinned with scheduling barriers (address
    // arithmetic may still move): each slice issues the next slice's fragment reads right after its
    // first products, so they land while the matrix core works.  The last slice holds the stage
    // barrier; after it the next stage's first fragments are read and the direct loads of stage kt + 2
    // are interleaved with the slice's remaining products, so the matrix core is fed while the loads
    // queue.  MODE 0: barrier and loads; 1: barrier, no loads (stage kt + 2 does not exist); 2: the
    // tile's last stage (neither).
    // Weight rows multiplied before the barrier.  Per-token tiles issue all of the last slice's products
    // after it (1.7 % faster over the DiT stack); the g128 and block-scale tiles keep one row before it
    // (none there is 0.5 % and 3 % slower, two 0.4 % and 2.5 % slower).
    constexpr int PRE = G128 ? 1 : 0;
    // the g128 fold (not the rescaled running sum) with one group per stage: every stage starts its partials
    // in its first products, so the fold leaves them as they are
    constexpr bool FRESH = G128 && !RESCALE && STAGES_PER_GROUP == 1;
    constexpr int POST_MFMA = (TN - PRE) * TM;
    constexpr int VM_LOADS = A_KB + B_KB + SC_PER_WAVE;
    constexpr int VM_PER = (VM_LOADS + POST_MFMA - 1) / POST_MFMA;  // POST_MFMA >= TM > 0
    auto stage_body = [&](int kt, int buf, auto mode_c) __attribute__((always_inline)) {
      constexpr int MODE = decltype(mode_c)::value;
      const char* stage = smem + SCR + buf * STAGE;
      // RESCALE: the factor from the previous group's scale product (carried from the previous stage) to this
      // one's (1 at the tile's first stage).
      float rs[TM];
      if constexpr (RESCALE) {
        static_assert(STAGES_PER_GROUP == 1, "one group per stage");
        const float* sc = reinterpret_cast<const float*>(smem + (kt % (NS + 1)) * SC_BYTES);
        const float swc = sc[wn * TN * 32];  // the wave's one weight scale
#pragma unroll
        for (int j = 0; j < TM; j++) {
          // this group's scale product; the previous group's is carried in ss_last.  The ratio comes from the
          // hardware reciprocal with one Newton step (within an ulp or two of the quotient; the running sum
          // rounds once per group anyway)
          const float den = sc[BN + wrow_m + j * 32] * swc;
          const float r0 = __builtin_amdgcn_rcpf(den);
          const float r = __builtin_fmaf(__builtin_fmaf(-den, r0, 1.0f), r0, r0);
          rs[j] = kt > 0 ? ss_last[j] * r : 1.0f;
          ss_last[j] = den;
        }
      }
#pragma unroll
      for (int s = 0; s < SLICES; s++) {
        const int cur = s & 1;
        const float* rsc = RESCALE && s == 0 ? rs : nullptr;
        // g128 fold with one group per stage: the stage's first slice starts every partial afresh
        const bool fresh = FRESH && s == 0;
        if (s + 1 < SLICES) {
          mfma_rows(cur, 0, 1, rsc, fresh);
          __builtin_amdgcn_sched_barrier(0x6);
          read_frags(cur ^ 1, stage, s + 1);
          __builtin_amdgcn_sched_barrier(0x6);
          mfma_rows(cur, 1, TN, rsc, fresh);
          __builtin_amdgcn_sched_barrier(0x6);
        } else if constexpr (MODE == 2) {
          mfma_rows(cur, 0, TN, nullptr, fresh);
        } else {
          mfma_rows(cur, 0, PRE, nullptr, fresh);
          // (the waits and the barrier are scalar instructions: nothing may cross them)
          __builtin_amdgcn_sched_barrier(0);
          // stage kt + 1 (the only loads in flight) has landed for this wave and its reads of stage kt
          // are complete; the barrier publishes both facts, then stage kt + 2 may refill `buf`
          wait_vmcnt<0>();
          __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
          barrier();
          __builtin_amdgcn_sched_barrier(0);
          read_frags(cur ^ 1, smem + SCR + (buf ^ 1) * STAGE, 0);
          if constexpr (MODE == 0) issue_stage(kt + 2, buf);
          mfma_rows(cur, PRE, TN, nullptr, fresh);
          // reads first, then products and loads alternating
          __builtin_amdgcn_sched_group_barrier(0x100, TN + TM, 0);
#pragma unroll
          for (int r = 0; r < POST_MFMA; r++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if constexpr (MODE == 0) __builtin_amdgcn_sched_group_barrier(0x020, VM_PER, 0);
          }
          __builtin_amdgcn_sched_barrier(0x6);
        }
      }
      if constexpr (RESCALE) {
        // (ss_last holds this group's scale product: after the last stage, the epilogue's factor)
      } else if constexpr (G128) {
        if ((kt + 1) % STAGES_PER_GROUP == 0) {
          const float* sc = reinterpret_cast<const float*>(smem + (kt % (NS + 1)) * SC_BYTES);
          const float swb = WBLK ? sc[wn * TN * 32] : 0.0f;  // the wave's one weight scale (block layout)
          // Per-channel scales: lane l needs the scale of channel 32 i + 8 rr + 4 (l >> 5) + q for each
          // (i, rr, q), the same for the 32 lanes of a half-wave.  Lane (row R = l >> 4, s = l & 15) loads
          // the one of channel 32 i + 8 (s >> 2) + 4 (R >> 1) + (s & 3), and the fma reads it with a DPP
          // row broadcast of lane s = 4 rr + q (one LDS read per lane per i instead of 16 bytes per output
          // quad).
          float swc[WBLK ? 1 : TN];
          if constexpr (!WBLK) {
#pragma unroll
            for (int i = 0; i < TN; i++)
              swc[i] = sc[wn * TN * 32 + i * 32 + ((lane & 15) >> 2) * 8 + (lane >> 5) * 4 + (lane & 3)];
          }
#pragma unroll
          for (int j = 0; j < TM; j++) {
            const float sam = sc[BN + wrow_m + j * 32];
            const float ss = sam * swb;
#pragma unroll
            for (int i = 0; i < TN; i++) {
              if constexpr (WBLK) {
#pragma unroll
                for (int r = 0; r < 16; r++)
                  facc[i][j][r] = __builtin_fmaf(MF::to_f32(acc[i][j][r]), ss, facc[i][j][r]);
              } else {
                fold_row_bcast(facc[i][j], acc[i][j], sam, swc[i], std::make_integer_sequence<int, 16>());
              }
            }
          }
          if constexpr (!FRESH) {
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
              for (int j = 0; j < TM; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
          }
        }
      }
    };
    // BMAJ state: the group partials of two consecutive blocks, and the fold scales of the current group:
    // per token block the lane's token scale (times the wave's weight scale with block weight scales) and,
    // per channel block, the lane's DPP source of the per-channel scales.  The tile's first stage folds the
    // zero partial of "the previous group's last block" with zero scales, which leaves the running sum +0.
    Acc part[BMAJ ? 2 : 1];
    float c_sa[TM], c_sw[TN];
#pragma unroll
    for (int j = 0; j < TM; j++) c_sa[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < TN; i++) c_sw[i] = 0.0f;
    auto read_scales = [&](int kt) __attribute__((always_inline)) {
      const float* sc = reinterpret_cast<const float*>(smem + (kt % (NS + 1)) * SC_BYTES);
#pragma unroll
      for (int j = 0; j < TM; j++) {
        const float sam = sc[BN + wrow_m + j * 32];
        c_sa[j] = WBLK ? sam * sc[wn * TN * 32] : sam;
      }
      if constexpr (!WBLK) {
        // lane (row R = l >> 4, s = l & 15) holds the scale of channel 32 i + 8 (s >> 2) + 4 (R >> 1) + (s & 3),
        // which register s of every lane in its row needs (read with a DPP row broadcast)
#pragma unroll
        for (int i = 0; i < TN; i++)
          c_sw[i] = sc[wn * TN * 32 + i * 32 + ((lane & 15) >> 2) * 8 + (lane >> 5) * 4 + (lane & 3)];
      }
    };
    if constexpr (BMAJ) {
#pragma unroll
      for (int r = 0; r < 16; r++) part[1][r] = 0;
    }
    // outputs [R0, R0 + RN) of one block's fold: facc = fma(float(p) * sa, sw, facc), or with block weight
    // scales facc = fma(float(p), sa * sw_block, facc)
    auto fold_chunk = [&](v16f& f, const Acc& p, float fsa, float fsw, auto r0_c, auto rn_c) __attribute__((always_inline)) {
      constexpr int R0 = decltype(r0_c)::value, RN = decltype(rn_c)::value;
      if constexpr (WBLK) {
#pragma unroll
        for (int r = R0; r < R0 + RN; r++) f[r] = __builtin_fmaf(MF::to_f32(p[r]), fsa, f[r]);
      } else {
        fold_rows_bcast<R0>(f, p, fsa, fsw, std::make_integer_sequence<int, RN>());
      }
    };
    constexpr int NB = TN * TM;            // blocks per wave, channel block outer
    constexpr int FOLD_PER = 16 / SLICES;  // outputs folded after each product
    constexpr int LAST = (TN - 1) * TM;    // first block of the last channel block
    // One stage.  The compiler waits for all outstanding LDS reads (lgkmcnt 0) before a product whose
    // fragments are pending, so reads are issued as early as their registers allow, and each slice issues
    // its reads before its share of the fold: the group's scales after the first product, the next channel
    // block's weight fragments (slice by slice, as the last token block releases them).  The last channel
    // block follows the stage barrier, reads the next stage's activation fragments as its products release
    // them, and spreads the direct loads of stage kt + 2 over its products.
    auto bm_stage = [&](int kt, int buf, auto mode_c) __attribute__((always_inline)) {
      constexpr int MODE = decltype(mode_c)::value;
      const char* stage = smem + SCR + buf * STAGE;
      const char* next = smem + SCR + (buf ^ 1) * STAGE;
      // the previous group's last block is folded during this stage's first block, with that group's scales
      const float p_sa = c_sa[TM - 1], p_sw = c_sw[TN - 1];
      static_assert(NB % 2 == 0, "blocks alternate between the two partial sets, block 0 in set 0");
      static_for<NB>([&](auto b_c) __attribute__((always_inline)) {
        constexpr int b = decltype(b_c)::value, i = b / TM, j = b % TM, cur = b & 1;
        constexpr int pb = (b + NB - 1) % NB, pi = pb / TM, pj = pb % TM;  // the block folded meanwhile
        if constexpr (b == LAST && MODE != 2) {
          // every wave's reads of this stage are done and stage kt + 1 has landed: the barrier publishes
          // both, then the next stage's fragments are read and stage kt + 2 refills `buf`
          __builtin_amdgcn_sched_barrier(0);
          wait_vmcnt<0>();
          __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
          barrier();
          __builtin_amdgcn_sched_barrier(0);
        }
        static_for<SLICES>([&](auto s_c) __attribute__((always_inline)) {
          constexpr int s = decltype(s_c)::value;
          if constexpr (s == 0) part[cur] = MF::run(fas[s], fbs[j][s], Acc{});
          else part[cur] = MF::run(fas[s], fbs[j][s], part[cur]);
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (b == 0 && s == 0) read_scales(kt);
          if constexpr (j == TM - 1) {  // slice s of the weight fragments is free
            if constexpr (i + 1 < TN) fas[s] = MF::template load<BK>(stage, wrow_n + (i + 1) * 32, s, lane);
            else if constexpr (MODE != 2) fas[s] = MF::template load<BK>(next, wrow_n, s, lane);
          }
          if constexpr (i == TN - 1 && MODE != 2) {
            fbs[j][s] = MF::template load<BK>(next + A_BYTES, wrow_m + j * 32, s, lane);
            if constexpr (MODE == 0) {
              constexpr int slot = j * SLICES + s, SLOTS = TM * SLICES;
#pragma unroll
              for (int q = slot * LOADS / SLOTS; q < (slot + 1) * LOADS / SLOTS; q++) issue_load(kt + 2, buf, q);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
          const float fsa = b == 0 ? p_sa : c_sa[pj];
          const float fsw = b == 0 ? p_sw : c_sw[pi];
          fold_chunk(facc[pi][pj], part[cur ^ 1], fsa, fsw, std::integral_constant<int, s * FOLD_PER>(),
                     std::integral_constant<int, FOLD_PER>());
          __builtin_amdgcn_sched_barrier(0);
        });
      });
    };
    int kt = 0;
    if constexpr (BMAJ) {
      for (; kt + 2 < nk; kt++) bm_stage(kt, kt & 1, std::integral_constant<int, 0>());
      if (kt + 1 < nk) {
        bm_stage(kt, kt & 1, std::integral_constant<int, 1>());
        kt++;
      }
      bm_stage(kt, kt & 1, std::integral_constant<int, 2>());
    } else {
      for (; kt + 2 < nk; kt++) stage_body(kt, kt & 1, std::integral_constant<int, 0>());
      if (kt + 1 < nk) {
        stage_body(kt, kt & 1, std::integral_constant<int, 1>());
        kt++;
      }
      if constexpr (EARLY_EP) {  // the next tile's epilogue operands land during the last stage
        if (t + nwx < t_end) {
          int64_t nm0, nn0;
          tile_origin(t + nwx, nm0, nn0);
          fetch_ep(nm0, nn0);
        }
      }
      stage_body(kt, kt & 1, std::integral_constant<int, 2>());
    }
    // every wave is done reading the stage buffers (and the scale ring) of this tile
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    barrier();

    // ---- next tile's first stage, then this tile's epilogue
    const int64_t em0 = m0, en0 = n0;
    t += nwx;
    const bool more = t < t_end;
    if (more) {
      tile_origin(t, m0, n0);
      plan_loads(m0, n0, tl);
      krev = !krev;
      issue_stage(0, 0);
      if constexpr (EARLY_EP) write_ep(epb ^ 1);  // its last reader was the previous epilogue
    }
    if constexpr (BMAJ) {  // the last group's last block, while the next tile's first stage lands
      fold_chunk(facc[TN - 1][TM - 1], part[(TN * TM - 1) & 1], c_sa[TM - 1], c_sw[TN - 1],
                 std::integral_constant<int, 0>(), std::integral_constant<int, 16>());
    }

    // Tile-local coordinates (32-bit): lane holds token ml = wrow_m + 32 j and channels
    // nl = wn*TN*32 + 32 i + 8 rr + 4 (lane >> 5) + q (q = 0..3) in register rr * 4 + q of tile (i, j);
    // rows ml < mrem and channels nl < nrem exist.
    const int64_t mleft = a.M - em0, nleft = a.N - en0;
    const int mrem = mleft < BM ? (int)mleft : BM, nrem = nleft < BN ? (int)nleft : BN;
    stores_full = mrem == BM && nrem == BN;
    const int nloc = wn * TN * 32 + (tl >> 5) * 4;
    const int erow_m = wm * TM * 32 + (tl & 31);
    if constexpr (EPI == HN_EPI_ACC32) {
      int32_t* obase = reinterpret_cast<int32_t*>(a.out) + em0 * a.ldo + en0;
#pragma unroll
      for (int j = 0; j < TM; j++) {
        const int ml = erow_m + j * 32;
        if (ml < mrem) {
#pragma unroll
          for (int i = 0; i < TN; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
              const int nl = nloc + i * 32 + (r >> 2) * 8 + (r & 3);
              if (nl < nrem) obase[(uint32_t)(ml * (int)a.ldo + nl)] = (int32_t)acc[i][j][r];
            }
        }
      }
    } else if constexpr (EPI == HN_EPI_SWIGLU_QUANT) {
      // per-channel bias and per-token scale of this tile (written at the tile top)
      const float* ep = reinterpret_cast<const float*>(smem + EP_OFF + (EARLY_EP ? epb * EP_BYTES : 0));
      constexpr int JH = TM / 2;
      // every output of the wave to its bf16 value: gate_proj(x) on wave wn = 0, up_proj(x) on wn = 1
#pragma unroll
      for (int j = 0; j < TM; j++) {
        const float sam = G128 ? 0.0f : ep[2 * BN + erow_m + j * 32];
#pragma unroll
        for (int i = 0; i < TN; i++) {
#pragma unroll
          for (int rr = 0; rr < 4; rr++) {
            const float4 sw4 = *reinterpret_cast<const float4*>(ep + nloc + i * 32 + rr * 8);
            const float4 b4 = *reinterpret_cast<const float4*>(ep + BN + nloc + i * 32 + rr * 8);
            const float swq[4] = {sw4.x, sw4.y, sw4.z, sw4.w};
            const float bq[4] = {b4.x, b4.y, b4.z, b4.w};
            // bf16 rounding two at a time with the hardware pack: rbf16 for every non-NaN value, and a NaN
            // stays a NaN of its sign (as under rbf16, bar the top payloads, which it carries into a zero);
            // the codes below read at most that sign (the peak skips NaN)
#pragma unroll
            for (int q = 0; q < 4; q += 2) {
              float v[2];
#pragma unroll
              for (int t = 0; t < 2; t++) {
                const int r = rr * 4 + q + t;
                if constexpr (RESCALE) v[t] = MF::get(acc[i][j], r) * ss_last[j];
                else if constexpr (G128) v[t] = facc[i][j][r];
                else v[t] = __builtin_fmaf(MF::to_f32(acc[i][j][r]) * sam, swq[q + t], 0.0f);
                v[t] = v[t] + bq[q + t];
              }
              const uint32_t pb = bf16x2_finite(v[0], v[1]);
              MF::put(acc[i][j], rr * 4 + q, __uint_as_float(pb << 16));
              MF::put(acc[i][j], rr * 4 + q + 1, __uint_as_float(pb & 0xffff0000u));
            }
          }
        }
      }
      // The partner wave (wave ^ 1) holds the other operand of every product in the same lane and
      // register.  Each wave writes the token half it does not finish (wn = 0 finishes j < JH, wn = 1 the
      // rest) as packed bf16 pairs: 16 bytes per lane per 8 registers, lane-contiguous, conflict-free.
      auto send = [&](auto jc) __attribute__((always_inline)) {
        constexpr int J0 = decltype(jc)::value;
        char* slot = smem + STG_OFF + wave * XCH_WAVE + tl * 16;
#pragma unroll
        for (int jj = 0; jj < JH; jj++)
#pragma unroll
          for (int i = 0; i < TN; i++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
              uint32_t w[4];
#pragma unroll
              for (int e = 0; e < 4; e++)
                w[e] = __builtin_amdgcn_perm(__float_as_uint(MF::get(acc[i][J0 + jj], h * 8 + 2 * e + 1)),
                                             __float_as_uint(MF::get(acc[i][J0 + jj], h * 8 + 2 * e)), 0x07060302u);
              *reinterpret_cast<v4i*>(slot + ((jj * TN + i) * 2 + h) * 1024) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            }
      };
      if (wn == 0) send(std::integral_constant<int, JH>());
      else send(std::integral_constant<int, 0>());
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      barrier();
      // h = bf16(bf16(silu(g)) * u), then the codes of each token's 128-channel group (lanes l and l^32).
      // Pairs of values share one hardware bf16 pack; the fp8 per-channel variant keeps one value at a
      // time, since its paired form does not fit the register file.
      constexpr bool PAIRED = !(KIND == HN_KIND_FP8 && !RESCALE);
      auto finish = [&](auto jc, auto gate_c) __attribute__((always_inline)) {
        constexpr int J0 = decltype(jc)::value;
        constexpr bool OWN_GATE = decltype(gate_c)::value;
        const char* pslot = smem + STG_OFF + (wave ^ 1) * XCH_WAVE + tl * 16;
#pragma unroll
        for (int jj = 0; jj < JH; jj++) {
          const int j = J0 + jj;
          float peak = 0.0f;
#pragma unroll
          for (int i = 0; i < TN; i++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
              const v4i p = *reinterpret_cast<const v4i*>(pslot + ((jj * TN + i) * 2 + h) * 1024);
              if constexpr (!PAIRED) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                  const int r = h * 8 + e;
                  const uint32_t pw = (uint32_t)p[e >> 1];
                  const float other = __uint_as_float((e & 1) ? (pw & 0xffff0000u) : (pw << 16));
                  const float own = MF::get(acc[i][J0 + jj], r);
                  const float g = OWN_GATE ? own : other, u = OWN_GATE ? other : own;
                  const float hv = rbf16(silu_bf16(g) * u);
                  MF::put(acc[i][J0 + jj], r, hv);
                  peak = __builtin_fmaxf(peak, __builtin_fabsf(hv));
                }
                continue;
              }
#pragma unroll
              for (int e = 0; e < 8; e += 2) {
                const int r = h * 8 + e;
                const uint32_t pw = (uint32_t)p[e >> 1];
                const float other0 = __uint_as_float(pw << 16), other1 = __uint_as_float(pw & 0xffff0000u);
                const float own0 = MF::get(acc[i][J0 + jj], r), own1 = MF::get(acc[i][J0 + jj], r + 1);
                const float g0 = OWN_GATE ? own0 : other0, u0 = OWN_GATE ? other0 : own0;
                const float g1 = OWN_GATE ? own1 : other1, u1 = OWN_GATE ? other1 : own1;
                float s0, s1;
                silu_bf16x2(g0, g1, s0, s1);
                // bf16(silu * up) two at a time with the hardware pack (as above)
                const uint32_t ph = bf16x2_finite(s0 * u0, s1 * u1);
                const float hv0 = __uint_as_float(ph << 16), hv1 = __uint_as_float(ph & 0xffff0000u);
                MF::put(acc[i][J0 + jj], r, hv0);
                MF::put(acc[i][J0 + jj], r + 1, hv1);
                peak = __builtin_fmaxf(peak, __builtin_fmaxf(__builtin_fabsf(hv0), __builtin_fabsf(hv1)));
              }
            }
          peak = __builtin_fmaxf(peak, shfl_xor_f(peak, 32));
          const float gs = KIND == HN_KIND_FP8 ? fp8_scale(peak) : int8_scale(peak);
          const bool fast = FastQuot<KIND>::ok(peak);  // h holds bf16 values: the exact fast quotient applies
          const typename FastQuot<KIND>::Div div(gs);
          const int ml = erow_m + j * 32;
          if (ml < mrem) {
            uint8_t* o = reinterpret_cast<uint8_t*>(a.out) + em0 * a.ldo + en0 / 2;
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
              for (int rr = 0; rr < 4; rr++) {
                const int nl = (tl >> 5) * 4 + i * 32 + rr * 8;
                float y[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                  const float v = MF::get(acc[i][J0 + jj], rr * 4 + q);
                  y[q] = __builtin_expect(fast, 1) ? div(v) : v / gs;
                }
                uint32_t w;
                if constexpr (KIND == HN_KIND_FP8) {
                  // fast groups: finite quotients, the hardware conversion; others the software encoder
                  w = __builtin_expect(fast, 1) ? e4m3_pack4_hw(y[0], y[1], y[2], y[3])
                                                : pack4_i8(e4m3_encode(y[0]), e4m3_encode(y[1]), e4m3_encode(y[2]),
                                                           e4m3_encode(y[3]));
                } else {
                  w = pack4_i8(round_half_away_i8(y[0]), round_half_away_i8(y[1]), round_half_away_i8(y[2]),
                               round_half_away_i8(y[3]));
                }
                *reinterpret_cast<uint32_t*>(o + (uint32_t)(ml * (int)a.ldo + nl)) = w;
              }
            if (tl < 32) a.qs[(em0 + ml) * a.ldqs + en0 / 256] = gs;
          }
        }
      };
      if (wn == 0) finish(std::integral_constant<int, 0>(), std::true_type());
      else finish(std::integral_constant<int, JH>(), std::false_type());
    } else {
      // per-channel scale and bias, and per-token scale, of this tile (written at the tile top)
      const float* ep = reinterpret_cast<const float*>(smem + EP_OFF + (EARLY_EP ? epb * EP_BYTES : 0));
#pragma unroll
      for (int j = 0; j < TM; j++) {
        const int ml = erow_m + j * 32;
        const bool m_ok = ml < mrem;
        const float sam = G128 ? 0.0f : ep[2 * BN + ml];
        // dequantize + bias (+ GELU) in place; the results overwrite the accumulator registers as fp32 bits
#pragma unroll
        for (int i = 0; i < TN; i++) {
#pragma unroll
          for (int rr = 0; rr < 4; rr++) {
            const float4 sw4 = *reinterpret_cast<const float4*>(ep + nloc + i * 32 + rr * 8);
            const float4 b4 = *reinterpret_cast<const float4*>(ep + BN + nloc + i * 32 + rr * 8);
            const float swq[4] = {sw4.x, sw4.y, sw4.z, sw4.w};
            const float bq[4] = {b4.x, b4.y, b4.z, b4.w};
            constexpr bool GELU = EPI == HN_EPI_GELU || EPI == HN_EPI_GELU_QUANT;
            // GELU: both bf16 roundings two values at a time with the hardware pack (rbf16 for every
            // non-NaN value; a NaN stays a NaN of its sign)
#pragma unroll
            for (int q = 0; q < 4; q += GELU ? 2 : 1) {
              float v[2];
#pragma unroll
              for (int t = 0; t < (GELU ? 2 : 1); t++) {
                const int r = rr * 4 + q + t;
                if constexpr (RESCALE) v[t] = MF::get(acc[i][j], r) * ss_last[j];
                else if constexpr (G128) v[t] = facc[i][j][r];
                else v[t] = __builtin_fmaf(MF::to_f32(acc[i][j][r]) * sam, swq[q + t], 0.0f);
                v[t] = v[t] + bq[q + t];
              }
              if constexpr (GELU) {
                const uint32_t px = bf16x2_finite(v[0], v[1]);
                const uint32_t pg = bf16x2_finite(gelu_tanh(__uint_as_float(px << 16)),
                                                  gelu_tanh(__uint_as_float(px & 0xffff0000u)));
                MF::put(acc[i][j], rr * 4 + q, __uint_as_float(pg << 16));
                MF::put(acc[i][j], rr * 4 + q + 1, __uint_as_float(pg & 0xffff0000u));
              } else {
                MF::put(acc[i][j], rr * 4 + q, v[0]);
              }
            }
          }
        }
        if constexpr (EPI == kEpiQkvHeads) {
          // q and k heads (hy_nomas/fused.py:65-91 on the bf16 projection output): r = 1/sqrt(mean(x^2) + eps)
          // over the head's 128 channels (lanes l and l^32 hold them), n = bf16(bf16(x r) w), then the
          // interleaved rotation of the pairs (2i, 2i + 1), which lie in one lane
          const int64_t c0 = en0 + wn * 128;
          const int part = (int)(c0 / a.hm_hidden);
          if (part < 2) {
            const float* wt = part == 0 ? a.hm_wq : a.hm_wk;
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
              for (int r = 0; r < 16; r++) {
                const float xv = rbf16(MF::get(acc[i][j], r));
                MF::put(acc[i][j], r, xv);
                ss = __builtin_fmaf(xv, xv, ss);
              }
            ss += shfl_xor_f(ss, 32);
            const float rs = 1.0f / __builtin_sqrtf(ss / 128.0f + a.hm_eps);
            const uint32_t mg = (uint32_t)(em0 + (ml < mrem ? ml : mrem - 1));
            const uint32_t tok = mg % (uint32_t)a.hm_L;
            const bool rope = a.hm_cos != nullptr;
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
              for (int rr = 0; rr < 4; rr++) {
                const int d = i * 32 + rr * 8 + (tl >> 5) * 4;
                const float4 w4 = *reinterpret_cast<const float4*>(wt + d);
                float nq[4];
                nq[0] = rbf16(rbf16(MF::get(acc[i][j], rr * 4 + 0) * rs) * w4.x);
                nq[1] = rbf16(rbf16(MF::get(acc[i][j], rr * 4 + 1) * rs) * w4.y);
                nq[2] = rbf16(rbf16(MF::get(acc[i][j], rr * 4 + 2) * rs) * w4.z);
                nq[3] = rbf16(rbf16(MF::get(acc[i][j], rr * 4 + 3) * rs) * w4.w);
                if (rope) {
                  const float4 c4 = *reinterpret_cast<const float4*>(a.hm_cos + (int64_t)tok * 128 + d);
                  const float4 s4 = *reinterpret_cast<const float4*>(a.hm_sin + (int64_t)tok * 128 + d);
                  const float o0 = nq[0] * c4.x - nq[1] * s4.x, o1 = nq[1] * c4.y + nq[0] * s4.y;
                  const float o2 = nq[2] * c4.z - nq[3] * s4.z, o3 = nq[3] * c4.w + nq[2] * s4.w;
                  nq[0] = o0; nq[1] = o1; nq[2] = o2; nq[3] = o3;
                }
#pragma unroll
                for (int q = 0; q < 4; q++) MF::put(acc[i][j], rr * 4 + q, nq[q]);
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
          // the GELU outputs are bf16 values: the exact two-op int8 quotient applies to the group (hn_common.h)
          const bool fast = fast_group_i8(peak);
          const FastDivI8 div(gs);
          if (m_ok) {
            int8_t* o = reinterpret_cast<int8_t*>(a.out) + em0 * a.ldo + en0;
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
              for (int rr = 0; rr < 4; rr++) {
                const int nl = nloc + i * 32 + rr * 8;
                const float v0 = MF::get(acc[i][j], rr * 4 + 0), v1 = MF::get(acc[i][j], rr * 4 + 1);
                const float v2 = MF::get(acc[i][j], rr * 4 + 2), v3 = MF::get(acc[i][j], rr * 4 + 3);
                uint32_t w;
                if (__builtin_expect(fast, 1))
                  w = pack4_i8(round_half_away_i8_inrange(div(v0)), round_half_away_i8_inrange(div(v1)),
                               round_half_away_i8_inrange(div(v2)), round_half_away_i8_inrange(div(v3)));
                else
                  w = pack4_i8(round_half_away_i8(v0 / gs), round_half_away_i8(v1 / gs), round_half_away_i8(v2 / gs),
                               round_half_away_i8(v3 / gs));
                if (nl < nrem) *reinterpret_cast<uint32_t*>(o + (uint32_t)(ml * (int)a.ldo + nl)) = w;
              }
            // N % 128 == 0, so the group is either wholly inside N or wholly past it
            if (tl < 32 && wn * 128 < nrem) a.qs[(em0 + ml) * a.ldqs + (en0 + wn * 128) / 128] = gs;
          }
        } else if (STAGED && (EPI == kEpiQkvHeads || a.stage_store)) {
          char* wst = smem + STG_OFF + wave * 32 * OPITCH;
          bool to_vt = false;
          if constexpr (EPI == kEpiQkvHeads) to_vt = a.hm_vt != nullptr && en0 + wn * 128 >= 2 * a.hm_hidden;
          if (to_vt) {
            // A v head to V^T: the wave's 128 dims x 32 tokens staged dim-major (row d of 64 bytes holds the
            // 32 tokens in the 16-key-group order: bits 2 and 3 of the token index swapped), then each row's 64
            // bytes written to its V^T row.  Lanes t and t ^ 1 (tokens 2p, 2p + 1) swap two of their four dims
            // with a DPP move, so each writes one dim of both tokens as a packed pair: the even lane dims
            // d0, d0 + 1, the odd lane d0 + 2, d0 + 3.
            const int tk = tl & 31;
            const bool odd = (tk & 1) != 0;
            const int te = tk & ~1;
            const int pcol = ((te & ~12) | ((te & 4) << 1) | ((te & 8) >> 1)) * 2;
#pragma unroll
            for (int i = 0; i < TN; i++)
#pragma unroll
              for (int rr = 0; rr < 4; rr++) {
                const int d0 = i * 32 + rr * 8 + (tl >> 5) * 4;
                const float v0 = MF::get(acc[i][j], rr * 4 + 0), v1 = MF::get(acc[i][j], rr * 4 + 1);
                const float v2 = MF::get(acc[i][j], rr * 4 + 2), v3 = MF::get(acc[i][j], rr * 4 + 3);
                const float r0 = dpp_f<0xB1>(odd ? v0 : v2), r1 = dpp_f<0xB1>(odd ? v1 : v3);  // lane t ^ 1
                const int da = d0 + (odd ? 2 : 0);
                *reinterpret_cast<uint32_t*>(wst + da * 64 + pcol) =
                    cvt2_out<HN_DTYPE_BF16>(odd ? r0 : v0, odd ? v2 : r0);
                *reinterpret_cast<uint32_t*>(wst + (da + 1) * 64 + pcol) =
                    cvt2_out<HN_DTYPE_BF16>(odd ? r1 : v1, odd ? v3 : r1);
              }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes have landed
            __builtin_amdgcn_wave_barrier();
            const int mb = wm * TM * 32 + j * 32;  // the block's first token (the block lies in one batch)
            // the block's tokens and the wave's head exist (N % 128 == 0: a head is wholly inside N or past it)
            if (mb < mrem && wn * TN * 32 < nrem) {
              const uint32_t mg = (uint32_t)(em0 + mb);
              const uint32_t bb = mg / (uint32_t)a.hm_L, ll = mg - bb * (uint32_t)a.hm_L;
              const int64_t h = (en0 + wn * 128 - 2 * a.hm_hidden) / 128;
              uint16_t* vb = a.hm_vt + bb * a.hm_svb + h * a.hm_svh + a.hm_loff + ll;
#pragma unroll
              for (int n = 0; n < 8; n++) {
                const int row = n * 16 + (tl >> 2), ch = tl & 3;
                const v4i v = *reinterpret_cast<const v4i*>(wst + row * 64 + ch * 16);
                __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(vb + row * a.hm_svd + ch * 8));
              }
            }
          } else {
          // token row (tl & 31) of this wave's staging block, then a 16-byte-per-lane write-back of the
          // block's 32 rows x TN*32 channels, non-temporal so the output stream does not evict the operand
          // panels other tiles are still reading from L2
          char* ob = wst + (tl & 31) * OPITCH;
#pragma unroll
          for (int i = 0; i < TN; i++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
              const int ocol = i * 32 + rr * 8 + (tl >> 5) * 4;
              *reinterpret_cast<uint2*>(ob + ocol * 2) =
                  make_uint2(cvt2_out<OUT_DT>(MF::get(acc[i][j], rr * 4 + 0), MF::get(acc[i][j], rr * 4 + 1)),
                             cvt2_out<OUT_DT>(MF::get(acc[i][j], rr * 4 + 2), MF::get(acc[i][j], rr * 4 + 3)));
            }
          __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's staging writes have landed
          __builtin_amdgcn_wave_barrier();
          constexpr int LPR = TN * 32 * 2 / 16, RPI = 64 / LPR;  // lanes per token row, rows per instruction
          uint16_t* obase = reinterpret_cast<uint16_t*>(a.out) + em0 * a.ldo + en0;
          // head-major QKV: the wave's head (part, h) block of out, rows at token hm_loff + l of batch b
          uint16_t* hbase = nullptr;
          if constexpr (EPI == kEpiQkvHeads) {
            const int64_t c0 = en0 + wn * 128;
            const int64_t part = c0 / a.hm_hidden, h = (c0 % a.hm_hidden) / 128;
            hbase = reinterpret_cast<uint16_t*>(a.out) + (part * a.hm_B * (a.hm_hidden / 128) + h) * a.hm_Ltot * 128;
          }
#pragma unroll
          for (int r0 = 0; r0 < 32; r0 += RPI) {
            const int orow = r0 + tl / LPR, ocol = (tl % LPR) * 8;
            const v4i v = *reinterpret_cast<const v4i*>(wst + orow * OPITCH + ocol * 2);
            const int ml2 = wm * TM * 32 + j * 32 + orow, nl = wn * TN * 32 + ocol;
            if (ml2 < mrem && nl < nrem) {
              if constexpr (EPI == kEpiQkvHeads) {
                const uint32_t mg = (uint32_t)(em0 + ml2);
                const uint32_t bb = mg / (uint32_t)a.hm_L, ll = mg - bb * (uint32_t)a.hm_L;
                uint16_t* o = hbase + ((int64_t)bb * (a.hm_hidden / 128) * a.hm_Ltot + a.hm_loff + ll) * 128 + ocol;
                __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(o));
              } else {
                __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(obase + (uint32_t)(ml2 * (int)a.ldo + nl)));
              }
            }
          }
          }
        } else if (m_ok) {
#pragma unroll
          for (int i = 0; i < TN; i++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
              const int nl = nloc + i * 32 + rr * 8;
              const uint32_t off = (uint32_t)(ml * (int)a.ldo + nl);
              const float v0 = MF::get(acc[i][j], rr * 4 + 0), v1 = MF::get(acc[i][j], rr * 4 + 1), v2 = MF::get(acc[i][j], rr * 4 + 2), v3 = MF::get(acc[i][j], rr * 4 + 3);
              if constexpr (OUT_DT == HN_DTYPE_F32) {
                float* o = reinterpret_cast<float*>(a.out) + em0 * a.ldo + en0 + off;
                if (a.vec_store && nl + 3 < nrem) {
                  *reinterpret_cast<float4*>(o) = make_float4(v0, v1, v2, v3);
                } else {
                  if (nl < nrem) o[0] = v0;
                  if (nl + 1 < nrem) o[1] = v1;
                  if (nl + 2 < nrem) o[2] = v2;
                  if (nl + 3 < nrem) o[3] = v3;
                }
              } else {
                uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + em0 * a.ldo + en0 + off;
                const uint32_t lo = cvt2_out<OUT_DT>(v0, v1), hi = cvt2_out<OUT_DT>(v2, v3);
                if (a.vec_store && nl + 3 < nrem) {
                  *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
                } else {
                  if (nl < nrem) o[0] = (uint16_t)(lo & 0xffffu);
                  if (nl + 1 < nrem) o[1] = (uint16_t)(lo >> 16);
                  if (nl + 2 < nrem) o[2] = (uint16_t)(hi & 0xffffu);
                  if (nl + 3 < nrem) o[3] = (uint16_t)(hi >> 16);
                }
              }
            }
        }
      }
    }
    if constexpr (EARLY_EP) epb ^= 1;
    if (!more) break;
    // the next tile's load offsets again (recomputed rather than kept live across the epilogue)
    int tl2 = lane;
    asm volatile("" : "+v"(tl2));
    plan_loads(m0, n0, tl2);
  }
}

}  // namespace hn
