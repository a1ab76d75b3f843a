// Softmax attention on the gfx950 bf16 matrix cores: the attention backend of the double-stream block
// (hy_nomas/model.py:145-150 `attention`, the scaled-dot-product attention the reference hands to ComfyUI's
// backend), in one pass over the keys with an online softmax.
//
//   out[b, i, h, :] = sum_j softmax_j(q[b, i, h, :] . k[b, j, h, :] * scale) v[b, j, h, :]
//
// Head dim 128, bf16 q / k / v / out, fp32 scores, running max and sums, bf16 probabilities for the
// second product (as flash attention does), no mask.
//
// Work split.  A workgroup of 4 waves owns 128 queries of one (batch, head); each wave 32.  Keys are walked
// in tiles of 64, staged in LDS by gfx950's direct-to-LDS loads one tile ahead (two buffers, one barrier per
// tile).
//
// Layouts.  The scores are computed transposed, S^T = K Q^T (keys as the MFMA A rows, queries as the B
// columns), so each lane's accumulators hold one query and 16 keys of each 32-key block: the row statistics
// of a query are in-lane reductions plus one exchange with lane l ^ 32, which holds the other 16 keys.  Each
// lane keeps its own partial row sum and the two are added once at the end.  The output is accumulated
// transposed too, O^T = V^T P^T, with the probabilities as the B operand straight from the score registers:
// an MFMA's operands run along the reduced dimension (here the keys), so the 8 keys of a lane's B fragment
// are the ones its score registers hold, keys 16 g + 8 (e / 4) + 4 h + e % 4 (e = 0..7) of 16-key group g in
// lane half h.  V^T therefore comes with the keys of each 16-key group stored in the order 0-3, 8-11, 4-7,
// 12-15 (`hn_attention`'s V^T layout): lane half h's 8 keys are then one 16-byte chunk, read with one
// ds_read_b128.
//
// LDS.  K tile: 64 rows of 256 bytes, 16-byte chunk c of row r at c ^ (r & 15); V^T tile: 128 rows of 128
// bytes, chunk c of row r at c ^ ((r >> 1) & 7).  Both are read conflict-free (16 lanes per 256-byte pass hit
// 16 different bank quads).  The direct loads write 1 KB per wave instruction in lane order, so the swizzle
// is applied on the global side (the lane fetches the logical chunk of its physical slot).
//
// Lazy rescale.  The running reference max m moves only when a tile's max exceeds it by more than 8 (base-2
// units), so the probabilities exp2(s - m) stay below 2^8 and the accumulators are rescaled only a few times
// per query instead of whenever the max grows.  The result is the same quotient: numerator and denominator
// share the reference.
#include "hn_common.h"

namespace hn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int v4i_a __attribute__((ext_vector_type(4)));
typedef float v16f_a __attribute__((ext_vector_type(16)));

constexpr int kHeadDim = 128;
constexpr int kBQ = 128;                        // queries per workgroup
constexpr int kBK = 64;                         // keys per tile
constexpr int kAttnWaves = 4;
constexpr int kKTile = kBK * kHeadDim * 2;      // 16 KB
constexpr int kVTile = kHeadDim * kBK * 2;      // 16 KB
constexpr int kAttnStage = kKTile + kVTile;
constexpr float kSlack = 8.0f;                  // headroom of the lazy max (base-2 units)

struct AttnArgs {
  const uint16_t* q;
  int64_t sqb, sqh, sqi;  // element strides of batch, head, token (dims contiguous)
  const uint16_t* k;
  int64_t skb, skh, skj;
  const uint16_t* vt;     // V^T: element (b, h, d, key position p) at vt + b svb + h svh + d svd + p
  int64_t svb, svh, svd;
  uint16_t* o;
  int64_t sob, soh, soi;
  int H;
  int64_t Lq, Lk;
  float scale_log2;       // softmax scale times log2(e): the scores are exponentiated base 2
  int qblocks;
};

__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }

// max of x over lanes l and l ^ 32 (one v_permlane32_swap instead of an LDS permute)
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                  false, false);
  return __builtin_fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}

__global__ __launch_bounds__(kAttnWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attention_kernel(const AttnArgs a) {
  __shared__ __align__(16) char smem[2 * kAttnStage];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h2 = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.x / a.qblocks, qb = blockIdx.x % a.qblocks;
  const int64_t b = bh / a.H, hh = bh % a.H;
  const uint16_t* qbase = a.q + b * a.sqb + hh * a.sqh;
  const char* kbase = reinterpret_cast<const char*>(a.k + b * a.skb + hh * a.skh);
  const char* vbase = reinterpret_cast<const char*>(a.vt + b * a.svb + hh * a.svh);
  const uint32_t kstride = (uint32_t)(a.skj * 2), vstride = (uint32_t)(a.svd * 2);  // bytes per key / dim row
  const int64_t q0 = (int64_t)qb * kBQ + wave * 32;
  const int64_t qi = q0 + l32 < a.Lq ? q0 + l32 : a.Lq - 1;

  // the wave's 32 queries: B fragments of S^T = K Q^T for the 8 steps of 16 dims (query l32, dims 16 ks + 8 h2 ..)
  bf16x8 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ks++) qf[ks] = *reinterpret_cast<const bf16x8*>(qbase + qi * a.sqi + 16 * ks + 8 * h2);

  // direct loads of one tile: wave w fills the 1 KB blocks w, w + 4, w + 8, w + 12 of the K tile (4 rows of
  // 256 bytes each) and of the V^T tile (8 rows of 128 bytes), each lane 16 bytes at a fixed 32-bit offset
  // from the tile's buffer descriptor (wave-uniform base: no per-lane 64-bit address arithmetic)
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int krow = (wave + 4 * u) * 4 + lane / 16, kphys = lane % 16;
    koff[u] = (uint32_t)krow * kstride + (uint32_t)((kphys ^ (krow & 15)) << 4);
    const int vrow = (wave + 4 * u) * 8 + lane / 8, vphys = lane % 8;
    voff[u] = (uint32_t)vrow * vstride + (uint32_t)((vphys ^ ((vrow >> 1) & 7)) << 4);
  }
  auto issue_tile = [&](int64_t j0, int buf) {
    char* kt = smem + buf * kAttnStage;
    char* vt = kt + kKTile;
    const __amdgpu_buffer_rsrc_t kr = buffer_rsrc(kbase + j0 * kstride);
    const __amdgpu_buffer_rsrc_t vr = buffer_rsrc(vbase + j0 * 2);
    if (j0 + kBK <= a.Lk) {
#pragma unroll
      for (int u = 0; u < 4; u++) b2lds16(kr, koff[u], 0, kt + (wave + 4 * u) * 1024);
    } else {
      // the last tile: rows past the last key re-read it (their scores are masked)
      const int last = (int)(a.Lk - 1 - j0);
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int krow = (wave + 4 * u) * 4 + lane / 16, kphys = lane % 16;
        const int r = krow < last ? krow : last;
        b2lds16(kr, (uint32_t)r * kstride + (uint32_t)((kphys ^ (krow & 15)) << 4), 0, kt + (wave + 4 * u) * 1024);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; u++) b2lds16(vr, voff[u], 0, vt + (wave + 4 * u) * 1024);
  };

  v16f_a oacc[4];
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int r = 0; r < 16; r++) oacc[db][r] = 0.0f;
  float m = -__builtin_inff();  // reference max of the scaled scores (base-2 units), shared by lanes l, l ^ 32
  // -m / (scale log2(e)) in every register: the score products start from it, so the scores come out already
  // relative to the reference and a probability is exp2(s scale log2(e)).  0 until the first tile sets m.
  v16f_a mref;
#pragma unroll
  for (int r = 0; r < 16; r++) mref[r] = 0.0f;
  const float inv_scale = 1.0f / a.scale_log2;
  float mref_m = 0.0f;  // the reference mref holds (m', base-2 units)
  float lsum = 0.0f;            // this lane's partial sum of the probabilities
  float pv[32];                 // the last tile's probabilities, not yet in lsum
#pragma unroll
  for (int i = 0; i < 32; i++) pv[i] = 0.0f;
  const int kswz = l32 & 15, vswz = (l32 >> 1) & 7;   // the lane's rows' swizzles (rows 32 i + l32)

  const int64_t nt = (a.Lk + kBK - 1) / kBK;
  // tile t in stage buffer BUF (a constant, so the buffer offset rides in the LDS reads' immediate field
  // and the lane's fragment offsets stay fixed across the loop)
  auto tile = [&](int64_t t, auto buf_c) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_c)::value;
    // tile t has landed for every wave, and every wave is done with the buffer tile t + 1 refills
    wait_vm0();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (t + 1 < nt) issue_tile((t + 1) * kBK, BUF ^ 1);
    const char* kt = smem + BUF * kAttnStage;
    const char* vt = kt + kKTile;
    const int64_t j0 = t * kBK;

    // S^T for the tile's two 32-key blocks (interleaved): lane holds query l32, keys 32 kb + 8 (r / 4) + 4 h2 + r % 4
    v16f_a s[2];
    // the K fragments two steps ahead of their products (a ring of three), so each read has two steps of
    // products to land in
    bf16x8 kf[3][2];
    auto read_k = [&](int ks, bf16x8* f) __attribute__((always_inline)) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
        f[kb] = *reinterpret_cast<const bf16x8*>(kt + (32 * kb + l32) * 256 + (((2 * ks + h2) ^ kswz) << 4));
    };
    read_k(0, kf[0]);
    read_k(1, kf[1]);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks % 3][kb], qf[ks], ks == 0 ? mref : s[kb], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      if (ks + 2 < 8) {
        read_k(ks + 2, kf[(ks + 2) % 3]);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      // the previous tile's probabilities join the running sum while the matrix core works (the
      // reference m' has not moved since they were formed: a move below rescales lsum after this)
#pragma unroll
      for (int i = 0; i < 4; i++) lsum += pv[4 * ks + i];
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
    if (j0 + kBK > a.Lk) {  // the last tile: keys past the end take no weight
      // register r of block kb holds key j0 + 32 kb + 8 (r / 4) + (r % 4) + 4 h2: a constant per register
      // against one per-lane limit
      const int lim = (int)(a.Lk - j0) - 4 * h2;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (32 * kb + 8 * (r / 4) + (r % 4) >= lim) s[kb][r] = -__builtin_inff();
    }
    // online softmax: the tile's max for this query (both lanes), then the lazy move of the reference max.
    // The scores hold s - m' / (scale log2(e)), m' the reference their products started from (m after the
    // first tile), so the tile's max in base-2 units is mx scale log2(e) + m'.
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) mx = __builtin_fmaxf(mx, s[kb][r]);
    const float mrel = max_xor32(mx) * a.scale_log2;  // the tile's max relative to m'
    // m' = m outside the move below; the first tile (m = -inf) always moves it
    if (__builtin_amdgcn_ballot_w64(!(mrel + mref_m <= m + kSlack)) != 0) {
      const float mt = mrel + mref_m;
      const bool grow = mt > m + kSlack;
      const float mnew = grow ? mt : m;
      const float alpha = __builtin_amdgcn_exp2f(m - mnew);  // 1 where m stays, 0 for the first tile
      m = mnew;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 4; db++)
#pragma unroll
        for (int r = 0; r < 16; r++) oacc[db][r] *= alpha;
      // this tile's scores moved to the new reference, and the next tiles' products start from it
      const float delta = (mref_m - m) * inv_scale;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) s[kb][r] += delta;
      mref_m = m;
      const float mr = -m * inv_scale;
#pragma unroll
      for (int r = 0; r < 16; r++) mref[r] = mr;
    }
    // probabilities exp2(s scale log2(e)) against the reference, this lane's sum, bf16 pairs
    uint32_t pk[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int p = 0; p < 8; p++) {
        const float e0 = __builtin_amdgcn_exp2f(s[kb][2 * p] * a.scale_log2);
        const float e1 = __builtin_amdgcn_exp2f(s[kb][2 * p + 1] * a.scale_log2);
        pv[16 * kb + 2 * p] = e0;
        pv[16 * kb + 2 * p + 1] = e1;
        pk[kb][p] = bf16x2_finite(e0, e1);
      }
    // O^T += V^T P^T over the four 16-key groups g = 2 kb + ks2: the B fragment is score registers
    // 8 ks2 .. 8 ks2 + 7 of block kb, the A fragment chunk 2 g + h2 of each V^T row (the keys in the same order)
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ks2++) {
        const v4i_a bi = {(int)pk[kb][4 * ks2], (int)pk[kb][4 * ks2 + 1], (int)pk[kb][4 * ks2 + 2],
                          (int)pk[kb][4 * ks2 + 3]};
        const int chunk = (4 * kb + 2 * ks2 + h2) ^ vswz;
#pragma unroll
        for (int db = 0; db < 4; db++) {
          const bf16x8 af = *reinterpret_cast<const bf16x8*>(vt + (32 * db + l32) * 128 + (chunk << 4));
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, __builtin_bit_cast(bf16x8, bi), oacc[db], 0, 0, 0);
        }
      }
  };
  issue_tile(0, 0);
  for (int64_t t = 0; t < nt; t += 2) {
    tile(t, std::integral_constant<int, 0>());
    if (t + 1 < nt) tile(t + 1, std::integral_constant<int, 1>());
  }
#pragma unroll
  for (int i = 0; i < 32; i++) lsum += pv[i];
  // normalize and store: lane holds query l32, dims 32 db + 8 rr + 4 h2 + 0..3 in registers 4 rr .. 4 rr + 3
  const float ltot = lsum + __shfl_xor(lsum, 32);
  const float inv = 1.0f / ltot;
  if (q0 + l32 < a.Lq) {
    uint16_t* orow = a.o + b * a.sob + hh * a.soh + (q0 + l32) * a.soi;
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const int d = 32 * db + 8 * rr + 4 * h2;
        const uint2 w = make_uint2(bf16x2_finite(oacc[db][4 * rr] * inv, oacc[db][4 * rr + 1] * inv),
                                   bf16x2_finite(oacc[db][4 * rr + 2] * inv, oacc[db][4 * rr + 3] * inv));
        *reinterpret_cast<uint2*>(orow + d) = w;
      }
  }
}

}  // namespace
}  // namespace hn

extern "C" int hn_attention(const void* q, int64_t sqb, int64_t sqh, int64_t sqi, const void* k, int64_t skb,
                            int64_t skh, int64_t skj, const void* vt, int64_t svb, int64_t svh, int64_t svd,
                            void* out, int64_t sob, int64_t soh, int64_t soi, int64_t B, int64_t H, int64_t Lq,
                            int64_t Lk, int64_t D, float scale, void* stream) {
  using namespace hn;
  HN_REQUIRE(B >= 0 && H > 0 && Lq >= 0 && Lk > 0, "hn_attention: bad shape B=%lld H=%lld Lq=%lld Lk=%lld",
             (long long)B, (long long)H, (long long)Lq, (long long)Lk);
  HN_REQUIRE(D == kHeadDim, "hn_attention: head dim %lld (128 only)", (long long)D);
  HN_REQUIRE(q && k && vt && out, "hn_attention: null pointer");
  HN_REQUIRE(svd >= (Lk + kBK - 1) / kBK * kBK,
             "hn_attention: V^T rows must hold ceil(Lk / 64) * 64 keys (svd=%lld for Lk=%lld)", (long long)svd,
             (long long)Lk);
  HN_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)vt & 15) == 0 &&
                 ((uintptr_t)out & 7) == 0,
             "hn_attention: q, k, v^T must be 16-byte and out 8-byte aligned");
  HN_REQUIRE(sqi % 8 == 0 && skj % 8 == 0 && svd % 8 == 0 && sqh % 8 == 0 && skh % 8 == 0 && svh % 8 == 0 &&
                 sqb % 8 == 0 && skb % 8 == 0 && svb % 8 == 0 && soi % 4 == 0 && soh % 4 == 0 && sob % 4 == 0,
             "hn_attention: strides must keep rows 16-byte aligned (out 8-byte)");
  HN_REQUIRE(skj > 0 && skj <= (1 << 23) && svd > 0 && svd <= (1 << 22),
             "hn_attention: key stride %lld / V^T row stride %lld out of range (tile offsets are 32-bit)",
             (long long)skj, (long long)svd);
  HN_REQUIRE(scale > 0.0f && scale < 1e30f, "hn_attention: bad scale");
  if (B == 0 || Lq == 0) return HN_OK;
  const int64_t qblocks = (Lq + kBQ - 1) / kBQ;
  const int64_t grid = B * H * qblocks;
  HN_REQUIRE(grid <= 0x7fffffff && qblocks <= 0x7fffffff && H <= 0x7fffffff, "hn_attention: problem too large");
  AttnArgs a{};
  a.q = (const uint16_t*)q; a.sqb = sqb; a.sqh = sqh; a.sqi = sqi;
  a.k = (const uint16_t*)k; a.skb = skb; a.skh = skh; a.skj = skj;
  a.vt = (const uint16_t*)vt; a.svb = svb; a.svh = svh; a.svd = svd;
  a.o = (uint16_t*)out; a.sob = sob; a.soh = soh; a.soi = soi;
  a.H = (int)H; a.Lq = Lq; a.Lk = Lk;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.qblocks = (int)qblocks;
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)grid), dim3(kAttnWaves * 64), 0, (hipStream_t)stream, a);
  return HN_LAUNCH_CHECK("attention_kernel");
}
