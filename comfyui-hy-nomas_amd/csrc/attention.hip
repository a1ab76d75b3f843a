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
// of a query are in-lane sums plus one exchange with lane l ^ 32, which holds the other 16 keys.  Each lane
// keeps its own partial row sum and the two are added once at the end.  The output is accumulated transposed
// too, O^T = V^T P^T, with the probabilities as the B operand straight from the score registers: an MFMA's
// operands run along the reduced dimension (here the keys), so the 16 keys of a B fragment are taken in the
// order the score accumulators hold them, and the V^T fragment reads the same keys, two runs of 4.  V is
// therefore read from V^T (keys contiguous for each of the 128 dims).
//
// LDS.  K tile: 64 rows of 256 bytes, 16-byte chunk c of row r at c ^ (r & 15); V^T tile: 128 rows of 128 bytes,
// chunk c of row r at c ^ ((r >> 1) & 7).  The direct loads write 1 KB per wave instruction in lane order, so
// the swizzle is applied on the global side (the lane fetches the logical chunk of its physical slot).
#include "hn_common.h"

namespace hn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int v4i_a __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;
constexpr int kBQ = 128;                        // queries per workgroup
constexpr int kBK = 64;                         // keys per tile
constexpr int kAttnWaves = 4;
constexpr int kKTile = kBK * kHeadDim * 2;      // 16 KB
constexpr int kVTile = kHeadDim * kBK * 2;      // 16 KB
constexpr int kAttnStage = kKTile + kVTile;

struct AttnArgs {
  const uint16_t* q;
  int64_t sqb, sqh, sqi;  // element strides of batch, head, token (dims contiguous)
  const uint16_t* k;
  int64_t skb, skh, skj;
  const uint16_t* vt;     // V^T: element (b, h, d, j) at vt + b svb + h svh + d svd + j
  int64_t svb, svh, svd;
  uint16_t* o;
  int64_t sob, soh, soi;
  int H;
  int64_t Lq, Lk;
  float scale_log2;       // softmax scale times log2(e): the scores are exponentiated base 2
  int qblocks;
};

typedef __attribute__((address_space(3))) void* lds_ptr_a;

__device__ __forceinline__ void g2lds16_a(const void* g, char* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_a)lds_wave_base, 16, 0, 0);
}

__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); }

__device__ __forceinline__ float fmax_f(float a, float b) { return __builtin_fmaxf(a, b); }

__global__ __launch_bounds__(kAttnWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attention_kernel(const AttnArgs a) {
  __shared__ __align__(16) char smem[2 * kAttnStage];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h2 = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.x / a.qblocks, qb = blockIdx.x % a.qblocks;
  const int64_t b = bh / a.H, hh = bh % a.H;
  const uint16_t* qbase = a.q + b * a.sqb + hh * a.sqh;
  const uint16_t* kbase = a.k + b * a.skb + hh * a.skh;
  const uint16_t* vbase = a.vt + b * a.svb + hh * a.svh;
  const int64_t q0 = (int64_t)qb * kBQ + wave * 32;
  const int64_t qi = q0 + l32 < a.Lq ? q0 + l32 : a.Lq - 1;

  // the wave's 32 queries: B fragments of S^T = K Q^T for the 8 steps of 16 dims (query l32, dims 16 ks + 8 h2 ..)
  bf16x8 qf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ks++) qf[ks] = *reinterpret_cast<const bf16x8*>(qbase + qi * a.sqi + 16 * ks + 8 * h2);

  // direct loads of one tile: wave w fills the 1 KB blocks w, w + 4, w + 8, w + 12 of the K tile (4 rows of
  // 256 bytes each) and of the V^T tile (8 rows of 128 bytes)
  auto issue_tile = [&](int64_t j0, int buf) {
    char* kt = smem + buf * kAttnStage;
    char* vt = kt + kKTile;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int blk = wave + 4 * u;
      const int row = blk * 4 + lane / 16, phys = lane % 16;
      const int logical = phys ^ (row & 15);
      const int64_t key = j0 + row < a.Lk ? j0 + row : a.Lk - 1;
      g2lds16_a(kbase + key * a.skj + logical * 8, kt + blk * 1024);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int blk = wave + 4 * u;
      const int row = blk * 8 + lane / 8, phys = lane % 8;
      const int logical = phys ^ ((row >> 1) & 7);
      g2lds16_a(vbase + row * a.svd + j0 + logical * 8, vt + blk * 1024);
    }
  };

  typedef float v16f_a __attribute__((ext_vector_type(16)));
  v16f_a oacc[4];
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int r = 0; r < 16; r++) oacc[db][r] = 0.0f;
  float m = -__builtin_inff();  // running max of the scaled scores (base-2 units), shared by lanes l, l ^ 32
  float lsum = 0.0f;            // this lane's partial sum of the probabilities

  const int64_t nt = (a.Lk + kBK - 1) / kBK;
  issue_tile(0, 0);
  for (int64_t t = 0; t < nt; t++) {
    const int buf = (int)(t & 1);
    // tile t has landed for every wave, and every wave is done with the buffer tile t + 1 refills
    wait_vm0();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (t + 1 < nt) issue_tile((t + 1) * kBK, buf ^ 1);
    const char* kt = smem + buf * kAttnStage;
    const char* vt = kt + kKTile;
    const int64_t j0 = t * kBK;

    // S^T for the tile's two 32-key blocks: lane holds query l32, keys 32 kb + 8 (r / 4) + 4 h2 + r % 4
    v16f_a s[2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
#pragma unroll
      for (int r = 0; r < 16; r++) s[kb][r] = 0.0f;
      const int row = 32 * kb + l32;
#pragma unroll
      for (int ks = 0; ks < 8; ks++) {
        const bf16x8 af = *reinterpret_cast<const bf16x8*>(kt + row * 256 + (((2 * ks + h2) ^ (row & 15)) << 4));
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, qf[ks], s[kb], 0, 0, 0);
      }
    }
    if (j0 + kBK > a.Lk) {  // the last tile: keys past the end take no weight
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int64_t key = j0 + 32 * kb + 8 * (r / 4) + 4 * h2 + (r % 4);
          if (key >= a.Lk) s[kb][r] = -__builtin_inff();
        }
    }
    // online softmax: the tile's max for this query (both lanes), the rescale of what came before
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) mx = fmax_f(mx, s[kb][r]);
    mx = fmax_f(mx, __shfl_xor(mx, 32));
    const float mnew = fmax_f(m, mx * a.scale_log2);
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);  // 0 for the first tile (m = -inf)
    m = mnew;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 4; db++)
#pragma unroll
        for (int r = 0; r < 16; r++) oacc[db][r] *= alpha;
    }
    // probabilities (base-2 exponent of the scaled score minus the max), this lane's sum, bf16 pairs
    uint32_t pk[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int p = 0; p < 8; p++) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][2 * p], a.scale_log2, -mnew));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][2 * p + 1], a.scale_log2, -mnew));
        lsum += e0 + e1;
        pk[kb][p] = bf16x2_finite(e0, e1);
      }
    // O^T += V^T P^T: step (kb, ks2) takes the 16 keys 32 kb + 16 ks2 + 8 (e / 4) + 4 h2 + e % 4 of element
    // e of lane half h2, i.e. registers 8 ks2 .. 8 ks2 + 7 of block kb, and the V^T row's keys in the same order
#pragma unroll
    for (int db = 0; db < 4; db++) {
      const int row = 32 * db + l32;
      const int swz = (row >> 1) & 7;
      const char* vrow = vt + row * 128 + 8 * h2;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ks2++) {
          const int c0 = 4 * kb + 2 * ks2;
          const uint2 lo = *reinterpret_cast<const uint2*>(vrow + ((c0 ^ swz) << 4));
          const uint2 hi = *reinterpret_cast<const uint2*>(vrow + (((c0 + 1) ^ swz) << 4));
          const v4i_a ai = {(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
          const v4i_a bi = {(int)pk[kb][4 * ks2], (int)pk[kb][4 * ks2 + 1], (int)pk[kb][4 * ks2 + 2],
                            (int)pk[kb][4 * ks2 + 3]};
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ai),
                                                             __builtin_bit_cast(bf16x8, bi), oacc[db], 0, 0, 0);
        }
    }
  }
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
