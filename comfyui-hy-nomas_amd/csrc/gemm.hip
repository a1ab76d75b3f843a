// Dispatch and C ABI of the block-scaled 8-bit GEMM (hy_nomas/kernels.py:152-170, block_gemm).
// The kernel template and its design notes are in gemm_kernel.h.
#include <atomic>

#include "gemm_kernel.h"
#include "skinny_kernel.h"

namespace hn {

// int8 codes lie in [-128, 127], so a whole-K int32 dot product is exact for K < 2^17.
constexpr int64_t kWholeKInt32Limit = 131072;

// ---------------------------------------------------------------------------------------------
// configurations

// Compute units of the current device (the persistent grid has at most one workgroup per CU).
// The per-device cache may be filled by several host threads at once; they store the same value.
static int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// WPE: waves per SIMD the kernel is compiled for; above WN * WM / 4, several workgroups share a CU and the
// persistent grid grows to match.
template <int KIND, int EPI, bool G128, int WN, int WM, int TN, int TM, int OUT_DT, int BK, int NS, bool WBLK = false,
          int WPE = WN * WM / 4>
static int launch_cfg(GemmArgs& a, hipStream_t st) {
  constexpr int BN = WN * TN * 32, BM = WM * TM * 32;
  const int64_t tm = (a.M + BM - 1) / BM, tn = (a.N + BN - 1) / BN;
  if (tm * tn > 0x7fffffff) {
    set_error("hn_block_gemm: problem too large (%lld tiles)", (long long)(tm * tn));
    return HN_ERR_UNSUPPORTED;
  }
  a.tiles_m = (int)tm;
  a.tiles_n = (int)tn;
  const int64_t slots = (int64_t)cu_count() * (WPE * 4 / (WN * WM));
  const int64_t grid = tm * tn < slots ? tm * tn : slots;
  hipLaunchKernelGGL((block_gemm_kernel<KIND, EPI, G128, WN, WM, TN, TM, OUT_DT, BK, NS, WBLK, WPE>),
                     dim3((unsigned)grid), dim3(WN * WM * 64), 0, st, a);
  return HN_LAUNCH_CHECK("block_gemm_kernel");
}

// The rows of a problem, as two launches: a.M rows from row 0 with the big tile, then the rest with a 128 x 128
// tile.  Tile rows are independent and every output keeps its fold order, so the results do not depend on
// where the split falls.
enum class TileSplit { kBig, kSmall, kBoth };

// Which tiles serve an M x N problem whose big tile is bm x bn with `slots` workgroups resident (one round of
// tiles), and for kBoth the rows the big tile takes.  A persistent grid runs ceil(tiles / slots) rounds of
// tiles; when the last round would leave more than half of the compute units idle, its rows go to 128 x 128
// tiles (four per big tile, on every compute unit).  A problem with fewer big tiles than half a round runs on
// small tiles alone.
static TileSplit choose_tiles(int64_t M, int64_t N, int bm, int bn, int64_t slots, int64_t* big_rows) {
  const int64_t tm = (M + bm - 1) / bm, tn = (N + bn - 1) / bn, tiles = tm * tn;
  const int64_t full = tiles / slots, rem = tiles % slots;
  if (rem == 0 || rem > slots / 2) return TileSplit::kBig;
  if (full == 0) return TileSplit::kSmall;
  const int64_t rows = (full * slots / tn) * bm;  // whole tile rows of the full rounds
  if (rows <= 0 || rows >= M) return TileSplit::kBig;
  *big_rows = rows;
  return TileSplit::kBoth;
}

// Launch the big-tile configuration BIG or the small one SMALL (each a launch_cfg instantiation) over the rows
// choose_tiles assigns them.
template <int BM, int BN, int WN, int WM, int WPE, typename Big, typename Small>
static int launch_split(GemmArgs& a, int out_esz, hipStream_t st, Big big, Small small) {
  const int64_t slots = (int64_t)cu_count() * (WPE * 4 / (WN * WM));
  int64_t rows = 0;
  const TileSplit how = choose_tiles(a.M, a.N, BM, BN, slots, &rows);
  if (how == TileSplit::kBig) return big(a);
  if (how == TileSplit::kSmall) return small(a);
  GemmArgs head = a, tail = a;
  head.M = rows;
  tail.M = a.M - rows;
  tail.qa = a.qa + rows * a.lda;
  tail.sa = a.sa + rows * a.ldsa;
  tail.out = static_cast<char*>(a.out) + rows * a.ldo * out_esz;
  const int rc = big(head);
  return rc != HN_OK ? rc : small(tail);
}

// per-token / per-channel: 256 x 256 tile, 8 waves of 128 x 64.  fp8 with block weight scales: the same
// tile (the running sum is rescaled in place, so there is no second accumulator set).  Other g128 layouts:
// 256 x 128, 8 waves of 128 x 32 (the int32 group partial and the fp32 running sum both fit in 256
// VGPRs).  128-byte K stages in two LDS buffers.  The plain and GELU epilogues also have 128 x 128 tiles of
// four waves (64 x 64 each, or 128 x 32 with block weight scales) for problems, or tails of problems, that
// would leave most compute units idle with the big tile (choose_tiles); two such workgroups share a compute
// unit (about 70 KB of LDS each).
template <int KIND, int EPI, int OUT_DT>
static int launch_group(GemmArgs& a, bool g128, hipStream_t st) {
  constexpr bool SWIGLU = EPI == HN_EPI_SWIGLU_QUANT;
  constexpr bool SMALL_OK = EPI == HN_EPI_NONE || EPI == HN_EPI_GELU;
  constexpr int ESZ = OUT_DT == HN_DTYPE_F32 ? 4 : 2;
  if (!g128) {
    auto big = [&](GemmArgs& x) { return launch_cfg<KIND, EPI, false, 2, 4, 4, 2, OUT_DT, 128, 2>(x, st); };
    if constexpr (SMALL_OK) {
      auto small = [&](GemmArgs& x) { return launch_cfg<KIND, EPI, false, 2, 2, 2, 2, OUT_DT, 128, 2, false, 2>(x, st); };
      return launch_split<256, 256, 2, 4, 2>(a, ESZ, st, big, small);
    }
    return big(a);
  }
  if constexpr (KIND == HN_KIND_FP8) {
    if (a.sw_rows == 128) {
      auto big = [&](GemmArgs& x) { return launch_cfg<KIND, EPI, true, 2, 4, 4, 2, OUT_DT, 128, 2, true>(x, st); };
      if constexpr (SMALL_OK) {
        auto small = [&](GemmArgs& x) {
          return launch_cfg<KIND, EPI, true, 1, 4, 4, 1, OUT_DT, 128, 2, true, 2>(x, st);
        };
        return launch_split<256, 256, 2, 4, 2>(a, ESZ, st, big, small);
      }
      return big(a);
    }
  }
  if constexpr (!SWIGLU) {
    if constexpr (KIND == HN_KIND_INT8) {  // (fp8 block scales took the branch above)
      if (a.sw_rows == 128) return launch_cfg<KIND, EPI, true, 2, 4, 4, 1, OUT_DT, 128, 2, true>(a, st);
    }
    auto big = [&](GemmArgs& x) { return launch_cfg<KIND, EPI, true, 2, 4, 4, 2, OUT_DT, 128, 2>(x, st); };
    if constexpr (SMALL_OK) {
      auto small = [&](GemmArgs& x) { return launch_cfg<KIND, EPI, true, 2, 2, 2, 2, OUT_DT, 128, 2, false, 2>(x, st); };
      return launch_split<256, 256, 2, 4, 2>(a, ESZ, st, big, small);
    }
    return big(a);
  }
  set_error("hn_block_gemm: swiglu_quant needs per-token scales or fp8 with 128 x 128 block weight scales");
  return HN_ERR_UNSUPPORTED;
}

template <int KIND, int EPI>
static int launch_out(GemmArgs& a, bool g128, int out_dtype, hipStream_t st) {
  if constexpr (EPI == HN_EPI_GELU_QUANT || EPI == HN_EPI_ACC32 || EPI == HN_EPI_SWIGLU_QUANT) {
    return launch_group<KIND, EPI, HN_DTYPE_BF16>(a, g128, st);
  } else {
    if (out_dtype == HN_DTYPE_BF16) return launch_group<KIND, EPI, HN_DTYPE_BF16>(a, g128, st);
    if (out_dtype == HN_DTYPE_F16) return launch_group<KIND, EPI, HN_DTYPE_F16>(a, g128, st);
    return launch_group<KIND, EPI, HN_DTYPE_F32>(a, g128, st);
  }
}

template <int KIND>
static int launch_kind(GemmArgs& a, bool g128, int epilogue, int out_dtype, hipStream_t st) {
  switch (epilogue) {
    case HN_EPI_NONE: return launch_out<KIND, HN_EPI_NONE>(a, g128, out_dtype, st);
    case HN_EPI_GELU: return launch_out<KIND, HN_EPI_GELU>(a, g128, out_dtype, st);
    case HN_EPI_GELU_QUANT: return launch_out<KIND, HN_EPI_GELU_QUANT>(a, g128, out_dtype, st);
    case HN_EPI_SWIGLU_QUANT: return launch_out<KIND, HN_EPI_SWIGLU_QUANT>(a, g128, out_dtype, st);
    default: break;
  }
  set_error("hn_block_gemm: bad epilogue %d", epilogue);
  return HN_ERR_ARG;
}

// M <= 4 int8 (the per-sample linears): one wave per 4 weight rows, v_dot4 on the streamed weights.
template <int MT, int MODE, int EPI>
static int launch_skinny_out(GemmArgs& a, int out_dtype, hipStream_t st) {
  constexpr int64_t ROWS = kSkinnyRows * kSkinnyWaves;
  const int64_t grid = (a.N + ROWS - 1) / ROWS;
  if (grid > 0x7fffffff) {
    set_error("hn_block_gemm: problem too large (N=%lld)", (long long)a.N);
    return HN_ERR_UNSUPPORTED;
  }
  const dim3 g((unsigned)grid), b(kSkinnyWaves * 64);
  if (out_dtype == HN_DTYPE_BF16) hipLaunchKernelGGL((skinny_gemm_kernel<MT, MODE, EPI, HN_DTYPE_BF16>), g, b, 0, st, a);
  else if (out_dtype == HN_DTYPE_F16) hipLaunchKernelGGL((skinny_gemm_kernel<MT, MODE, EPI, HN_DTYPE_F16>), g, b, 0, st, a);
  else hipLaunchKernelGGL((skinny_gemm_kernel<MT, MODE, EPI, HN_DTYPE_F32>), g, b, 0, st, a);
  return HN_LAUNCH_CHECK("skinny_gemm_kernel");
}

template <int MT, int MODE>
static int launch_skinny_epi(GemmArgs& a, int epilogue, int out_dtype, hipStream_t st) {
  if (epilogue == HN_EPI_GELU) return launch_skinny_out<MT, MODE, HN_EPI_GELU>(a, out_dtype, st);
  return launch_skinny_out<MT, MODE, HN_EPI_NONE>(a, out_dtype, st);
}

template <int MODE>
static int launch_skinny_mode(GemmArgs& a, int epilogue, int out_dtype, hipStream_t st) {
  if (a.M == 1) return launch_skinny_epi<1, MODE>(a, epilogue, out_dtype, st);
  if (a.M == 2) return launch_skinny_epi<2, MODE>(a, epilogue, out_dtype, st);
  return launch_skinny_epi<4, MODE>(a, epilogue, out_dtype, st);
}

}  // namespace hn

extern "C" int hn_block_gemm(const void* qa, int64_t lda, const float* sa, int64_t ldsa, const void* qw, int64_t ldw,
                             const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype, int64_t M, int64_t N,
                             int64_t K, int64_t group, int kind, int epilogue, void* out, int out_dtype, int64_t ldo,
                             float* qs, int64_t ldqs, void* stream) {
  using namespace hn;
  HN_REQUIRE(M >= 0 && N > 0 && K > 0, "hn_block_gemm: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
             (long long)K);
  HN_REQUIRE(K % 128 == 0, "hn_block_gemm: K=%lld is not a multiple of 128", (long long)K);
  HN_REQUIRE(group == 128 || group == K, "hn_block_gemm: group must be 128 or K (got %lld)", (long long)group);
  HN_REQUIRE(kind == HN_KIND_INT8 || kind == HN_KIND_FP8, "hn_block_gemm: bad kind %d", kind);
  HN_REQUIRE(epilogue >= HN_EPI_NONE && epilogue <= HN_EPI_SWIGLU_QUANT, "hn_block_gemm: bad epilogue %d", epilogue);
  HN_REQUIRE(epilogue != HN_EPI_ACC32 || kind == HN_KIND_INT8, "hn_block_gemm: ACC32 is int8 only");
  // whole-K int8 accumulation holds the exact dot product in int32: |sum| <= 128 * 128 * K < 2^31
  HN_REQUIRE(kind != HN_KIND_INT8 || (group != K && epilogue != HN_EPI_ACC32) || K < kWholeKInt32Limit,
             "hn_block_gemm: int8 with one scale group over K=%lld would overflow the int32 accumulator "
             "(K < %lld; use group 128)", (long long)K, (long long)kWholeKInt32Limit);
  HN_REQUIRE(epilogue != HN_EPI_GELU_QUANT || (N % 128 == 0 && qs != nullptr && ldqs >= N / 128),
             "hn_block_gemm: gelu_quant needs N %% 128 == 0 and qs [M, N/128]");
  HN_REQUIRE(out_dtype >= HN_DTYPE_BF16 && out_dtype <= HN_DTYPE_F32, "hn_block_gemm: bad out dtype %d", out_dtype);
  HN_REQUIRE(bias == nullptr || (bias_dtype >= HN_DTYPE_BF16 && bias_dtype <= HN_DTYPE_F32),
             "hn_block_gemm: bad bias dtype %d", bias_dtype);
  HN_REQUIRE(epilogue != HN_EPI_SWIGLU_QUANT || (N % 256 == 0 && qs != nullptr && ldqs >= N / 256),
             "hn_block_gemm: swiglu_quant needs N %% 256 == 0 (gate and up interleaved in 128-row blocks) and "
             "qs [M, N/256]");
  HN_REQUIRE((epilogue != HN_EPI_GELU_QUANT && epilogue != HN_EPI_SWIGLU_QUANT) ||
                 (ldo % 4 == 0 && ((uintptr_t)out & 3) == 0),
             "hn_block_gemm: quantized outputs are stored 4 codes at a time: ldo %% 4 == 0, 4-byte aligned out");
  HN_REQUIRE(lda >= K && ldw >= K && ldo >= (epilogue == HN_EPI_SWIGLU_QUANT ? N / 2 : N),
             "hn_block_gemm: row strides smaller than the rows");
  HN_REQUIRE(lda % 16 == 0 && ldw % 16 == 0, "hn_block_gemm: code row strides must be multiples of 16 bytes");
  HN_REQUIRE(lda < (1 << 22) && ldw < (1 << 22) && ldsa < (1 << 22) && ldsw < (1 << 22) && ldo < (1 << 22),
             "hn_block_gemm: row strides must be below 2^22 elements");
  HN_REQUIRE(sw_rows == 1 || (sw_rows == 128 && group == 128 && epilogue != HN_EPI_ACC32),
             "hn_block_gemm: sw_rows must be 1, or 128 with group 128 (got %lld)", (long long)sw_rows);
  HN_REQUIRE(qa && qw && out, "hn_block_gemm: null pointer");
  HN_REQUIRE(((uintptr_t)qa & 15) == 0 && ((uintptr_t)qw & 15) == 0, "hn_block_gemm: codes must be 16-byte aligned");
  if (epilogue != HN_EPI_ACC32) {
    HN_REQUIRE(sa && sw, "hn_block_gemm: null scales");
    HN_REQUIRE(ldsa >= K / group && ldsw >= K / group, "hn_block_gemm: scale row strides too small");
  }
  if (M == 0) return HN_OK;
  GemmArgs a{};
  a.qa = (const uint8_t*)qa; a.lda = lda; a.sa = sa; a.ldsa = ldsa;
  a.qw = (const uint8_t*)qw; a.ldw = ldw; a.sw = sw; a.ldsw = ldsw; a.sw_rows = (int)sw_rows;
  a.bias = bias; a.bias_dtype = bias_dtype;
  a.M = M; a.N = N; a.K = K;
  a.out = out; a.ldo = ldo; a.qs = qs; a.ldqs = ldqs;
  const int esz = out_dtype == HN_DTYPE_F32 ? 4 : 2;
  a.vec_store = (N % 4 == 0) && (ldo % 4 == 0) && ((((uintptr_t)out) & (4 * esz - 1)) == 0);
  a.stage_store = esz == 2 && (N % 8 == 0) && (ldo % 8 == 0) && ((((uintptr_t)out) & 15) == 0);
  hipStream_t st = (hipStream_t)stream;
  // per-token mode also serves a single-group K == 128 problem with one scale row per channel
  const bool g128 = group == 128 && (K != 128 || sw_rows == 128);
  if (epilogue == HN_EPI_ACC32) return launch_group<HN_KIND_INT8, HN_EPI_ACC32, HN_DTYPE_BF16>(a, false, st);
  if (kind == HN_KIND_INT8 && M <= kSkinnyMaxM && (epilogue == HN_EPI_NONE || epilogue == HN_EPI_GELU)) {
    if (!g128) return launch_skinny_mode<0>(a, epilogue, out_dtype, st);
    if (sw_rows == 128) return launch_skinny_mode<2>(a, epilogue, out_dtype, st);
    return launch_skinny_mode<1>(a, epilogue, out_dtype, st);
  }
  if (kind == HN_KIND_INT8) return launch_kind<HN_KIND_INT8>(a, g128, epilogue, out_dtype, st);
  return launch_kind<HN_KIND_FP8>(a, g128, epilogue, out_dtype, st);
}

static int qkv_heads_impl(const void* qa, int64_t lda, const float* sa, int64_t ldsa, const void* qw, int64_t ldw,
                          const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype, int64_t B,
                          int64_t L, int64_t hidden, int64_t K, int64_t group, int kind, const float* q_norm_w,
                          const float* k_norm_w, const float* cos_t, const float* sin_t, float eps, void* out,
                          int64_t L_total, int64_t l_offset, void* vt, int64_t svb, int64_t svh, int64_t svd,
                          void* stream) {
  using namespace hn;
  HN_REQUIRE(B >= 0 && L >= 0 && hidden > 0 && K > 0, "hn_qkv_heads: bad shape");
  HN_REQUIRE(hidden % 128 == 0, "hn_qkv_heads: hidden=%lld is not a multiple of the head dim 128", (long long)hidden);
  HN_REQUIRE(K % 128 == 0, "hn_qkv_heads: K=%lld is not a multiple of 128", (long long)K);
  HN_REQUIRE(group == 128 || group == K, "hn_qkv_heads: group must be 128 or K (got %lld)", (long long)group);
  HN_REQUIRE(kind == HN_KIND_INT8 || kind == HN_KIND_FP8, "hn_qkv_heads: bad kind %d", kind);
  HN_REQUIRE(sw_rows == 1 || (sw_rows == 128 && group == 128), "hn_qkv_heads: sw_rows must be 1, or 128 with group 128");
  HN_REQUIRE(kind != HN_KIND_INT8 || group != K || K < kWholeKInt32Limit,
             "hn_qkv_heads: int8 with one scale group over K=%lld would overflow the int32 accumulator (K < %lld)",
             (long long)K, (long long)kWholeKInt32Limit);
  HN_REQUIRE(l_offset >= 0 && L_total >= l_offset + L, "hn_qkv_heads: tokens [%lld, %lld) exceed L_total=%lld",
             (long long)l_offset, (long long)(l_offset + L), (long long)L_total);
  HN_REQUIRE(B * L < ((int64_t)1 << 31), "hn_qkv_heads: B * L must be below 2^31");
  HN_REQUIRE(lda >= K && ldw >= K && lda % 16 == 0 && ldw % 16 == 0, "hn_qkv_heads: bad code row strides");
  HN_REQUIRE(lda < (1 << 22) && ldw < (1 << 22) && ldsa < (1 << 22) && ldsw < (1 << 22),
             "hn_qkv_heads: row strides must be below 2^22 elements");
  HN_REQUIRE(ldsa >= K / group && ldsw >= K / group, "hn_qkv_heads: scale row strides too small");
  HN_REQUIRE(bias == nullptr || (bias_dtype >= HN_DTYPE_BF16 && bias_dtype <= HN_DTYPE_F32), "hn_qkv_heads: bad bias dtype");
  HN_REQUIRE(qa && sa && qw && sw && q_norm_w && k_norm_w && out, "hn_qkv_heads: null pointer");
  HN_REQUIRE((cos_t == nullptr) == (sin_t == nullptr), "hn_qkv_heads: cos and sin must both be given or both NULL");
  HN_REQUIRE(((uintptr_t)qa & 15) == 0 && ((uintptr_t)qw & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                 ((uintptr_t)q_norm_w & 15) == 0 && ((uintptr_t)k_norm_w & 15) == 0 &&
                 ((uintptr_t)cos_t & 15) == 0 && ((uintptr_t)sin_t & 15) == 0,
             "hn_qkv_heads: codes, output, norm weights and rope tables must be 16-byte aligned");
  if (B * L == 0) return HN_OK;
  GemmArgs a{};
  a.qa = (const uint8_t*)qa; a.lda = lda; a.sa = sa; a.ldsa = ldsa;
  a.qw = (const uint8_t*)qw; a.ldw = ldw; a.sw = sw; a.ldsw = ldsw; a.sw_rows = (int)sw_rows;
  a.bias = bias; a.bias_dtype = bias_dtype;
  a.M = B * L; a.N = 3 * hidden; a.K = K;
  a.out = out; a.ldo = 3 * hidden;
  a.stage_store = 1;
  a.hm_L = L; a.hm_Ltot = L_total; a.hm_loff = l_offset; a.hm_hidden = hidden; a.hm_B = B;
  a.hm_wq = q_norm_w; a.hm_wk = k_norm_w; a.hm_cos = cos_t; a.hm_sin = sin_t; a.hm_eps = eps;
  a.hm_vt = (uint16_t*)vt; a.hm_svb = svb; a.hm_svh = svh; a.hm_svd = svd;
  hipStream_t st = (hipStream_t)stream;
  const bool g128 = group == 128 && (K != 128 || sw_rows == 128);
  if (kind == HN_KIND_INT8) return launch_group<HN_KIND_INT8, kEpiQkvHeads, HN_DTYPE_BF16>(a, g128, st);
  return launch_group<HN_KIND_FP8, kEpiQkvHeads, HN_DTYPE_BF16>(a, g128, st);
}

extern "C" int hn_qkv_heads(const void* qa, int64_t lda, const float* sa, int64_t ldsa, const void* qw, int64_t ldw,
                            const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype, int64_t B,
                            int64_t L, int64_t hidden, int64_t K, int64_t group, int kind, const float* q_norm_w,
                            const float* k_norm_w, const float* cos_t, const float* sin_t, float eps, void* out,
                            int64_t L_total, int64_t l_offset, void* stream) {
  return qkv_heads_impl(qa, lda, sa, ldsa, qw, ldw, sw, ldsw, sw_rows, bias, bias_dtype, B, L, hidden, K, group, kind,
                        q_norm_w, k_norm_w, cos_t, sin_t, eps, out, L_total, l_offset, nullptr, 0, 0, 0, stream);
}

extern "C" int hn_qkv_heads_vt(const void* qa, int64_t lda, const float* sa, int64_t ldsa, const void* qw, int64_t ldw,
                               const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype,
                               int64_t B, int64_t L, int64_t hidden, int64_t K, int64_t group, int kind,
                               const float* q_norm_w, const float* k_norm_w, const float* cos_t, const float* sin_t,
                               float eps, void* out, int64_t L_total, int64_t l_offset, void* vt, int64_t svb,
                               int64_t svh, int64_t svd, void* stream) {
  HN_REQUIRE(vt != nullptr && ((uintptr_t)vt & 15) == 0, "hn_qkv_heads_vt: V^T must be a 16-byte aligned pointer");
  HN_REQUIRE(L % 32 == 0 && l_offset % 16 == 0,
             "hn_qkv_heads_vt: L=%lld must be a multiple of 32 and l_offset=%lld of 16", (long long)L,
             (long long)l_offset);
  HN_REQUIRE(svd % 8 == 0 && svh % 8 == 0 && svb % 8 == 0 && svd >= l_offset + L && svh >= 128 * svd &&
                 svb >= (hidden / 128) * svh,
             "hn_qkv_heads_vt: V^T strides (%lld, %lld, %lld) must be multiples of 8 holding [B, H, 128, >= %lld]",
             (long long)svb, (long long)svh, (long long)svd, (long long)(l_offset + L));
  return qkv_heads_impl(qa, lda, sa, ldsa, qw, ldw, sw, ldsw, sw_rows, bias, bias_dtype, B, L, hidden, K, group, kind,
                        q_norm_w, k_norm_w, cos_t, sin_t, eps, out, L_total, l_offset, vt, svb, svh, svd, stream);
}
