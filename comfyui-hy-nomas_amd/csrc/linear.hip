// One-call W8A8 linear: dynamic activation quantization, then the block-scaled GEMM
// (hy_nomas/kernels.py:210-222, block_linear).  The activation codes and their scales are scratch: they
// live in a workspace the caller passes in, laid out as
//   [0, M * K)                       codes, row stride K (int8 or e4m3)
//   [codes_end rounded up to 256, +) scales, fp32 [M, K / group]
#include "hn_common.h"

namespace hn {

// Bytes of the codes and the offset of the scales in a workspace of an M x K linear.
static int64_t linear_scales_offset(int64_t M, int64_t K) { return (M * K + 255) / 256 * 256; }
int64_t linear_workspace_bytes(int64_t M, int64_t K, int64_t group) {
  return linear_scales_offset(M, K) + M * (K / group) * (int64_t)sizeof(float);
}

// Shapes and pointers checked before any launch (the callees check the rest: strides, alignment, dtypes).
int check_linear(const char* who, const void* x, int64_t M, int64_t N, int64_t K, int64_t group, int kind,
                 const void* qw, const float* sw, const void* out) {
  HN_REQUIRE(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%lld N=%lld K=%lld", who, (long long)M, (long long)N,
             (long long)K);
  HN_REQUIRE(K % 128 == 0, "%s: K=%lld is not a multiple of 128", who, (long long)K);
  HN_REQUIRE(group == 128 || group == K, "%s: group must be 128 or K (got %lld)", who, (long long)group);
  HN_REQUIRE(kind == HN_KIND_INT8 || kind == HN_KIND_FP8, "%s: bad kind %d", who, kind);
  HN_REQUIRE(M == 0 || (x && qw && sw && out), "%s: null pointer", who);
  return HN_OK;
}

// Quantize x into the workspace, then run the GEMM from it (both enqueued on `stream`).
int run_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind, int rounding,
               const void* qw, int64_t ldw, const float* sw, int64_t ldsw, int64_t sw_rows, const void* bias,
               int bias_dtype, int64_t N, void* out, int out_dtype, int64_t ldo, uint8_t* ws, void* stream) {
  if (M == 0) return HN_OK;
  float* s = reinterpret_cast<float*>(ws + linear_scales_offset(M, K));
  const int64_t ng = K / group;
  int rc = hn_quantize_act(x, x_dtype, ldx, M, K, group, kind, rounding, ws, K, s, ng, stream);
  if (rc != HN_OK) return rc;
  return hn_block_gemm(ws, K, s, ng, qw, ldw, sw, ldsw, sw_rows, bias, bias_dtype, M, N, K, group, kind, HN_EPI_NONE,
                       out, out_dtype, ldo, nullptr, 0, stream);
}

}  // namespace hn

extern "C" int64_t hn_block_linear_workspace_bytes(int64_t M, int64_t K, int64_t group) {
  if (M < 0 || K <= 0 || K % 128 || (group != 128 && group != K)) return -1;
  return hn::linear_workspace_bytes(M, K, group);
}

extern "C" int hn_block_linear(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group, int kind,
                               int rounding, const void* qw, int64_t ldw, const float* sw, int64_t ldsw, int64_t sw_rows,
                               const void* bias, int bias_dtype, int64_t N, void* out, int out_dtype, int64_t ldo,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace hn;
  int rc = check_linear("hn_block_linear", x, M, N, K, group, kind, qw, sw, out);
  if (rc != HN_OK) return rc;
  const int64_t need = linear_workspace_bytes(M, K, group);
  HN_REQUIRE(workspace_bytes >= need, "hn_block_linear: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
             (long long)need);
  HN_REQUIRE(M == 0 || (workspace && ((uintptr_t)workspace & 255) == 0),
             "hn_block_linear: workspace must be 256-byte aligned");
  return run_linear(x, x_dtype, ldx, M, K, group, kind, rounding, qw, ldw, sw, ldsw, sw_rows, bias, bias_dtype, N, out,
                    out_dtype, ldo, (uint8_t*)workspace, stream);
}
