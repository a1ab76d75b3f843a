// The one-call linear without allocation or workspace argument: the activation codes and scales go to a
// fixed scratch array in device memory that the library owns, for callers that cannot allocate (code
// under HIP graph capture, serving loops that forbid allocation).
//
// `scratch` is a file-scope device array: each GPU the library runs on holds its own copy, at its own
// address, for the life of the process.  In host code its name is only a stand-in, so the device address
// is looked up once per device (hipGetSymbolAddress, with that device current) and that pointer is what
// the kernels receive.  Every call on one GPU shares its array: calls that overlap on one GPU (different
// streams, or threads) race on it, and must be serialized by the caller.  Nothing in it needs to start at
// zero: each call's quantizer writes every code and scale its GEMM reads.
#include <mutex>

#include "hn_common.h"

namespace hn {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[HN_NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_lock;
static void* g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch array (looked up on the first call on that device).
static int scratch_address(void** out) {
  int dev = 0;
  int rc = hip_status(hipGetDevice(&dev), "hn_block_linear_noalloc: hipGetDevice");
  if (rc != HN_OK) return rc;
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("hn_block_linear_noalloc: device %d beyond the %d the library tracks", dev, kMaxDevices);
    return HN_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hn_block_linear_noalloc: hipGetSymbolAddress");
    if (rc != HN_OK) return rc;
    if (p == nullptr || ((uintptr_t)p & 255) != 0) {
      set_error("hn_block_linear_noalloc: scratch array at an unusable address %p", p);
      return HN_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HN_OK;
}

}  // namespace hn

extern "C" int hn_block_linear_noalloc(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t group,
                                       int kind, int rounding, const void* qw, int64_t ldw, const float* sw,
                                       int64_t ldsw, int64_t sw_rows, const void* bias, int bias_dtype, int64_t N,
                                       void* out, int out_dtype, int64_t ldo, void* stream) {
  using namespace hn;
  int rc = check_linear("hn_block_linear_noalloc", x, M, N, K, group, kind, qw, sw, out);
  if (rc != HN_OK) return rc;
  const int64_t need = linear_workspace_bytes(M, K, group);
  HN_REQUIRE(need <= (int64_t)HN_NOALLOC_SCRATCH_BYTES,
             "hn_block_linear_noalloc: M=%lld x K=%lld needs %lld bytes of scratch, beyond the %lld the library holds",
             (long long)M, (long long)K, (long long)need, (long long)HN_NOALLOC_SCRATCH_BYTES);
  if (M == 0) return HN_OK;
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc != HN_OK) return rc;
  return run_linear(x, x_dtype, ldx, M, K, group, kind, rounding, qw, ldw, sw, ldsw, sw_rows, bias, bias_dtype, N, out,
                    out_dtype, ldo, (uint8_t*)ws, stream);
}
