// jq_quantized_matmul_noalloc: the workspace form of the dense matmul with its scratch in a
// fixed device array of this library instead of a caller workspace, for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops).
//
// The array `scratch` is a file-scope __device__ variable: each GPU the library runs on holds
// its own copy from module load until the process ends. Its device address comes from
// hipGetSymbolAddress, once per device with that device current, and only that address is
// passed to kernels (the array's name in host code is a host-side stand-in, not a device
// address). Every call on one GPU shares the array: calls that overlap on a GPU race, and the
// array keeps the last call's contents. The K-split kernel writes every partial it later reads
// within the same call, and the prefill GEMM every f16 activation row and exponent it reads,
// so nothing needs clearing between calls.
#include <mutex>

#include "jq_common.h"

namespace {

constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[JQ_NOALLOC_SCRATCH_BYTES];

std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device (NULL until looked up)

// The current device's address of `scratch` (looked up on the first call on that device).
int scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return JQ_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return JQ_ERR_LAUNCH;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return JQ_OK;
}

}  // namespace

extern "C" {

int jq_quantized_matmul_noalloc(const void* x, int x_dtype, const uint32_t* codes,
                                const void* scales, const void* biases, int sb_dtype, int bits,
                                int group_size, int64_t M, int64_t N, int64_t K, void* y,
                                int y_dtype, jq_stream_t stream) {
  const int64_t need = jq_quantized_matmul_workspace_size(M, N, K, bits, group_size, x_dtype,
                                                          sb_dtype);
  if (need <= 0)  // no scratch used (or invalid sizes, which the matmul reports)
    return jq_quantized_matmul(x, x_dtype, codes, scales, biases, sb_dtype, bits, group_size, M,
                               N, K, y, y_dtype, stream);
  // The workspace form checks the array's size before any launch: the K-split decode needs
  // its whole workspace (JQ_ERR_WORKSPACE otherwise), the prefill GEMM runs its activation
  // rows in passes of whole 256-row tiles that fit.
  void* ws = nullptr;
  const int s = scratch_ptr(&ws);
  if (s) return s;
  return jq_quantized_matmul_ws(x, x_dtype, codes, scales, biases, sb_dtype, bits, group_size, M,
                                N, K, y, y_dtype, ws, (int64_t)JQ_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
