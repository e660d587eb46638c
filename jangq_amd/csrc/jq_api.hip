// Dense matmul entry points: dispatch between the vector-ALU decode GEMV (M <= 4), the
// decode-batch matrix-core kernels (up to 64 rows: 4x4x4 blocks for long rows, the
// LDS-streamed 16x16x32 kernel for K <= 4096, the register-streamed one otherwise), the
// prefill GEMM and, for shapes none of those takes, the older LDS-tiled GEMM or the generic
// GEMV.
#include <mutex>
#include <vector>

#include "jq_common.h"
#include "jq_qmv.h"

namespace jqh {

namespace {
struct Occ {
  const void* kern;
  int threads;
  size_t lds;
  int dev;
  int nb;  // resident blocks per CU; -1: dynamic LDS opt-in recorded
};
std::mutex g_geo_mu;
std::vector<Occ> g_geo;
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices];  // 0: not queried yet

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
  return dev;
}
}  // namespace

int cus() {
  const int dev = current_device();
  std::lock_guard<std::mutex> lk(g_geo_mu);
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
      n = 256;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

int blocks_per_cu(const void* kern, int threads, size_t lds) {
  const int dev = current_device();
  std::lock_guard<std::mutex> lk(g_geo_mu);
  for (const Occ& o : g_geo)
    if (o.kern == kern && o.threads == threads && o.lds == lds && o.dev == dev && o.nb > 0)
      return o.nb;
  int nb = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, threads, lds) != hipSuccess || nb < 1)
    nb = 1;
  g_geo.push_back(Occ{kern, threads, lds, dev, nb});
  return nb;
}

bool set_lds(const void* kern, size_t lds) {
  if (lds <= 64 * 1024) return true;
  const int dev = current_device();
  std::lock_guard<std::mutex> lk(g_geo_mu);
  for (const Occ& o : g_geo)
    if (o.kern == kern && o.lds == lds && o.dev == dev && o.nb == -1) return true;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return false;
  g_geo.push_back(Occ{kern, 0, lds, dev, -1});
  return true;
}

}  // namespace jqh

namespace {

// Activation rows from which the 256 x 256-tile prefill GEMM takes over (measured on MI355X
// at K = 4096, N = 14336: faster than the 128-row-tile GEMM from 384 rows on).
constexpr int64_t kGemmMinRows = 384;
// Activation rows up to which the persistent decode-batch kernel runs (in passes of
// 2 * 16/(128/gs) rows, the weights re-read from the last-level cache after the first).
constexpr int64_t kDecpMaxRows = 64;
// The 4x4x4 matrix-core GEMV takes the decode batches whose rows are too long for the
// persistent kernel to stage a full MFMA block of activations (measured on MI355X at
// K = 14336: 28 vs 39 us for 8 rows of the 2-bit down projection, 112 vs 154 us for 32).
constexpr int64_t kQmv4MinK = 8192;
inline bool use_qmv4(int64_t M, int64_t K) { return M <= kDecpMaxRows && K >= kQmv4MinK; }

inline bool al(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

// The f16 prefill GEMM takes large-M shapes whose operands it can copy in whole dwords
// (activation rows in 16-byte pieces); it needs a workspace for the f16 activations.
inline bool gemm16_shape(int64_t M, int64_t K, int bits, int gs, int xd, int sb) {
  return M >= kGemmMinRows && jqk::gemm16_ok(M, K, bits, gs, xd, sb);
}
inline bool use_gemm16(const void* x, const uint32_t* codes, const void* scales,
                       const void* biases, int64_t M, int64_t K, int bits, int gs, int xd,
                       int sb) {
  return gemm16_shape(M, K, bits, gs, xd, sb) && al(x, 16) && al(codes, 4) && al(scales, 4) &&
         al(biases, 4);
}

jqk::QmmProblem dense_problem(const void* x, const uint32_t* codes, const void* scales,
                              const void* biases, int64_t M, int64_t N, int64_t K, void* y) {
  jqk::QmmProblem p;
  p.x = x; p.codes = codes; p.scales = scales; p.biases = biases; p.y = y;
  p.M = M; p.N = N; p.K = K;
  p.expert_stride_codes = 0;
  p.expert_stride_sb = 0;
  return p;
}

// The vector-ALU GEMV serves up to 4 activation rows (2 at 2 bits); from 3 rows, outputs of
// more than kGemvRowsMax rows run faster on the matrix-core kernel. Measured on MI355X (graph,
// rotated weights): gate|up 2 x 14336 x 4096 3-bit at 3 / 4 rows 25.9 / 26.5 -> 18.1 /
// 18.6 us; 4096-row outputs within 5% either way (o 6-bit 8.8 against 9.2 us: kept).
constexpr int64_t kGemvRowsMax = 8192;
bool prefer_gemv(int M, int64_t K, int64_t maxN, int bits, int gs, int xd, int sb) {
  if (!jqk::gemv_ok(M, K, maxN, bits, gs, xd, sb)) return false;
  return M <= 2 || maxN <= kGemvRowsMax || !jqk::dmx_ok(M, K, maxN, bits, gs, xd, sb, 1);
}

int dense_one(const void* x, int xd, const uint32_t* codes, const void* scales,
              const void* biases, int sb, int bits, int gs, int64_t M, int64_t N, int64_t K,
              void* y, int yd, hipStream_t st) {
  const bool mfma_ok = (xd == JQ_BF16 || xd == JQ_F16) && K % 128 == 0;
  const int Mi = (int)(M < (1 << 30) ? M : (1 << 30));
  if (prefer_gemv(Mi, K, N, bits, gs, xd, sb)) {
    jqk::QmvBatch b;
    b.M = Mi;
    b.K = (int)K;
    b.p[0].x = x; b.p[0].codes = codes; b.p[0].scales = scales; b.p[0].biases = biases;
    b.p[0].y = y; b.p[0].N = N;
    return jqk::gemv_launch(b, 1, bits, gs, xd, sb, yd, st);
  }
  if (use_qmv4(M, K) && jqk::qmv4_ok(Mi, K, N, bits, gs, xd, sb)) {
    jqk::QmvBatch b;
    b.M = Mi;
    b.K = (int)K;
    b.p[0].x = x; b.p[0].codes = codes; b.p[0].scales = scales; b.p[0].biases = biases;
    b.p[0].y = y; b.p[0].N = N;
    return jqk::qmv4_launch(b, 1, bits, gs, xd, sb, yd, st);
  }
  if (M <= kDecpMaxRows && jqk::dmx_ok(Mi, K, N, bits, gs, xd, sb, 1)) {
    jqk::QmvBatch b;
    b.M = Mi;
    b.K = (int)K;
    b.p[0].x = x; b.p[0].codes = codes; b.p[0].scales = scales; b.p[0].biases = biases;
    b.p[0].y = y; b.p[0].N = N;
    return jqk::dmx_launch(b, 1, bits, gs, xd, sb, yd, st);
  }
  if (M <= kDecpMaxRows && jqk::decp_ok(Mi, K, N, xd, sb)) {
    jqk::QmvBatch b;
    b.M = Mi;
    b.K = (int)K;
    b.p[0].x = x; b.p[0].codes = codes; b.p[0].scales = scales; b.p[0].biases = biases;
    b.p[0].y = y; b.p[0].N = N;
    return jqk::decp_launch(b, 1, bits, gs, xd, sb, yd, st);
  }
  if (use_gemm16(x, codes, scales, biases, M, K, bits, gs, xd, sb)) {
    // No caller workspace here: a stream-ordered allocation for the f16 activations.
    const int64_t need = jqk::gemm16_workspace(M, N, K, gs);
    void* ws = nullptr;
    if (hipMallocAsync(&ws, (size_t)need, st) == hipSuccess) {
      const int s = jqk::gemm16_launch(dense_problem(x, codes, scales, biases, M, N, K, y), bits,
                                       gs, xd, sb, yd, ws, need, st);
      const hipError_t f = hipFreeAsync(ws, st);
      return s ? s : (f == hipSuccess ? JQ_OK : JQ_ERR_LAUNCH);
    }
    (void)hipGetLastError();  // out of memory: the workspace-free GEMM below
  }
  if (M >= kGemmMinRows && jqk::gemm_ok(M, K, bits, gs, xd, sb)) {
    jqk::QmmProblem p;
    p.x = x; p.codes = codes; p.scales = scales; p.biases = biases; p.y = y;
    p.M = M; p.N = N; p.K = K;
    p.expert_stride_codes = 0;
    p.expert_stride_sb = 0;
    return jqk::gemm_launch(p, bits, gs, xd, sb, yd, st);
  }
  if (M > 4 && mfma_ok) {
    jqk::QmmProblem p;
    p.x = x; p.codes = codes; p.scales = scales; p.biases = biases; p.y = y;
    p.M = M; p.N = N; p.K = K;
    p.expert_stride_codes = 0;
    p.expert_stride_sb = 0;
    return jqk::qmm_launch(p, bits, gs, xd, sb, yd, st);
  }
  // GEMV in slices of at most 4 token rows.
  const int xs = jqh::dtype_size(xd), ys = jqh::dtype_size(yd);
  for (int64_t m0 = 0; m0 < M; m0 += 4) {
    jqk::QmvBatch b;
    b.M = (int)(M - m0 < 4 ? M - m0 : 4);
    b.K = (int)K;
    b.p[0].x = (const char*)x + m0 * K * xs;
    b.p[0].codes = codes;
    b.p[0].scales = scales;
    b.p[0].biases = biases;
    b.p[0].N = N;
    b.p[0].y = (char*)y + m0 * N * ys;
    const int s = jqk::qmv_launch(b, 1, bits, gs, xd, sb, yd, st);
    if (s) return s;
  }
  return JQ_OK;
}

int check_dense(const void* x, int xd, const uint32_t* codes, const void* scales,
                const void* biases, int sb, int bits, int gs, int64_t M, int64_t N, int64_t K,
                void* y, int yd) {
  int s = jqh::check_qshape(bits, gs, N, K);
  if (s) return s;
  if (M < 0 || M > ((int64_t)1 << 31)) return JQ_ERR_SHAPE;
  if (!jqh::dtype_ok(xd) || !jqh::dtype_ok(sb) || !jqh::dtype_ok(yd)) return JQ_ERR_DTYPE;
  if (M > 0 && N > 0 && K > 0 && (!x || !codes || !scales || !biases || !y)) return JQ_ERR_NULL;
  if (M > 0 && N > 0 && K == 0 && !y) return JQ_ERR_NULL;
  return JQ_OK;
}

__global__ void fill_zero_kernel(void* y, int64_t n, int es) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (es == 4) ((float*)y)[i] = 0.f;
    else ((uint16_t*)y)[i] = 0;
  }
}

}  // namespace

extern "C" {

int jq_quantized_matmul(const void* x, int x_dtype, const uint32_t* codes, const void* scales,
                        const void* biases, int sb_dtype, int bits, int group_size, int64_t M,
                        int64_t N, int64_t K, void* y, int y_dtype, jq_stream_t stream) {
  int s = check_dense(x, x_dtype, codes, scales, biases, sb_dtype, bits, group_size, M, N, K, y,
                      y_dtype);
  if (s) return s;
  if (M == 0 || N == 0) return JQ_OK;
  hipStream_t st = (hipStream_t)stream;
  if (K == 0) {  // empty contraction: y = 0
    const int64_t n = M * N;
    fill_zero_kernel<<<(unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536), 256, 0, st>>>(
        y, n, jqh::dtype_size(y_dtype));
    return jqh::launch_status();
  }
  return dense_one(x, x_dtype, codes, scales, biases, sb_dtype, bits, group_size, M, N, K, y,
                   y_dtype, st);
}

// Workspace-taking form of jq_quantized_matmul: decode batches (5..64 rows) of long rows
// (K > 4096) split K over the matrix-core items and sum fp32 partials in the workspace.
static bool use_split(int64_t M, int64_t N, int64_t K, int bits, int gs, int xd, int sb) {
  const int Mi = (int)(M < (1 << 30) ? M : (1 << 30));
  return M > 4 && M <= kDecpMaxRows && !jqk::gemv_ok(Mi, K, N, bits, gs, xd, sb) &&
         jqk::dmx_split_workspace(Mi, K, N, bits, gs, xd, sb) > 0;
}

int64_t jq_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int bits,
                                           int group_size, int x_dtype, int sb_dtype) {
  if (M < 0 || N < 0 || K < 0) return -1;
  if (M > 0 && N > 0 && gemm16_shape(M, K, bits, group_size, x_dtype, sb_dtype))
    return jqk::gemm16_workspace(M, N, K, group_size);
  if (!use_split(M, N, K, bits, group_size, x_dtype, sb_dtype)) return 0;
  return jqk::dmx_split_workspace((int)M, K, N, bits, group_size, x_dtype, sb_dtype);
}

int jq_quantized_matmul_ws(const void* x, int x_dtype, const uint32_t* codes, const void* scales,
                           const void* biases, int sb_dtype, int bits, int group_size, int64_t M,
                           int64_t N, int64_t K, void* y, int y_dtype, void* workspace,
                           int64_t workspace_bytes, jq_stream_t stream) {
  int s = check_dense(x, x_dtype, codes, scales, biases, sb_dtype, bits, group_size, M, N, K, y,
                      y_dtype);
  if (s) return s;
  if (M > 0 && N > 0 && K > 0 &&
      use_gemm16(x, codes, scales, biases, M, K, bits, group_size, x_dtype, sb_dtype))
    return jqk::gemm16_launch(dense_problem(x, codes, scales, biases, M, N, K, y), bits,
                              group_size, x_dtype, sb_dtype, y_dtype, workspace, workspace_bytes,
                              (hipStream_t)stream);
  if (M == 0 || N == 0 || K == 0 || !use_split(M, N, K, bits, group_size, x_dtype, sb_dtype))
    return jq_quantized_matmul(x, x_dtype, codes, scales, biases, sb_dtype, bits, group_size, M,
                               N, K, y, y_dtype, stream);
  jqk::QmvBatch b;
  b.M = (int)M;
  b.K = (int)K;
  b.p[0].x = x; b.p[0].codes = codes; b.p[0].scales = scales; b.p[0].biases = biases;
  b.p[0].y = y; b.p[0].N = N;
  return jqk::dmx_split_launch(b, bits, group_size, x_dtype, sb_dtype, y_dtype, workspace,
                               workspace_bytes, (hipStream_t)stream);
}

int jq_quantized_matmul_multi(int count, const void* const* x, int x_dtype,
                              const uint32_t* const* codes, const void* const* scales,
                              const void* const* biases, int sb_dtype, const int* bits,
                              const int* group_size, const int64_t* M, const int64_t* N,
                              const int64_t* K, void* const* y, int y_dtype, jq_stream_t stream) {
  if (count < 0) return JQ_ERR_SHAPE;
  if (count == 0) return JQ_OK;
  if (!x || !codes || !scales || !biases || !bits || !group_size || !M || !N || !K || !y)
    return JQ_ERR_NULL;
  for (int i = 0; i < count; ++i) {
    int s = check_dense(x[i], x_dtype, codes[i], scales[i], biases[i], sb_dtype, bits[i],
                        group_size[i], M[i], N[i], K[i], y[i], y_dtype);
    if (s) return s;
  }
  hipStream_t st = (hipStream_t)stream;
  bool same = count <= jqk::kMaxProblems;
  for (int i = 1; i < count && same; ++i)
    same = bits[i] == bits[0] && group_size[i] == group_size[0] && M[i] == M[0] && K[i] == K[0];
  const int M0 = (int)(M[0] < (1 << 30) ? M[0] : (1 << 30));
  int64_t maxN = 0;
  for (int i = 0; i < count; ++i) maxN = N[i] > maxN ? N[i] : maxN;
  const bool gemv = same && prefer_gemv(M0, K[0], maxN, bits[0], group_size[0], x_dtype, sb_dtype);
  const bool q4 = same && !gemv && use_qmv4(M[0], K[0]) &&
                  jqk::qmv4_ok(M0, K[0], maxN, bits[0], group_size[0], x_dtype, sb_dtype);
  const bool dmx = same && !gemv && !q4 && M[0] <= kDecpMaxRows &&
                   jqk::dmx_ok(M0, K[0], maxN, bits[0], group_size[0], x_dtype, sb_dtype, 1);
  const bool dec = same && M[0] <= kDecpMaxRows && jqk::decp_ok(M0, K[0], maxN, x_dtype, sb_dtype);
  if (q4 || gemv || dmx || dec || (same && M[0] >= 1 && M[0] <= 4 && K[0] > 0)) {
    jqk::QmvBatch b;
    b.M = (int)M[0];
    b.K = (int)K[0];
    int n = 0;
    for (int i = 0; i < count; ++i) {
      if (N[i] == 0) continue;
      b.p[n].x = x[i];
      b.p[n].codes = codes[i];
      b.p[n].scales = scales[i];
      b.p[n].biases = biases[i];
      b.p[n].y = y[i];
      b.p[n].N = N[i];
      ++n;
    }
    if (gemv) return jqk::gemv_launch(b, n, bits[0], group_size[0], x_dtype, sb_dtype, y_dtype, st);
    if (q4) return jqk::qmv4_launch(b, n, bits[0], group_size[0], x_dtype, sb_dtype, y_dtype, st);
    if (dmx) return jqk::dmx_launch(b, n, bits[0], group_size[0], x_dtype, sb_dtype, y_dtype, st);
    if (dec) return jqk::decp_launch(b, n, bits[0], group_size[0], x_dtype, sb_dtype, y_dtype, st);
    return jqk::qmv_launch(b, n, bits[0], group_size[0], x_dtype, sb_dtype, y_dtype, st);
  }
  for (int i = 0; i < count; ++i) {
    int s = jq_quantized_matmul(x[i], x_dtype, codes[i], scales[i], biases[i], sb_dtype, bits[i],
                                group_size[i], M[i], N[i], K[i], y[i], y_dtype, stream);
    if (s) return s;
  }
  return JQ_OK;
}

}  // extern "C"
