/*
 * jangq_amd — C ABI of the MI355X (gfx950) quantized-weight matmul path.
 *
 * Storage contract (JANG v2 / MLX affine, reference FORMAT.md:57-90, format/spec.py:6-30):
 *   codes   uint32 [rows, K*bits/32]   LSB-first bitstream of `bits`-bit codes along K
 *                                      (jang-tools/jang_tools/pack.py:12-149); 3/5/6-bit
 *                                      codes straddle word boundaries.
 *   scales  [rows, K/group_size]       bf16, f16 or f32 (JQ_BF16 / JQ_F16 / JQ_F32)
 *   biases  [rows, K/group_size]       same dtype as scales
 *   w[r,k] = fl(fl(q[r,k] * scale[r,k/gs]) + bias[r,k/gs])   in fp32
 *                                      (jang-tools/jang_tools/affine.py:445-463)
 *   bits in {2,3,4,5,6,8}, group_size in {32,64,128}, K % group_size == 0.
 *   3-D expert stacks are [E, rows, ...] and contiguous.
 *
 * Conventions
 *   - Every pointer argument is caller-owned device memory (except where noted as host).
 *     No entry point allocates device memory, synchronises the stream or keeps state
 *     between calls, except the documented workspace arguments.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL is the default stream).
 *   - Return value: JQ_OK (0) or a negative JQ_ERR_* code. Nothing throws across the ABI.
 *     Shapes, bits, group sizes and dtypes are validated on the host before any launch.
 */
#ifndef JANGQ_AMD_H
#define JANGQ_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* jq_stream_t; /* == hipStream_t */

#define JQ_ABI_VERSION 2

enum jq_status {
  JQ_OK = 0,
  JQ_ERR_BITS = -1,        /* bits not in {2,3,4,5,6,8} */
  JQ_ERR_GROUP_SIZE = -2,  /* group_size not in {32,64,128} or K % group_size != 0 */
  JQ_ERR_SHAPE = -3,       /* a dimension is negative, too large or inconsistent */
  JQ_ERR_DTYPE = -4,       /* unsupported dtype code for this argument */
  JQ_ERR_NULL = -5,        /* a required pointer is NULL while its extent is non-zero */
  JQ_ERR_LAUNCH = -6,      /* the HIP runtime reported an error at launch */
  JQ_ERR_WORKSPACE = -7,   /* workspace missing or smaller than the size query returned */
  JQ_ERR_INDEX = -8,       /* an index argument is out of range (checked where cheap) */
};

enum jq_dtype {
  JQ_F32 = 0,
  JQ_BF16 = 1,
  JQ_F16 = 2,
};

/* ABI version of the loaded library (JQ_ABI_VERSION at build time). */
int jq_abi_version(void);

/* Static string for a status code. */
const char* jq_status_string(int status);

/*
 * Unpack codes to one uint8 per element: out[r, k] = q[r, k].
 * Replaces jang-tools/jang_tools/pack.py:85-149 (unpack_bits) applied to a packed uint32
 * matrix viewed as bytes (affine.py:457).
 */
int jq_unpack(const uint32_t* codes, int bits, int64_t rows, int64_t K,
              uint8_t* out, jq_stream_t stream);

/*
 * Dequantize: out[r, k] = fl(fl(q*s) + b) in fp32, stored as out_dtype (bf16/f16 are the
 * round-to-nearest-even of that fp32 value). Bit-exact with the fp32 reference.
 * Replaces jang-tools/jang_tools/affine.py:445-463 (dequantize_affine_numpy) and the
 * mx.dequantize call at jang-tools/jang_tools/loader.py:469.
 */
int jq_dequantize(const uint32_t* codes, const void* scales, const void* biases,
                  int sb_dtype, int bits, int group_size, int64_t rows, int64_t K,
                  void* out, int out_dtype, jq_stream_t stream);

/*
 * Affine group quantization with MLX's rule (dominant edge, signed scale, eps 1e-7,
 * round-half-even), codes packed LSB-first. w_dtype is the source dtype (converted to fp32
 * exactly). sb_dtype: JQ_BF16 (MLX runtime sidecars), JQ_F16 (converter sidecars, with the
 * non-zero f16 scale guard) or JQ_F32.
 * Replaces jang-tools/jang_tools/affine.py:193-276 (quantize_native_affine_numpy, the CPU
 * mirror of mx.quantize) as called from jang-tools/jang_tools/convert.py:602-645.
 */
int jq_quantize(const void* w, int w_dtype, int bits, int group_size, int64_t rows,
                int64_t K, uint32_t* codes, void* scales, void* biases, int sb_dtype,
                jq_stream_t stream);

/*
 * Lossless expansion of 1-bit storage codes to 2-bit runtime codes: `words` uint32 words of an
 * LSB-first 1-bit stream (32 codes each) become 2*words words of the 2-bit stream of the same
 * codes (scales and biases are unchanged). Rows stay rows: a [rows, K/32] 1-bit matrix becomes
 * [rows, K/16].
 * Replaces jang-tools/jang_tools/affine.py:402-416 (expand_packed_1bit_to_2bit_numpy / _mlx),
 * applied per shard at load time by affine.py:527-544.
 */
int jq_expand_1bit_to_2bit(const uint32_t* src, int64_t words, uint32_t* dst,
                           jq_stream_t stream);

/*
 * y[M, N] = x[M, K] @ dequant(W)[N, K]^T  (transpose=True), fp32 accumulation.
 * x_dtype: JQ_BF16 / JQ_F16 / JQ_F32; y_dtype likewise (MLX returns x.dtype).
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits) as
 * called from jang-tools/jang_tools/jangrt/linear.py:41-45 and
 * jang-tools/jang_tools/dots3/ops.py:44-51. Small M runs the decode GEMV kernels, larger
 * M the matrix-core GEMM; from 384 rows the f16 prefill GEMM, whose f16 activation copy this
 * entry point takes from a stream-ordered allocation (hipMallocAsync / hipFreeAsync on
 * `stream`; jq_quantized_matmul_ws takes it from the caller instead).
 */
int jq_quantized_matmul(const void* x, int x_dtype, const uint32_t* codes,
                        const void* scales, const void* biases, int sb_dtype, int bits,
                        int group_size, int64_t M, int64_t N, int64_t K, void* y,
                        int y_dtype, jq_stream_t stream);

/*
 * jq_quantized_matmul with a caller workspace (same reference call: mx.quantized_matmul at
 * jang-tools/jang_tools/jangrt/linear.py:41-45). Decode batches of long rows (5..64 rows,
 * K > 4096) split K over the matrix-core kernel and sum fp32 partials in the workspace
 * (a smaller workspace returns JQ_ERR_WORKSPACE). Prefill shapes (384 rows and more, group
 * size 64 or 128) hold their activations as f16 rows in the workspace (M*K*2 bytes plus
 * 4 bytes per row of x and of W); a smaller workspace runs the rows in passes of whole
 * 256-row tiles, and one below 256 rows' worth returns JQ_ERR_WORKSPACE. Every other shape
 * runs exactly as jq_quantized_matmul. The size query returns the bytes for one pass (0: no
 * workspace used, -1: invalid sizes).
 */
int64_t jq_quantized_matmul_workspace_size(int64_t M, int64_t N, int64_t K, int bits,
                                           int group_size, int x_dtype, int sb_dtype);
int jq_quantized_matmul_ws(const void* x, int x_dtype, const uint32_t* codes,
                           const void* scales, const void* biases, int sb_dtype, int bits,
                           int group_size, int64_t M, int64_t N, int64_t K, void* y,
                           int y_dtype, void* workspace, int64_t workspace_bytes,
                           jq_stream_t stream);

/*
 * jq_quantized_matmul_ws without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid it); it has no
 * counterpart in the reference. The K-split partials of decode batches of long rows and the
 * prefill GEMM's f16 activation rows go to a fixed array inside the library,
 * JQ_NOALLOC_SCRATCH_BYTES per GPU, held from the first call on a GPU until the process ends;
 * a K-split shape that needs more returns JQ_ERR_WORKSPACE (the size query
 * jq_quantized_matmul_workspace_size tells it beforehand), a prefill shape runs in passes of
 * rows that fit. Every other shape runs as jq_quantized_matmul. It calls no allocator. Calls that overlap on one GPU (other streams or
 * threads) share the array and race; the array keeps the last call's contents, and each call
 * writes every partial it reads.
 */
#define JQ_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)
int jq_quantized_matmul_noalloc(const void* x, int x_dtype, const uint32_t* codes,
                                const void* scales, const void* biases, int sb_dtype, int bits,
                                int group_size, int64_t M, int64_t N, int64_t K, void* y,
                                int y_dtype, jq_stream_t stream);

/*
 * Grouped form of jq_quantized_matmul: `count` independent problems sharing x_dtype,
 * y_dtype and sb_dtype, in ONE launch when they share M, K, bits and group_size (q/k/v or
 * gate/up projections of one token batch). Each array has `count` entries.
 * No reference counterpart as one call: it replaces `count` consecutive
 * mx.quantized_matmul calls on the same x (jang-tools/jang_tools/dots3/ops.py:79-93).
 */
int jq_quantized_matmul_multi(int count, const void* const* x, int x_dtype,
                              const uint32_t* const* codes, const void* const* scales,
                              const void* const* biases, int sb_dtype, const int* bits,
                              const int* group_size, const int64_t* M, const int64_t* N,
                              const int64_t* K, void* const* y, int y_dtype,
                              jq_stream_t stream);

/*
 * OCP MX modes as MLX stores them (mode "mxfp4" = 4, "mxfp8" = 8; group size 32, no biases):
 *   W[n, k] = value(code[n, k]) * 2^(scales[n, k/32] - 127)
 *   codes   uint32 [rows, K*mode/32], little-endian bytes: mxfp4 two E2M1 codes per byte
 *           (element 2i in the low nibble), mxfp8 one E4M3 (FN) byte per element
 *   scales  uint8 [rows, K/32] E8M0 exponents (255 = NaN)
 * jq_mx_dequantize writes W (out_dtype; exact in fp32). jq_mx_quantized_matmul computes
 * y[M, N] = x[M, K] @ W^T (x bf16/f16, fp32 accumulation, K <= 16384) as decode GEMVs, one
 * launch per activation row. Replace mx.dequantize / mx.quantized_matmul with mode
 * "mxfp4"/"mxfp8", the modes the loader switches a module to when its scales are uint8
 * (jang-tools/jang_tools/loader.py:1877-1912); format per
 * jang-tools/jang_tools/mimo_v2/mxfp4_codec.py:1-50.
 */
int jq_mx_dequantize(const uint32_t* codes, const uint8_t* scales, int mode, int64_t rows,
                     int64_t K, void* out, int out_dtype, jq_stream_t stream);
int jq_mx_quantized_matmul(const void* x, int x_dtype, const uint32_t* codes,
                           const uint8_t* scales, int mode, int64_t M, int64_t N, int64_t K,
                           void* y, int y_dtype, jq_stream_t stream);

/*
 * gather_qmm over MX-mode expert stacks (codes [E, N, K*mode/32], E8M0 scales uint8
 * [E, N, K/32], no biases; format as jq_mx_dequantize): out[i*M + m] = x[lhs[i]*M + m] @
 * W[rhs[i]]^T for pairs i < n_pairs and rows m < M (lhs NULL: i). x [x_batch, M, K] bf16/f16,
 * out [n_pairs, M, N]; n_pairs * M < 65536. A pair whose expert id is >= E is not written.
 * Replaces mx.gather_qmm(..., mode="mxfp4"/"mxfp8") as called from
 * jang-tools/jang_tools/dots3/ops.py:181-188 on the expert stacks the loader switches to an
 * MX mode (jang-tools/jang_tools/loader.py:1866-1912).
 */
int jq_mx_gather_qmm(const void* x, int x_dtype, int64_t x_batch, int64_t M,
                     const uint32_t* codes, const uint8_t* scales, int mode, int64_t E,
                     int64_t N, int64_t K, const uint32_t* lhs, const uint32_t* rhs,
                     int64_t n_pairs, void* out, int y_dtype, jq_stream_t stream);

/*
 * Elementwise SwiGLU of two projections already rounded to dtype: h = round(silu(g) * u),
 * with the clamp gate = min(g, L), up = clip(u, -L, L) when swiglu_limit > 0.
 * No MLX operator as one call: silu(gate) * up of mlx_lm SwitchGLU (restated at
 * jang-tools/jang_tools/dots3/ops.py:215) and jang-tools/jang_tools/dsv41/model.py:1214-1219.
 */
int jq_swiglu(const void* g, const void* u, int64_t n, float swiglu_limit, void* h, int dtype,
              jq_stream_t stream);

/*
 * Router: probs = softmax(logits) in fp32 (max-subtracted, "precise"), top-k expert ids
 * per token (ties -> lower id first), weights = their probabilities, optionally divided
 * by their sum (norm_topk_prob). logits f32 [T, E]; idx uint32 [T, k]; weights f32 [T, k].
 * Ids are written in descending-probability order.
 * Replaces the caller-side routing of jang-tools/jang_tools/qwen4_exp/modeling.py:587-593
 * (softmax(precise=True) -> argpartition -> take_along_axis -> renorm).
 */
int jq_moe_route(const float* logits, int64_t T, int64_t E, int k, int renorm,
                 uint32_t* idx, float* weights, jq_stream_t stream);

/*
 * Router options (jq_moe_route_ex, jq_moe_block). A NULL options pointer means softmax scores
 * with renormalisation (norm_topk_prob), no bias, no groups, scaling 1.
 *   score       JQ_SCORE_SOFTMAX      softmax(logits) in fp32, max-subtracted
 *                                     (jang-tools/jang_tools/qwen4_exp/modeling.py:587-593,
 *                                     jang-tools/jang_tools/mistral4_mlx.py:359-387)
 *               JQ_SCORE_SIGMOID      sigmoid(logits) (jang-tools/jang_tools/dots3/ops.py:149-162,
 *                                     jang-tools/jang_tools/laguna/model.py:50-62)
 *               JQ_SCORE_SQRTSOFTPLUS sqrt(softplus(logits)) (jang-tools/jang_tools/dsv41/model.py:1184-1190)
 *   score_bias  f32 [E] device array added to the scores for the selection only
 *               (e_score_correction_bias); the weights are the unbiased scores
 *   n_group, topk_group  group-limited selection (n_group > 1, E % n_group == 0, n_group <= 64):
 *               the topk_group groups of E/n_group consecutive experts with the largest
 *               maximum selection value are kept; every other expert gets selection value 0
 *               and score 0 (mistral4_mlx.py:363-375)
 *   renorm      weights /= (sum of the k weights + renorm_eps): 0 for the softmax routers,
 *               1e-20 for the sigmoid-type ones (dots3/ops.py:160, laguna/model.py:59)
 *   scaling     routed_scaling_factor, multiplies the weights last (mistral4_mlx.py:383-385)
 * The k experts come in descending selection order, ties to the lower expert id.
 */
enum jq_score_func {
  JQ_SCORE_SOFTMAX = 0,
  JQ_SCORE_SIGMOID = 1,
  JQ_SCORE_SQRTSOFTPLUS = 2,
};

typedef struct jq_route_opts {
  int score;
  int renorm;
  float renorm_eps;
  float scaling;
  const float* score_bias;
  int n_group;
  int topk_group;
} jq_route_opts;

/*
 * jq_moe_route with the router options above: logits [T, E] of logits_dtype (JQ_F32, or the
 * bf16 / f16 output of the router linear, read exactly) -> idx uint32 [T, k] and weights f32
 * [T, k]; scores and weights are computed in fp32. E <= 4096, k <= 64.
 * Replaces the router functions cited at jq_route_opts.
 */
int jq_moe_route_ex(const void* logits, int logits_dtype, int64_t T, int64_t E, int k,
                    const jq_route_opts* opts, uint32_t* idx, float* weights, jq_stream_t stream);

/*
 * Workspace bytes needed by jq_gather_qmm for n_pairs (token, expert) pairs over E experts
 * with M activation rows per pair (jq_switch_glu: M = 1, n_pairs = T*k). Host-only.
 * Returns -1 for invalid arguments.
 */
int64_t jq_gather_workspace_size(int64_t n_pairs, int64_t E, int64_t M);

/*
 * out[i] = x[lhs[i]] @ dequant(W[rhs[i]])^T for i < n_pairs.
 *   x     [x_batch, M, K]   (x_dtype)
 *   W     codes [E, N, K*bits/32], scales/biases [E, N, K/gs]
 *   lhs   uint32 [n_pairs] (NULL means lhs[i] = i, x_batch must be >= n_pairs)
 *   rhs   uint32 [n_pairs] expert ids (< E)
 *   out   [n_pairs, M, N]  (y_dtype)
 * Pairs are grouped by expert on the device so each selected expert's packed weights are
 * streamed once per call whatever the order of rhs; `sorted_indices` is accepted for
 * signature parity and changes nothing (the device grouping is always exact). Pairs whose
 * expert id is >= E are skipped (their output rows are not written).
 * Replaces mx.gather_qmm(x, w, scales, biases, lhs_indices, rhs_indices, transpose=True,
 * group_size, bits, sorted_indices) as called from jang-tools/jang_tools/dsv41/model.py:855-857
 * and jang-tools/jang_tools/dots3/ops.py:168-192.
 */
int jq_gather_qmm(const void* x, int x_dtype, int64_t x_batch, int64_t M,
                  const uint32_t* codes, const void* scales, const void* biases,
                  int sb_dtype, int bits, int group_size, int64_t E, int64_t N, int64_t K,
                  const uint32_t* lhs, const uint32_t* rhs, int64_t n_pairs,
                  int sorted_indices, void* out, int y_dtype, void* workspace,
                  int64_t workspace_bytes, jq_stream_t stream);

/*
 * SwitchGLU over stacked experts: for every (token t, slot j) pair with e = idx[t, j]:
 *   h = silu(x[t] @ Wg[e]^T) * (x[t] @ Wu[e]^T)     (each projection rounded to y_dtype
 *                                                    first, as three gather_qmm calls do)
 *   out[t, j] = h @ Wd[e]^T
 * x [T, H] (x_dtype); idx uint32 [T, k]; out [T, k, H] (y_dtype).
 * gate/up codes [E, I, H*bits_gu/32], scales/biases [E, I, H/gs];
 * down codes [E, H, I*bits_d/32], scales/biases [E, H, I/gs].
 * h_buf: caller scratch of T*k*I elements of y_dtype (the SwiGLU activations).
 * One grouped launch computes gate+up+SwiGLU for all active experts, a second the down
 * projection. Replaces mlx_lm SwitchGLU.__call__ as restated at
 * jang-tools/jang_tools/dots3/ops.py:195-223 and jang-tools/jang_tools/jangrt/switchglu_decode.py:161-183
 * (both the sorted and unsorted branches compute the same values).
 */
int jq_switch_glu(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                  const uint32_t* idx, int k,
                  const uint32_t* gate_codes, const void* gate_scales, const void* gate_biases,
                  const uint32_t* up_codes, const void* up_scales, const void* up_biases,
                  int bits_gu,
                  const uint32_t* down_codes, const void* down_scales, const void* down_biases,
                  int bits_d, int sb_dtype, int group_size, void* h_buf, void* out,
                  int y_dtype, void* workspace, int64_t workspace_bytes, jq_stream_t stream);

/*
 * Weighted combine of the routed experts' outputs (and the shared expert's):
 *   out[t, :] = round(sum_j w[t, j] * y[t, j, :])        fp32 in slot order j = 0 .. k-1
 *   out[t, :] = round(out[t, :] + shared[t, :])           if shared != NULL
 * y [T, k, H], shared [T, H] and out [T, H] of `dtype` (JQ_BF16 / JQ_F16 / JQ_F32); w f32 [T, k].
 * No MLX operator: one launch for the caller-side composition (y * scores[..., None]).sum(-2)
 * (+ shared_expert(x)) of jang-tools/jang_tools/qwen4_exp/modeling.py:594-597, with the same
 * two roundings as those array operations.
 */
int jq_moe_combine(const void* y, const float* w, const void* shared, int64_t T, int k,
                   int64_t H, void* out, int dtype, jq_stream_t stream);

/*
 * SwitchGLU followed by the weighted combine, one call for the routed part of a MoE block:
 *   out[t, :] = jq_moe_combine(jq_switch_glu(x, idx)[t, :, :], weights[t, :], shared[t, :])
 * with the same values and roundings as those two calls (y_buf [T, k, H] of y_dtype is the
 * caller scratch for the per-slot expert outputs, weights f32 [T, k], shared [T, H] or NULL,
 * out [T, H]). At decode sizes the combine runs inside the down-projection launch (one block
 * sums a row's k expert outputs in slot order), so the routed experts take two launches and
 * y_buf is not written; elsewhere it is the two calls. An expert id >= E contributes 0 in the
 * fused form (jq_switch_glu leaves such rows unwritten).
 * Replaces the routed half of the fused affine MoE decode of
 * jang-tools/jang_tools/dsv41/metal_decode.py:334-503 (gate|up and down+combine dispatches)
 * and the caller-side composition of jang-tools/jang_tools/qwen4_exp/modeling.py:594-597.
 */
int jq_switch_glu_combine(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I,
                          int64_t E, const uint32_t* idx, const float* weights, int k,
                          const uint32_t* gate_codes, const void* gate_scales,
                          const void* gate_biases, const uint32_t* up_codes,
                          const void* up_scales, const void* up_biases, int bits_gu,
                          const uint32_t* down_codes, const void* down_scales,
                          const void* down_biases, int bits_d, int sb_dtype, int group_size,
                          void* h_buf, void* y_buf, const void* shared, void* out, int y_dtype,
                          void* workspace, int64_t workspace_bytes, jq_stream_t stream);

/*
 * Routing plus the routed experts of a MoE block: jq_moe_route(logits -> idx, weights), then
 * jq_switch_glu_combine with them; idx uint32 [T, k] and weights f32 [T, k] are outputs (the
 * same values jq_moe_route writes), logits f32 [T, E]. At decode sizes (E <= 512) the gate|up
 * launch computes each token's top-k itself, so routing, gate|up and down+combine take two
 * launches instead of three.
 * Replaces qwen4_exp/modeling.py:587-597 after the router GEMV (jang-tools/jang_tools), the
 * dispatches of dsv41/metal_decode.py:334-503.
 */
int jq_moe_experts(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E,
                   const float* logits, int k, int renorm, uint32_t* idx, float* weights,
                   const uint32_t* gate_codes, const void* gate_scales, const void* gate_biases,
                   const uint32_t* up_codes, const void* up_scales, const void* up_biases,
                   int bits_gu, const uint32_t* down_codes, const void* down_scales,
                   const void* down_biases, int bits_d, int sb_dtype, int group_size,
                   void* h_buf, void* y_buf, const void* shared, void* out, int y_dtype,
                   void* workspace, int64_t workspace_bytes, jq_stream_t stream);

/*
 * SwiGLU projection pair of a dense MLP: h = silu(round(x @ Wg^T)) * round(x @ Wu^T), each
 * product rounded to y_dtype first (as two quantized_matmul calls returning y_dtype give),
 * h rounded to y_dtype. Gate and up share bits, group size, N and K.
 * up_buf: caller scratch of M*N elements of y_dtype, required when M is above the decode
 * sizes (M > 4; 2-bit: M > 2); NULL is accepted for decode sizes (one launch, no scratch).
 * At 5..64 rows with K <= 4096, group size 64 or 128 and x and scales of one 16-bit dtype,
 * for 8-bit codes or at most 16 / (128 / group_size) rows, the pair also runs as one launch
 * (matrix-core kernel with the SiLU * up epilogue) and leaves up_buf untouched.
 * No MLX operator as one call: replaces gate_proj(x), up_proj(x) and silu(g) * u of the
 * shared-expert MLP (jang-tools/jang_tools/qwen4_exp/modeling.py:597,
 * jang-tools/jang_tools/dsv41/metal_decode.py:355-371 for the shared slot).
 */
int jq_quantized_swiglu(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                        const uint32_t* gate_codes, const void* gate_scales,
                        const void* gate_biases, const uint32_t* up_codes,
                        const void* up_scales, const void* up_biases, int sb_dtype, int bits,
                        int group_size, void* h, void* up_buf, int y_dtype,
                        jq_stream_t stream);

/*
 * jq_quantized_swiglu with the SwiGLU clamp of the fused MoE decode: with swiglu_limit > 0,
 * gate = min(round(g), L) and up = clip(round(u), -L, L) before silu(gate) * up
 * (jang-tools/jang_tools/dsv41/model.py:1239-1244 for the shared expert,
 * jang-tools/jang_tools/dsv41/metal_decode.py:362-366).
 */
int jq_quantized_swiglu_ex(const void* x, int x_dtype, int64_t M, int64_t N, int64_t K,
                           const uint32_t* gate_codes, const void* gate_scales,
                           const void* gate_biases, const uint32_t* up_codes,
                           const void* up_scales, const void* up_biases, int sb_dtype, int bits,
                           int group_size, float swiglu_limit, void* h, void* up_buf,
                           int y_dtype, jq_stream_t stream);

/* A quantized weight: 2-D [rows, K*bits/32], or an expert stack [E, rows, K*bits/32]. */
typedef struct jq_qweight {
  const uint32_t* codes;
  const void* scales;  /* [.., rows, K/group_size] of sb_dtype */
  const void* biases;  /* same shape and dtype */
  int sb_dtype;
  int bits;
  int group_size;
} jq_qweight;

/*
 * Where the routing weights enter a MoE block:
 *   JQ_COMBINE_AFTER_DOWN   out = round(round(sum_j w_j * y_j) + s')   (mlx_lm / qwen-style:
 *       jang-tools/jang_tools/qwen4_exp/modeling.py:594-599), y_j = round(down_j(h_j)),
 *       h_j = round(silu(g_j) * u_j); s' = round(round(sigmoid(gate_logit)) * s) with a shared
 *       gate, else s; the weighted sum is fp32 in slot order
 *   JQ_COMBINE_BEFORE_DOWN  h_j = round(silu(g_j) * u_j * w_j), out = round(sum_j y_j + s)
 *       (fp32, slot order; jang-tools/jang_tools/dsv41/model.py:1214-1245 and its two-dispatch
 *       fusion, dsv41/metal_decode.py:334-503)
 * where g_j, u_j are rounded to the activation dtype (and clamped with swiglu_limit > 0), and
 * s = round(down_s(round(silu(g_s) * u_s))) is the shared expert's output (same clamp).
 */
enum jq_moe_combine_mode {
  JQ_COMBINE_AFTER_DOWN = 0,
  JQ_COMBINE_BEFORE_DOWN = 1,
};

typedef struct jq_moe_opts {
  int combine;         /* jq_moe_combine_mode */
  float swiglu_limit;  /* > 0: the SwiGLU clamp, routed and shared experts */
} jq_moe_opts;

/*
 * Bytes of the caller workspace of jq_moe_block (-1: invalid sizes). Host-only.
 */
int64_t jq_moe_block_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int k,
                                    int64_t shared_I, int x_dtype);

/*
 * A whole MoE block after the router GEMV: routing (jq_route_opts), the routed experts
 * (SwitchGLU over gate/up/down stacks [E, I, H*b/32], [E, I, H*b/32], [E, H, I*b/32], one group
 * size), an optional shared expert (dense SwiGLU MLP of intermediate size shared_I; NULL
 * weights when shared_I == 0) with an optional sigmoid gate (shared_gate_logits [T] of x_dtype:
 * the output of the 1-row shared_expert_gate linear), and the combine of jq_moe_combine_mode.
 * x [T, H] bf16/f16; logits [T, E] of logits_dtype; outputs idx uint32 [T, k], weights f32 [T, k] (as
 * jq_moe_route_ex writes them) and out [T, H] of x_dtype. E <= 4096, k <= 64.
 * At decode sizes the routed experts take two launches (gate|up routing for itself, then down
 * with the combine inside).
 * Replaces the MoE block bodies of jang-tools/jang_tools/qwen4_exp/modeling.py:586-599,
 * jang-tools/jang_tools/dsv41/model.py:1166-1245 (with dsv41/metal_decode.py:334-503),
 * jang-tools/jang_tools/mistral4_mlx.py:355-387 and jang-tools/jang_tools/dots3/ops.py:149-223
 * after their router GEMV.
 */
int jq_moe_block(const void* x, int x_dtype, int64_t T, int64_t H, int64_t I, int64_t E, int k,
                 const void* logits, int logits_dtype, const jq_route_opts* route,
                 const jq_qweight* gate,
                 const jq_qweight* up, const jq_qweight* down, int64_t shared_I,
                 const jq_qweight* shared_gate_proj, const jq_qweight* shared_up_proj,
                 const jq_qweight* shared_down_proj, const void* shared_gate_logits,
                 const jq_moe_opts* opts, uint32_t* idx, float* weights, void* out,
                 void* workspace, int64_t workspace_bytes, jq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JANGQ_AMD_H */
