/*
 * Bit-level C restatement of the JANG affine codec — TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (and nothing in the product) to cross-check the numpy oracle with an
 * independent algorithm: codes are read one bit at a time from the LSB-first row stream
 * (jang-tools/jang_tools/pack.py:85-149 defines the stream), dequantization rounds the
 * product and the sum separately (jang-tools/jang_tools/affine.py:458-463; this file is
 * compiled with -ffp-contract=off), and the GEMV accumulates in double.
 */
#include <stdint.h>
#include <string.h>

/* Bit `pos` of a little-endian uint32 word stream. */
static inline uint32_t bit_at(const uint32_t* w, int64_t pos) {
  return (w[pos >> 5] >> (pos & 31)) & 1u;
}

/* codes [rows, K] from packed [rows, K*bits/32]. */
void jqo_unpack(const uint32_t* w, int bits, int64_t rows, int64_t K, uint8_t* out) {
  const int64_t P = K * bits / 32;
  for (int64_t r = 0; r < rows; ++r) {
    const uint32_t* row = w + r * P;
    for (int64_t k = 0; k < K; ++k) {
      uint32_t v = 0;
      for (int b = 0; b < bits; ++b) v |= bit_at(row, k * bits + b) << b;
      out[r * K + k] = (uint8_t)v;
    }
  }
}

/* packed [rows, K*bits/32] from codes [rows, K] (values must fit `bits`). */
void jqo_pack(const uint8_t* codes, int bits, int64_t rows, int64_t K, uint32_t* w) {
  const int64_t P = K * bits / 32;
  memset(w, 0, (size_t)(rows * P) * sizeof(uint32_t));
  for (int64_t r = 0; r < rows; ++r) {
    uint32_t* row = w + r * P;
    for (int64_t k = 0; k < K; ++k) {
      for (int b = 0; b < bits; ++b) {
        const int64_t pos = k * bits + b;
        row[pos >> 5] |= (uint32_t)((codes[r * K + k] >> b) & 1u) << (pos & 31);
      }
    }
  }
}

/* out[r, k] = fl(fl(q * s) + b), s/b fp32 [rows, K/gs]. */
void jqo_dequant(const uint32_t* w, const float* s, const float* b, int bits, int gs,
                 int64_t rows, int64_t K, float* out) {
  const int64_t P = K * bits / 32, G = K / gs;
  for (int64_t r = 0; r < rows; ++r) {
    const uint32_t* row = w + r * P;
    for (int64_t k = 0; k < K; ++k) {
      uint32_t v = 0;
      for (int j = 0; j < bits; ++j) v |= bit_at(row, k * bits + j) << j;
      const float sc = s[r * G + k / gs], bi = b[r * G + k / gs];
      volatile float prod = (float)v * sc;
      out[r * K + k] = prod + bi;
    }
  }
}

/* y[m, n] = sum_k x[m, k] * W[n, k] in double (W already dequantized, fp32). */
void jqo_gemm_f64(const float* x, const float* W, int64_t M, int64_t N, int64_t K, double* y) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) acc += (double)x[m * K + k] * (double)W[n * K + k];
      y[m * N + n] = acc;
    }
}
