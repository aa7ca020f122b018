/*
 * Plain-C brute-force GEMM and IEEE decoding -- TEST INFRASTRUCTURE ONLY.
 * Used by tests/ to pin oracle/gemm_oracle.py independently of numpy/BLAS.
 *
 *   oracle_gemm_f64: C[m*ldc+n] = sum_{k ascending} A[m*lda+k] * B(k, n), where
 *     B(k, n) = B[k*ldb+n] (layout 0, the reference's [K,N] operand,
 *     src/cuda/fp16_matmul.cu:311-313) or B[n*ldb+k] (layout 1, the Linear
 *     weight [N,K], src/main.cpp:172-182).  Triple loop, one double accumulator.
 *   oracle_f16_bits_to_f64 / oracle_bf16_bits_to_f64: decode binary16 and
 *     bfloat16 bit patterns from the IEEE 754 field definitions.
 *   oracle_f64_to_bf16_bits: round a binary32 value to bfloat16, nearest even.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

void oracle_gemm_f64(int layout, const double* A, int64_t lda, const double* B, int64_t ldb, double* C,
                     int64_t ldc, int M, int N, int K) {
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      double s = 0.0;
      for (int k = 0; k < K; ++k) {
        const double b = layout == 0 ? B[(int64_t)k * ldb + n] : B[(int64_t)n * ldb + k];
        s += A[(int64_t)m * lda + k] * b;
      }
      C[(int64_t)m * ldc + n] = s;
    }
  }
}

double oracle_f16_bits_to_f64(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int exp = (h >> 10) & 0x1F;
  const int man = h & 0x3FF;
  double v;
  if (exp == 0) {
    v = ldexp((double)man, -24); /* subnormal: man * 2^-14 * 2^-10 */
  } else if (exp == 31) {
    v = man ? NAN : INFINITY;
  } else {
    v = ldexp((double)(man | 0x400), exp - 25); /* (1.man) * 2^(exp-15) */
  }
  return sign ? -v : v;
}

double oracle_bf16_bits_to_f64(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int exp = (h >> 7) & 0xFF;
  const int man = h & 0x7F;
  double v;
  if (exp == 0) {
    v = ldexp((double)man, -133); /* man * 2^-126 * 2^-7 */
  } else if (exp == 255) {
    v = man ? NAN : INFINITY;
  } else {
    v = ldexp((double)(man | 0x80), exp - 134); /* (1.man) * 2^(exp-127) */
  }
  return sign ? -v : v;
}

uint16_t oracle_f32_to_bf16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}
