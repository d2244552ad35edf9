/*
 * ORACLE ONLY (test infrastructure): CPU restatement of the 4-bit group-64
 * quantized matmul. Not linked into, or called by, the product library.
 *
 * Layout (MLX affine, quant/quantize.py:71-75): row n of w is a little-endian
 * bit stream of 4-bit codes; code k sits at bits 4*(k%8) of word k/8
 * (engine/kernels.py:159-166). Dequant w = scale*q + bias per 64-wide group.
 */
#include <math.h>
#include <stdlib.h>
#include <stddef.h>
#include <string.h>

#include "oracle.h"

static inline float bf2f(uint16_t h) {
  uint32_t u = ((uint32_t)h) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* engine/kernels.py:121 (formula), experiments/native/qmv_spike.mm:118-124 (fp64 loop).
 * Each weight row is dequantized once into fp64 and dotted with every x row in
 * k order; rows are independent (OpenMP over n), so the result does not depend
 * on the thread count. */
void orc_qmv_w4g64_f64(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                       const uint16_t* biases, double* y, int M, int N, int K) {
  const int KW = K / 8, G = K / 64;
  double* xd = (double*)malloc(sizeof(double) * (size_t)M * K);
  for (size_t i = 0; i < (size_t)M * K; ++i) xd[i] = (double)bf2f(x[i]);
#pragma omp parallel
  {
    double* wrow = (double*)malloc(sizeof(double) * (size_t)K);
#pragma omp for schedule(static)
    for (int n = 0; n < N; ++n) {
      for (int k = 0; k < K; ++k) {
        const uint32_t q = (w[(size_t)n * KW + k / 8] >> (4 * (k % 8))) & 0xFu;
        const double s = bf2f(scales[(size_t)n * G + k / 64]);
        const double b = bf2f(biases[(size_t)n * G + k / 64]);
        wrow[k] = s * (double)q + b;
      }
      /* up to 8 x rows at a time: independent sums, each still in k order */
      for (int m0 = 0; m0 < M; m0 += 8) {
        const int mb = M - m0 < 8 ? M - m0 : 8;
        double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int k = 0; k < K; ++k) {
          const double wk = wrow[k];
          for (int j = 0; j < mb; ++j) acc[j] += wk * xd[(size_t)(m0 + j) * K + k];
        }
        for (int j = 0; j < mb; ++j) y[(size_t)(m0 + j) * N + n] = acc[j];
      }
    }
    free(wrow);
  }
  free(xd);
}

/* engine/kernels.py:146-172: per group d = sum q*x, acc += s*d + b*sum(x); fp32 */
void orc_qmv_w4g64_f32(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                       const uint16_t* biases, uint16_t* y, int M, int N, int K, int threads) {
  const int KW = K / 8, G = K / 64;
  /* x widened once, plus per-group sums */
  float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
  float* xs = (float*)malloc(sizeof(float) * (size_t)M * G);
  for (int m = 0; m < M; ++m)
    for (int g = 0; g < G; ++g) {
      float s = 0.0f;
      for (int i = 0; i < 64; ++i) {
        const float v = bf2f(x[(size_t)m * K + g * 64 + i]);
        xf[(size_t)m * K + g * 64 + i] = v;
        s += v;
      }
      xs[(size_t)m * G + g] = s;
    }
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int n = 0; n < N; ++n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint32_t* wr = w + (size_t)n * KW;
    for (int g = 0; g < G; ++g) {
      float q[64];
      for (int j = 0; j < 8; ++j) {
        const uint32_t word = wr[g * 8 + j];
        for (int i = 0; i < 8; ++i) q[j * 8 + i] = (float)((word >> (4 * i)) & 0xFu);
      }
      const float s = bf2f(scales[(size_t)n * G + g]);
      const float b = bf2f(biases[(size_t)n * G + g]);
      for (int m = 0; m < M && m < 8; ++m) {
        const float* xr = xf + (size_t)m * K + g * 64;
        float d = 0.0f;
        for (int i = 0; i < 64; ++i) d += q[i] * xr[i];
        acc[m] += s * d + b * xs[(size_t)m * G + g];
      }
    }
    for (int m = 0; m < M && m < 8; ++m) y[(size_t)m * N + n] = f2bf(acc[m]);
  }
  free(xf);
  free(xs);
}
