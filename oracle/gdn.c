/*
 * ORACLE ONLY (test infrastructure): CPU restatement of the Gated DeltaNet
 * recurrence, following engine/kernels.py:34-63 operation by operation:
 *   x = a + dt_bias; sp = x > 20 ? x : log(1 + exp(x)); g = exp(-exp(A_log) * sp)
 *   beta = 1 / (1 + exp(-b)); S *= g; kv = S.k; delta = (v - kv) * beta;
 *   S += k * delta; y = S.q
 * with GQA head hk = hv / (Hv / Hk) (engine/kernels.py:15).
 * Snapshot t is the state after token t (the reference keeps only the one
 * before the last token, engine/kernels.py:69-75; here every token's is kept).
 */
#include <math.h>
#include <stddef.h>

#include "oracle.h"

void orc_gated_delta_f64(const float* q, const float* k, const float* v, const float* a,
                         const float* b, const float* A_log, const float* dt_bias,
                         double* state, double* y, double* snaps,
                         int B, int T, int Hk, int Hv, int Dk, int Dv) {
  const int rep = Hv / Hk;
  for (int bi = 0; bi < B; ++bi)
    for (int hv = 0; hv < Hv; ++hv) {
      const int hk = hv / rep;
      const double A = exp((double)A_log[hv]);
      const double dt = dt_bias[hv];
      for (int dv = 0; dv < Dv; ++dv) {
        double* st = state + (((size_t)bi * Hv + hv) * Dv + dv) * Dk;
        for (int t = 0; t < T; ++t) {
          const size_t qk_off = (((size_t)bi * T + t) * Hk + hk) * Dk;
          const size_t g_off = ((size_t)bi * T + t) * Hv + hv;
          const double xx = (double)a[g_off] + dt;
          const double sp = xx > 20.0 ? xx : log(1.0 + exp(xx));
          const double g = exp(-A * sp);
          const double beta = 1.0 / (1.0 + exp(-(double)b[g_off]));
          double kv = 0.0;
          for (int i = 0; i < Dk; ++i) {
            st[i] *= g;
            kv += st[i] * (double)k[qk_off + i];
          }
          const double delta = ((double)v[(((size_t)bi * T + t) * Hv + hv) * Dv + dv] - kv) * beta;
          double o = 0.0;
          for (int i = 0; i < Dk; ++i) {
            st[i] += (double)k[qk_off + i] * delta;
            o += st[i] * (double)q[qk_off + i];
          }
          y[(((size_t)bi * T + t) * Hv + hv) * Dv + dv] = o;
          if (snaps) {
            double* sn = snaps + ((((size_t)t * B + bi) * Hv + hv) * Dv + dv) * Dk;
            for (int i = 0; i < Dk; ++i) sn[i] = st[i];
          }
        }
      }
    }
}

void orc_gated_delta_f32(const float* q, const float* k, const float* v, const float* a,
                         const float* b, const float* A_log, const float* dt_bias,
                         float* state, float* y, float* snaps,
                         int B, int T, int Hk, int Hv, int Dk, int Dv, int threads) {
  const int rep = Hv / Hk;
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads > 0 ? threads : 1)
  for (int bi = 0; bi < B; ++bi)
    for (int hv = 0; hv < Hv; ++hv) {
      const int hk = hv / rep;
      const float A = expf(A_log[hv]);
      const float dt = dt_bias[hv];
      for (int dv = 0; dv < Dv; ++dv) {
        float* st = state + (((size_t)bi * Hv + hv) * Dv + dv) * Dk;
        for (int t = 0; t < T; ++t) {
          const size_t qk_off = (((size_t)bi * T + t) * Hk + hk) * Dk;
          const size_t g_off = ((size_t)bi * T + t) * Hv + hv;
          const float xx = a[g_off] + dt;
          const float sp = xx > 20.0f ? xx : logf(1.0f + expf(xx));
          const float g = expf(-A * sp);
          const float beta = 1.0f / (1.0f + expf(-b[g_off]));
          float kv = 0.0f;
          for (int i = 0; i < Dk; ++i) {
            st[i] *= g;
            kv += st[i] * k[qk_off + i];
          }
          const float delta = (v[(((size_t)bi * T + t) * Hv + hv) * Dv + dv] - kv) * beta;
          float o = 0.0f;
          for (int i = 0; i < Dk; ++i) {
            st[i] += k[qk_off + i] * delta;
            o += st[i] * q[qk_off + i];
          }
          y[(((size_t)bi * T + t) * Hv + hv) * Dv + dv] = o;
          if (snaps) {
            float* sn = snaps + ((((size_t)t * B + bi) * Hv + hv) * Dv + dv) * Dk;
            for (int i = 0; i < Dk; ++i) sn[i] = st[i];
          }
        }
      }
    }
}
