/*
 * CPU restatement of the reference's hot-path arithmetic (test infrastructure).
 *
 * ORACLE ONLY: this library is the checker for the HIP kernels of libqvex.so.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it;
 * the product path never does.
 *
 * bf16 values are uint16_t bit patterns, as in include/qvex.h.
 */
#ifndef QVEX_ORACLE_H
#define QVEX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* y[m,n] = sum_k x[m,k] * (s[n,k/64] * q[n,k] + b[n,k/64]) in fp64
 * (engine/kernels.py:121-125, experiments/native/qmv_spike.mm:115-125). */
void orc_qmv_w4g64_f64(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                       const uint16_t* biases, double* y, int M, int N, int K);

/* Same sum in fp32 with the s*sum(q*x) + b*sum(x) group factoring
 * (engine/kernels.py:168-171), bf16 output; OpenMP over rows. The CPU baseline. */
void orc_qmv_w4g64_f32(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                       const uint16_t* biases, uint16_t* y, int M, int N, int K, int threads);

/* Gated DeltaNet recurrence in fp64 following engine/kernels.py:34-63 op for op.
 * q,k [B,T,Hk,Dk] v [B,T,Hv,Dv] (fp32 values of the bf16 inputs), a,b [B,T,Hv],
 * A_log, dt_bias [Hv], state [B,Hv,Dv,Dk] (in/out, fp64),
 * y [B,T,Hv,Dv] fp64, snaps [T,B,Hv,Dv,Dk] fp64 (may be NULL). */
void orc_gated_delta_f64(const float* q, const float* k, const float* v, const float* a,
                         const float* b, const float* A_log, const float* dt_bias,
                         double* state, double* y, double* snaps,
                         int B, int T, int Hk, int Hv, int Dk, int Dv);

/* fp32 GDN recurrence (same op order), OpenMP over (b, hv): the CPU baseline. */
void orc_gated_delta_f32(const float* q, const float* k, const float* v, const float* a,
                         const float* b, const float* A_log, const float* dt_bias,
                         float* state, float* y, float* snaps,
                         int B, int T, int Hk, int Hv, int Dk, int Dv, int threads);

/* Speculative acceptance (fp32 emulation of the GPU reduction order; see spec.c). */
void orc_spec_accept(const float* target, const float* draft, const int32_t* draft_ids,
                     const float* u_accept, const float* u_sample, float temperature,
                     int32_t* n_accept, int32_t* out_token, int S, int k, int V, int threads);

/* The same with the target rows filtered as Sampler.scores (presence penalty
 * with `seen` [V] or NULL, top_k (0 or >= V: off), top_p; see spec.c). */
void orc_spec_accept_filtered(const float* target, const float* draft, const int32_t* draft_ids,
                              const float* u_accept, const float* u_sample, float inv_temp, const float* seen,
                              float presence_penalty, int top_k, float top_p, int32_t* n_accept,
                              int32_t* out_token, int S, int k, int V, int threads);

/* Philox4x32-10 block (Salmon et al. 2011): out = philox(ctr, key). */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* The sampler's uniforms of draw event `event` (see rng.c): n values in [0, 1). */
void orc_philox_uniforms(uint64_t seed, uint64_t event, int n, float* out);

/* The filter record (c_0, S_p, cutoff) of one target row (see spec.c); an
 * unfiltered row gives cutoff = -inf and (max, sum exp) from the part order. */
void orc_row_filter(const float* row, int V, float inv_temp, const float* seen, float presence_penalty, int top_k,
                    float top_p, float out[3]);

/* exp used by the sampler on both sides (Cody-Waite reduction + Taylor, fmaf). */
float orc_expf(float x);

#ifdef __cplusplus
}
#endif

#endif
