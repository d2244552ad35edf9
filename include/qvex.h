/*
 * qvex.h — C ABI of libqvex.so, the MI355X (gfx950) kernels of QVex's MTP
 * speculative-decoding verify step.
 *
 * Conventions (every entry point):
 *   - returns 0 (QVEX_OK) or a qvex_status code; qvex_last_error() gives a
 *     thread-local message for the last failure on the calling thread;
 *   - all pointers are device pointers (HBM) unless stated otherwise; buffers
 *     are dense row-major with the shapes given; bf16 tensors are passed as
 *     uint16_t bit patterns;
 *   - outputs and workspaces are allocated by the caller; the library never
 *     allocates device memory;
 *   - work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *     is asynchronous; nothing synchronizes the host.
 *
 * Each declaration names the reference interface it replaces
 * (paths are into the QVex-3.5 source tree).
 */
#ifndef QVEX_H
#define QVEX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum qvex_status {
  QVEX_OK = 0,
  QVEX_EINVAL = 1,   /* bad shape, pointer alignment or argument */
  QVEX_EHIP = 2,     /* HIP runtime error (launch or query) */
  QVEX_ENOTSUP = 3   /* shape outside what the kernels implement */
};

/* Message of the last failed call on this thread ("" if none). */
const char* qvex_last_error(void);

/* ABI version: bumped whenever a signature changes. */
int qvex_abi_version(void);

/* ------------------------------------------------------------------------
 * 4-bit group-64 quantized matmul (MLX affine layout).
 *
 *   y[m, n] = sum_k x[m, k] * (scales[n, k/64] * q[n, k] + biases[n, k/64])
 *   q[n, k] = (w[n, k/8] >> (4 * (k % 8))) & 0xF
 *
 * x: bf16 [M, K]; w: uint32 [N, K/8]; scales, biases: bf16 [N, K/64];
 * y: bf16 [M, N]. fp32 accumulation, one bf16 rounding of the output.
 * Requires 1 <= M <= 8, K % 64 == 0, N >= 1; x, w 16-byte aligned.
 *
 * Replaces mx.quantized_matmul(x, w, scales, biases, transpose=True,
 * group_size=64, bits=4) as called by QLinear.__call__
 * (engine/model.py:87-91) and qmv_multi (engine/kernels.py:197-211).
 * ------------------------------------------------------------------------ */
int qvex_qmv_w4g64(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                   const uint16_t* biases, uint16_t* y, int M, int N, int K,
                   void* stream);

/* Same as qvex_qmv_w4g64 with an explicit tile: rows_per_wave in {1,2,4,8}
 * weight rows per wave, k_split in {1,2,4} waves sharing one row group along
 * K. Used by tile sweeps; qvex_qmv_w4g64 picks the tile from (M, N, K). */
int qvex_qmv_w4g64_tiled(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                         const uint16_t* biases, uint16_t* y, int M, int N, int K,
                         int rows_per_wave, int k_split, void* stream);

/* Same product through the MFMA form of the kernel (16-row tiles, block-
 * diagonal activation operand): tiles_per_wave in {1,2,4} 16-row tiles per
 * wave, wave_ksplit in {1,2,4} waves of a block splitting K. Requires
 * K % 256 == 0 for M <= 4 and K % 128 == 0 for M <= 8. */
int qvex_qmv_w4g64_mfma(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                        const uint16_t* biases, uint16_t* y, int M, int N, int K,
                        int tiles_per_wave, int wave_ksplit, void* stream);

/* ------------------------------------------------------------------------
 * Gated DeltaNet recurrence (verify form), one state snapshot per token.
 *
 * For each batch b, value head hv (key head hk = hv / (Hv/Hk)), value row dv:
 *   g = exp(-exp(A_log[hv]) * softplus(a + dt_bias[hv])), beta = sigmoid(b)
 *   S *= g; kv = S.k; delta = (v - kv) * beta; S += k * delta; y = S.q
 * q, k: bf16 [B,T,Hk,Dk]; v: bf16 [B,T,Hv,Dv]; a, b: bf16 [B,T,Hv];
 * A_log: fp32 [Hv]; dt_bias: bf16 [Hv]; state_in: fp32 [B,Hv,Dv,Dk];
 * y: bf16 [B,T,Hv,Dv]; snapshots: fp32 [T,B,Hv,Dv,Dk] when snap_every != 0
 * (slot t = state after token t), else [1,B,Hv,Dv,Dk] (final state).
 * state_in may alias a snapshot slot. Requires Dk == 128, Dv % 16 == 0.
 *
 * Replaces gated_delta(q,k,v,a,b,A_log,dt_bias,state,keep_mid)
 * (engine/kernels.py:92-116) and its Metal source (engine/kernels.py:11-75);
 * rollback to an accepted length L is then snapshots[L-1] (state_in for L=0)
 * instead of RecurrentCache.rollback's single saved state
 * (engine/model.py:189-193).
 * ------------------------------------------------------------------------ */
int qvex_gdn_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       const uint16_t* a, const uint16_t* b, const float* A_log,
                       const uint16_t* dt_bias, const float* state_in, float* snapshots,
                       int snap_every, uint16_t* y, int B, int T, int Hk, int Hv, int Dk,
                       int Dv, void* stream);

/* Ring form of qvex_gdn_recurrent for stream/graph replay: ring is
 * fp32 [n_slots,B,Hv,Dv,Dk]; the state is read from slot c = *cur_slot (a device
 * int32) and the state after token t goes to slot (c + 1 + t) % n_slots.
 * Committing L accepted tokens is then cur_slot = (c + L) % n_slots, a device-side
 * update (see qvex_commit_step). Requires n_slots >= T + 1. Same reference
 * interface as qvex_gdn_recurrent. */
int qvex_gdn_recurrent_ring(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const uint16_t* a, const uint16_t* b, const float* A_log,
                            const uint16_t* dt_bias, float* ring, int n_slots,
                            const int32_t* cur_slot, uint16_t* y, int B, int T, int Hk,
                            int Hv, int Dk, int Dv, void* stream);

/* ------------------------------------------------------------------------
 * Fused speculative acceptance sampling for S independent verify steps.
 *
 * target: fp32 [S, k+1, V] logits of the verify rows; draft: fp32 [S, k, V]
 * logits of the draft distribution, or NULL when the drafts are greedy (q is
 * one-hot at the draft id); draft_ids: int32 [S, k]; u_accept: fp32 [S, k];
 * u_sample: fp32 [S]; inv_temp = 1/temperature (<= 0 selects greedy: accept iff
 * argmax matches, token = argmax). With z = logits * inv_temp, p = softmax(z):
 *   accept d_i iff u_i * q_i(d_i) < p_i(d_i)  (evaluated division-free);
 *   n_accept[s] = index of the first rejection (k if none);
 *   out_token[s] ~ max(0, p_n - q_n) at the first rejection, else ~ p_k.
 * The reduction order is fixed (see csrc/spec.hip), so results are
 * reproducible bit for bit given identical logits and uniforms. Requires
 * V % 4 == 0, V <= 1,179,648, k <= 32; workspace of
 * qvex_spec_accept_workspace_bytes(S, k, V, draft != NULL) bytes.
 *
 * Replaces the accept/resample/bonus block of decode()
 * (engine/speculative.py:74-81) with Sampler.scores/pick at temperature only
 * (engine/sampler.py:30-58; top-k/top-p filtering is not applied).
 * ------------------------------------------------------------------------ */
uint64_t qvex_spec_accept_workspace_bytes(int S, int k, int V, int has_draft);
int qvex_spec_accept(const float* target, const float* draft, const int32_t* draft_ids,
                     const float* u_accept, const float* u_sample, float inv_temp,
                     int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                     void* workspace, uint64_t workspace_bytes, void* stream);

/* Pure streaming read of `bytes` bytes (multiple of 16) from `buf`, folding
 * them into `sink` (64 uint32 words). Measures the achievable HBM read rate;
 * the counterpart of read_roof (experiments/native/qmv_spike.mm:21-32). */
int qvex_read_roof(const void* buf, uint64_t bytes, uint32_t* sink, int blocks,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QVEX_H */
