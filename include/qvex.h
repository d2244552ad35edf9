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
 * wave, wave_ksplit in {1,2,4,8} waves of a block splitting K. Requires
 * K % 256 == 0 for M <= 4 and K % 128 == 0 for M <= 8. */
int qvex_qmv_w4g64_mfma(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                        const uint16_t* biases, uint16_t* y, int M, int N, int K,
                        int tiles_per_wave, int wave_ksplit, void* stream);

/* ------------------------------------------------------------------------
 * Other widths and groups of the MLX affine layout: bits in {2,3,4,5,6,8},
 * group_size in {32,64,128} (per-module overrides, Config.qparams at
 * engine/model.py:68-71; mixed 4/3-bit models from quant/build.py:67-68).
 * Each weight row is a little-endian bit stream of K codes (quant/quantize.py:
 * 71-75): q[n, k] = bits [k*bits, (k+1)*bits) of row n's stream, w: uint32
 * [N, K*bits/32]; scales, biases: bf16 [N, K/group_size].
 *
 * y[M, N] = x[M, K] @ dequant(W)^T, fp32 accumulation per 32-code chunk
 * (sum q*x and sum x, folded with the group's scale and bias), one bf16
 * rounding: mx.quantized_matmul(..., group_size, bits) in QLinear.__call__
 * (engine/model.py:87-91). 1 <= M <= 8, K % group_size == 0, x and w 16-byte
 * aligned. */
int qvex_qmv_affine(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                    const uint16_t* biases, uint16_t* y, int M, int N, int K, int bits,
                    int group_size, void* stream);
/* out[l, :] = bf16(s * q + b) of row ids[l] (clamped to [0, V)): mx.dequantize
 * of the gathered rows in QEmbedding.__call__ (engine/model.py:126-130).
 * H % group_size == 0; w, out 16-byte aligned. */
int qvex_embed_affine(const int32_t* ids, int L, const uint32_t* w, const uint16_t* scales,
                      const uint16_t* biases, int V, int H, int bits, int group_size,
                      uint16_t* out, void* stream);
/* Lossless re-encoding of a bits <= 4, group 64 or 128 weight in the 4-bit
 * group-64 layout (codes unchanged in nibbles, a group-128 scale and bias
 * repeated for both halves): w4 uint32 [N, K/8], scales4, biases4 bf16
 * [N, K/64]; every 4-bit group-64 entry point then computes the same
 * products. No reference counterpart (a layout step of this library). */
int qvex_affine_widen_w4g64(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                            int N, int K, int bits, int group_size, uint32_t* w4,
                            uint16_t* scales4, uint16_t* biases4, void* stream);

/* ------------------------------------------------------------------------
 * Tile-packed weights: the QLinear triplet (engine/model.py:83-85) re-laid
 * once, at layer construction, as records of (16 rows x 256 k): 2048 bytes of
 * 4-bit words in the order the MFMA lanes consume them (nibbles reordered so
 * even k sit in the low half-word) followed by 256 bytes of (scale, bias)
 * bf16 pairs. Rows past N are zero. K must be a multiple of 256.
 * qvex_w4g64_packed_bytes() = ceil(N/16) * (K/256) * 2304 (0 if unsupported). */
uint64_t qvex_w4g64_packed_bytes(int N, int K);
int qvex_w4g64_pack(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    int N, int K, void* packed, uint64_t packed_bytes, void* stream);

/* y[M, N] = x[M, K] @ dequant(W)^T from the packed copy, M = 1..8: the product
 * of mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size=64,
 * bits=4) in QLinear.__call__ (engine/model.py:87-91), on MFMA with fully
 * coalesced record loads. The tile depends on (N, K) only, so each output row
 * is bitwise the same for every M. x, packed 16-byte aligned. */
int qvex_qmv_w4g64_packed(const uint16_t* x, const void* packed, uint16_t* y, int M, int N,
                          int K, void* stream);
/* SwiGLU variant for the fused gate/up projection of the MLP (gate rows
 * [0, N/2), up rows [N/2, N), engine/model.py:294-302): pack with the gate/up
 * interleave (each 16-row tile holds 8 gate rows and their 8 up rows), then
 * y[M, N/2] = bf16(silu(g) * u) with g, u the bf16-rounded products, i.e.
 * qvex_qmv_w4g64_packed followed by qvex_swiglu (_swiglu,
 * engine/model.py:134-135) up to the order of the per-set fp32 sums (a row
 * sits in another block of the interleaved pack). N % 16 == 0. */
int qvex_w4g64_pack_swiglu(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                           int N, int K, void* packed, uint64_t packed_bytes, void* stream);
int qvex_qmv_w4g64_packed_swiglu(const uint16_t* x, const void* packed, uint16_t* y, int M,
                                 int N, int K, void* stream);
/* Residual RMSNorm folded into the products around it (the residual adds and
 * mx.fast.rms_norm of the decoder layer, engine/model.py:309-317):
 *
 * qvex_qmv_w4g64_packed_resid - a product that ends a sub-block (o_proj,
 *   out_proj, down): delta = bf16(x W^T) as qvex_qmv_w4g64_packed, then
 *   h = bf16(resid + delta) -> h_out [M, N], u = bf16(h * norm_w) -> u_out
 *   [M, N] (norm_w: the NEXT norm's weight), and per row r and 16-row tile j
 *   the sum of h^2 over the tile -> sq_parts[r * ceil(N/16) + j].
 * qvex_qmv_w4g64_packed_rstd - the product that starts the next sub-block
 *   (in_proj, qkv, gate_up with swiglu != 0, lm_head) on x = u: output row r is
 *   scaled by rsqrt(S_r / dim + eps) before rounding, S_r the sum of the row's
 *   nparts = ceil(dim/16) partials (a multiple of 4, <= 256, i.e. dim <= 4096).
 *   This equals rms_norm(h) W^T up to where the bf16 roundings fall.
 * qvex_rms_parts - u and the partials for a residual row no product made
 *   (the embedding): u = bf16(x * norm_w), sq_parts as above, x [M, D]. */
int qvex_qmv_w4g64_packed_resid(const uint16_t* x, const void* packed, int M, int N, int K,
                                const uint16_t* resid, const uint16_t* norm_w, uint16_t* h_out,
                                uint16_t* u_out, float* sq_parts, void* stream);
int qvex_qmv_w4g64_packed_rstd(const uint16_t* u, const void* packed, uint16_t* y, int M, int N,
                               int K, const float* sq_parts, int nparts, int dim, float eps,
                               int swiglu, void* stream);
/* qvex_qmv_w4g64_packed_rstd (swiglu 0) that also writes, per row r and 16-row
 * tile j, the largest bf16 output of the tile to tile_max[r * ceil(N/16) + j]
 * (bf16; 16-byte aligned): the verify lm_head's logits and the tile maxima
 * qvex_spec_accept_tiles_bf16 starts from, in one launch (mx.quantized_matmul
 * of the lm_head, engine/model.py:330-336, with the sampler's first reduction
 * in its epilogue). */
int qvex_qmv_w4g64_packed_rstd_tilemax(const uint16_t* u, const void* packed, uint16_t* y, int M,
                                       int N, int K, const float* sq_parts, int nparts, int dim,
                                       float eps, uint16_t* tile_max, void* stream);
int qvex_rms_parts(const uint16_t* x, const uint16_t* norm_w, uint16_t* u_out, float* sq_parts,
                   int M, int D, void* stream);
/* out_proj after the split GatedDeltaNet mixer (qvex_gdn_decode_split): the
 * gated RMSNorm's per-(token, head) scale (_gated_rmsnorm, engine/model.py:
 * 138-143, before out_proj at engine/model.py:288-290) applied inside the
 * product. u [M, K] bf16 is silu(z) * w * y per 128-column head, unscaled;
 * head h's share of row r of u W^T is multiplied in fp32 by
 * rsqrt(S_rh / 128 + eps), S_rh the sum of the seg_nb (1, 2, 4 or 8) partials
 * seg_ss[(r * K/128 + h) * seg_nb + b]; then the residual epilogue of
 * qvex_qmv_w4g64_packed_resid. This equals out_proj(gated_rmsnorm(y, z)) up
 * to where the bf16 roundings fall. */
int qvex_qmv_w4g64_packed_gnorm_resid(const uint16_t* u, const void* packed, int M, int N, int K,
                                      const float* seg_ss, int seg_nb, float seg_eps,
                                      const uint16_t* resid, const uint16_t* norm_w, uint16_t* h_out,
                                      uint16_t* u_out, float* sq_parts, void* stream);
/* Greedy drafting on the lm_head (the argmax of `_argmax` / Sampler.pick with
 * temperature 0, engine/sampler.py:30-58, over mx.quantized_matmul's bf16
 * logits): out_token[r] = the first index of the largest bf16-rounded output
 * of row r of x W^T, without writing the product. The packed kernel's epilogue
 * keeps each 16-row tile's (max, first index); a one-block-per-row kernel
 * takes the first tile holding the row maximum. With sq_parts the rows are
 * scaled as qvex_qmv_w4g64_packed_rstd does (x = u of the final norm).
 * workspace: qvex_qmv_w4g64_argmax_workspace_bytes(M, N) = M * ceil(N/16) * 8.
 * With out_token NULL only the product runs: the workspace then holds row r's
 * per-tile pairs at float offset r * ceil(N/16) * 2, for qvex_mtp_input or
 * qvex_embed_rms_parts to reduce inside their own launch. */
uint64_t qvex_qmv_w4g64_argmax_workspace_bytes(int M, int N);
int qvex_qmv_w4g64_packed_argmax(const uint16_t* x, const void* packed, int M, int N, int K,
                                 const float* sq_parts, int nparts, int dim, float eps,
                                 int32_t* out_token, void* workspace, uint64_t workspace_bytes,
                                 void* stream);
/* The same with an explicit tile: tiles_per_wave in {1,2,4} 16-row tiles,
 * wave_ksplit in {1,2,4,8} (16 with one tile) waves splitting the 256-k sets,
 * and the load pipeline: prefetch_sets = 0 keeps two sets in flight per wave,
 * 2/4/6/8 issues all of a wave's sets (at least ceil(K/256 / wave_ksplit)) at
 * once, -1 picks as qvex_qmv_w4g64_packed does. Same bits for every pipeline.
 * For tile sweeps and tests. */
int qvex_qmv_w4g64_packed_tiled(const uint16_t* x, const void* packed, uint16_t* y, int M,
                                int N, int K, int tiles_per_wave, int wave_ksplit,
                                int prefetch_sets, void* stream);

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
 * fp32 [n_slots,B,Hv,Dv,Dk]; with c = *cur_slot mod n_slots (cur_slot a device
 * int32, typically the layer's token count), the state is read from slot c and
 * the state after token t goes to slot (c + 1 + t) % n_slots (every token when
 * snap_every != 0, else only the last). Keeping L tokens then means advancing
 * the counter by L: no state is copied. Requires n_slots >= T + 1 with
 * snapshots. Same reference interface as qvex_gdn_recurrent. */
int qvex_gdn_recurrent_ring(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const uint16_t* a, const uint16_t* b, const float* A_log,
                            const uint16_t* dt_bias, float* ring, int n_slots,
                            const int32_t* cur_slot, int snap_every, uint16_t* y, int B, int T,
                            int Hk, int Hv, int Dk, int Dv, void* stream);

/* The whole GatedDeltaNet mixer between in_proj and out_proj for a verify or
 * decode step of T <= 8 tokens, one launch (GatedDeltaNet.__call__,
 * engine/model.py:259-290, with gated_delta from engine/kernels.py:92-116 and
 * _gated_rmsnorm from engine/model.py:138-143): qvex_gdn_conv_qk, then
 * qvex_gdn_recurrent_ring, then qvex_gated_rmsnorm, with bitwise the same
 * outputs, conv ring and state ring as those three calls. proj [T, p_stride]
 * bf16 holds the conv channels (conv_dim = 2 * key_dim + Hv * 128), z at
 * z_offset and b, a at ab_offset; `counter` is the layer's token count (conv
 * ring row and state slot, as in the two ring forms); out bf16 [T, Hv * 128]
 * is the input of out_proj. B = 1, Dk = Dv = 128, key_dim = Hk * 128. */
int qvex_gdn_decode_fused(const uint16_t* proj, long p_stride, uint16_t* conv_ring, int ring_rows,
                          const int32_t* counter, const uint16_t* conv_w, int kernel_size, int conv_dim,
                          int key_dim, float q_scale, float k_scale, float qk_eps, const float* A_log,
                          const uint16_t* dt_bias, int z_offset, int ab_offset, float* state_ring,
                          int n_slots, int snap_every, const uint16_t* norm_w, float norm_eps,
                          uint16_t* out, int T, int Hk, int Hv, int Dk, int Dv, void* stream);
/* The same mixer with each value head split over blocks_per_head (2, 4 or 8)
 * workgroups of 128 / blocks_per_head state rows, so that the recurrence
 * spreads over Hv * blocks_per_head CUs. The gated norm's per-head scale needs
 * all 128 rows of a head, so it is left to the out_proj
 * (qvex_qmv_w4g64_packed_gnorm_resid): u_out [T, Hv * 128] bf16 receives
 * silu(z) * (norm_w * y) with y the bf16 recurrence output, and
 * ss_parts [T, Hv, blocks_per_head] fp32 each workgroup's sum of y^2. The conv
 * ring and state ring are bitwise those of qvex_gdn_decode_fused. Same
 * reference interface as qvex_gdn_decode_fused. */
int qvex_gdn_decode_split(const uint16_t* proj, long p_stride, uint16_t* conv_ring, int ring_rows,
                          const int32_t* counter, const uint16_t* conv_w, int kernel_size, int conv_dim,
                          int key_dim, float q_scale, float k_scale, float qk_eps, const float* A_log,
                          const uint16_t* dt_bias, int z_offset, int ab_offset, float* state_ring,
                          int n_slots, int snap_every, const uint16_t* norm_w, uint16_t* u_out,
                          float* ss_parts, int T, int Hk, int Hv, int Dk, int Dv, int blocks_per_head,
                          void* stream);

/* Chunked (prefill) form of the same recurrence, chunk = 64 tokens, on MFMA:
 * gated_delta over a long prompt (engine/kernels.py:92-116 as called by
 * GatedDeltaNet.__call__ during prefill, engine/model.py:282-286). Phase 1
 * (all chunks in parallel) builds each chunk's WY form W, U~ and the masked
 * Q K^T in `workspace`; phase 2 scans the chunks in order with the fp32 state
 * in registers. state_in fp32 [B,Hv,Dv,Dk] -> state_out (may be the same
 * buffer), y bf16 [B,T,Hv,Dv]. Dk = Dv = 128, chunk = 64. Operands of the
 * products are bf16, accumulation fp32. workspace:
 * qvex_gdn_chunked_workspace_bytes() = B * Hv * ceil(T/64) * 73984 bytes. */
uint64_t qvex_gdn_chunked_workspace_bytes(int B, int T, int Hv, int Dk, int Dv, int chunk);
int qvex_gdn_chunked(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                     const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                     const float* state_in, float* state_out, uint16_t* y, int B, int T, int Hk,
                     int Hv, int Dk, int Dv, int chunk, void* workspace, uint64_t workspace_bytes,
                     void* stream);

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

/* The same with the target rows filtered as Sampler.scores
 * (engine/sampler.py:30-52): presence penalty x - penalty * s(j), s(j) = 1 for
 * the tokens of `seen` (fp32 [V], 0/1, or NULL) and, in verify row i, for the
 * drafts d_0..d_{i-1}; when sampling, top-k (0 < top_k < V; 0 or >= V = off)
 * and top-p (0 < top_p < 1, over the top-k values or, without top-k, over the
 * whole vocabulary: engine/sampler.py:44-50). top_k <= 64 merges per-part lists;
 * larger top_k and whole-vocabulary top-p find the cutoff by exact radix
 * descents (csrc/spec.hip). Greedy scores are only penalised. Draft logits,
 * when given, are not filtered. Ties at the cutoff are all kept.
 * workspace: qvex_spec_accept_filtered_workspace_bytes(S, k, V, has_draft, top_k). */
uint64_t qvex_spec_accept_filtered_workspace_bytes(int S, int k, int V, int has_draft, int top_k);
int qvex_spec_accept_filtered(const float* target, const float* draft, const int32_t* draft_ids,
                              const float* u_accept, const float* u_sample, float inv_temp,
                              const float* seen, float presence_penalty, int top_k, float top_p,
                              int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                              void* workspace, uint64_t workspace_bytes, void* stream);
/* The same on bf16 logits as the lm_head writes them (target and draft both
 * bf16): every value widens exactly to fp32 on load, so the results equal
 * qvex_spec_accept_filtered on the fp32 copies (Sampler.scores' astype(float32),
 * engine/sampler.py:33) without making them. */
int qvex_spec_accept_filtered_bf16(const uint16_t* target, const uint16_t* draft,
                                   const int32_t* draft_ids, const float* u_accept,
                                   const float* u_sample, float inv_temp, const float* seen,
                                   float presence_penalty, int top_k, float top_p,
                                   int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                                   void* workspace, uint64_t workspace_bytes, void* stream);

/* qvex_spec_accept_filtered_bf16 for the decode cycle's call (the verify rows'
 * accept and draw of engine/speculative.py:74-81 with Sampler.scores'
 * filtering, engine/sampler.py:30-52) given tile_max [S*(k+1), V/16] bf16: the
 * largest logit of each 16-column tile of each target row, as
 * qvex_qmv_w4g64_packed_rstd_tilemax writes it with the logits (or
 * qvex_tile_max_bf16 computes it). Without draft logits, with no presence
 * penalty, 1 <= top_k <= 64 when sampling, V a multiple of 128 up to 262,144,
 * one kernel with one block per target row does the work: the top_k-th
 * largest of 256 thread maxima of the tile maxima bounds the row's k-th value
 * from below, so only the tiles whose maximum reaches it are read (a few
 * hundred logits instead of the row); rows where too many tiles or values
 * reach it run the two-kernel path's work inside the same block. Other calls
 * are qvex_spec_accept_filtered_bf16's. Results are identical to that call's
 * (no reference counterpart: this is the same interface fed by the lm_head's
 * epilogue). workspace as there (qvex_spec_accept_filtered_workspace_bytes),
 * zero-filled before its first use (and outside any graph capture that uses
 * it): the call counts each step's finished rows in it and leaves the count
 * at zero. */
int qvex_spec_accept_tiles_bf16(const uint16_t* target, const uint16_t* tile_max, const int32_t* draft_ids,
                                const float* u_accept, const float* u_sample, float inv_temp,
                                const float* seen, float presence_penalty, int top_k, float top_p,
                                int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                                void* workspace, uint64_t workspace_bytes, void* stream);
/* 1 when qvex_spec_accept_tiles_bf16 runs its one-kernel form for a call with
 * these arguments (and tile maxima), else 0 (no reference counterpart: the
 * dispatch test of the entry above, for callers that choose before a graph
 * capture). */
int qvex_spec_accept_tiles_applies(int S, int k, int V, float inv_temp, int top_k, float presence_penalty);
/* The one-kernel form of qvex_spec_accept_tiles_bf16 without the step
 * decision: each target row r leaves rows[2 r] = its accept flag (rows r < k;
 * 0 for the bonus row k) and rows[2 r + 1] = its draw (the residual draw at a rejection,
 * the bonus draw for row k) in rows [S * (k+1)][2] int32; the step's (n, token)
 * is the first row with flag 0 and its draw, as qvex_cycle_finish_ex decides it
 * from rows (the accept loop of engine/speculative.py:74-81). Only for calls
 * where qvex_spec_accept_tiles_applies is 1 (else QVEX_EINVAL); the workspace
 * needs no zero fill (no counter is used). No reference counterpart: it splits
 * the reference's accept loop between two launches of the decode cycle. */
int qvex_spec_accept_tiles_rows_bf16(const uint16_t* target, const uint16_t* tile_max, const int32_t* draft_ids,
                                     const float* u_accept, const float* u_sample, float inv_temp,
                                     const float* seen, float presence_penalty, int top_k, float top_p,
                                     int32_t* rows, int S, int k, int V, void* workspace,
                                     uint64_t workspace_bytes, void* stream);
/* tile_max[r][t] = the largest of x[r][16 t .. 16 t + 15] for bf16 rows x
 * [rows, V] (bf16 out [rows, ceil(V/16)]): the tile maxima of
 * qvex_spec_accept_tiles_bf16 for logits that no tile-maxima epilogue wrote. */
int qvex_tile_max_bf16(const uint16_t* x, int rows, int V, uint16_t* out, void* stream);

/* Sampler.scores (engine/sampler.py:30-52) for R rows of V logits (bf16 when
 * logits_bf16, else fp32; 16-byte aligned) into out fp32 [R, V]: the presence
 * penalty x - penalty * seen[j] (seen fp32 [V] 0/1 or NULL; the caller marks
 * extra_seen in it), then greedy (inv_temp <= 0): the penalised logits; else
 * z = x * inv_temp filtered by top-k / top-p exactly as the accept entry
 * points filter their target rows (same cutoff), and out = z - c_0 - log(S) on
 * the kept set (c_0 the row maximum, S the kept sum of exp(z - c_0)), -inf
 * elsewhere. workspace: qvex_sampler_scores_workspace_bytes(R, V, top_k). */
uint64_t qvex_sampler_scores_workspace_bytes(int R, int V, int top_k);
int qvex_sampler_scores(const void* logits, int logits_bf16, int R, int V, const float* seen,
                        float presence_penalty, float inv_temp, int top_k, float top_p, float* out,
                        void* workspace, uint64_t workspace_bytes, void* stream);

/* qvex_spec_accept_filtered_bf16 without a workspace argument and without any
 * allocation: the workspace is a static device array of QVEX_SPEC_SCRATCH_BYTES
 * (4 MiB) per GPU, held until the process ends, whose address is looked up
 * once per device on the first call there. No counterpart in the reference:
 * this is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). Calls whose
 * qvex_spec_accept_filtered_workspace_bytes(S, k, V, draft != NULL, top_k)
 * exceeds the array return QVEX_EINVAL (one verify step of k = 3 drafts over
 * the 9B vocabulary of 248,320 needs about 140 KB with top-k 20, about 33 KB
 * unfiltered). Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (different streams, threads) race and must be ordered
 * by the caller. Results equal qvex_spec_accept_filtered_bf16's bit for bit. */
#define QVEX_SPEC_SCRATCH_BYTES (4u << 20)
int qvex_spec_accept_filtered_bf16_noalloc(const uint16_t* target, const uint16_t* draft,
                                           const int32_t* draft_ids, const float* u_accept,
                                           const float* u_sample, float inv_temp, const float* seen,
                                           float presence_penalty, int top_k, float top_p,
                                           int32_t* n_accept, int32_t* out_token, int S, int k, int V,
                                           void* stream);

/* ------------------------------------------------------------------------
 * Verify-forward glue (Qwen3.5 hybrid stack, engine/model.py). bf16 storage,
 * fp32 arithmetic, one bf16 rounding per output.
 * ------------------------------------------------------------------------ */

/* out[l, :] = dequant(w[ids[l], :]) (QEmbedding.__call__, engine/model.py:126-130);
 * ids outside [0, V) are clamped. w uint32 [V, H/8]; scales/biases bf16 [V, H/64]. */
int qvex_embed_w4g64(const int32_t* ids, int L, const uint32_t* w, const uint16_t* scales,
                     const uint16_t* biases, int V, int H, uint16_t* out, void* stream);

/* out[r] = w * (x[r] * rsqrt(mean(x[r]^2) + eps)) * scale, w optional (NULL = 1)
 * (mx.fast.rms_norm at engine/model.py:218-219, 276-277, 314-316, 335; the
 * weightless q/k scaling of engine/model.py:275-277 uses scale). D % 8 == 0,
 * D <= 8192; strides in elements, multiples of 8; pointers 16-byte aligned. */
int qvex_rmsnorm(const uint16_t* x, long x_stride, const uint16_t* w, uint16_t* out,
                 long out_stride, int R, int D, float eps, float scale, void* stream);

/* Two qvex_rmsnorm calls in one launch: out0 = rms_norm(x0) * w0 and
 * out1 = rms_norm(x1) * w1, R rows each of width D (same rules as qvex_rmsnorm,
 * scale 1). The MTP head's input norms (engine/mtp.py:63-65: rms of the
 * embedding and of the hidden, concatenated): out0, out1 are the two halves of
 * the fc input row, sharing out_stride. */
int qvex_rmsnorm_pair(const uint16_t* x0, long x0_stride, const uint16_t* w0, uint16_t* out0,
                      const uint16_t* x1, long x1_stride, const uint16_t* w1, uint16_t* out1,
                      long out_stride, int R, int D, float eps, void* stream);

/* The MTP head's input for one draft step in one launch (MTPHead.__call__,
 * engine/mtp.py:61-63): x_in[r, 0:H] = rms_norm(embed(tok_r)) * w_emb and
 * x_in[r, H:2H] = rms_norm(hid[s_r]) * w_hid, bit-identical to qvex_embed_w4g64
 * + qvex_rmsnorm_pair. tok_r = ids[r], or, for T = 1 with am_parts, the greedy
 * token of the previous step's lm_head: the argmax of the per-tile pairs that
 * qvex_qmv_w4g64_packed_argmax left in its workspace (out_token NULL), row
 * *am_row (NULL: row 0), stored to *ids_out (as that call's reduction would
 * store it). s_r = *hid_sel (device row index; NULL: r). With counters, the
 * launch also adds *n_accept (NULL: 0) + extra to counters[0 .. ncnt) (the
 * previous step's qvex_commit_step). Same layout rules as those calls. */
int qvex_mtp_input(const int32_t* ids, int T, const float* am_parts, int am_tiles, const int32_t* am_row,
                   int32_t* ids_out, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                   int V, int H, const uint16_t* w_emb, const uint16_t* hid, long hid_stride,
                   const int32_t* hid_sel, const uint16_t* w_hid, uint16_t* x_in, long x_stride, float eps,
                   int32_t* counters, int ncnt, const int32_t* n_accept, int extra, void* stream);

/* The verify rows' input in one launch (QEmbedding.__call__, engine/model.py:
 * 126-130, then the first layer's input norm, engine/model.py:309-310): h_out =
 * embed(ids), and u_out, parts as qvex_rms_parts(h_out, norm_w) writes them,
 * bit-identical to those two calls. With am_parts, ids[am_slot] is first
 * replaced by the argmax of the per-tile pairs of row *am_row (NULL: row 0)
 * that qvex_qmv_w4g64_packed_argmax left in its workspace (the last draft). */
int qvex_embed_rms_parts(int32_t* ids, int L, const float* am_parts, int am_tiles, const int32_t* am_row,
                         int am_slot, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                         int V, int H, const uint16_t* norm_w, uint16_t* h_out, uint16_t* u_out,
                         float* parts, void* stream);

/* h = bf16(x + delta); out = rms_norm(h) * w: the residual add and the next
 * pre-norm of Layer.__call__ (engine/model.py:313-316) in one pass. [R, D],
 * D % 8 == 0, D <= 8192, pointers 16-byte aligned. */
int qvex_add_rmsnorm(const uint16_t* x, const uint16_t* delta, uint16_t* h_out,
                     const uint16_t* w, uint16_t* out, int R, int D, float eps, void* stream);

/* GatedDeltaNet input stage (engine/model.py:259-277). The conv input history
 * is a ring of ring_rows rows [ring_rows, C] keyed by the layer's token count
 * p = *pos (device int32): the conv state is rows p-K+1 .. p-1 (mod ring_rows),
 * token t is stored at row p + t, so keeping L tokens is p += L and rollback
 * copies nothing (generalises RecurrentCache.conv/conv_prev, engine/model.py:
 * 179-193). Computes causal depthwise conv (conv_w [C, K]) + SiLU; q, k heads
 * of 128 rms-normalised (no weight, eps) times q_scale / k_scale; v; and the b, a
 * gate inputs copied from proj[:, ab_offset : ab_offset + 2*Hv] into [T, Hv].
 * Requires ring_rows >= T + K - 1. */
int qvex_gdn_conv_qk(const uint16_t* proj, long p_stride, uint16_t* conv_ring, int ring_rows,
                     const int32_t* pos, const uint16_t* conv_w, int kernel_size, uint16_t* q,
                     uint16_t* k, uint16_t* v, uint16_t* a_out, uint16_t* b_out, int T, int C,
                     int key_dim, int Hv, int ab_offset, float q_scale, float k_scale, float eps,
                     void* stream);

/* counters[i] += n_accept[0] + extra for i < n: advances every cache counter
 * past the kept verify tokens on the device (the commit half of decode()'s
 * accept/rollback, engine/speculative.py:85-101), so a captured cycle needs no
 * host round trip. */
int qvex_commit_step(int32_t* counters, int n, const int32_t* n_accept, int extra, void* stream);

/* out = silu(z) * rms_norm(y, w) per head row of D (_gated_rmsnorm,
 * engine/model.py:138-143); y [R, D], z rows of `heads` heads with z_stride. */
int qvex_gated_rmsnorm(const uint16_t* y, const uint16_t* z, long z_stride, int heads,
                       const uint16_t* w, uint16_t* out, int R, int D, float eps, void* stream);

/* out[l, i] = silu(gu[l, i]) * gu[l, I + i] (MLP with the fused gate_up,
 * engine/model.py:133-135, 300-302). */
int qvex_swiglu(const uint16_t* gu, uint16_t* out, int L, int I, void* stream);

/* fp32 copy of bf16 values (Sampler.scores' astype(float32), engine/sampler.py:33). */
int qvex_bf16_to_f32(const uint16_t* in, float* out, long n, void* stream);

/* KV cache layouts (cap a multiple of 32; K and V each hold Hkv * cap * D bf16),
 * tiled so that each wave load instruction of the attention kernels reads 1 KiB
 * of consecutive bytes:
 *   K: key p, dim d of kv head h at
 *      (((h * cap/16 + p/16) * D/32 + d/32) * 64 + ((d % 32) / 8) * 16 + p % 16) * 8 + d % 8
 *   V: (((h * cap/32 + p/32) * D + d) * 32 + p % 32
 * (the reference keeps [B, Hkv, cap, D] arrays, engine/model.py:149-176).
 *
 * Attention input stage (engine/model.py:213-226): q and k rms-normalised per
 * head with q_norm / k_norm, NeoX-form RoPE on the first rot_dim dims at
 * positions *pos0 + l (pos0 a device int32), q written to q_out [L, Hq, D],
 * k and v appended to the caches at those positions (KVCache.update,
 * engine/model.py:156-170). proj row = [Hq x (q | gate) | Hkv x k | Hkv x v].
 * rope: NULL, or a qvex_rope_table() of rope_rows positions for rot_dim and
 * theta, whose (cos, sin) pairs are then loaded instead of evaluated (the same
 * values, so the same results; positions past rope_rows are evaluated). */
int qvex_attn_qk_rope(const uint16_t* proj, long p_stride, const uint16_t* q_norm,
                      const uint16_t* k_norm, const int32_t* pos0, int L, int Hq, int Hkv, int D,
                      int rot_dim, float theta, float eps, uint16_t* q_out, uint16_t* k_cache,
                      uint16_t* v_cache, int cap, const float* rope, int rope_rows, void* stream);

/* Causal GQA attention of L queries over the cache (query l sees keys
 * 0 .. *pos0 + l), scale 1/sqrt(D), output times sigmoid(gate) from the q_proj
 * rows: mx.fast.scaled_dot_product_attention + o * sigmoid(gate)
 * (engine/model.py:228-232). Split-K over keys_per_split keys per block
 * (a multiple of 128: 4 waves x 32 keys per step); max_keys bounds *pos0 + L,
 * and only the splits below *pos0 + L do work. Splits below known_keys (keys
 * visible on every call: max_keys for a one-off call, the position at capture
 * for a captured graph) request their first keys before reading *pos0, the
 * others read it first and load nothing when past it; results do not depend on
 * known_keys. D is 128 or 256. workspace: qvex_attn_workspace_bytes(). */
uint64_t qvex_attn_workspace_bytes(int L, int Hq, int Hkv, int D, int max_keys, int keys_per_split);
int qvex_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                   const int32_t* pos0, int L, int Hq, int Hkv, int D, int cap, int max_keys,
                   int known_keys, int keys_per_split, const uint16_t* gate, long gate_stride,
                   uint16_t* out, void* workspace, uint64_t workspace_bytes, void* stream);

/* The decode / verify step of the attention block in two launches: the input
 * stage of qvex_attn_qk_rope (q and k norms, RoPE, the cache append) folded
 * into qvex_attention's split kernel, for L = 1..8 new tokens
 * (engine/model.py:213-232 on the speculative verify, engine/speculative.py:86).
 * Each split block computes its query rows and, where its keys include this
 * call's, those keys itself; splits past *pos0 + L load nothing (a graph may be
 * captured with max_keys = cap). rot_dim / 2 must be a multiple of D / 16.
 * The rotation's (cos, sin) come from a table of qvex_rope_table() covering at
 * least cap positions (the same values qvex_attn_qk_rope computes); L * rot_dim / 2
 * must be at most 256. The norms' sums of squares run in another order than
 * qvex_attn_qk_rope's, so cached keys can differ from its in the last bit.
 * Workspace as qvex_attention's. */
int qvex_attention_decode(const uint16_t* proj, long p_stride, const uint16_t* q_norm,
                          const uint16_t* k_norm, const int32_t* pos0, int L, int Hq, int Hkv, int D,
                          int rot_dim, float eps, const float* rope, int rope_rows, uint16_t* k_cache,
                          uint16_t* v_cache, int cap, int max_keys, int keys_per_split, uint16_t* out,
                          void* workspace, uint64_t workspace_bytes, void* stream);

/* RoPE table for qvex_attn_qk_rope and qvex_attention_decode: table[p][i] = (cos, sin) of
 * p * theta^(-2i / rot_dim), p < rows, i < rot_dim / 2 (float pairs); the angle
 * of mx.fast.rope(traditional=False) at position p (engine/model.py:222-225). */
int qvex_rope_table(int rot_dim, float theta, int rows, float* table, void* stream);

/* ------------------------------------------------------------------------
 * Device-side cycle bookkeeping (host side of decode(),
 * engine/speculative.py:82-102), so a whole MTP cycle can be captured once in a
 * HIP graph and replayed with one host synchronisation.
 * ------------------------------------------------------------------------ */

/* dst[0:H) = src[clamp(*idx, 0, rows-1) * row_stride + 0:H): the row of the
 * last valid pending pair, selected on the device. */
int qvex_gather_row(const uint16_t* src, long row_stride, const int32_t* idx, int rows,
                    uint16_t* dst, int H, void* stream);

/* ids = [*feed, drafts[0] .. drafts[k-1]]: the verify input. */
int qvex_assemble_ids(const int32_t* feed, const int32_t* drafts, int k, int32_t* ids, void* stream);

/* After the accept: pend_ids = [d_0 .. d_{n-1}, token, 0 ...] (k + 1 slots),
 * *feed = token, *n_prev = n, out = [n, token, d_0 .. d_{k-1}] for the host. */
int qvex_cycle_finish(const int32_t* drafts, int k, const int32_t* n_accept, const int32_t* token,
                      int32_t* pend_ids, int32_t* feed, int32_t* n_prev, int32_t* out, void* stream);

/* qvex_cycle_finish and the rest of a captured cycle's bookkeeping in one
 * launch: ids_next[0] = token (the next verify input's first id, the drafts
 * then being written straight into ids_next[1..k]), main_counters[i] +=
 * n + main_extra for i < n_main (the verify commit of decode(),
 * engine/speculative.py:94-101), mtp_counters[i] += mtp_delta (the draft
 * steps' net advance), and u_out[0:u_width) = the uniforms of draw event
 * *u_counter under u_seed (as qvex_philox_uniforms), then *u_counter += 1 (the
 * next cycle's uniforms). Null pointers skip a part; every read happens before
 * any write, so drafts may alias ids_next + 1. done (optional, one int32, may
 * be pinned host memory): set to 1 after every entry of `out` is visible
 * system-wide, so a host that zeroes it before the launch and polls it reads
 * the cycle's result without a stream synchronisation (the reference's one
 * read per cycle, engine/speculative.py:82-85). rows (optional, [k + 1][2]
 * int32, as qvex_spec_accept_tiles_rows_bf16 leaves them): when given,
 * n_accept and token are not read (may be NULL) and the step is decided here,
 * as decode() does with the verify's accept flags (engine/speculative.py:74-81):
 * n = the first r < k whose flag is 0 (k when none), token = row n's draw. */
int qvex_cycle_finish_ex(const int32_t* drafts, int k, const int32_t* n_accept, const int32_t* token,
                         int32_t* pend_ids, int32_t* feed, int32_t* n_prev, int32_t* out,
                         int32_t* ids_next, int32_t* main_counters, int n_main, int main_extra,
                         int32_t* mtp_counters, int n_mtp, int mtp_delta, uint64_t u_seed,
                         uint64_t* u_counter, int u_width, float* u_out, int32_t* done,
                         const int32_t* rows, void* stream);

/* The sampler's uniforms (the draws of engine/speculative.py:79-81 and
 * Sampler.pick's categorical, engine/sampler.py:57-58, which use MLX's
 * generator): out[i] = u(*counter, i) for i < n (1..256), then *counter += 1,
 * where draw event c under seed s gives
 *   u(c, i) = (philox4x32_10({c_lo, c_hi, i / 4, 0}, {s_lo, s_hi})[i % 4] >> 8) * 2^-24
 * (Philox4x32-10, Salmon et al., SC 2011). counter: one device uint64. The
 * stream never repeats, and a draw needs no host work, so it can be captured. */
int qvex_philox_uniforms(uint64_t seed, uint64_t* counter, int n, float* out, void* stream);

/* Presence tracking (Sampler.observe, engine/sampler.py:60-62): seen[ids[q]] = 1
 * for q < min(max_ids, (n_ptr ? *n_ptr : 0) + n_offset); ids outside [0, V) are
 * skipped. With n_ptr = the cycle result [n, token, drafts...] and
 * ids = result + 1, n_offset = 1 it marks the token and the n accepted drafts. */
int qvex_mark_seen(float* seen, int V, const int32_t* ids, int max_ids, const int32_t* n_ptr,
                   int n_offset, void* stream);

/* Pure streaming read of `bytes` bytes (multiple of 16) from `buf`, folding
 * them into `sink` (64 uint32 words). Measures the achievable HBM read rate;
 * the counterpart of read_roof (experiments/native/qmv_spike.mm:21-32). */
int qvex_read_roof(const void* buf, uint64_t bytes, uint32_t* sink, int blocks,
                   void* stream);

/* Read-ceiling probe with a fixed access pattern and a choice of load path:
 * waves of `waves_per_block` (4 or 8) each read `iters` (2, 4, 8 or 16) 1 KiB
 * units, all issued before the first wait; lds = 1 lands them in LDS through
 * global_load_lds_dwordx4, lds = 0 in VGPRs. bytes must be a multiple of
 * 1 KiB * iters * waves_per_block. A measurement aid beside qvex_read_roof
 * (experiments/native/qmv_spike.mm:21-32 measures its own read roof). */
int qvex_read_probe(const void* buf, uint64_t bytes, uint32_t* sink, int iters, int lds,
                    int waves_per_block, void* stream);

/* Dense bf16 copy of an MLX 4-bit group-64 weight: out[n, k] =
 * bf16(s[n, k/64] * q[n, k] + b[n, k/64]) with the product and sum in fp32
 * (one rounding). The long (prefill) calls of QLinear (engine/model.py:87-91
 * with many rows, mx.quantized_matmul's prefill case) then run as a plain
 * library GEMM on it. out [N, K] bf16, 16-byte aligned; K % 64 == 0. */
int qvex_w4g64_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N, int K,
                       uint16_t* out, void* stream);

/* Prefill products from the packed copy: y[M, N] = x[M, K] @ W^T for prompt
 * chunks (mx.quantized_matmul in QLinear.__call__, engine/model.py:87-91, on
 * the 512-token chunks of engine/engine.py:232-248). x bf16 [M, K] row-major
 * (16-byte aligned), packed from qvex_w4g64_pack, y bf16 [M, N]. Each weight is
 * dequantized in registers to bf16(s * q + b) (as qvex_w4g64_dequant) and the
 * products accumulate in fp32 on the matrix cores; any M >= 1, K % 256 == 0. */
int qvex_w4g64_packed_gemm(const uint16_t* x, const void* packed, uint16_t* y, int M, int N, int K,
                           void* stream);
/* The same on a weight packed by qvex_w4g64_pack_swiglu (fused [gate; up], N
 * rows): y [M, N/2] = bf16(silu(g) * u) with g and u the bf16-rounded products
 * (MLP.__call__'s _swiglu, engine/model.py:133-135, 300-302). N % 16 == 0. */
int qvex_w4g64_packed_gemm_swiglu(const uint16_t* x, const void* packed, uint16_t* y, int M, int N, int K,
                                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QVEX_H */
