// Fused inputs of the decode cycle: the greedy draft token, its embedding row and
// the norms that feed the first product, in one launch each.
//
// Reference: QEmbedding.__call__ (engine/model.py:126-130) followed by the first
// layer's input norm (engine/model.py:309-310, mx.fast.rms_norm) for the verify
// rows; MTPHead.__call__'s input x = fc([rms(embed(tok)), rms(h)])
// (engine/mtp.py:61-63) for a draft step; the greedy draft of the previous step
// (the argmax of the shared lm_head's logits, engine/speculative.py:57).
//
// Each kernel does exactly the arithmetic of the launches it replaces, so the
// results are theirs bit for bit:
//   the token: the first index of the largest bf16 output, from the per-tile
//     (max, first index) pairs the lm_head's argmax epilogue wrote (the
//     reduction of argmax_parts_kernel: a maximum and a smallest index are
//     order-free);
//   the embedding row: bf16(s * q + b) per element, as embed_kernel;
//   the MTP norms: rms_row256's reduction over the row held in registers;
//   the verify row's norm inputs: u = bf16(h * w) and the per-16-column sums of
//     h^2 with rms_parts_kernel's lane layout and DPP tree.
#include "qvex_common.h"
#include "rms_row.h"

namespace {

constexpr int IN_T = 1024;   // threads per block (the argmax reads up to 16384 tiles per round)
constexpr int IN_PER = 16;   // tile pairs per thread per round

// The token of one row from its per-tile (max, first index) pairs, in every thread.
__device__ int block_argmax(const float* __restrict__ parts, int tiles, float* sh_v, int* sh_j) {
  const int t = threadIdx.x;
  const float2* p = reinterpret_cast<const float2*>(parts);
  float bv = -__builtin_inff();
  int bj = 0x7fffffff;
  for (int q0 = 0; q0 < tiles; q0 += IN_T * IN_PER) {
    float2 v[IN_PER];
#pragma unroll
    for (int i = 0; i < IN_PER; ++i) {
      const int q = q0 + t + IN_T * i;
      v[i] = q < tiles ? p[q] : make_float2(-__builtin_inff(), __int_as_float(0x7fffffff));
    }
#pragma unroll
    for (int i = 0; i < IN_PER; ++i) {
      const int j = __float_as_int(v[i].y);
      if (v[i].x > bv || (v[i].x == bv && j < bj)) {
        bv = v[i].x;
        bj = j;
      }
    }
  }
  const float m = wave_allmax(bv);
  int c = bv == m ? bj : 0x7fffffff;
  c = wave_allmin(c);
  if ((t & 63) == 0) {
    sh_v[t >> 6] = m;
    sh_j[t >> 6] = c;
  }
  __syncthreads();
  // the waves' (max, first index) pairs combined the same way by wave 0: the
  // largest value, then the smallest index holding it
  if (t < 64) {
    const float v = t < IN_T / 64 ? sh_v[t] : -__builtin_inff();
    const int j = t < IN_T / 64 ? sh_j[t] : 0x7fffffff;
    const float mm = wave_allmax(v);
    const int cc = wave_allmin(v == mm ? j : 0x7fffffff);
    if (t == 0) sh_j[IN_T / 64] = cc == 0x7fffffff ? 0 : cc;
  }
  __syncthreads();
  return sh_j[IN_T / 64];
}

// Embedding row `id` into registers: thread t < 256 holds chunks t + 256 c
// (8 elements each, one packed word), bf16-rounded as embed_kernel stores them.
__device__ __forceinline__ void embed_row_regs(int id, const uint32_t* __restrict__ w, const uint16_t* __restrict__ sc,
                                               const uint16_t* __restrict__ bi, int H, float (&v)[RMS_MAXC][8],
                                               u32x4 (&packed)[RMS_MAXC]) {
  const int t = threadIdx.x;
  const int KW = H / 8, G = H / 64;
  // every chunk's words, scales and biases requested first (chunks past the row
  // re-read chunk 0, never used), then dequantized: loads used inside their own
  // chunk's branch would each be waited for there, one round trip per chunk
  uint32_t wq[RMS_MAXC], sq[RMS_MAXC], bq[RMS_MAXC];
  if (t < 256) {
#pragma unroll
    for (int c = 0; c < RMS_MAXC; ++c) {
      const int wi = t + 256 * c, wc = wi < KW ? wi : 0;
      wq[c] = w[(size_t)id * KW + wc];
      sq[c] = sc[(size_t)id * G + wc / 8];
      bq[c] = bi[(size_t)id * G + wc / 8];
    }
  }
#pragma unroll
  for (int c = 0; c < RMS_MAXC; ++c) {
    const int wi = t + 256 * c;
    if (t < 256 && wi < KW) {
      const uint32_t word = wq[c];
      const float s = bf16_to_f32((uint16_t)sq[c]);
      const float b = bf16_to_f32((uint16_t)bq[c]);
      uint32_t pk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v0 = fmaf(s, (float)((word >> (8 * j)) & 0xF), b);
        const float v1 = fmaf(s, (float)((word >> (8 * j + 4)) & 0xF), b);
        pk[j] = pack_bf16x2(v0, v1);
      }
      packed[c] = u32x4{pk[0], pk[1], pk[2], pk[3]};
      unpack8(packed[c], v[c]);
    }
  }
}

__device__ __forceinline__ int clamp_id(int id, int V) { return id < 0 ? 0 : (id >= V ? V - 1 : id); }

// MTP draft-step input, grid (T, 2). Block (r, 0): token r (ids[r], or for T = 1
// the argmax of am_parts row *am_row, also stored to *ids_out), its embedding
// row, x_in[r, 0:H] = rms(embedding) * w_emb. Block (r, 1): x_in[r, H:2H] =
// rms(hid row (hid_sel ? *hid_sel : r)) * w_hid, and block (0, 1) advances the
// cache counters by *n_accept + extra (the previous step's commit).
__global__ __launch_bounds__(IN_T) void mtp_input_kernel(
    const int32_t* __restrict__ ids, const float* __restrict__ am_parts, int am_tiles,
    const int32_t* __restrict__ am_row, int32_t* __restrict__ ids_out, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi, int V, int H,
    const uint16_t* __restrict__ w_emb, const uint16_t* __restrict__ hid, long hid_stride,
    const int32_t* __restrict__ hid_sel, const uint16_t* __restrict__ w_hid, uint16_t* __restrict__ x_in,
    long x_stride, float eps, int32_t* __restrict__ counters, int ncnt, const int32_t* __restrict__ n_accept,
    int extra) {
  __shared__ float red[4];
  __shared__ float sh_v[IN_T / 64];
  __shared__ int sh_j[IN_T / 64 + 1];
  const int row = blockIdx.x;
  if (blockIdx.y == 1) {
    const int hr = hid_sel ? *hid_sel : row;
    rms_row256<false>(hid + (size_t)hr * hid_stride, nullptr, nullptr, w_hid, x_in + (size_t)row * x_stride + H, H,
                      eps, 1.0f, red);
    if (counters && row == 0 && threadIdx.x == 0) {
      const int add = (n_accept ? *n_accept : 0) + extra;
      for (int i = 0; i < ncnt; ++i) counters[i] += add;
    }
    return;
  }
  int id;
  if (am_parts) {
    id = block_argmax(am_parts + (size_t)(am_row ? *am_row : 0) * am_tiles * 2, am_tiles, sh_v, sh_j);
    if (threadIdx.x == 0) *ids_out = id;
  } else {
    id = ids[row];
  }
  id = clamp_id(id, V);
  float v[RMS_MAXC][8];
  u32x4 packed[RMS_MAXC];
  embed_row_regs(id, w, sc, bi, H, v, packed);
  rms_vals256(v, w_emb, x_in + (size_t)row * x_stride, H, eps, 1.0f, red);
}

// Verify input, one block per row: token r (ids[r]; for r == am_slot the argmax
// of am_parts row *am_row, stored back to ids[r]), the embedding row into h_out
// (the residual stream), then u = bf16(h * norm_w) and the per-16-column sums of
// h^2 (what the first layer's products read as their folded input norm).
__global__ __launch_bounds__(IN_T) void embed_parts_kernel(int32_t* __restrict__ ids, const float* __restrict__ am_parts,
                                                           int am_tiles, const int32_t* __restrict__ am_row,
                                                           int am_slot, const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ sc,
                                                           const uint16_t* __restrict__ bi, int V, int H,
                                                           const uint16_t* __restrict__ norm_w,
                                                           uint16_t* __restrict__ h_out, uint16_t* __restrict__ u_out,
                                                           float* __restrict__ parts) {
  __shared__ float sh_v[IN_T / 64];
  __shared__ int sh_j[IN_T / 64 + 1];
  __shared__ u32x4 rowbuf[256 * RMS_MAXC];   // the bf16 row (H <= 8192)
  const int row = blockIdx.x;
  int id;
  if (am_parts && row == am_slot) {
    id = block_argmax(am_parts + (size_t)(am_row ? *am_row : 0) * am_tiles * 2, am_tiles, sh_v, sh_j);
    if (threadIdx.x == 0) ids[row] = id;
  } else {
    id = ids[row];
  }
  id = clamp_id(id, V);
  float v[RMS_MAXC][8];
  u32x4 packed[RMS_MAXC];
  embed_row_regs(id, w, sc, bi, H, v, packed);
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < RMS_MAXC; ++c) {
    const int wi = t + 256 * c;
    if (t < 256 && wi < H / 8) {
      *reinterpret_cast<u32x4*>(h_out + (size_t)row * H + wi * 8) = packed[c];
      rowbuf[wi] = packed[c];
    }
  }
  __syncthreads();
  // rms_parts_kernel's layout: column n on lane n % 16 of a DPP row
  const uint16_t* rb = reinterpret_cast<const uint16_t*>(rowbuf);
  const int tiles = H / 16;
  // the norm weights of this thread's columns requested together, before the loop
  // (H <= 8192: at most 8 per thread; columns past H re-read column 0, never used)
  uint16_t nw[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int n = t + IN_T * q;
    nw[q] = norm_w[n < H ? n : 0];
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int n = t + IN_T * q;
    if (n < H) {
      const float hv = bf16_to_f32(rb[n]);
      const float sq = row16_allsum(hv * hv);
      u_out[(size_t)row * H + n] = f32_to_bf16(hv * bf16_to_f32(nw[q]));
      if ((n & 15) == 0) parts[(size_t)row * tiles + n / 16] = sq;
    }
  }
}

}  // namespace

extern "C" int qvex_mtp_input(const int32_t* ids, int T, const float* am_parts, int am_tiles, const int32_t* am_row,
                              int32_t* ids_out, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                              int V, int H, const uint16_t* w_emb, const uint16_t* hid, long hid_stride,
                              const int32_t* hid_sel, const uint16_t* w_hid, uint16_t* x_in, long x_stride,
                              float eps, int32_t* counters, int ncnt, const int32_t* n_accept, int extra,
                              void* stream) {
  const char* fn = "qvex_mtp_input";
  QVEX_CHECK_ARG(w && scales && biases && hid && x_in && (ids || am_parts), "%s: null pointer", fn);
  QVEX_CHECK_ARG(T >= 1 && V >= 1 && H >= 64 && H % 64 == 0 && H <= 256 * 8 * RMS_MAXC, "%s: T=%d V=%d H=%d", fn, T,
                 V, H);
  QVEX_CHECK_ARG(!am_parts || (T == 1 && ids_out && am_tiles >= 1), "%s: the argmax input needs T = 1 and ids_out",
                 fn);
  QVEX_CHECK_ARG(hid_stride >= H && hid_stride % 8 == 0 && x_stride >= 2 * H && x_stride % 8 == 0,
                 "%s: strides %ld / %ld", fn, hid_stride, x_stride);
  QVEX_CHECK_ARG(qvex_aligned(hid, 16) && qvex_aligned(x_in, 16) && qvex_aligned(w, 4) &&
                     (!w_emb || qvex_aligned(w_emb, 16)) && (!w_hid || qvex_aligned(w_hid, 16)) &&
                     (!am_parts || qvex_aligned(am_parts, 8)),
                 "%s: hid, x_in and the norm weights must be 16-byte aligned", fn);
  QVEX_CHECK_ARG(!counters || (ncnt >= 1 && ncnt <= 64), "%s: ncnt=%d", fn, ncnt);
  hipLaunchKernelGGL(mtp_input_kernel, dim3(T, 2), dim3(IN_T), 0, (hipStream_t)stream, ids, am_parts, am_tiles,
                     am_row, ids_out, w, scales, biases, V, H, w_emb, hid, hid_stride, hid_sel, w_hid, x_in, x_stride,
                     eps, counters, ncnt, n_accept, extra);
  QVEX_CHECK_LAUNCH(fn);
  return QVEX_OK;
}

extern "C" int qvex_embed_rms_parts(int32_t* ids, int L, const float* am_parts, int am_tiles, const int32_t* am_row,
                                    int am_slot, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                                    int V, int H, const uint16_t* norm_w, uint16_t* h_out, uint16_t* u_out,
                                    float* parts, void* stream) {
  const char* fn = "qvex_embed_rms_parts";
  QVEX_CHECK_ARG(ids && w && scales && biases && norm_w && h_out && u_out && parts, "%s: null pointer", fn);
  QVEX_CHECK_ARG(L >= 1 && V >= 1 && H >= 64 && H % 64 == 0 && H <= 256 * 8 * RMS_MAXC, "%s: L=%d V=%d H=%d", fn, L,
                 V, H);
  QVEX_CHECK_ARG(!am_parts || (am_slot >= 0 && am_slot < L && am_tiles >= 1), "%s: am_slot=%d outside 0..%d", fn,
                 am_slot, L - 1);
  QVEX_CHECK_ARG(qvex_aligned(h_out, 16) && qvex_aligned(w, 4) && (!am_parts || qvex_aligned(am_parts, 8)),
                 "%s: h_out must be 16-byte aligned", fn);
  hipLaunchKernelGGL(embed_parts_kernel, dim3(L), dim3(IN_T), 0, (hipStream_t)stream, ids, am_parts, am_tiles, am_row,
                     am_parts ? am_slot : -1, w, scales, biases, V, H, norm_w, h_out, u_out, parts);
  QVEX_CHECK_LAUNCH(fn);
  return QVEX_OK;
}
