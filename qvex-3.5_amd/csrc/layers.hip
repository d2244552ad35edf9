// Verify-forward glue kernels of the Qwen3.5 hybrid layer stack.
//
// Reference (engine/model.py): QEmbedding (121-130), mx.fast.rms_norm
// (218-219, 276-277, 314-316, 335), _swiglu (133-135), _gated_rmsnorm (138-143),
// GatedDeltaNet conv1d + SiLU + q/k norms (257-277), Attention q/k norm +
// partial RoPE + KV append + SDPA + sigmoid gate (210-232). All arithmetic is
// fp32 with bf16 storage; each kernel rounds its outputs to bf16 once.
//
// Layout: activations are row-major [rows, features] bf16; KV caches are
// [Hkv, cap, D] bf16 per layer (one contiguous key run per kv head); the
// GDN conv input window [3 + T, C] is kept per call so that the conv state
// after L accepted tokens is rows L..L+2 of it (a pointer pick on rollback).
#include "qvex_common.h"
#include "rms_row.h"

#include <math.h>

#include <algorithm>

namespace {

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------- embedding gather + dequant

// out[l, k] = bf16(s[id, k/64] * q[id, k] + b[id, k/64]); one block per token.
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ ids, const uint32_t* __restrict__ w,
                                                    const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi,
                                                    uint16_t* __restrict__ out, int V, int H) {
  const int l = blockIdx.x;
  int id = ids[l];
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);
  const int KW = H / 8, G = H / 64;
  const uint32_t* wr = w + (size_t)id * KW;
  for (int wi = threadIdx.x; wi < KW; wi += blockDim.x) {
    const uint32_t word = wr[wi];
    const int g = wi / 8;
    const float s = bf16_to_f32(sc[(size_t)id * G + g]);
    const float b = bf16_to_f32(bi[(size_t)id * G + g]);
    u32x4 o;
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v0 = fmaf(s, (float)((word >> (8 * j)) & 0xF), b);
      const float v1 = fmaf(s, (float)((word >> (8 * j + 4)) & 0xF), b);
      pk[j] = pack_bf16x2(v0, v1);
    }
    o.x = pk[0]; o.y = pk[1]; o.z = pk[2]; o.w = pk[3];
    *reinterpret_cast<u32x4*>(out + (size_t)l * H + wi * 8) = o;
  }
}

// ---------------------------------------------------------------- RMSNorm family
//
// One 256-thread block per row (rms_row256 in rms_row.h); with ADD the row is
// first h = bf16(x + delta), stored, and normalised.
template <bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, long x_stride,
                                                      const uint16_t* __restrict__ delta, long d_stride,
                                                      uint16_t* __restrict__ h_out, long h_stride,
                                                      const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                      long o_stride, int R, int D, float eps, float scale) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  rms_row256<ADD>(x + row * x_stride, ADD ? delta + row * d_stride : nullptr, ADD ? h_out + row * h_stride : nullptr,
                  w, out + row * o_stride, D, eps, scale, red);
}

// Two independent row sets in one launch (grid.y selects the set): the MTP
// head's two input norms, each written into its half of the fc input.
__global__ __launch_bounds__(256) void rmsnorm_pair_kernel(const uint16_t* __restrict__ x0, long x0_stride,
                                                           const uint16_t* __restrict__ w0,
                                                           uint16_t* __restrict__ out0,
                                                           const uint16_t* __restrict__ x1, long x1_stride,
                                                           const uint16_t* __restrict__ w1,
                                                           uint16_t* __restrict__ out1, long o_stride, int D,
                                                           float eps) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const bool second = blockIdx.y != 0;
  rms_row256<false>((second ? x1 : x0) + row * (second ? x1_stride : x0_stride), nullptr, nullptr,
                    second ? w1 : w0, (second ? out1 : out0) + row * o_stride, D, eps, 1.0f, red);
}

// ---------------------------------------------------------------- GDN: conv1d + SiLU + q/k norm
//
// The conv input history is a ring of R rows per layer keyed by the token count
// p = *pos: the state is rows (p-3, p-2, p-1) mod R, new token t goes to row
// (p + t) mod R. Window row j of token t is ring[(p + t - (K-1) + j) mod R] for
// t + j < K-1, else proj[t + j - (K-1)]. Keeping L tokens is p += L, so rollback
// moves no data. conv[t, c] = sum_j window[t + j, c] * cw[c, j]
// (cross-correlation, MLX conv1d with groups = C); silu; q and k heads
// rms-normalised (no weight, eps) and scaled; b, a copied out of the
// projection row into contiguous [T, Hv] arrays.
// Grid (T, C / 512); block 256 = 4 waves; each wave owns one 128-channel head
// with 2 channels per lane, so the head's norm is one wave reduction.
__global__ __launch_bounds__(256) void conv_silu_qk_kernel(
    const uint16_t* __restrict__ proj, long p_stride, uint16_t* __restrict__ ring, int R,
    const int32_t* __restrict__ pos, const uint16_t* __restrict__ cw, int KC, uint16_t* __restrict__ q,
    uint16_t* __restrict__ k, uint16_t* __restrict__ v, uint16_t* __restrict__ a_out,
    uint16_t* __restrict__ b_out, int T, int C, int key_dim, int Hv, int ab_off, float q_scale,
    float k_scale, float eps) {
  const int t = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int head = blockIdx.y * 4 + wave;      // 128-channel head index over C
  const int c0 = head * 128 + 2 * lane;
  if (c0 >= C) return;
  const int W = KC - 1;  // state rows
  const long p0 = *pos;
  float acc0 = 0.0f, acc1 = 0.0f;
  for (int j = 0; j < KC; ++j) {
    const int r = t + j;   // window row
    uint32_t p;
    if (r < W) {
      long rr = (p0 + r - W) % R;
      if (rr < 0) rr += R;
      p = *reinterpret_cast<const uint32_t*>(ring + rr * C + c0);
    } else {
      p = *reinterpret_cast<const uint32_t*>(proj + (size_t)(r - W) * p_stride + c0);
    }
    acc0 = fmaf(bf16_lo(p), bf16_to_f32(cw[(size_t)c0 * KC + j]), acc0);
    acc1 = fmaf(bf16_hi(p), bf16_to_f32(cw[(size_t)(c0 + 1) * KC + j]), acc1);
  }
  {
    long rr = (p0 + t) % R;
    if (rr < 0) rr += R;
    *reinterpret_cast<uint32_t*>(ring + rr * C + c0) =
        *reinterpret_cast<const uint32_t*>(proj + (size_t)t * p_stride + c0);
  }
  float s0 = silu(acc0), s1 = silu(acc1);
  if (c0 < 2 * key_dim) {
    // q or k head: weightless RMSNorm over the 128 channels, then the scale
    float ss = wave_allsum(fmaf(s0, s0, s1 * s1));
    const float inv = rsqrtf(ss / 128.0f + eps);
    const bool isq = c0 < key_dim;
    const float sc = isq ? q_scale : k_scale;
    s0 = s0 * inv * sc;
    s1 = s1 * inv * sc;
    uint16_t* dst = isq ? q + (size_t)t * key_dim + c0 : k + (size_t)t * key_dim + (c0 - key_dim);
    *reinterpret_cast<uint32_t*>(dst) = pack_bf16x2(s0, s1);
  } else {
    const int vd = C - 2 * key_dim;
    *reinterpret_cast<uint32_t*>(v + (size_t)t * vd + (c0 - 2 * key_dim)) = pack_bf16x2(s0, s1);
  }
  if (blockIdx.y == 0 && threadIdx.x < Hv) {
    b_out[(size_t)t * Hv + threadIdx.x] = proj[(size_t)t * p_stride + ab_off + threadIdx.x];
    a_out[(size_t)t * Hv + threadIdx.x] = proj[(size_t)t * p_stride + ab_off + Hv + threadIdx.x];
  }
}

// ---------------------------------------------------------------- gated RMSNorm
// out = bf16(silu(z) * bf16(w * (y * rsqrt(mean(y^2) + eps)))), rows of D = 128.
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const uint16_t* __restrict__ y,
                                                            const uint16_t* __restrict__ z, long z_stride,
                                                            int heads, const uint16_t* __restrict__ w,
                                                            uint16_t* __restrict__ out, int R, int D, float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= R) return;
  const int t = row / heads, h = row % heads;
  const uint16_t* yr = y + (size_t)row * D;
  const uint16_t* zr = z + (size_t)t * z_stride + (size_t)h * D;
  float ss = 0.0f;
  for (int i = 2 * lane; i < D; i += 128) {
    const uint32_t p = *reinterpret_cast<const uint32_t*>(yr + i);
    ss = fmaf(bf16_lo(p), bf16_lo(p), fmaf(bf16_hi(p), bf16_hi(p), ss));
  }
  ss = wave_allsum(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
  for (int i = 2 * lane; i < D; i += 128) {
    const uint32_t p = *reinterpret_cast<const uint32_t*>(yr + i);
    const uint32_t wp = *reinterpret_cast<const uint32_t*>(w + i);
    const uint32_t zp = *reinterpret_cast<const uint32_t*>(zr + i);
    const float n0 = bf16_to_f32(f32_to_bf16(bf16_lo(wp) * (bf16_lo(p) * inv)));
    const float n1 = bf16_to_f32(f32_to_bf16(bf16_hi(wp) * (bf16_hi(p) * inv)));
    const float z0 = bf16_lo(zp), z1 = bf16_hi(zp);
    *reinterpret_cast<uint32_t*>(out + (size_t)row * D + i) = pack_bf16x2(silu(z0) * n0, silu(z1) * n1);
  }
}

// ---------------------------------------------------------------- SwiGLU
// out[l, i] = silu(gu[l, i]) * gu[l, I + i]
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                     int L, int I) {
  const long n2 = (long)L * I / 2;
  for (long p = (long)blockIdx.x * blockDim.x + threadIdx.x; p < n2; p += (long)gridDim.x * blockDim.x) {
    const long e = 2 * p;
    const int l = (int)(e / I), i = (int)(e % I);
    const uint32_t g = *reinterpret_cast<const uint32_t*>(gu + (size_t)l * 2 * I + i);
    const uint32_t u = *reinterpret_cast<const uint32_t*>(gu + (size_t)l * 2 * I + I + i);
    *reinterpret_cast<uint32_t*>(out + e) =
        pack_bf16x2(silu(bf16_lo(g)) * bf16_lo(u), silu(bf16_hi(g)) * bf16_hi(u));
  }
}

__global__ __launch_bounds__(256) void bf16_to_f32_kernel(const uint16_t* __restrict__ in, float* __restrict__ out,
                                                          long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    out[i] = bf16_to_f32(in[i]);
}

// KV cache layouts, tiled so that every load of the attention kernels reads
// 1 KiB of consecutive bytes per wave instruction (cap a multiple of 32):
//   K [Hkv][cap / 16][D / 32][64][8]: key p, dim d at block p / 16, step d / 32,
//     lane 16 ((d % 32) / 8) + p % 16, element d % 8 -- exactly the B operand of
//     the score MFMA (lane l: key l % 16, dims 32 step + 8 (l / 16) .. +7);
//   V [Hkv][cap / 32][D][32]: key p, dim d at block p / 32, row d, column p % 32
//     -- the B operand of the P.V MFMA (lane l: dim l % 16 of a 16-dim tile, keys
//     8 (l / 16) .. +7 of a 32-key block).
__host__ __device__ __forceinline__ size_t kt_index(int kh, int cap, int D, int p, int d) {
  return ((((size_t)kh * (cap / 16) + p / 16) * (D / 32) + d / 32) * 64 + ((d % 32) / 8) * 16 + p % 16) * 8 + d % 8;
}
__host__ __device__ __forceinline__ size_t vt_index(int kh, int cap, int D, int p, int d) {
  return (((size_t)kh * (cap / 32) + p / 32) * D + d) * 32 + p % 32;
}

// ---------------------------------------------------------------- attention: q/k norm + partial RoPE + KV append
//
// proj row l = [Hq x (q D | gate D) | Hkv x k D | Hkv x v D]. One wave per
// (token, head); lane holds elements lane + 64 i. RoPE (NeoX form, the
// non-traditional mx.fast.rope): for i < rot/2, (x_i, x_{i+rot/2}) rotated by
// pos * theta^(-2i/rot); dims >= rot pass through. pos = *pos0 + l.
// PER = D / 64 elements per lane, a template parameter so that every load of the
// wave (row, norm weights, the V row) is issued before the first is waited on.
// With a table of rope_table_kernel (rows >= pos + 1) the lane's (cos, sin) is
// loaded as soon as the position arrives, alongside the row, instead of being
// evaluated after the norm (powf and sincosf of a large angle: ~1 us of the
// wave's ~2 us); the table holds the same values, so the results are the same.
template <int PER>
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ proj, long p_stride, const uint16_t* __restrict__ q_norm,
    const uint16_t* __restrict__ k_norm, const int32_t* __restrict__ pos0, int Hq, int Hkv, int D,
    int rot, float theta, float eps, uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, int cap, const float2* __restrict__ rope, int rope_rows) {
  const int l = blockIdx.x, h = blockIdx.y;  // h < Hq: query head; else kv head h - Hq
  const int lane = threadIdx.x;
  const int pos = *pos0 + l;
  const int half = rot / 2;
  const bool tab = rope != nullptr && pos >= 0 && pos < rope_rows;   // uniform over the wave
  float2 cs_tab = make_float2(1.0f, 0.0f);
  if (tab && lane < rot) cs_tab = rope[(size_t)pos * half + lane % half];
  const bool isq = h < Hq;
  const int kh = h - Hq;
  const uint16_t* src = isq ? proj + (size_t)l * p_stride + (size_t)h * 2 * D
                            : proj + (size_t)l * p_stride + (size_t)Hq * 2 * D + (size_t)kh * D;
  const uint16_t* nw = isq ? q_norm : k_norm;
  const uint16_t* vs = proj + (size_t)l * p_stride + (size_t)Hq * 2 * D + (size_t)Hkv * D + (size_t)kh * D;
  float x[PER];
  uint16_t wv[PER], vv[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    x[i] = bf16_to_f32(src[lane + 64 * i]);
    wv[i] = nw[lane + 64 * i];
    vv[i] = isq ? (uint16_t)0 : vs[lane + 64 * i];
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) ss = fmaf(x[i], x[i], ss);
  ss = wave_allsum(ss);
  const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
  for (int i = 0; i < PER; ++i) x[i] = bf16_to_f32(f32_to_bf16(bf16_to_f32(wv[i]) * (x[i] * inv)));
  // rotary part lives in element slot 0 (lane < 64 <= rot requires rot <= 64);
  // lane i < half pairs with lane i + half (an explicit index: an xor by half
  // pairs the right lanes only when half is a power of two)
  if (rot > 0) {
    const float partner = __shfl(x[0], lane < half ? lane + half : lane - half, 64);
    if (lane < rot) {
      float sn, cs;
      if (tab) {
        cs = cs_tab.x;
        sn = cs_tab.y;
      } else {
        const int i = lane % half;
        const float inv_freq = powf(theta, -2.0f * (float)i / (float)rot);
        sincosf((float)pos * inv_freq, &sn, &cs);
      }
      x[0] = lane < half ? x[0] * cs - partner * sn : partner * sn + x[0] * cs;
    }
  }
  if (isq) {
    uint16_t* dst = q_out + ((size_t)l * Hq + h) * D;
#pragma unroll
    for (int i = 0; i < PER; ++i) dst[lane + 64 * i] = f32_to_bf16(x[i]);
  } else if (pos >= 0 && pos < cap) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      k_cache[kt_index(kh, cap, D, pos, lane + 64 * i)] = f32_to_bf16(x[i]);
      v_cache[vt_index(kh, cap, D, pos, lane + 64 * i)] = vv[i];
    }
  }
}

// ---------------------------------------------------------------- attention: split-K over the cache (MFMA)
//
// One wave per (kv head, query tile, key split). The tile's 16 rows are GQ query
// heads x QT positions (row r = head r / QT, position tile*QT + r % QT); query l
// sees keys [0, *pos0 + l]. For each 16-key block:
//   S[16 x 16] = Q[16 x D] K^T with v_mfma_f32_16x16x32_bf16 (D/32 steps; lane l
//   holds Q row l%16 dims 8(l/16).. and key l%16 of the block, same dims);
//   the accumulator puts rows 4(l/16)+r in lane l at key l%16, so row max / sum
//   are 16-lane DPP reductions; online softmax rescales O in place;
//   P (bf16) goes through the wave's own LDS tile into the A layout, and O[16 x D] += P V
//   with V stored dim-major, so lane l reads 8 consecutive keys of dim l%16.
// Partials (m, l, O) per row go to the workspace; attn_combine merges splits.
typedef __bf16 att_bf16x8 __attribute__((ext_vector_type(8)));
typedef float att_f32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dpp_row16(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_row16<0xB1>(v));
  v = fmaxf(v, dpp_row16<0x4E>(v));
  v = fmaxf(v, dpp_row16<0x124>(v));
  v = fmaxf(v, dpp_row16<0x128>(v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_row16<0xB1>(v);
  v += dpp_row16<0x4E>(v);
  v += dpp_row16<0x124>(v);
  v += dpp_row16<0x128>(v);
  return v;
}

__device__ __forceinline__ att_bf16x8 as_att8(const u32x4 v) { return __builtin_bit_cast(att_bf16x8, v); }

// One block of 4 waves per (kv head, 16-row tile, split of keys_per_split keys).
// Per iteration each wave takes the next 32 keys of the split (the 4 waves cover
// 128 adjacent keys), loads their K rows and dim-major V columns in one round
// trip, scores them with MFMA, runs an online softmax per row and accumulates
// P V with MFMA. The 4 waves' (max, sum, O) are then merged in LDS and written as
// one partial per block: ws [kv head][tile][split] = ([16 rows][m, l], [16 rows][O[D]]).
template <int D>
__global__ __launch_bounds__(256) void attn_mfma_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ pos0, int L, int Hq, int Hkv, int cap, int QT, int keys_per_split, int known_keys,
    float scale, float* __restrict__ ws) {
  constexpr int KS = D / 32;     // MFMA steps over head dims
  constexpr int NT = D / 16;     // 16-dim output tiles of O
  const int kh = blockIdx.x, tile = blockIdx.y, split = blockIdx.z;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int GQ = Hq / Hkv;
  const int k_lo = split * keys_per_split;
  const uint16_t* kbase = k_cache + (size_t)kh * cap * D;
  const uint16_t* vbase = v_cache + (size_t)kh * D * cap;

  // K keys kb + 16h + li and V keys kb + 8lg .. +7 of a 128-key window (tiled
  // layouts above), issued together (keys past k_hi are masked out of the
  // softmax and get P = 0). The first window does not depend on the device
  // position, so its loads go out before the position is read (this kernel runs
  // the prefill, where the grid holds only visible splits).
  // A operand: Q row li, dims step*32 + 8*lg .. +7 (the 1/sqrt(D) scale is applied
  // to the scores). Requested first: loads complete in order, so the scores can
  // start once Q and K are in while the V columns still stream
  u32x4 qa[KS];
  {
    const int g = li / QT, lq = tile * QT + li % QT;
    const bool ok = g < GQ && lq < L;
    const uint16_t* qp = q + ((size_t)(ok ? lq : 0) * Hq + kh * GQ + (ok ? g : 0)) * D + 8 * lg;
#pragma unroll
    for (int s = 0; s < KS; ++s) qa[s] = ok ? load16(qp + 32 * s) : u32x4{0, 0, 0, 0};
  }
  u32x4 kr[2][KS], vr[NT];
  auto load_kv = [&](int kb) {
    kb = min(kb, cap - 32);      // whole 32-key blocks in bounds (keys past k_hi are masked)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint16_t* kp = kbase + ((size_t)(kb / 16 + h) * KS * 64 + lane) * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) kr[h][s] = load16(kp + (size_t)s * 512);
    }
    const uint16_t* vp = vbase + (size_t)(kb / 32) * D * 32 + li * 32 + 8 * lg;
#pragma unroll
    for (int t = 0; t < NT; ++t) vr[t] = load16(vp + (size_t)t * 512);
  };
  // splits below known_keys hold visible keys on every call: their first
  // window goes out before the position is read; the others read it first and
  // exit without loading when their keys are past it (a captured graph spans the
  // whole capacity)
  const bool early = k_lo < known_keys;      // uniform over the block
  if (early) load_kv(k_lo + 32 * w);

  const int p0 = *pos0;
  const int kend_tile = p0 + min(L, (tile + 1) * QT);
  const int k_hi = min(k_lo + keys_per_split, kend_tile);
  if (k_lo >= k_hi) return;      // split past the visible keys: the combine never reads it
  if (!early) load_kv(k_lo + 32 * w);

  __shared__ __align__(16) uint32_t ps[4][16][20];   // per-wave P tile, bf16 pairs [row][key pair], 80-byte rows
  __shared__ float4 obv[4][NT][4][16];   // per-wave O for the merge: [wave][dim tile][row group][dim] x 4 rows
  __shared__ float ml[4][16][2];         // per-wave (m, l)
  __shared__ __align__(16) float fac[4][16];   // merge factors e^{m_w - m}

  // the 4 rows this lane owns in accumulator layout: r = 4*lg + j
  int rlim[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * lg + j;
    const int g = r / QT, lq = tile * QT + r % QT;
    rlim[j] = (g < GQ && lq < L) ? p0 + lq : -1;     // last visible key, -1 = dead row
  }

  float m_r[4], l_r[4];
  att_f32x4 o[NT];
#pragma unroll
  for (int j = 0; j < 4; ++j) { m_r[j] = -INFINITY; l_r[j] = 0.0f; }
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = att_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int n_it = (k_hi - k_lo + 127) / 128;          // uniform over the block (LDS barriers below)
  for (int it = 0; it < n_it; ++it) {
    const int kb = k_lo + 128 * it + 32 * w;
    if (it > 0) load_kv(kb);

    att_f32x4 sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      att_f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < KS; ++s) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_att8(qa[s]), as_att8(kr[h][s]), c, 0, 0, 0);
      sc[h] = c;
    }
    // online softmax per row (row = 4*lg + j, keys across the 16 lanes of the group)
    float p[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float mx = -INFINITY;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int key = kb + 16 * h + li;
        const bool vis = key < k_hi && key <= rlim[j];
        sc[h][j] = vis ? sc[h][j] * scale : -INFINITY;
        mx = fmaxf(mx, sc[h][j]);
      }
      mx = row16_max(mx);
      const float mnew = fmaxf(m_r[j], mx);
      const float corr = (mnew == -INFINITY) ? 1.0f : expf(m_r[j] - mnew);
      float sum = 0.0f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        p[h][j] = (sc[h][j] == -INFINITY) ? 0.0f : expf(sc[h][j] - mnew);
        sum += p[h][j];
      }
      l_r[j] = l_r[j] * corr + row16_sum(sum);
      m_r[j] = mnew;
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t][j] *= corr;
    }
    // P to the A layout through this wave's own LDS tile (in-order LDS within
    // the wave: no block barrier), read back as one 16-byte row slice
    {
      uint16_t* ps16 = reinterpret_cast<uint16_t*>(&ps[w][0][0]);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) ps16[(4 * lg + j) * 40 + 16 * h + li] = f32_to_bf16(p[h][j]);
    }
    u32x4 pa;
    __builtin_memcpy(&pa, &ps[w][li][4 * lg], sizeof(pa));   // alias-safe (the tile is written as bf16)
    // O += P V: B operand = keys kb + 8*lg .. +7 of dim t*16 + li
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_att8(pa), as_att8(vr[t]), o[t], 0, 0, 0);
  }

  // merge the 4 waves: m = max_w m_w, l = sum_w l_w e^{m_w-m}, O = sum_w O_w e^{m_w-m} (fixed order w = 0..3).
  // A lane's 4 rows of a dim go to LDS as one float4 (16 b128 writes per lane)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * lg + j;
    if (li == 0) { ml[w][r][0] = m_r[j]; ml[w][r][1] = l_r[j]; }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) obv[w][t][lg][li] = make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
  __syncthreads();
  float* wsb = ws + (((size_t)kh * gridDim.y + tile) * gridDim.z + split) * 16 * (D + 2);
  if (threadIdx.x < 16) {
    const int r = threadIdx.x;
    const float m = fmaxf(fmaxf(ml[0][r][0], ml[1][r][0]), fmaxf(ml[2][r][0], ml[3][r][0]));
    float l = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float f = ml[v][r][0] == -INFINITY ? 0.0f : expf(ml[v][r][0] - m);
      fac[v][r] = f;
      l += ml[v][r][1] * f;
    }
    wsb[2 * r] = m;
    wsb[2 * r + 1] = l;
  }
  __syncthreads();
  // thread (row group rg, dim d): rows 4 rg .. 4 rg + 3 of dim d, one b128 read per wave
  for (int e = threadIdx.x; e < 4 * D; e += 256) {
    const int rg = e / D, d = e % D, t = d >> 4, dl = d & 15;
    float4 ov[4], fv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      ov[v] = obv[v][t][rg][dl];
      fv[v] = *reinterpret_cast<const float4*>(&fac[v][4 * rg]);
    }
    const float a0 = ((ov[0].x * fv[0].x + ov[1].x * fv[1].x) + ov[2].x * fv[2].x) + ov[3].x * fv[3].x;
    const float a1 = ((ov[0].y * fv[0].y + ov[1].y * fv[1].y) + ov[2].y * fv[2].y) + ov[3].y * fv[3].y;
    const float a2 = ((ov[0].z * fv[0].z + ov[1].z * fv[1].z) + ov[2].z * fv[2].z) + ov[3].z * fv[3].z;
    const float a3 = ((ov[0].w * fv[0].w + ov[1].w * fv[1].w) + ov[2].w * fv[2].w) + ov[3].w * fv[3].w;
    float* op = wsb + 32 + (size_t)(4 * rg) * D + d;
    op[0] = a0;
    op[D] = a1;
    op[2 * D] = a2;
    op[3 * D] = a3;
  }
}

// (cos, sin) of p * theta^(-2i/rot) for positions p < rows and i < rot / 2, as
// qk_norm_rope_kernel evaluates them (same expressions, so the same bits):
// table[p][i] = (cos, sin).
__global__ __launch_bounds__(256) void rope_table_kernel(int rot, float theta, long n, float2* __restrict__ table) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int half = rot / 2;
  const int p = (int)(e / half), i = (int)(e % half);
  const float inv_freq = powf(theta, -2.0f * (float)i / (float)rot);
  float sn, cs;
  sincosf((float)p * inv_freq, &sn, &cs);
  table[e] = make_float2(cs, sn);
}

// ---------------------------------------------------------------- attention: decode step, fused
//
// The decode / verify step (L <= 8 new tokens) as one launch plus the combine.
// Each block (kv head, 16-row tile, split) first reads the token count, so the
// splits past the visible keys exit before loading anything (a captured graph is
// sized for the whole capacity), then does for itself what qk_norm_rope does:
//   Q: its 16 rows from the projection row, RMS-normed (q_norm) and rotated, into
//      LDS in the A-operand layout (16 threads per row, D / 16 dims each; the row
//      sum of squares is a DPP sum over the 16 threads; rotation partners are
//      rot / 2 dims apart, D / 16 divides rot / 2, so a partner is a lane shift);
//   new keys p0 .. p0 + L - 1 (blocks whose split holds any): K normed (k_norm)
//      and rotated, V copied, into LDS; the lanes whose cache keys are new take
//      them from there, and the block of the split holding key p0 + j and of the
//      tile (j / QT) whose rows first see it writes it to the caches (each key
//      written once; every block computes the same bits).
// Rounding follows qk_norm_rope: bf16(w * (x * rstd)), rotation in fp32 on
// those values, bf16 result (the sum of squares runs in another order).
// The key loop, softmax, merge and partials are attn_mfma_partial_kernel's.
template <int D>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const int32_t* __restrict__ pos0, const uint16_t* __restrict__ proj, long p_stride,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache, float* __restrict__ ws, const float2* __restrict__ rope, int rope_rows, int L,
    int Hq, int Hkv, int cap, int QT, int keys_per_split, int rot, float eps, float scale) {
  constexpr int KS = D / 32;       // MFMA steps over head dims
  constexpr int NT = D / 16;       // 16-dim output tiles of O
  constexpr int DPT = D / 16;      // dims per thread in the norm passes
  constexpr int QROW = D + 8;      // bf16 per LDS row (16-byte pad: the 16 rows of an A read hit distinct banks)
  const int kh = blockIdx.x, tile = blockIdx.y, split = blockIdx.z;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int GQ = Hq / Hkv;
  const int k_lo = split * keys_per_split;
  const int p0 = *pos0;

  // raw inputs of the norm pass, requested before the position is waited for:
  // thread (row nr = tid / 16, slice nc = tid % 16) -> dims nc * DPT .. + DPT - 1
  const int nr = threadIdx.x >> 4, nc = threadIdx.x & 15;
  const int qg = nr / QT, qlq = tile * QT + nr % QT;
  const bool qok = qg < GQ && qlq < L;
  u32x4 qraw[DPT / 8], qwt[DPT / 8];
  {
    const uint16_t* src = proj + (size_t)(qok ? qlq : 0) * p_stride + (size_t)(kh * GQ + (qok ? qg : 0)) * 2 * D + nc * DPT;
#pragma unroll
    for (int i = 0; i < DPT / 8; ++i) {
      qraw[i] = load16(src + 8 * i);
      qwt[i] = load16(q_norm + nc * DPT + 8 * i);
    }
  }
  // the new keys' raw K and V slices (row nr = token nr; rows past L re-read the
  // last), loaded with no condition and before the K / V window: a later or
  // conditional load would make the norm pass wait for the whole window
  u32x4 kraw[DPT / 8], kwt[DPT / 8], vraw[DPT / 8];
  {
    const uint16_t* src = proj + (size_t)min(nr, L - 1) * p_stride + (size_t)Hq * 2 * D + (size_t)kh * D + nc * DPT;
#pragma unroll
    for (int i = 0; i < DPT / 8; ++i) {
      kraw[i] = load16(src + 8 * i);
      vraw[i] = load16(src + (size_t)Hkv * D + 8 * i);
      kwt[i] = load16(k_norm + nc * DPT + 8 * i);
    }
  }

  const int kend_tile = p0 + min(L, (tile + 1) * QT);
  const int k_hi = min(k_lo + keys_per_split, kend_tile);
  if (k_lo >= k_hi) return;      // split past the visible keys: the combine never reads it
  const bool has_new = k_hi > max(p0, k_lo);   // this split holds keys of this call (uniform)
  // rotation (cos, sin) of this call's tokens (the Q rows' positions are the new
  // keys' positions) from the table, requested before the K / V window so that
  // the norm pass waits only for them
  // (no condition: a load under a branch is waited for at the end of the
  // branch; the workspace stands in for the table when there is no rotation)
  const int half = rot / 2;
  const bool rthr = (int)threadIdx.x < L * half;
  const float2 rcs = [&]() {
    const int hs = max(half, 1), e = rthr ? (int)threadIdx.x : 0, j = e / hs, i = e % hs;
    const float2* src = half > 0 ? rope + (size_t)min(p0 + j, rope_rows - 1) * half + i
                                 : reinterpret_cast<const float2*>(ws);
    return *src;
  }();
  __builtin_amdgcn_sched_barrier(0);     // the table load goes out before the K / V window

  const uint16_t* kbase = k_cache + (size_t)kh * cap * D;
  const uint16_t* vbase = v_cache + (size_t)kh * D * cap;
  u32x4 kr[2][KS], vr[NT];
  auto load_kv = [&](int kb) {
    kb = min(kb, cap - 32);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint16_t* kp = kbase + ((size_t)(kb / 16 + h) * KS * 64 + lane) * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) kr[h][s] = load16(kp + (size_t)s * 512);
    }
    const uint16_t* vp = vbase + (size_t)(kb / 32) * D * 32 + li * 32 + 8 * lg;
#pragma unroll
    for (int t = 0; t < NT; ++t) vr[t] = load16(vp + (size_t)t * 512);
  };
  load_kv(k_lo + 32 * w);


  // LDS: Q rows, new K / V rows and the rotation table while the keys are
  // scored; the wave merge after the loop reuses it
  constexpr int OBV_BYTES = 4 * NT * 4 * 16 * 16;
  constexpr int TAB_BYTES = 2 * 8 * (D / 2) * 4;
  constexpr int PRE_BYTES = (16 + 2 * 8) * QROW * 2 + TAB_BYTES;
  constexpr int VT_BYTES = 2 * NT * 64 * 16;            // two waves' V operand tiles
  constexpr int LOOP_BYTES = PRE_BYTES + VT_BYTES;
  __shared__ __align__(16) unsigned char smem[OBV_BYTES > LOOP_BYTES ? OBV_BYTES : LOOP_BYTES];
  uint16_t* qs = reinterpret_cast<uint16_t*>(smem);               // [16][QROW]
  uint16_t* nk = qs + 16 * QROW;                                   // [8][QROW]
  uint16_t* nv = nk + 8 * QROW;                                    // [8][QROW]
  float* tab_c = reinterpret_cast<float*>(nv + 8 * QROW);          // [8][rot / 2] cos, then sin
  float* tab_s = tab_c + 8 * (D / 2);
  float4 (*obv)[NT][4][16] = reinterpret_cast<float4 (*)[NT][4][16]>(smem);
  __shared__ __align__(16) uint32_t ps[4][16][20];   // per-wave P tile, bf16 pairs [row][key pair], 80-byte rows
  __shared__ float ml[4][16][2];                      // per-wave (m, l)
  __shared__ __align__(16) float fac[4][16];          // merge factors e^{m_w - m}

  if (half > 0 && rthr) {
    const int j = threadIdx.x / half, i = threadIdx.x % half;
    tab_c[j * (D / 2) + i] = rcs.x;
    tab_s[j * (D / 2) + i] = rcs.y;
  }
  __syncthreads();

  // RMS norm + rotation of one 16-thread row slice (tok = its token's index in the call)
  // (the row's 16 threads are lanes of one wave: the normed slices go to the
  // row in LDS, each thread reads its rotation partner's slice back, and LDS
  // runs in order within a wave)
  auto norm_rope = [&](const u32x4 (&raw)[DPT / 8], const u32x4 (&wt)[DPT / 8], int tok, uint16_t* row) {
    float x[DPT], wv[DPT];
#pragma unroll
    for (int i = 0; i < DPT / 8; ++i) {
      const uint32_t r4[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
      const uint32_t w4[4] = {wt[i].x, wt[i].y, wt[i].z, wt[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * i + 2 * j] = bf16_lo(r4[j]);
        x[8 * i + 2 * j + 1] = bf16_hi(r4[j]);
        wv[8 * i + 2 * j] = bf16_lo(w4[j]);
        wv[8 * i + 2 * j + 1] = bf16_hi(w4[j]);
      }
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < DPT; ++e) ss = fmaf(x[e], x[e], ss);
    ss = row16_sum(ss);
    const float inv = rsqrtf(ss / (float)D + eps);
    auto store = [&](uint16_t* dst) {
#pragma unroll
      for (int i = 0; i < DPT / 8; ++i) {
        u32x4 o;
        o.x = (uint32_t)f32_to_bf16(x[8 * i]) | ((uint32_t)f32_to_bf16(x[8 * i + 1]) << 16);
        o.y = (uint32_t)f32_to_bf16(x[8 * i + 2]) | ((uint32_t)f32_to_bf16(x[8 * i + 3]) << 16);
        o.z = (uint32_t)f32_to_bf16(x[8 * i + 4]) | ((uint32_t)f32_to_bf16(x[8 * i + 5]) << 16);
        o.w = (uint32_t)f32_to_bf16(x[8 * i + 6]) | ((uint32_t)f32_to_bf16(x[8 * i + 7]) << 16);
        *reinterpret_cast<u32x4*>(dst + 8 * i) = o;
      }
    };
    const int d0 = nc * DPT;
#pragma unroll
    for (int e = 0; e < DPT; ++e) x[e] = bf16_to_f32(f32_to_bf16(wv[e] * (x[e] * inv)));
    store(row + d0);
    if (rot > 0) {
      const int pd0 = d0 < half ? d0 + half : d0 - half;    // partner slice (half % DPT == 0)
      const int i0 = d0 < rot ? d0 % half : 0;
      u32x4 pr[DPT / 8];
#pragma unroll
      for (int i = 0; i < DPT / 8; ++i) pr[i] = *reinterpret_cast<const u32x4*>(row + (d0 < rot ? pd0 : d0) + 8 * i);
#pragma unroll
      for (int e = 0; e < DPT; ++e) {
        const uint32_t pw = e % 8 < 2 ? pr[e / 8].x : e % 8 < 4 ? pr[e / 8].y : e % 8 < 6 ? pr[e / 8].z : pr[e / 8].w;
        const float partner = (e & 1) ? bf16_hi(pw) : bf16_lo(pw);
        const float cs = tab_c[tok * (D / 2) + i0 + e], sn = tab_s[tok * (D / 2) + i0 + e];
        const int d = d0 + e;
        const float r = d < half ? x[e] * cs - partner * sn : partner * sn + x[e] * cs;
        x[e] = d < rot ? r : x[e];
      }
      store(row + d0);
    }
  };
  if (qok) {
    norm_rope(qraw, qwt, qlq, qs + nr * QROW);
  } else {
#pragma unroll
    for (int i = 0; i < DPT / 8; ++i) *reinterpret_cast<u32x4*>(qs + nr * QROW + nc * DPT + 8 * i) = u32x4{0u, 0u, 0u, 0u};
  }
  if (has_new && nr < 8) {     // uniform per 16-thread row: the row16 sum stays within live lanes
    if (nr < L) {
      norm_rope(kraw, kwt, nr, nk + nr * QROW);
#pragma unroll
      for (int i = 0; i < DPT / 8; ++i) *reinterpret_cast<u32x4*>(nv + nr * QROW + nc * DPT + 8 * i) = vraw[i];
    }
  }
  __syncthreads();

  // the new keys to the caches: key p0 + j by the split holding it, in the tile whose rows first see it
  if (has_new) {
    for (int e = threadIdx.x; e < 8 * (D / 8); e += 256) {
      const int j = e / (D / 8), c8 = (e % (D / 8)) * 8, p = p0 + j;
      if (j < L && j / QT == tile && p >= k_lo && p < k_lo + keys_per_split && p < cap) {
        *reinterpret_cast<u32x4*>(k_cache + kt_index(kh, cap, D, p, c8)) =
            *reinterpret_cast<const u32x4*>(nk + j * QROW + c8);
#pragma unroll
        for (int q = 0; q < 8; ++q) v_cache[vt_index(kh, cap, D, p, c8 + q)] = nv[j * QROW + c8 + q];
      }
    }
  }

  u32x4 qa[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qa[s] = *reinterpret_cast<const u32x4*>(qs + li * QROW + 32 * s + 8 * lg);

  // the 4 rows this lane owns in accumulator layout: r = 4*lg + j
  int rlim[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * lg + j;
    const int g = r / QT, lq = tile * QT + r % QT;
    rlim[j] = (g < GQ && lq < L) ? p0 + lq : -1;     // last visible key, -1 = dead row
  }

  float m_r[4], l_r[4];
  att_f32x4 o[NT];
#pragma unroll
  for (int j = 0; j < 4; ++j) { m_r[j] = -INFINITY; l_r[j] = 0.0f; }
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = att_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int n_it = (k_hi - k_lo + 127) / 128;          // uniform over the block
  for (int it = 0; it < n_it; ++it) {
    const int kb = k_lo + 128 * it + 32 * w;
    if (it > 0) load_kv(kb);
    if (has_new && kb + 31 >= p0 && kb < p0 + L) {     // this wave's window holds new keys (uniform per wave)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = kb + 16 * h + li - p0;
        if (j >= 0 && j < L) {
#pragma unroll
          for (int s = 0; s < KS; ++s) kr[h][s] = *reinterpret_cast<const u32x4*>(nk + j * QROW + 32 * s + 8 * lg);
        }
      }
      // V: the window's B operands through a wave-private LDS tile, the new
      // keys' values written over theirs (at most two adjacent waves hold new
      // keys: tiles w & 1), read back; LDS is in order within a wave
      u32x4* vt = reinterpret_cast<u32x4*>(smem + PRE_BYTES) + (w & 1) * NT * 64;
#pragma unroll
      for (int t = 0; t < NT; ++t) vt[t * 64 + lane] = vr[t];
      uint16_t* vt16 = reinterpret_cast<uint16_t*>(vt);
      for (int e = lane; e < L * D; e += 64) {
        const int j = e / D, d = e % D, k = p0 + j - kb;
        if (k >= 0 && k < 32) vt16[((d >> 4) * 64 + (k >> 3) * 16 + (d & 15)) * 8 + (k & 7)] = nv[j * QROW + d];
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) vr[t] = vt[t * 64 + lane];
    }

    att_f32x4 sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      att_f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < KS; ++s) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_att8(qa[s]), as_att8(kr[h][s]), c, 0, 0, 0);
      sc[h] = c;
    }
    float p[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float mx = -INFINITY;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int key = kb + 16 * h + li;
        const bool vis = key < k_hi && key <= rlim[j];
        sc[h][j] = vis ? sc[h][j] * scale : -INFINITY;
        mx = fmaxf(mx, sc[h][j]);
      }
      mx = row16_max(mx);
      const float mnew = fmaxf(m_r[j], mx);
      const float corr = (mnew == -INFINITY) ? 1.0f : expf(m_r[j] - mnew);
      float sum = 0.0f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        p[h][j] = (sc[h][j] == -INFINITY) ? 0.0f : expf(sc[h][j] - mnew);
        sum += p[h][j];
      }
      l_r[j] = l_r[j] * corr + row16_sum(sum);
      m_r[j] = mnew;
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t][j] *= corr;
    }
    {
      uint16_t* ps16 = reinterpret_cast<uint16_t*>(&ps[w][0][0]);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) ps16[(4 * lg + j) * 40 + 16 * h + li] = f32_to_bf16(p[h][j]);
    }
    u32x4 pa;
    __builtin_memcpy(&pa, &ps[w][li][4 * lg], sizeof(pa));
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_att8(pa), as_att8(vr[t]), o[t], 0, 0, 0);
  }

  // merge the 4 waves as attn_mfma_partial_kernel does (the merge buffer reuses the Q / new-key LDS)
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * lg + j;
    if (li == 0) { ml[w][r][0] = m_r[j]; ml[w][r][1] = l_r[j]; }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) obv[w][t][lg][li] = make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
  __syncthreads();
  float* wsb = ws + (((size_t)kh * gridDim.y + tile) * gridDim.z + split) * 16 * (D + 2);
  if (threadIdx.x < 16) {
    const int r = threadIdx.x;
    const float m = fmaxf(fmaxf(ml[0][r][0], ml[1][r][0]), fmaxf(ml[2][r][0], ml[3][r][0]));
    float l = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float f = ml[v][r][0] == -INFINITY ? 0.0f : expf(ml[v][r][0] - m);
      fac[v][r] = f;
      l += ml[v][r][1] * f;
    }
    wsb[2 * r] = m;
    wsb[2 * r + 1] = l;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 4 * D; e += 256) {
    const int rg = e / D, d = e % D, t = d >> 4, dl = d & 15;
    float4 ov[4], fv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      ov[v] = obv[v][t][rg][dl];
      fv[v] = *reinterpret_cast<const float4*>(&fac[v][4 * rg]);
    }
    const float a0 = ((ov[0].x * fv[0].x + ov[1].x * fv[1].x) + ov[2].x * fv[2].x) + ov[3].x * fv[3].x;
    const float a1 = ((ov[0].y * fv[0].y + ov[1].y * fv[1].y) + ov[2].y * fv[2].y) + ov[3].y * fv[3].y;
    const float a2 = ((ov[0].z * fv[0].z + ov[1].z * fv[1].z) + ov[2].z * fv[2].z) + ov[3].z * fv[3].z;
    const float a3 = ((ov[0].w * fv[0].w + ov[1].w * fv[1].w) + ov[2].w * fv[2].w) + ov[3].w * fv[3].w;
    float* op = wsb + 32 + (size_t)(4 * rg) * D + d;
    op[0] = a0;
    op[D] = a1;
    op[2 * D] = a2;
    op[3 * D] = a3;
  }
}

// out[lq, (kh*GQ + g)*D + d] = bf16(sigmoid(gate) * sum_s o_s e^{m_s-m} / sum_s l_s e^{m_s-m})
// over the splits that hold visible keys (the count follows from the device position).
// One 256-thread block per (kv head, tile, row, slice of D / DS dims): NG groups of
// D / (4 DS) threads, thread (g, j) owns dims 4j..4j+3 of the slice for splits g,
// g + NG, ... The gate and the first CB splits of each thread (m, l and its 4
// values) are requested before the position is read; splits past the active count
// are dropped by selects (the workspace may hold anything there). Each thread
// merges its splits against its own maximum, the groups then merge in LDS in a
// fixed order. A split whose keys are all invisible to the row (m = -inf) adds
// nothing, so a row's bits do not depend on the other rows of the call.
template <int D, int DS>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ ws, int nsplit, int ntile,
                                                           int keys_per_split, const int32_t* __restrict__ pos0,
                                                           int L, int Hq, int Hkv, int QT,
                                                           const uint16_t* __restrict__ gate, long g_stride,
                                                           uint16_t* __restrict__ out) {
  constexpr int DSL = D / DS;           // dims per block
  constexpr int TPG = DSL / 4;          // threads per split group
  constexpr int NG = 256 / TPG;         // split groups
  constexpr int CB = 8;                 // splits per thread per batch
  const int kh = blockIdx.x, tile = blockIdx.y, r = blockIdx.z / DS, ds = blockIdx.z % DS;
  const int GQ = Hq / Hkv;
  if (r >= GQ * QT) return;
  const int g = r / QT, lq = tile * QT + r % QT;
  if (lq >= L) return;
  const int h = kh * GQ + g;
  const size_t rec = (size_t)16 * (D + 2);
  const float* base = ws + ((size_t)kh * ntile + tile) * nsplit * rec;
  const int tid = threadIdx.x;
  const int grp = tid / TPG, j = tid % TPG;
  const int d0 = ds * DSL;
  __shared__ float gm[NG], gl[NG];
  __shared__ __align__(16) float part[NG][DSL];

  const float gt = tid < DSL ? bf16_to_f32(gate[(size_t)lq * g_stride + (size_t)h * 2 * D + D + d0 + tid]) : 0.0f;
  float ms[CB], ls[CB];
  float4 os[CB];
  auto load_batch = [&](int s0, int lim) {
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int s = s0 + grp + NG * i;
      const bool ok = s < lim;
      const float* rp = base + (size_t)(ok ? s : 0) * rec;
      ms[i] = ok ? rp[2 * r] : -INFINITY;
      ls[i] = ok ? rp[2 * r + 1] : 0.0f;
      os[i] = ok ? *reinterpret_cast<const float4*>(rp + 32 + (size_t)r * D + d0 + 4 * j)
                 : float4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  load_batch(0, nsplit);
  const int kend_tile = *pos0 + min(L, (tile + 1) * QT);
  const int nact = min(nsplit, (kend_tile + keys_per_split - 1) / keys_per_split);

  // this thread's splits, merged against its running maximum
  float m = -INFINITY, l = 0.0f;
  float4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < nact; s0 += CB * NG) {
    if (s0 > 0) load_batch(s0, nact);
    float mb = -INFINITY;
#pragma unroll
    for (int i = 0; i < CB; ++i)
      if (s0 + grp + NG * i < nact) mb = fmaxf(mb, ms[i]);
    if (mb == -INFINITY) continue;                  // nothing visible in this batch
    const float mn = fmaxf(m, mb);
    const float c = m == -INFINITY ? 0.0f : expf(m - mn);
    l *= c;
    o.x *= c; o.y *= c; o.z *= c; o.w *= c;
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      if (s0 + grp + NG * i < nact && ms[i] != -INFINITY) {
        const float f = expf(ms[i] - mn);
        l = fmaf(ls[i], f, l);
        o.x = fmaf(os[i].x, f, o.x);
        o.y = fmaf(os[i].y, f, o.y);
        o.z = fmaf(os[i].z, f, o.z);
        o.w = fmaf(os[i].w, f, o.w);
      }
    }
    m = mn;
  }
  if (j == 0) { gm[grp] = m; gl[grp] = l; }
  *reinterpret_cast<float4*>(&part[grp][4 * j]) = o;
  __syncthreads();
  if (tid < DSL) {   // wave 0 (DSL <= 64)
    float mx = gm[0];
#pragma unroll
    for (int q = 1; q < NG; ++q) mx = fmaxf(mx, gm[q]);
    // group q's factor evaluated once, in lane q, and read back per group
    // (the same value every lane computed before: one exp per lane, not NG)
    static_assert(NG <= DSL && DSL <= 64, "lane q of the active lanes holds group q's factor");
    const float gq = tid < NG ? gm[tid] : -INFINITY;
    const float fl = gq == -INFINITY ? 0.0f : expf(gq - mx);
    float acc = 0.0f, lt = 0.0f;
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      const float f = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fl), q));
      acc = fmaf(part[q][tid], f, acc);
      lt = fmaf(gl[q], f, lt);
    }
    const float invl = lt > 0.0f ? 1.0f / lt : 0.0f;
    out[(size_t)lq * Hq * D + (size_t)h * D + d0 + tid] = f32_to_bf16(acc * invl * sigmoidf_(gt));
  }
}

// counters[i] += n_accept[0] + 1 for every i (advance all caches past the kept tokens)
__global__ void commit_kernel(int32_t* __restrict__ counters, int n, const int32_t* __restrict__ n_accept,
                              int extra) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) counters[i] += n_accept[0] + extra;
}

}  // namespace

// ================================================================ C ABI

extern "C" int qvex_embed_w4g64(const int32_t* ids, int L, const uint32_t* w, const uint16_t* scales,
                                const uint16_t* biases, int V, int H, uint16_t* out, void* stream) {
  QVEX_CHECK_ARG(ids && w && scales && biases && out, "qvex_embed_w4g64: null pointer");
  QVEX_CHECK_ARG(L >= 1 && V >= 1 && H >= 64 && H % 64 == 0, "qvex_embed_w4g64: L=%d V=%d H=%d", L, V, H);
  QVEX_CHECK_ARG(qvex_aligned(out, 16) && qvex_aligned(w, 4), "qvex_embed_w4g64: out must be 16-byte aligned");
  hipLaunchKernelGGL(embed_kernel, dim3(L), dim3(256), 0, (hipStream_t)stream, ids, w, scales, biases, out, V, H);
  QVEX_CHECK_LAUNCH("qvex_embed_w4g64");
  return QVEX_OK;
}

extern "C" int qvex_rmsnorm(const uint16_t* x, long x_stride, const uint16_t* w, uint16_t* out, long out_stride,
                            int R, int D, float eps, float scale, void* stream) {
  QVEX_CHECK_ARG(x && out, "qvex_rmsnorm: null pointer");
  QVEX_CHECK_ARG(R >= 1 && D >= 8 && D % 8 == 0 && D <= 256 * 8 * RMS_MAXC && x_stride >= D && out_stride >= D &&
                     x_stride % 8 == 0 && out_stride % 8 == 0,
                 "qvex_rmsnorm: R=%d D=%d strides %ld/%ld (D %% 8 == 0, D <= 8192, strides %% 8 == 0)", R, D,
                 x_stride, out_stride);
  QVEX_CHECK_ARG(qvex_aligned(x, 16) && qvex_aligned(out, 16) && (!w || qvex_aligned(w, 16)),
                 "qvex_rmsnorm: x, w, out must be 16-byte aligned");
  hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(R), dim3(256), 0, (hipStream_t)stream, x, x_stride,
                     (const uint16_t*)nullptr, 0L, (uint16_t*)nullptr, 0L, w, out, out_stride, R, D, eps, scale);
  QVEX_CHECK_LAUNCH("qvex_rmsnorm");
  return QVEX_OK;
}

extern "C" int qvex_rmsnorm_pair(const uint16_t* x0, long x0_stride, const uint16_t* w0, uint16_t* out0,
                                 const uint16_t* x1, long x1_stride, const uint16_t* w1, uint16_t* out1,
                                 long out_stride, int R, int D, float eps, void* stream) {
  QVEX_CHECK_ARG(x0 && x1 && out0 && out1, "qvex_rmsnorm_pair: null pointer");
  QVEX_CHECK_ARG(R >= 1 && D >= 8 && D % 8 == 0 && D <= 256 * 8 * RMS_MAXC && x0_stride >= D && x1_stride >= D &&
                     out_stride >= D && x0_stride % 8 == 0 && x1_stride % 8 == 0 && out_stride % 8 == 0,
                 "qvex_rmsnorm_pair: R=%d D=%d strides %ld/%ld/%ld (D %% 8 == 0, D <= 8192, strides %% 8 == 0)", R,
                 D, x0_stride, x1_stride, out_stride);
  QVEX_CHECK_ARG(qvex_aligned(x0, 16) && qvex_aligned(x1, 16) && qvex_aligned(out0, 16) && qvex_aligned(out1, 16) &&
                     (!w0 || qvex_aligned(w0, 16)) && (!w1 || qvex_aligned(w1, 16)),
                 "qvex_rmsnorm_pair: pointers must be 16-byte aligned");
  hipLaunchKernelGGL(rmsnorm_pair_kernel, dim3(R, 2), dim3(256), 0, (hipStream_t)stream, x0, x0_stride, w0, out0,
                     x1, x1_stride, w1, out1, out_stride, D, eps);
  QVEX_CHECK_LAUNCH("qvex_rmsnorm_pair");
  return QVEX_OK;
}

extern "C" int qvex_add_rmsnorm(const uint16_t* x, const uint16_t* delta, uint16_t* h_out, const uint16_t* w,
                                uint16_t* out, int R, int D, float eps, void* stream) {
  QVEX_CHECK_ARG(x && delta && h_out && out, "qvex_add_rmsnorm: null pointer");
  QVEX_CHECK_ARG(R >= 1 && D >= 8 && D % 8 == 0 && D <= 256 * 8 * RMS_MAXC, "qvex_add_rmsnorm: R=%d D=%d", R, D);
  QVEX_CHECK_ARG(qvex_aligned(x, 16) && qvex_aligned(delta, 16) && qvex_aligned(h_out, 16) && qvex_aligned(out, 16) &&
                     (!w || qvex_aligned(w, 16)),
                 "qvex_add_rmsnorm: pointers must be 16-byte aligned");
  hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(R), dim3(256), 0, (hipStream_t)stream, x, (long)D, delta, (long)D,
                     h_out, (long)D, w, out, (long)D, R, D, eps, 1.0f);
  QVEX_CHECK_LAUNCH("qvex_add_rmsnorm");
  return QVEX_OK;
}

extern "C" int qvex_gdn_conv_qk(const uint16_t* proj, long p_stride, uint16_t* conv_ring, int ring_rows,
                                const int32_t* pos, const uint16_t* conv_w, int kernel_size, uint16_t* q,
                                uint16_t* k, uint16_t* v, uint16_t* a_out, uint16_t* b_out, int T, int C,
                                int key_dim, int Hv, int ab_offset, float q_scale, float k_scale, float eps,
                                void* stream) {
  QVEX_CHECK_ARG(proj && conv_ring && pos && conv_w && q && k && v && a_out && b_out,
                 "qvex_gdn_conv_qk: null pointer");
  QVEX_CHECK_ARG(T >= 1 && kernel_size >= 2 && C % 512 == 0 && key_dim % 128 == 0 && 2 * key_dim < C &&
                     Hv >= 1 && Hv <= 256 && ab_offset + 2 * Hv <= p_stride,
                 "qvex_gdn_conv_qk: T=%d K=%d C=%d key_dim=%d Hv=%d", T, kernel_size, C, key_dim, Hv);
  QVEX_CHECK_ARG(ring_rows >= T + kernel_size - 1, "qvex_gdn_conv_qk: ring_rows=%d < T + K - 1 = %d", ring_rows,
                 T + kernel_size - 1);
  hipLaunchKernelGGL(conv_silu_qk_kernel, dim3(T, C / 512), dim3(256), 0, (hipStream_t)stream, proj, p_stride,
                     conv_ring, ring_rows, pos, conv_w, kernel_size, q, k, v, a_out, b_out, T, C, key_dim, Hv,
                     ab_offset, q_scale, k_scale, eps);
  QVEX_CHECK_LAUNCH("qvex_gdn_conv_qk");
  return QVEX_OK;
}

extern "C" int qvex_gated_rmsnorm(const uint16_t* y, const uint16_t* z, long z_stride, int heads, const uint16_t* w,
                                  uint16_t* out, int R, int D, float eps, void* stream) {
  QVEX_CHECK_ARG(y && z && w && out, "qvex_gated_rmsnorm: null pointer");
  QVEX_CHECK_ARG(R >= 1 && D >= 2 && D % 2 == 0 && heads >= 1 && R % heads == 0, "qvex_gated_rmsnorm: R=%d D=%d", R, D);
  hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3((R + 3) / 4), dim3(256), 0, (hipStream_t)stream, y, z, z_stride,
                     heads, w, out, R, D, eps);
  QVEX_CHECK_LAUNCH("qvex_gated_rmsnorm");
  return QVEX_OK;
}

extern "C" int qvex_swiglu(const uint16_t* gu, uint16_t* out, int L, int I, void* stream) {
  QVEX_CHECK_ARG(gu && out && L >= 1 && I >= 2 && I % 2 == 0, "qvex_swiglu: L=%d I=%d", L, I);
  const long n2 = (long)L * I / 2;
  const int blocks = (int)std::min<long>((n2 + 255) / 256, 4096);
  hipLaunchKernelGGL(swiglu_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, gu, out, L, I);
  QVEX_CHECK_LAUNCH("qvex_swiglu");
  return QVEX_OK;
}

extern "C" int qvex_bf16_to_f32(const uint16_t* in, float* out, long n, void* stream) {
  QVEX_CHECK_ARG(in && out && n >= 1, "qvex_bf16_to_f32: n=%ld", n);
  const int blocks = (int)std::min<long>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(bf16_to_f32_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, in, out, n);
  QVEX_CHECK_LAUNCH("qvex_bf16_to_f32");
  return QVEX_OK;
}

extern "C" int qvex_attn_qk_rope(const uint16_t* proj, long p_stride, const uint16_t* q_norm, const uint16_t* k_norm,
                                 const int32_t* pos0, int L, int Hq, int Hkv, int D, int rot_dim, float theta,
                                 float eps, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, int cap,
                                 const float* rope, int rope_rows, void* stream) {
  QVEX_CHECK_ARG(proj && q_norm && k_norm && pos0 && q_out && k_cache && v_cache, "qvex_attn_qk_rope: null pointer");
  QVEX_CHECK_ARG(L >= 1 && Hq >= 1 && Hkv >= 1 && Hq % Hkv == 0 && D % 64 == 0 && D <= 512 && rot_dim >= 0 &&
                     rot_dim <= 64 && rot_dim % 2 == 0 && cap >= 32 && cap % 32 == 0,
                 "qvex_attn_qk_rope: L=%d Hq=%d Hkv=%d D=%d rot=%d cap=%d (cap a multiple of 32)", L, Hq, Hkv, D,
                 rot_dim, cap);
  QVEX_CHECK_ARG(p_stride >= (long)Hq * 2 * D + 2L * Hkv * D, "qvex_attn_qk_rope: p_stride too small");
  QVEX_CHECK_ARG(rope_rows >= 0 && (rope == nullptr || qvex_aligned(rope, 8)),
                 "qvex_attn_qk_rope: rope_rows=%d (the table 8-byte aligned)", rope_rows);
  decltype(&qk_norm_rope_kernel<1>) fn = nullptr;
  switch (D / 64) {
    case 1: fn = qk_norm_rope_kernel<1>; break;
    case 2: fn = qk_norm_rope_kernel<2>; break;
    case 3: fn = qk_norm_rope_kernel<3>; break;
    case 4: fn = qk_norm_rope_kernel<4>; break;
    case 5: fn = qk_norm_rope_kernel<5>; break;
    case 6: fn = qk_norm_rope_kernel<6>; break;
    case 7: fn = qk_norm_rope_kernel<7>; break;
    case 8: fn = qk_norm_rope_kernel<8>; break;
  }
  hipLaunchKernelGGL(fn, dim3(L, Hq + Hkv), dim3(64), 0, (hipStream_t)stream, proj, p_stride, q_norm, k_norm, pos0,
                     Hq, Hkv, D, rot_dim, theta, eps, q_out, k_cache, v_cache, cap,
                     reinterpret_cast<const float2*>(rope), rope ? rope_rows : 0);
  QVEX_CHECK_LAUNCH("qvex_attn_qk_rope");
  return QVEX_OK;
}

namespace {
constexpr int ATT_ROWS = 16;
constexpr int ATT_DSPLIT = 4;   // combine blocks per row, each over D / 4 dims (4 x the blocks in flight)
}

extern "C" uint64_t qvex_attn_workspace_bytes(int L, int Hq, int Hkv, int D, int max_keys, int keys_per_split) {
  if (L < 1 || Hkv < 1 || Hq % Hkv || keys_per_split < 1) return 0;
  const int GQ = Hq / Hkv;
  const int QT = ATT_ROWS / GQ < 1 ? 1 : ATT_ROWS / GQ;
  const int ntile = (L + QT - 1) / QT;
  const int nsplit = (max_keys + keys_per_split - 1) / keys_per_split;
  return (uint64_t)Hkv * ntile * nsplit * ATT_ROWS * (D + 2) * sizeof(float);
}

extern "C" int qvex_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                              const int32_t* pos0, int L, int Hq, int Hkv, int D, int cap, int max_keys,
                              int known_keys, int keys_per_split, const uint16_t* gate, long gate_stride,
                              uint16_t* out, void* workspace, uint64_t workspace_bytes, void* stream) {
  QVEX_CHECK_ARG(q && k_cache && v_cache && pos0 && gate && out && workspace, "qvex_attention: null pointer");
  QVEX_CHECK_ARG(L >= 1 && Hkv >= 1 && Hq % Hkv == 0 && Hq / Hkv <= ATT_ROWS, "qvex_attention: Hq=%d Hkv=%d", Hq, Hkv);
  QVEX_CHECK_ARG(D == 256 || D == 128, "qvex_attention: D=%d (128 or 256 supported)", D);
  QVEX_CHECK_ARG(max_keys >= 1 && max_keys <= cap && keys_per_split >= 128 && keys_per_split % 128 == 0 &&
                     cap % 32 == 0 && cap >= 32,
                 "qvex_attention: max_keys=%d cap=%d keys_per_split=%d (a multiple of 128; cap %% 32 == 0)", max_keys,
                 cap, keys_per_split);
  const uint64_t need = qvex_attn_workspace_bytes(L, Hq, Hkv, D, max_keys, keys_per_split);
  QVEX_CHECK_ARG(workspace_bytes >= need, "qvex_attention: workspace %llu < %llu bytes",
                 (unsigned long long)workspace_bytes, (unsigned long long)need);
  const int GQ = Hq / Hkv;
  const int QT = ATT_ROWS / GQ;
  const int ntile = (L + QT - 1) / QT;
  const int nsplit = (max_keys + keys_per_split - 1) / keys_per_split;
  QVEX_CHECK_ARG(ntile <= 65535 && nsplit <= 65535, "qvex_attention: grid too large");
  const float scale = 1.0f / sqrtf((float)D);
  hipStream_t st = (hipStream_t)stream;
  const dim3 pgrid(Hkv, ntile, nsplit);
  if (D == 256) {
    hipLaunchKernelGGL((attn_mfma_partial_kernel<256>), pgrid, dim3(256), 0, st, q, k_cache, v_cache, pos0, L, Hq,
                       Hkv, cap, QT, keys_per_split, known_keys, scale, (float*)workspace);
    QVEX_CHECK_LAUNCH("qvex_attention/partial");
    hipLaunchKernelGGL((attn_combine_kernel<256, ATT_DSPLIT>), dim3(Hkv, ntile, ATT_ROWS * ATT_DSPLIT), dim3(256), 0, st,
                       (const float*)workspace, nsplit, ntile, keys_per_split, pos0, L, Hq, Hkv, QT, gate,
                       gate_stride, out);
  } else {
    hipLaunchKernelGGL((attn_mfma_partial_kernel<128>), pgrid, dim3(256), 0, st, q, k_cache, v_cache, pos0, L, Hq,
                       Hkv, cap, QT, keys_per_split, known_keys, scale, (float*)workspace);
    QVEX_CHECK_LAUNCH("qvex_attention/partial");
    hipLaunchKernelGGL((attn_combine_kernel<128, ATT_DSPLIT>), dim3(Hkv, ntile, ATT_ROWS * ATT_DSPLIT), dim3(256), 0, st,
                       (const float*)workspace, nsplit, ntile, keys_per_split, pos0, L, Hq, Hkv, QT, gate,
                       gate_stride, out);
  }
  QVEX_CHECK_LAUNCH("qvex_attention/combine");
  return QVEX_OK;
}

extern "C" int qvex_rope_table(int rot_dim, float theta, int rows, float* table, void* stream) {
  QVEX_CHECK_ARG(table && rot_dim >= 2 && rot_dim % 2 == 0 && rows >= 1, "qvex_rope_table: rot_dim=%d rows=%d", rot_dim,
                 rows);
  const long n = (long)rows * (rot_dim / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, rot_dim,
                     theta, n, reinterpret_cast<float2*>(table));
  QVEX_CHECK_LAUNCH("qvex_rope_table");
  return QVEX_OK;
}

extern "C" int qvex_attention_decode(const uint16_t* proj, long p_stride, const uint16_t* q_norm,
                                     const uint16_t* k_norm, const int32_t* pos0, int L, int Hq, int Hkv, int D,
                                     int rot_dim, float eps, const float* rope, int rope_rows, uint16_t* k_cache,
                                     uint16_t* v_cache, int cap, int max_keys, int keys_per_split, uint16_t* out,
                                     void* workspace, uint64_t workspace_bytes, void* stream) {
  const char* fn = "qvex_attention_decode";
  QVEX_CHECK_ARG(proj && q_norm && k_norm && pos0 && k_cache && v_cache && out && workspace && (rope || rot_dim == 0),
                 "%s: null pointer", fn);
  QVEX_CHECK_ARG(rot_dim == 0 || (rope_rows >= cap && qvex_aligned(rope, 8)),
                 "%s: rope table of %d rows must cover cap=%d positions (8-byte aligned)", fn, rope_rows, cap);
  QVEX_CHECK_ARG(L >= 1 && L <= 8 && Hkv >= 1 && Hq % Hkv == 0 && Hq / Hkv <= ATT_ROWS, "%s: L=%d (1..8) Hq=%d Hkv=%d",
                 fn, L, Hq, Hkv);
  QVEX_CHECK_ARG(D == 256 || D == 128, "%s: D=%d (128 or 256 supported)", fn, D);
  QVEX_CHECK_ARG(rot_dim >= 0 && rot_dim <= D && rot_dim % 2 == 0 && (rot_dim == 0 || (rot_dim / 2) % (D / 16) == 0) &&
                     L * (rot_dim / 2) <= 256,
                 "%s: rot_dim=%d must be even, at most D, a multiple of 2 * D / 16 = %d, and L * rot_dim / 2 <= 256",
                 fn, rot_dim, D / 8);
  QVEX_CHECK_ARG(p_stride >= (long)Hq * 2 * D + 2L * Hkv * D && p_stride % 8 == 0,
                 "%s: p_stride=%ld too small or not a multiple of 8", fn, p_stride);
  QVEX_CHECK_ARG(qvex_aligned(proj, 16) && qvex_aligned(q_norm, 16) && qvex_aligned(k_norm, 16) &&
                     qvex_aligned(k_cache, 16) && qvex_aligned(v_cache, 16),
                 "%s: proj, norms and caches must be 16-byte aligned", fn);
  QVEX_CHECK_ARG(max_keys >= 1 && max_keys <= cap && keys_per_split >= 128 && keys_per_split % 128 == 0 &&
                     cap % 32 == 0 && cap >= 32,
                 "%s: max_keys=%d cap=%d keys_per_split=%d (a multiple of 128; cap %% 32 == 0)", fn, max_keys, cap,
                 keys_per_split);
  const uint64_t need = qvex_attn_workspace_bytes(L, Hq, Hkv, D, max_keys, keys_per_split);
  QVEX_CHECK_ARG(workspace_bytes >= need, "%s: workspace %llu < %llu bytes", fn, (unsigned long long)workspace_bytes,
                 (unsigned long long)need);
  const int GQ = Hq / Hkv;
  const int QT = ATT_ROWS / GQ;
  const int ntile = (L + QT - 1) / QT;
  const int nsplit = (max_keys + keys_per_split - 1) / keys_per_split;
  QVEX_CHECK_ARG(nsplit <= 65535, "%s: grid too large", fn);
  const float scale = 1.0f / sqrtf((float)D);
  hipStream_t st = (hipStream_t)stream;
  const dim3 pgrid(Hkv, ntile, nsplit);
  if (D == 256) {
    hipLaunchKernelGGL((attn_decode_kernel<256>), pgrid, dim3(256), 0, st, pos0, proj, p_stride, q_norm, k_norm,
                       k_cache, v_cache, (float*)workspace, reinterpret_cast<const float2*>(rope), rope_rows, L, Hq,
                       Hkv, cap, QT, keys_per_split, rot_dim, eps, scale);
    QVEX_CHECK_LAUNCH("qvex_attention_decode/partial");
    hipLaunchKernelGGL((attn_combine_kernel<256, ATT_DSPLIT>), dim3(Hkv, ntile, ATT_ROWS * ATT_DSPLIT), dim3(256), 0, st,
                       (const float*)workspace, nsplit, ntile, keys_per_split, pos0, L, Hq, Hkv, QT, proj, p_stride, out);
  } else {
    hipLaunchKernelGGL((attn_decode_kernel<128>), pgrid, dim3(256), 0, st, pos0, proj, p_stride, q_norm, k_norm,
                       k_cache, v_cache, (float*)workspace, reinterpret_cast<const float2*>(rope), rope_rows, L, Hq,
                       Hkv, cap, QT, keys_per_split, rot_dim, eps, scale);
    QVEX_CHECK_LAUNCH("qvex_attention_decode/partial");
    hipLaunchKernelGGL((attn_combine_kernel<128, ATT_DSPLIT>), dim3(Hkv, ntile, ATT_ROWS * ATT_DSPLIT), dim3(256), 0, st,
                       (const float*)workspace, nsplit, ntile, keys_per_split, pos0, L, Hq, Hkv, QT, proj, p_stride, out);
  }
  QVEX_CHECK_LAUNCH("qvex_attention_decode/combine");
  return QVEX_OK;
}

extern "C" int qvex_commit_step(int32_t* counters, int n, const int32_t* n_accept, int extra, void* stream) {
  QVEX_CHECK_ARG(counters && n_accept && n >= 1, "qvex_commit_step: null pointer or n=%d", n);
  hipLaunchKernelGGL(commit_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, counters, n, n_accept,
                     extra);
  QVEX_CHECK_LAUNCH("qvex_commit_step");
  return QVEX_OK;
}
