// Gated DeltaNet, chunked (prefill) form on MFMA.
//
// Reference: the same recurrence as engine/kernels.py:34-63 (gated_delta), per
// value head hv and state row i, token by token:
//   g = exp(-exp(A_log) * softplus(a + dt_bias)),  beta = sigmoid(b)
//   S *= g;  kv = S.k;  delta = (v - kv) * beta;  S += delta k^T;  y = S.q
// Prefill runs it over thousands of tokens; here it is regrouped in chunks of
// C = 64 tokens (the delta-rule chunking of Yang et al., "Gated Delta Networks",
// in its WY/UT form), so that everything but a short sequential scan is dense
// matrix products.
//
// Within a chunk, with l_t = sum_{s<=t} log g_s (inclusive, chunk-local) and
// S0 the state entering the chunk, the state after token t is
//   S_t = e^{l_t} S0 + sum_{s<=t} e^{l_t - l_s} u_s k_s^T,
//   u_t = beta_t (v_t - e^{l_t} S0 k_t - sum_{s<t} e^{l_t - l_s} (k_s.k_t) u_s).
// Collecting the rows: (I + A) U = diag(beta) (V - diag(e^l) K S0^T) with
// A[t][s] = beta_t e^{l_t - l_s} k_t.k_s (s < t). With T = (I + A)^{-1}:
//   W  = T diag(beta e^l) K,  U~ = T diag(beta) V,  U = U~ - W S0^T
//   Y  = diag(e^l) Q S0^T + P U,   P[t][s] = e^{l_t - l_s} q_t.k_s (s <= t)
//   S_C = e^{l_C} S0 + (diag(e^{l_C - l_t}) U)^T K
// W, U~, P and the chunk-local gates do not depend on the state, so they are
// computed for all chunks at once (phase 1); only the last three lines run in
// order over the chunks (phase 2). Exponents are always differences l_t - l_s
// with s <= t (never above 0), so nothing overflows.
//
// Phase 1, one 256-thread block per (chunk, value head, batch): K K^T and Q K^T
// on v_mfma_f32_16x16x32_bf16, the unit lower-triangular inverse in fp32 (16x16
// diagonal blocks by forward substitution, then block rows), W and U~ on MFMA.
// Results go to a workspace record per chunk in the layouts phase 2 reads.
//
// Phase 2, one block of NW waves per (value head, NW*16 state rows, batch):
// each wave keeps its 16 x 128 slice of S, transposed, in MFMA accumulators
// (fp32) for the whole sequence. Kept transposed, the state and U leave the
// accumulators as B operands without a trip through LDS: a pair of 16-row
// accumulator tiles is a k = 32 operand once both sides agree on the order of
// k, and phase 1 writes W, P and K^T in that order (fragment order, below).
// Per chunk the block stages W, Q, P, K^T and the gates in LDS, double-buffered
// (the next chunk's copy is staged after the current chunk's products, its
// loads in flight during them), one barrier per chunk. The blocks of one head
// are Hv apart in the linear block order, so with round-robin dispatch over 8
// XCDs (Hv a multiple of 8) they share an XCD and its L2.
//
// Operands are bf16 (the state is rounded to bf16 where it enters a product);
// accumulation and the state itself stay fp32.
#include "qvex_common.h"
#include "w4_dequant.h"

namespace {

constexpr int CH = 64;                 // tokens per chunk
constexpr int DD = 128;                // Dk = Dv
constexpr int KS_LD = DD + 8;          // bf16 row stride of [64][128] tiles in LDS
constexpr int KT_LD = CH + 8;          // bf16 row stride of [128][64] (transposed) tiles
constexpr int F_LD = CH + 4;           // fp32 row stride of [64][64] matrices
constexpr int P_LD = CH + 8;           // bf16 row stride of [64][64]

// workspace record per (batch, head, chunk)
constexpr long OFF_W = 0;              // bf16 [64][128], W in fragment order
constexpr long OFF_U = 16384;          // fp32 [4 row tiles][8 col tiles][64 lanes][4], U~ in accumulator order
constexpr long OFF_P = 49152;          // bf16 [64][64], P in fragment order
constexpr long OFF_KT = 57344;         // bf16 [128][64], K transposed, in fragment order
constexpr long OFF_G = 73728;          // fp32 [2][64]: e^{l_t}, then e^{l_C - l_t}
constexpr long REC = 74240;

struct ChunkArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* a;
  const uint16_t* b;
  const float* A_log;
  const uint16_t* dt_bias;
  const float* s_in;
  float* s_out;
  uint16_t* y;
  uint8_t* ws;
  int B, T, Hk, Hv, nchunk;
};

__device__ __forceinline__ bf16x8_t lds8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ bf16x8_t pack8(const float* v) {
  return as_bf16x8(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                   pack_bf16x2(v[6], v[7]));
}

__device__ __forceinline__ f32x4_t mfma(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// two floats to packed bf16, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// An accumulator tile pair (tiles 2m and 2m + 1 of 16 rows; lane li + 16 g
// holds rows 4g + r of each) as the B operand of a k = 32 product, k running
// over the pair's 32 rows in the order 4g + 0..3, 16 + 4g + 0..3.
__device__ __forceinline__ bf16x8_t pair_operand(f32x4_t lo, f32x4_t hi) {
  return as_bf16x8(cvt_pk(lo[0], lo[1]), cvt_pk(lo[2], lo[3]), cvt_pk(hi[0], hi[1]), cvt_pk(hi[2], hi[3]));
}

// Fragment order of a bf16 [R][K] matrix (K a multiple of 32) as the A operand
// of those products: [R/16 row tiles][K/32 k groups][64 lanes][8], lane
// li + 16 g holding row 16 rt + li and, of its k group, columns 4g + 0..3 then
// 16 + 4g + 0..3 - the k order of pair_operand. Element offset of (row, k):
__device__ __forceinline__ int frag_off(int row, int k, int nkg) {
  const int j = k & 31;
  return ((((row >> 4) * nkg + (k >> 5)) * 64 + (row & 15) + 16 * ((j >> 2) & 3)) << 3) + ((j >> 4) << 2) + (j & 3);
}

// ------------------------------------------------------------------ phase 1

__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(ChunkArgs p) {
  const int c = blockIdx.x, hv = blockIdx.y, bi = blockIdx.z;
  const int hk = hv / (p.Hv / p.Hk);
  const int t0 = c * CH;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, li = lane & 15, lg4 = lane >> 4;

  // LDS regions, each reused once its first tenant is dead, so that two blocks
  // fit on a CU (75 KB): Q -> T (Q dies with the K K^T / Q K^T products), A -> V^T
  // (A dies with the inverse; V waits in registers meanwhile); P goes straight
  // to the workspace record
  constexpr int SZ_KS = CH * KS_LD * 2, SZ_KT = DD * KT_LD * 2, SZ_F = CH * F_LD * 4;
  constexpr int SZ_R4 = SZ_KT > SZ_F ? SZ_KT : SZ_F;
  __shared__ __align__(16) unsigned char smem[SZ_KS + SZ_KT + SZ_KS + SZ_R4];
  uint16_t* Ks = reinterpret_cast<uint16_t*>(smem);                       // K row-major; reused for W
  uint16_t* Kt = reinterpret_cast<uint16_t*>(smem + SZ_KS);               // K transposed [dk][t]
  uint16_t* Qs = reinterpret_cast<uint16_t*>(smem + SZ_KS + SZ_KT);       // Q row-major, then:
  float* Tm = reinterpret_cast<float*>(smem + SZ_KS + SZ_KT);             //   T = (I + A)^{-1}
  float* Am = reinterpret_cast<float*>(smem + 2 * SZ_KS + SZ_KT);         // A, then:
  uint16_t* Vt = reinterpret_cast<uint16_t*>(smem + 2 * SZ_KS + SZ_KT);   //   V transposed [dv][t]
  static_assert(SZ_KS == SZ_F, "Q and T share a region");
  __shared__ float lgs[CH], bet[CH], gam[CH];
  __shared__ float Xs[4][16 * 17];
  uint8_t* rec = p.ws + (((long)bi * p.Hv + hv) * p.nchunk + c) * REC;
  uint16_t* Pg = reinterpret_cast<uint16_t*>(rec + OFF_P);

  // K, Q rows (row-major) and K transposed; V kept in registers until its
  // region is free; tokens past T are zero
  u32x4 vreg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;
    const int row = idx >> 4, col = (idx & 15) * 8;
    const int t = t0 + row;
    u32x4 kv = {0u, 0u, 0u, 0u}, qv = kv, vv = kv;
    if (t < p.T) {
      const long qk = (((long)bi * p.T + t) * p.Hk + hk) * DD + col;
      kv = load16(p.k + qk);
      qv = load16(p.q + qk);
      vv = load16(p.v + (((long)bi * p.T + t) * p.Hv + hv) * DD + col);
    }
    vreg[i] = vv;
    *reinterpret_cast<u32x4*>(&Ks[row * KS_LD + col]) = kv;
    *reinterpret_cast<u32x4*>(&Qs[row * KS_LD + col]) = qv;
    const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Kt[(col + 2 * e) * KT_LD + row] = (uint16_t)(kw[e] & 0xffffu);
      Kt[(col + 2 * e + 1) * KT_LD + row] = (uint16_t)(kw[e] >> 16);
    }
  }
  // gates, same formulas as the recurrent kernel; inclusive prefix sum of log g
  if (w == 0) {
    const int t = t0 + lane;
    float lgv = 0.0f, be = 0.0f;
    if (t < p.T) {
      const long ab = ((long)bi * p.T + t) * p.Hv + hv;
      const float x = bf16_to_f32(p.a[ab]) + bf16_to_f32(p.dt_bias[hv]);
      const float sp = x > 20.0f ? x : log1pf(expf(x));
      lgv = -expf(p.A_log[hv]) * sp;
      be = 1.0f / (1.0f + expf(-bf16_to_f32(p.b[ab])));
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(lgv, off, 64);
      if (lane >= off) lgv += o;
    }
    lgs[lane] = lgv;
    bet[lane] = be;
    gam[lane] = expf(lgv);
  }
  __syncthreads();

  // A = beta_t e^{l_t-l_s} K K^T (s < t) and P = e^{l_t-l_s} Q K^T (s <= t); wave w = row tile
  {
    const int rt = w;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      f32x4_t ckk = {0.0f, 0.0f, 0.0f, 0.0f}, cqk = ckk;
      if (ct <= rt) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const bf16x8_t ak = lds8(&Ks[(16 * rt + li) * KS_LD + 32 * ks + 8 * lg4]);
          const bf16x8_t aq = lds8(&Qs[(16 * rt + li) * KS_LD + 32 * ks + 8 * lg4]);
          const bf16x8_t bk = lds8(&Ks[(16 * ct + li) * KS_LD + 32 * ks + 8 * lg4]);
          ckk = mfma(ak, bk, ckk);
          cqk = mfma(aq, bk, cqk);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * rt + 4 * lg4 + r, s = 16 * ct + li;
        const float dA = (s <= t) ? expf(lgs[t] - lgs[s]) : 0.0f;
        Am[t * F_LD + s] = (s < t) ? bet[t] * dA * ckk[r] : 0.0f;
        Pg[frag_off(t, s, CH / 32)] = f32_to_bf16((s <= t) ? dA * cqk[r] : 0.0f);
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < CH * F_LD; i += 256) Tm[i] = 0.0f;     // Q is dead: its region becomes T
  __syncthreads();

  // T = (I + A)^{-1}: diagonal 16x16 blocks, wave w inverts block w (lane j = column j)
  if (lane < 16) {
    const int j = lane, o = 16 * w;
    float x[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float s = (t == j) ? 1.0f : 0.0f;
#pragma unroll
      for (int u = 0; u < t; ++u) s = fmaf(-Am[(o + t) * F_LD + o + u], x[u], s);
      x[t] = s;
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) Tm[(o + t) * F_LD + o + j] = x[t];
  }
  __syncthreads();
  // off-diagonal blocks, by distance d from the diagonal: T_ij = -T_ii sum_{m=j}^{i-1} A_im T_mj
  for (int d = 1; d < 4; ++d) {
    const int j = w, i = w + d;
    const int rho = lane >> 2, kap = 4 * (lane & 3);
    if (i < 4) {
      float x4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m = j; m < i; ++m) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const float av = Am[(16 * i + rho) * F_LD + 16 * m + u];
          const float* tr = &Tm[(16 * m + u) * F_LD + 16 * j + kap];
#pragma unroll
          for (int e = 0; e < 4; ++e) x4[e] = fmaf(av, tr[e], x4[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) Xs[w][rho * 17 + kap + e] = x4[e];
    }
    __syncthreads();
    if (i < 4) {
      float t4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float tv = Tm[(16 * i + rho) * F_LD + 16 * i + u];
#pragma unroll
        for (int e = 0; e < 4; ++e) t4[e] = fmaf(-tv, Xs[w][u * 17 + kap + e], t4[e]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) Tm[(16 * i + rho) * F_LD + 16 * j + kap + e] = t4[e];
    }
    __syncthreads();
  }

  // A is dead: V transposed into its region
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;
    const int row = idx >> 4, col = (idx & 15) * 8;
    const uint32_t vw[4] = {vreg[i].x, vreg[i].y, vreg[i].z, vreg[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Vt[(col + 2 * e) * KT_LD + row] = (uint16_t)(vw[e] & 0xffffu);
      Vt[(col + 2 * e + 1) * KT_LD + row] = (uint16_t)(vw[e] >> 16);
    }
  }
  __syncthreads();

  // W = T diag(beta e^l) K -> Ks (row-major staging); U~ = T diag(beta) V -> workspace (accumulator order)
  {
    const int rt = w;
    const int nks = rt >= 2 ? 2 : 1;     // T is lower triangular: token blocks past the row tile are zero
    bf16x8_t aW[2], aU[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (ks < nks) {
        float tv[8], wv[8], uv[8];
        const float* tr = &Tm[(16 * rt + li) * F_LD + 32 * ks + 8 * lg4];
#pragma unroll
        for (int e = 0; e < 8; ++e) tv[e] = tr[e];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int s = 32 * ks + 8 * lg4 + e;
          uv[e] = tv[e] * bet[s];
          wv[e] = uv[e] * gam[s];
        }
        aW[ks] = pack8(wv);
        aU[ks] = pack8(uv);
      }
    }
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
      f32x4_t cw = {0.0f, 0.0f, 0.0f, 0.0f}, cu = cw;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (ks < nks) {
          cw = mfma(aW[ks], lds8(&Kt[(16 * ct + li) * KT_LD + 32 * ks + 8 * lg4]), cw);
          cu = mfma(aU[ks], lds8(&Vt[(16 * ct + li) * KT_LD + 32 * ks + 8 * lg4]), cu);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) Ks[(16 * rt + 4 * lg4 + r) * KS_LD + 16 * ct + li] = f32_to_bf16(cw[r]);
      *reinterpret_cast<f32x4_t*>(rec + OFF_U + (((long)(rt * 8 + ct) * 64 + lane) * 16)) = cu;
    }
  }
  __syncthreads();
  // W [64][128] and K^T [128][64] to the record in fragment order: 16-byte piece
  // idx is lane idx % 64 of fragment idx / 64, gathered from two 8-byte runs
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i, f = idx >> 6, fl = idx & 63;
    const uint16_t* src = &Ks[(16 * (f >> 2) + (fl & 15)) * KS_LD + 32 * (f & 3) + 4 * (fl >> 4)];
    const u32x2 lo = *reinterpret_cast<const u32x2*>(src), hi = *reinterpret_cast<const u32x2*>(src + 16);
    *reinterpret_cast<u32x4*>(rec + OFF_W + (long)idx * 16) = u32x4{lo.x, lo.y, hi.x, hi.y};
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i, f = idx >> 6, fl = idx & 63;
    const uint16_t* src = &Kt[(16 * (f >> 1) + (fl & 15)) * KT_LD + 32 * (f & 1) + 4 * (fl >> 4)];
    const u32x2 lo = *reinterpret_cast<const u32x2*>(src), hi = *reinterpret_cast<const u32x2*>(src + 16);
    *reinterpret_cast<u32x4*>(rec + OFF_KT + (long)idx * 16) = u32x4{lo.x, lo.y, hi.x, hi.y};
  }
  if (tid < CH) {
    float* g = reinterpret_cast<float*>(rec + OFF_G);
    g[tid] = gam[tid];
    g[CH + tid] = expf(lgs[CH - 1] - lgs[tid]);
  }
}

// ------------------------------------------------------------------ phase 2

template <int NW>
__global__ __launch_bounds__(64 * NW) void gdn_chunk_scan_kernel(ChunkArgs p) {
  constexpr int NT = 64 * NW;
  constexpr int NR = 1024 / NT;          // 16-byte pieces per thread of a 16 KB tile
  constexpr int NP = 512 / NT;           // ... of the 8 KB P tile
  const int hv = blockIdx.x, slice = blockIdx.y, bi = blockIdx.z;
  const int hk = hv / (p.Hv / p.Hk);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, li = lane & 15, lg4 = lane >> 4;
  const int dvt = slice * NW + w;        // this wave's 16 columns of the state
  const int dv0 = 16 * dvt;

  // operand tiles in fragment order, double-buffered: chunk c + 1 is staged
  // while chunk c's products read the other buffer
  __shared__ __align__(16) uint16_t Wf[2][CH * DD];
  __shared__ __align__(16) uint16_t Qf[2][CH * DD];
  __shared__ __align__(16) uint16_t Kf[2][DD * CH];
  __shared__ __align__(16) uint16_t Pf[2][CH * CH];
  __shared__ __align__(16) float gam[2][CH];
  __shared__ __align__(16) float dec[2][CH];

  // the state slice, transposed, in accumulator layout: tile ct, lane li + 16 g,
  // element r holds S[dv0 + li][16 ct + 4 g + r], so that tile pairs are the
  // B operand of W S^T and Q S^T as they stand
  const long s_base = (((long)bi * p.Hv + hv) * DD + dv0 + li) * DD + 4 * lg4;
  f32x4_t S[8];
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) S[ct][r] = p.s_in[s_base + 16 * ct + r];

  const uint8_t* rec0 = p.ws + ((long)bi * p.Hv + hv) * p.nchunk * REC;
  u32x4 rW[NR], rQ[NR], rK[NR], rP[NP];
  f32x4_t rU[4];
  float rG = 0.0f, rD = 0.0f;

  auto fetch = [&](int c) {
    const uint8_t* rec = rec0 + (long)c * REC;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int idx = tid + NT * i;
      rW[i] = load16(rec + OFF_W + (long)idx * 16);
      rK[i] = load16(rec + OFF_KT + (long)idx * 16);
      // rows past T repeat row T - 1 (in bounds, no branch): they only reach
      // output rows that are never stored
      const int t = min(c * CH + (idx >> 4), p.T - 1);
      rQ[i] = load16(p.q + (((long)bi * p.T + t) * p.Hk + hk) * DD + (idx & 15) * 8);
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) rP[i] = load16(rec + OFF_P + (long)(tid + NT * i) * 16);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
      rU[rt] = *reinterpret_cast<const f32x4_t*>(rec + OFF_U + ((long)(rt * 8 + dvt) * 64 + lane) * 16);
    if (tid < CH) {
      rG = reinterpret_cast<const float*>(rec + OFF_G)[tid];
      rD = reinterpret_cast<const float*>(rec + OFF_G)[CH + tid];
    }
  };
  auto stage = [&](int b) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int idx = tid + NT * i;
      *reinterpret_cast<u32x4*>(&Wf[b][idx * 8]) = rW[i];
      *reinterpret_cast<u32x4*>(&Kf[b][idx * 8]) = rK[i];
      const int row = idx >> 4, col = (idx & 15) * 8;   // Q arrives row-major
      *reinterpret_cast<u32x2*>(&Qf[b][frag_off(row, col, DD / 32)]) = u32x2{rQ[i].x, rQ[i].y};
      *reinterpret_cast<u32x2*>(&Qf[b][frag_off(row, col + 4, DD / 32)]) = u32x2{rQ[i].z, rQ[i].w};
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) *reinterpret_cast<u32x4*>(&Pf[b][(tid + NT * i) * 8]) = rP[i];
    if (tid < CH) {                  // wave 0: chunk-local decay factors
      gam[b][tid] = rG;
      dec[b][tid] = rD;
    }
  };

  fetch(0);
  stage(0);
  f32x4_t U0[4] = {rU[0], rU[1], rU[2], rU[3]};
  if (p.nchunk > 1) fetch(1);
  __syncthreads();
  for (int c = 0; c < p.nchunk; ++c) {
    const int b = c & 1;
    const uint16_t* Wb = Wf[b] + lane * 8;
    const uint16_t* Qb = Qf[b] + lane * 8;
    const uint16_t* Kb = Kf[b] + lane * 8;
    const uint16_t* Pb = Pf[b] + lane * 8;

    // Operand fragments are read from LDS one step ahead of the products that
    // use them (fa / fb alternate; sched_barrier keeps the compiler from sinking
    // each read next to its product, which would expose every LDS latency).
    bf16x8_t fa[8], fb[8];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      fa[ks] = lds8(Wb + ks * 512);
      fa[4 + ks] = lds8(Qb + ks * 512);
    }
    bf16x8_t bS[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) bS[ks] = pair_operand(S[2 * ks], S[2 * ks + 1]);
    const float gC = gam[b][CH - 1];
    f32x4_t d4[4];                       // e^{l_C - l_t} for this lane's tokens, by row tile
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) d4[rt] = *reinterpret_cast<const f32x4_t*>(&dec[b][16 * rt + 4 * lg4]);
    __builtin_amdgcn_sched_barrier(0);

    // U = U~ - W S^T ;  Y = e^l (Q S^T); the state is scaled by e^{l_C} meanwhile
    f32x4_t U[4], Y[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      bf16x8_t* cur = (rt & 1) ? fb : fa;
      bf16x8_t* nxt = (rt & 1) ? fa : fb;
      // the decay row first: LDS reads complete in order, so a read queued
      // behind the prefetch would wait for all of it
      const f32x4_t g4 = *reinterpret_cast<const f32x4_t*>(&gam[b][16 * rt + 4 * lg4]);
      if (rt < 3) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          nxt[ks] = lds8(Wb + ((rt + 1) * 4 + ks) * 512);
          nxt[4 + ks] = lds8(Qb + ((rt + 1) * 4 + ks) * 512);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) nxt[j] = lds8(Kb + j * 512);     // K^T, state tiles 0..3
      }
      f32x4_t cw = {0.0f, 0.0f, 0.0f, 0.0f}, cq = cw;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        cw = mfma(cur[ks], bS[ks], cw);
        cq = mfma(cur[4 + ks], bS[ks], cq);
      }
#pragma unroll
      for (int ct = 2 * rt; ct < 2 * rt + 2; ++ct) S[ct] *= gC;
      U[rt] = U0[rt] - cw;
      Y[rt] = g4 * cq;
      __builtin_amdgcn_sched_barrier(0);
    }
    // U and diag(e^{l_C - l_t}) U as B operands over tokens
    bf16x8_t bU[2], bD[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bU[ks] = pair_operand(U[2 * ks], U[2 * ks + 1]);
      bD[ks] = pair_operand(U[2 * ks] * d4[2 * ks], U[2 * ks + 1] * d4[2 * ks + 1]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) fb[j] = lds8(Kb + (8 + j) * 512);         // K^T, state tiles 4..7
    __builtin_amdgcn_sched_barrier(0);

    // S^T = e^{l_C} S^T + K^T (D U)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) S[ct] = mfma(fa[2 * ct + ks], bD[ks], S[ct]);
    // P fragments (row tile, token group): (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
    fa[0] = lds8(Pb + 0 * 512);
    fa[1] = lds8(Pb + 2 * 512);
#pragma unroll
    for (int j = 2; j < 6; ++j) fa[j] = lds8(Pb + (j + 2) * 512);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ct = 4; ct < 8; ++ct)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) S[ct] = mfma(fb[2 * (ct - 4) + ks], bD[ks], S[ct]);

    // Y += P U (P lower triangular: no token group 1 for the first two row tiles)
    Y[0] = mfma(fa[0], bU[0], Y[0]);
    Y[1] = mfma(fa[1], bU[0], Y[1]);
    Y[2] = mfma(fa[3], bU[1], mfma(fa[2], bU[0], Y[2]));
    Y[3] = mfma(fa[5], bU[1], mfma(fa[4], bU[0], Y[3]));
    // Next chunk's tiles to the other buffer (its last readers finished before
    // the previous barrier), then this chunk's outputs, then the loads two
    // chunks ahead: the stage's wait for its loads (issued one chunk earlier)
    // then never includes the stores, which count in the same in-order counter.
    if (c + 1 < p.nchunk) {
      stage(b ^ 1);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) U0[rt] = rU[rt];
    }
    const bool full = (c + 1) * CH <= p.T;
    uint16_t* yp = p.y + (((long)bi * p.T + c * CH + 4 * lg4) * p.Hv + hv) * DD + dv0 + li;
    const long ystep = (long)p.Hv * DD;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const uint32_t y01 = cvt_pk(Y[rt][0], Y[rt][1]), y23 = cvt_pk(Y[rt][2], Y[rt][3]);
      const uint16_t yv[4] = {(uint16_t)y01, (uint16_t)(y01 >> 16), (uint16_t)y23, (uint16_t)(y23 >> 16)};
      if (full) {
#pragma unroll
        for (int r = 0; r < 4; ++r) yp[(16 * rt + r) * ystep] = yv[r];
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (c * CH + 16 * rt + 4 * lg4 + r < p.T) yp[(16 * rt + r) * ystep] = yv[r];
      }
    }
    if (c + 2 < p.nchunk) fetch(c + 2);
    __syncthreads();
  }
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) p.s_out[s_base + 16 * ct + r] = S[ct][r];
}

constexpr int SCAN_NW = 4;

}  // namespace

extern "C" uint64_t qvex_gdn_chunked_workspace_bytes(int B, int T, int Hv, int Dk, int Dv, int chunk) {
  if (B < 1 || T < 1 || Hv < 1 || Dk != DD || Dv != DD || chunk != CH) return 0;
  return (uint64_t)B * Hv * ((T + CH - 1) / CH) * REC;
}

extern "C" int qvex_gdn_chunked(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* a,
                                const uint16_t* b, const float* A_log, const uint16_t* dt_bias,
                                const float* state_in, float* state_out, uint16_t* y, int B, int T, int Hk,
                                int Hv, int Dk, int Dv, int chunk, void* workspace, uint64_t workspace_bytes,
                                void* stream) {
  QVEX_CHECK_ARG(q && k && v && a && b && A_log && dt_bias && state_in && state_out && y && workspace,
                 "qvex_gdn_chunked: null pointer");
  QVEX_CHECK_ARG(B >= 1 && T >= 1 && Hk >= 1 && Hv >= Hk && Hv % Hk == 0,
                 "qvex_gdn_chunked: B=%d T=%d Hk=%d Hv=%d", B, T, Hk, Hv);
  if (Dk != DD || Dv != DD || chunk != CH)
    return qvex::fail(QVEX_ENOTSUP, "qvex_gdn_chunked: needs Dk = Dv = 128 and chunk = 64 (got %d, %d, %d)", Dk,
                      Dv, chunk);
  QVEX_CHECK_ARG(qvex_aligned(q, 16) && qvex_aligned(k, 16) && qvex_aligned(v, 16) && qvex_aligned(workspace, 16),
                 "qvex_gdn_chunked: q, k, v and workspace must be 16-byte aligned");
  const uint64_t need = qvex_gdn_chunked_workspace_bytes(B, T, Hv, Dk, Dv, chunk);
  QVEX_CHECK_ARG(workspace_bytes >= need, "qvex_gdn_chunked: workspace %llu < %llu bytes",
                 (unsigned long long)workspace_bytes, (unsigned long long)need);
  const int nchunk = (T + CH - 1) / CH;
  QVEX_CHECK_ARG(nchunk <= 65535 && Hv <= 65535 && B <= 65535, "qvex_gdn_chunked: grid too large");
  ChunkArgs p{q, k, v, a, b, A_log, dt_bias, state_in, state_out, y, (uint8_t*)workspace, B, T, Hk, Hv, nchunk};
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(nchunk, Hv, B), dim3(256), 0, st, p);
  QVEX_CHECK_LAUNCH("qvex_gdn_chunked/prep");
  hipLaunchKernelGGL((gdn_chunk_scan_kernel<SCAN_NW>), dim3(Hv, DD / (16 * SCAN_NW), B), dim3(64 * SCAN_NW), 0, st, p);
  QVEX_CHECK_LAUNCH("qvex_gdn_chunked/scan");
  return QVEX_OK;
}
