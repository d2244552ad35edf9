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
// each wave keeps its 16 x 128 slice of S in MFMA accumulators (fp32) for the
// whole sequence. Per chunk the block stages W, Q, P, K^T and the gates in LDS
// (the next chunk's copy is in flight during the current chunk's products).
// The blocks of one head are consecutive in x, so with round-robin dispatch they
// share an XCD and its L2.
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
constexpr long OFF_W = 0;              // bf16 [64][128], W row-major
constexpr long OFF_U = 16384;          // fp32 [4 row tiles][8 col tiles][64 lanes][4], U~ in accumulator order
constexpr long OFF_P = 49152;          // bf16 [64][64], P row-major
constexpr long OFF_KT = 57344;         // bf16 [128][64], K transposed
constexpr long OFF_LG = 73728;         // fp32 [64], inclusive chunk-local log decay
constexpr long REC = 73984;

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
        Pg[t * CH + s] = f32_to_bf16((s <= t) ? dA * cqk[r] : 0.0f);
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
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;
    const int row = idx >> 4, col = (idx & 15) * 8;
    *reinterpret_cast<u32x4*>(rec + OFF_W + (row * DD + col) * 2) = *reinterpret_cast<const u32x4*>(&Ks[row * KS_LD + col]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + 256 * i;
    const int row = idx >> 3, col = (idx & 7) * 8;
    *reinterpret_cast<u32x4*>(rec + OFF_KT + (row * CH + col) * 2) = *reinterpret_cast<const u32x4*>(&Kt[row * KT_LD + col]);
  }
  if (tid < CH) reinterpret_cast<float*>(rec + OFF_LG)[tid] = lgs[tid];
}

// ------------------------------------------------------------------ phase 2

template <int NW>
__global__ __launch_bounds__(64 * NW) void gdn_chunk_scan_kernel(ChunkArgs p) {
  constexpr int NT = 64 * NW;
  constexpr int NR = 1024 / NT;          // 16-byte chunks per thread of a [64][128] or [128][64] bf16 tile
  constexpr int NP = 512 / NT;           // ... of the [64][64] P tile
  const int hv = blockIdx.x, slice = blockIdx.y, bi = blockIdx.z;
  const int hk = hv / (p.Hv / p.Hk);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, li = lane & 15, lg4 = lane >> 4;
  const int dvt = slice * NW + w;        // this wave's 16-row tile of the state
  const int dv0 = 16 * dvt;

  __shared__ __align__(16) uint16_t Ws[CH * KS_LD];
  __shared__ __align__(16) uint16_t Qs[CH * KS_LD];
  __shared__ __align__(16) uint16_t Ps[CH * P_LD];
  __shared__ __align__(16) uint16_t Kts[DD * KT_LD];
  __shared__ float gam[CH], dec[CH];
  __shared__ __align__(16) uint16_t Sb[NW][16 * KS_LD];
  __shared__ __align__(16) uint16_t Ub[NW][16 * KT_LD];
  __shared__ __align__(16) uint16_t DUb[NW][16 * KT_LD];

  // state slice S[dv0 + 4*lg4 + r][16*ct + li] in accumulator layout
  const long s_base = (((long)bi * p.Hv + hv) * DD + dv0) * DD;
  f32x4_t S[8];
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) S[ct][r] = p.s_in[s_base + (long)(4 * lg4 + r) * DD + 16 * ct + li];

  const uint8_t* rec0 = p.ws + ((long)bi * p.Hv + hv) * p.nchunk * REC;
  u32x4 rW[NR], rQ[NR], rK[NR], rP[NP];
  f32x4_t rU[4];
  float rL = 0.0f;

  auto fetch = [&](int c) {
    const uint8_t* rec = rec0 + (long)c * REC;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int idx = tid + NT * i;
      rW[i] = load16(rec + OFF_W + (long)idx * 16);
      rK[i] = load16(rec + OFF_KT + (long)idx * 16);
      const int row = idx >> 4, col = (idx & 15) * 8;
      const int t = c * CH + row;
      rQ[i] = t < p.T ? load16(p.q + (((long)bi * p.T + t) * p.Hk + hk) * DD + col) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) rP[i] = load16(rec + OFF_P + (long)(tid + NT * i) * 16);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
      rU[rt] = *reinterpret_cast<const f32x4_t*>(rec + OFF_U + ((long)(rt * 8 + dvt) * 64 + lane) * 16);
    if (tid < CH) rL = reinterpret_cast<const float*>(rec + OFF_LG)[tid];
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int idx = tid + NT * i;
      const int row = idx >> 4, col = (idx & 15) * 8;           // [64][128] tiles
      *reinterpret_cast<u32x4*>(&Ws[row * KS_LD + col]) = rW[i];
      *reinterpret_cast<u32x4*>(&Qs[row * KS_LD + col]) = rQ[i];
      const int krow = idx >> 3, kcol = (idx & 7) * 8;          // [128][64] tile
      *reinterpret_cast<u32x4*>(&Kts[krow * KT_LD + kcol]) = rK[i];
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int idx = tid + NT * i;
      const int row = idx >> 3, col = (idx & 7) * 8;
      *reinterpret_cast<u32x4*>(&Ps[row * P_LD + col]) = rP[i];
    }
    if (tid < CH) {                  // wave 0: chunk-local decay factors
      const float lC = __shfl(rL, CH - 1, 64);
      gam[tid] = expf(rL);
      dec[tid] = expf(lC - rL);
    }
  };

  fetch(0);
  for (int c = 0; c < p.nchunk; ++c) {
    __syncthreads();                     // every wave is done with the previous chunk's tiles
    stage();
    const f32x4_t U0[4] = {rU[0], rU[1], rU[2], rU[3]};
    __syncthreads();
    if (c + 1 < p.nchunk) fetch(c + 1);  // next chunk's loads overlap this chunk's products

    // S (bf16) in B-operand layout: Sb[dv][dk]
    uint16_t* sb = Sb[w];
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) sb[(4 * lg4 + r) * KS_LD + 16 * ct + li] = f32_to_bf16(S[ct][r]);
    bf16x8_t bS[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) bS[ks] = lds8(&sb[li * KS_LD + 32 * ks + 8 * lg4]);

    // U = U~ - W S^T ;  Y = e^l (Q S^T)
    f32x4_t U[4], Y[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      f32x4_t cw = {0.0f, 0.0f, 0.0f, 0.0f}, cq = cw;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        cw = mfma(lds8(&Ws[(16 * rt + li) * KS_LD + 32 * ks + 8 * lg4]), bS[ks], cw);
        cq = mfma(lds8(&Qs[(16 * rt + li) * KS_LD + 32 * ks + 8 * lg4]), bS[ks], cq);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * rt + 4 * lg4 + r;
        U[rt][r] = U0[rt][r] - cw[r];
        Y[rt][r] = gam[t] * cq[r];
      }
    }
    // U^T and (diag(e^{l_C - l_t}) U)^T in bf16: Ub[dv][t]
    uint16_t* ub = Ub[w];
    uint16_t* dub = DUb[w];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * rt + 4 * lg4 + r;
        ub[li * KT_LD + t] = f32_to_bf16(U[rt][r]);
        dub[li * KT_LD + t] = f32_to_bf16(U[rt][r] * dec[t]);
      }
    // Y += P U (P lower triangular: skip the zero token block of the first two row tiles)
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        if (ks == 0 || rt >= 2)
          Y[rt] = mfma(lds8(&Ps[(16 * rt + li) * P_LD + 32 * ks + 8 * lg4]), lds8(&ub[li * KT_LD + 32 * ks + 8 * lg4]), Y[rt]);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = c * CH + 16 * rt + 4 * lg4 + r;
        if (t < p.T) p.y[(((long)bi * p.T + t) * p.Hv + hv) * DD + dv0 + li] = f32_to_bf16(Y[rt][r]);
      }
    // S = e^{l_C} S + (D U)^T K
    const float gC = gam[CH - 1];
    bf16x8_t aDU[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) aDU[ks] = lds8(&dub[li * KT_LD + 32 * ks + 8 * lg4]);
#pragma unroll
    for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
      for (int r = 0; r < 4; ++r) S[ct][r] *= gC;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) S[ct] = mfma(aDU[ks], lds8(&Kts[(16 * ct + li) * KT_LD + 32 * ks + 8 * lg4]), S[ct]);
    }
  }
#pragma unroll
  for (int ct = 0; ct < 8; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) p.s_out[s_base + (long)(4 * lg4 + r) * DD + 16 * ct + li] = S[ct][r];
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
