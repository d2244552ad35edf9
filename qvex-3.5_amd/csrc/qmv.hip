// 4-bit group-64 quantized GEMV / skinny GEMM for M = 1..8 rows (MLX affine layout).
//
// Reference semantics: mx.quantized_matmul(transpose=True, group_size=64, bits=4)
// as used by QLinear (engine/model.py:87-91); the multi-row factoring
// sum_g s*sum(q*x) + b*sum(x) is the one of engine/kernels.py:121-125,171.
//
// MI355X design (bandwidth-bound, no MFMA: at M <= 8 there is no dense tile to feed):
//   * every lane streams 16-byte chunks (4 packed words = 32 nibbles = half a
//     quantization group) with global_load_dwordx4; a wave covers 1 KiB of one
//     weight row per load, fully coalesced;
//   * nibbles are turned into bf16 pairs with one v_and_or_b32 each:
//     (w >> 4j) & 0x000F000F | 0x43004300 = bf16(128 + q_j), bf16(128 + q_{j+4});
//     the matching x pairs (x_j, x_{j+4}) are permuted once per chunk and reused
//     for every weight row, and v_dot2c_f32_bf16 accumulates in fp32;
//   * the +128 offset is folded into the group bias: s*(D - 128*X) + b*X
//     = s*D + (b - 128*s)*X, with X = sum(x) over the chunk (also a dot2);
//   * cross-lane sums use DPP row_shr / row_bcast (no LDS round trip), and
//     KS waves can split K for short-N shapes, combining through LDS.
#include "qvex_common.h"
#include "w4_dequant.h"

namespace {

// Chunk = 32 consecutive k of one row = 4 uint32 words = 16 bytes.
// Block = 256 threads = 4 waves; KS waves share one row group of R rows and
// split the chunk sequence between them; 4/KS row groups per block.
template <int M, int R, int KS>
__global__ __launch_bounds__(256) void qmv_w4g64_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    uint16_t* __restrict__ y, int N, int K) {
  constexpr int RG = 4 / KS;
  // chunks per lane whose weight loads are issued together (2 measured no faster)
  constexpr int U = 1;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rg = wave / KS;
  const int ws = wave % KS;
  const int row0 = (blockIdx.x * RG + rg) * R;

  const int nchunk = K >> 5;
  const int KW = K >> 3;   // words per row
  const int G = K >> 6;    // groups per row
  const uint32_t magic = opaque_vgpr(kMagic);
  const uint32_t nib = opaque_sgpr(kNib);

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  for (int cbase = ws * 64; cbase < nchunk; cbase += 64 * KS * U) {
    // weights first: they are the long-latency stream; rows past N re-read
    // row N-1 (never stored), chunks past K are skipped
    u32x4 wv[U][R];
    uint32_t sb[U][R][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cbase + u * 64 * KS + lane;
      if (c < nchunk) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = min(row0 + r, N - 1);
          wv[u][r] = load_nt16(w + (size_t)row * KW + (size_t)c * 4);
          sb[u][r][0] = scales[(size_t)row * G + (c >> 1)];
          sb[u][r][1] = biases[(size_t)row * G + (c >> 1)];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cbase + u * 64 * KS + lane;
      if (c >= nchunk) continue;
      // x chunk of every activation row, permuted into (x_j, x_{j+4}) pairs
      uint32_t xp[M][16];
      float xs[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (size_t)m * K + (size_t)c * 32;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = load16(xr + 8 * i);
          xp[m][4 * i + 0] = (v.x & 0xffffu) | (v.z << 16);
          xp[m][4 * i + 1] = (v.x >> 16) | (v.z & 0xffff0000u);
          xp[m][4 * i + 2] = (v.y & 0xffffu) | (v.w << 16);
          xp[m][4 * i + 3] = (v.y >> 16) | (v.w & 0xffff0000u);
          sum = dot2(v.x, kOnes, sum);
          sum = dot2(v.y, kOnes, sum);
          sum = dot2(v.z, kOnes, sum);
          sum = dot2(v.w, kOnes, sum);
        }
        xs[m] = sum;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t ws4[4] = {wv[u][r].x, wv[u][r].y, wv[u][r].z, wv[u][r].w};
        float d[M];
#pragma unroll
        for (int m = 0; m < M; ++m) d[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t wd = ws4[i];
          const uint32_t p0 = and_or(wd, nib, magic);
          const uint32_t p1 = and_or(wd >> 4, nib, magic);
          const uint32_t p2 = and_or(wd >> 8, nib, magic);
          const uint32_t p3 = and_or(wd >> 12, nib, magic);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            d[m] = dot2(p0, xp[m][4 * i + 0], d[m]);
            d[m] = dot2(p1, xp[m][4 * i + 1], d[m]);
            d[m] = dot2(p2, xp[m][4 * i + 2], d[m]);
            d[m] = dot2(p3, xp[m][4 * i + 3], d[m]);
          }
        }
        const float sc = bf16_to_f32((uint16_t)sb[u][r][0]);
        const float bi = bf16_to_f32((uint16_t)sb[u][r][1]);
        const float bo = fmaf(-128.0f, sc, bi);
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = fmaf(sc, d[m], fmaf(bo, xs[m], acc[r][m]));
      }
    }
  }

  // lane reduction: lane 63 ends with the wave total
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = wave_sum_to_lane63(acc[r][m]);

  if constexpr (KS == 1) {
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row < N) {
#pragma unroll
          for (int m = 0; m < M; ++m) y[(size_t)m * N + row] = f32_to_bf16(acc[r][m]);
        }
      }
    }
  } else {
    __shared__ float red[4][R * M];
    if (lane == 63) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) red[wave][r * M + m] = acc[r][m];
    }
    __syncthreads();
    if (ws == 0 && lane < R * M) {
      const int r = lane / M, m = lane % M;
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < KS; ++j) s += red[rg * KS + j][lane];
      const int row = row0 + r;
      if (row < N) y[(size_t)m * N + row] = f32_to_bf16(s);
    }
  }
}

// ---------------------------------------------------------------- MFMA variant
//
// At M > 1 the VALU form above spends 16*M dot2 ops per 16 weight bytes and
// becomes issue-bound well below the HBM roof. This variant keeps the same
// one-op nibble dequant (bf16 128+q pairs) but hands the products to
// v_mfma_f32_16x16x32_bf16, so the VALU work per weight word is fixed (dequant +
// a group fold) whatever M is.
//
// Layout: one MFMA covers 16 weight rows (the 16 output columns n = lane%16)
// and 4 k-chunks of 8 (lane groups c = lane/16). A "set" is the span of K that
// the 4 lane groups cover together: MP = 4 (M <= 4) gives 4 groups per set, one
// per lane group (8 words = 32 B per lane, 8 MFMA steps); MP = 8 (M <= 8) gives
// 2 groups per set, each split over two lane groups (4 words, 4 steps). The
// activation operand is block-diagonal: A row i = (group slot i/MP, activation
// row i%MP) is non-zero only in the k-chunks of its own group, so the 16x16
// accumulator holds one group's partial dot product per (slot, activation row)
// - what the per-group scale/bias fold needs - and lane l's four accumulators
// belong to weight row l%16 and a single group slot, so the fold reads one
// scale and one bias. The bias term needs X = sum(x) per (group, activation
// row): the same A operand times an all-ones B gives it in exactly the fold's
// lane layout, one extra MFMA per step and no VALU work.
//
// Pipelining: a wave walks its group sets (stride WS) with two register
// buffers; the weights, scales, biases and the activation chunks of set i+1
// are in flight while set i is computed. TN 16-row tiles share each activation
// operand; WS waves of a block split the sets of the same tiles and combine
// through LDS in a fixed order, so results depend on (N, K, TN, WS) only.
// (x_0..x_7) as bf16 -> A operand pairs (x_0,x_4) (x_1,x_5) (x_2,x_6) (x_3,x_7),
// matching the order in which and_or() unpacks the nibbles of a word.
__device__ __forceinline__ bf16x8_t perm_x(const u32x4 v) {
  return as_bf16x8((v.x & 0xffffu) | (v.z << 16), (v.x >> 16) | (v.z & 0xffff0000u),
                   (v.y & 0xffffu) | (v.w << 16), (v.y >> 16) | (v.w & 0xffff0000u));
}

constexpr int mfma_block(int WS) { return WS >= 4 ? 64 * WS : 256; }

template <int MP, int TN, int WS>
__global__ __launch_bounds__(mfma_block(WS)) void qmv_mfma_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    uint16_t* __restrict__ y, int M, int N, int K) {
  constexpr int GPM = 16 / MP;     // groups per set
  constexpr int CPG = 4 / GPM;     // lane groups per group
  constexpr int NS = 8 / CPG;      // MFMA steps per set = words per lane per set
  constexpr int NL = NS / 4;       // 16-byte weight loads per lane per set
  constexpr int RG = mfma_block(WS) / 64 / WS;   // tile groups per block
  constexpr int LIVE = 16 * (MP / 4);            // lanes holding distinct (row, m) sums

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = wave / WS, ws = wave % WS;
  const int G = K >> 6;
  const int KW = K >> 3;
  const int GS = G / GPM;

  const uint32_t magic = opaque_vgpr(kMagic);
  const uint32_t nib = opaque_sgpr(kNib);
  const bf16x8_t ones = as_bf16x8(kOnes, kOnes, kOnes, kOnes);

  const int c = lane >> 4, i16 = lane & 15;
  const int cg = c / CPG;                 // group slot of lane group c
  const int cw = (c % CPG) * NS;          // first word (within the group) of lane group c
  const bool part = (i16 / MP) == cg && (i16 % MP) < M;   // A row i16 is live in chunk c
  const int am = i16 % MP;                // activation row fed by this lane
  const int tile0 = (blockIdx.x * RG + rg) * TN;

  float acc[TN][4];
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = 0.0f;

  u32x4 wb[2][TN][NL];
  uint32_t sbuf[2][TN][2];
  u32x4 xb[2][NS];

  auto issue = [&](int buf, int gs) {
    const int g = gs * GPM + cg;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      // rows past N re-read row N-1; their sums are never stored
      const int n = min((tile0 + t) * 16 + i16, N - 1);
      const uint32_t* wp = w + (size_t)n * KW + g * 8 + cw;
#pragma unroll
      for (int q = 0; q < NL; ++q) wb[buf][t][q] = load_nt16(wp + 4 * q);
      sbuf[buf][t][0] = scales[(size_t)n * G + g];
      sbuf[buf][t][1] = biases[(size_t)n * G + g];
    }
    const uint16_t* xp = x + (size_t)(part ? am : 0) * K + g * 64 + cw * 8;
#pragma unroll
    for (int s = 0; s < NS; ++s) xb[buf][s] = part ? load16(xp + 8 * s) : u32x4{0u, 0u, 0u, 0u};
  };

  auto compute = [&](int buf) {
    f32x4_t C[TN], CX = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < TN; ++t) C[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const bf16x8_t a = perm_x(xb[buf][s]);
      CX = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, CX, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const u32x4 wv = wb[buf][t][s / 4];
        const uint32_t wd = (s % 4 == 0) ? wv.x : (s % 4 == 1) ? wv.y : (s % 4 == 2) ? wv.z : wv.w;
        const bf16x8_t b = as_bf16x8(and_or(wd, nib, magic), and_or(wd >> 4, nib, magic),
                                     and_or(wd >> 8, nib, magic), and_or(wd >> 12, nib, magic));
        C[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, C[t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const float sc = bf16_to_f32((uint16_t)sbuf[buf][t][0]);
      const float bi = bf16_to_f32((uint16_t)sbuf[buf][t][1]);
      const float bo = fmaf(-128.0f, sc, bi);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(sc, C[t][r], fmaf(bo, CX[r], acc[t][r]));
    }
  };

  int gs = ws;
  if (gs < GS) issue(0, gs);
  while (gs < GS) {
    const int g1 = gs + WS;
    if (g1 < GS) issue(1, g1);
    compute(0);
    if (g1 >= GS) break;
    const int g2 = g1 + WS;
    if (g2 < GS) issue(0, g2);
    compute(1);
    gs = g2;
  }

  // combine the lane groups that share an activation row
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = acc[t][r];
      if constexpr (MP == 4) v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc[t][r] = v;
    }
  if constexpr (WS > 1) {
    __shared__ float red[RG * WS][TN][4][LIVE];
    if (lane < LIVE) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][t][r][lane] = acc[t][r];
    }
    __syncthreads();
    if (ws != 0) return;
    if (lane < LIVE) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = 0.0f;
#pragma unroll
          for (int j = 0; j < WS; ++j) v += red[rg * WS + j][t][r][lane];
          acc[t][r] = v;
        }
    }
  }
  if (lane < LIVE) {
    const int fm0 = (4 * c) % MP;         // activation row of accumulator 0
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int n = (tile0 + t) * 16 + i16;
      if (n < N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = fm0 + r;
          if (m < M) y[(size_t)m * N + n] = f32_to_bf16(acc[t][r]);
        }
      }
    }
  }
}

// Pure read roof: grid-stride 16-byte loads, folded with xor so nothing is dead.
__global__ __launch_bounds__(256) void read_roof_kernel(const u32x4* __restrict__ buf, uint64_t n16,
                                                        uint32_t* __restrict__ sink) {
  uint32_t a = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = load_nt16(buf + i);
    a ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (a == 0x9e3779b9u) sink[threadIdx.x & 63] = a;  // practically never taken
}

// Read-ceiling probe of one launch, two load paths with the same access
// pattern: W waves each read ITERS 1 KiB units (unit u = wave + i * W, so the
// waves of one step read adjacent KiB), every load issued before the first is
// waited on; LDS = true lands the bytes in LDS with gfx950's
// global_load_lds_dwordx4 (no VGPRs), LDS = false in VGPRs. The host sizes the
// grid so that the buffer is exactly W * ITERS units.
template <int ITERS, bool LDS, int WPB>
__global__ __launch_bounds__(64 * WPB) void read_probe_kernel(const u32x4* __restrict__ buf,
                                                              uint32_t* __restrict__ sink) {
  __shared__ __align__(16) u32x4 ring[LDS ? WPB : 1][LDS ? ITERS : 1][64];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint64_t W = (uint64_t)gridDim.x * WPB;
  const uint64_t gw = (uint64_t)blockIdx.x * WPB + w;
  uint32_t a = 0;
  if constexpr (LDS) {
#pragma unroll
    for (int i = 0; i < ITERS; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(buf + (gw + i * W) * 64 + lane),
                                       (__attribute__((address_space(3))) void*)&ring[w][i][0], 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int i = 0; i < ITERS; ++i) {
      const u32x4 v = ring[w][i][lane];
      a ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  } else {
    u32x4 r[ITERS];
#pragma unroll
    for (int i = 0; i < ITERS; ++i) r[i] = load_nt16(buf + (gw + i * W) * 64 + lane);
#pragma unroll
    for (int i = 0; i < ITERS; ++i) a ^= r[i].x ^ r[i].y ^ r[i].z ^ r[i].w;
  }
  if (a == 0x9e3779b9u) sink[lane] = a;  // practically never taken
}

typedef void (*qmv_fn)(const uint16_t*, const uint32_t*, const uint16_t*, const uint16_t*,
                       uint16_t*, int, int);

template <int M, int R>
qmv_fn pick_ks(int ks) {
  switch (ks) {
    case 1: return qmv_w4g64_kernel<M, R, 1>;
    case 2: return qmv_w4g64_kernel<M, R, 2>;
    case 4: return qmv_w4g64_kernel<M, R, 4>;
  }
  return nullptr;
}

template <int M>
qmv_fn pick_r(int r, int ks) {
  switch (r) {
    case 1: return pick_ks<M, 1>(ks);
    case 2: return pick_ks<M, 2>(ks);
    case 4: return pick_ks<M, 4>(ks);
    case 8: return pick_ks<M, 8>(ks);
  }
  return nullptr;
}

qmv_fn pick(int M, int r, int ks) {
  switch (M) {
    case 1: return pick_r<1>(r, ks);
    case 2: return pick_r<2>(r, ks);
    case 3: return pick_r<3>(r, ks);
    case 4: return pick_r<4>(r, ks);
    case 5: return pick_r<5>(r, ks);
    case 6: return pick_r<6>(r, ks);
    case 7: return pick_r<7>(r, ks);
    case 8: return pick_r<8>(r, ks);
  }
  return nullptr;
}

typedef void (*qmv_mfma_fn)(const uint16_t*, const uint32_t*, const uint16_t*, const uint16_t*,
                            uint16_t*, int, int, int);

template <int MP, int TN>
qmv_mfma_fn pick_mfma_ws(int ws) {
  switch (ws) {
    case 1: return qmv_mfma_kernel<MP, TN, 1>;
    case 2: return qmv_mfma_kernel<MP, TN, 2>;
    case 4: return qmv_mfma_kernel<MP, TN, 4>;
    case 8: return qmv_mfma_kernel<MP, TN, 8>;
  }
  return nullptr;
}

template <int MP>
qmv_mfma_fn pick_mfma_tn(int tn, int ws) {
  switch (tn) {
    case 1: return pick_mfma_ws<MP, 1>(ws);
    case 2: return pick_mfma_ws<MP, 2>(ws);
    case 4: return pick_mfma_ws<MP, 4>(ws);
  }
  return nullptr;
}

int launch_mfma(const uint16_t* x, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                uint16_t* y, int M, int N, int K, int TN, int WS, hipStream_t stream) {
  QVEX_CHECK_ARG(M >= 1 && M <= 8, "qvex_qmv_w4g64: M=%d outside 1..8", M);
  QVEX_CHECK_ARG(N >= 1, "qvex_qmv_w4g64: N=%d", N);
  const int MP = M <= 4 ? 4 : 8;
  const int set_k = 64 * (16 / MP);
  QVEX_CHECK_ARG(K >= set_k && K % set_k == 0, "qvex_qmv_w4g64 (mfma): K=%d must be a multiple of %d", K, set_k);
  QVEX_CHECK_ARG(x && w && scales && biases && y, "qvex_qmv_w4g64: null pointer");
  QVEX_CHECK_ARG(qvex_aligned(x, 16) && qvex_aligned(w, 16), "qvex_qmv_w4g64: x and w must be 16-byte aligned");
  QVEX_CHECK_ARG(qvex_aligned(scales, 2) && qvex_aligned(biases, 2) && qvex_aligned(y, 2),
                 "qvex_qmv_w4g64: scales/biases/y must be 2-byte aligned");
  qmv_mfma_fn fn = MP == 4 ? pick_mfma_tn<4>(TN, WS) : pick_mfma_tn<8>(TN, WS);
  QVEX_CHECK_ARG(fn != nullptr, "qvex_qmv_w4g64 (mfma): unsupported tile TN=%d WS=%d", TN, WS);
  const int threads = WS >= 4 ? 64 * WS : 256;
  const int rows_per_block = 16 * TN * (threads / 64 / WS);
  const int blocks = (N + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(threads), 0, stream, x, w, scales, biases, y, M, N, K);
  QVEX_CHECK_LAUNCH("qvex_qmv_w4g64 (mfma)");
  return QVEX_OK;
}

// Default tile: rows per wave shrink as M grows (x pairs cost 16*M VGPRs); the
// K split depends on (N, K) only, so a row's summation order - and its bits -
// do not change with the number of activation rows.
void default_tile(int M, int N, int K, int* R, int* KS) {
  const int r = M <= 4 ? 4 : 2;
  const int nchunk = K / 32;
  int ks = 1;
  const long target_waves = 4096;  // 16 waves per CU on 256 CUs
  while (ks < 4 && (long)((N + 3) / 4) * ks < target_waves && nchunk >= 64 * ks * 2) ks *= 2;
  *R = r;
  *KS = ks;
}

int launch(const uint16_t* x, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
           uint16_t* y, int M, int N, int K, int R, int KS, hipStream_t stream) {
  QVEX_CHECK_ARG(M >= 1 && M <= 8, "qvex_qmv_w4g64: M=%d outside 1..8", M);
  QVEX_CHECK_ARG(N >= 1, "qvex_qmv_w4g64: N=%d", N);
  QVEX_CHECK_ARG(K >= 64 && K % 64 == 0, "qvex_qmv_w4g64: K=%d must be a positive multiple of 64", K);
  QVEX_CHECK_ARG(x && w && scales && biases && y, "qvex_qmv_w4g64: null pointer");
  QVEX_CHECK_ARG(qvex_aligned(x, 16) && qvex_aligned(w, 16), "qvex_qmv_w4g64: x and w must be 16-byte aligned");
  QVEX_CHECK_ARG(qvex_aligned(scales, 2) && qvex_aligned(biases, 2) && qvex_aligned(y, 2),
                 "qvex_qmv_w4g64: scales/biases/y must be 2-byte aligned");
  qmv_fn fn = pick(M, R, KS);
  QVEX_CHECK_ARG(fn != nullptr, "qvex_qmv_w4g64: unsupported tile R=%d KS=%d", R, KS);
  const int rows_per_block = R * (4 / KS);
  const int blocks = (N + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), 0, stream, x, w, scales, biases, y, N, K);
  QVEX_CHECK_LAUNCH("qvex_qmv_w4g64");
  return QVEX_OK;
}

// W[n, k] = bf16(s * q + b) in fp32 (one rounding), for the dense GEMM of long
// (prefill) calls. One thread per uint32 word: eight codes of one group, one
// 16-byte store.
__global__ __launch_bounds__(256) void dequant_w4g64_kernel(const uint32_t* __restrict__ w,
                                                            const uint16_t* __restrict__ scales,
                                                            const uint16_t* __restrict__ biases,
                                                            uint16_t* __restrict__ out, long words, int K) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int KW = K / 8;
  const long n = i / KW;
  const int kw = (int)(i - n * KW);
  const int g = kw / 8;                       // 64 codes = 8 words per group
  const float sc = bf16_to_f32(scales[n * (K / 64) + g]);
  const float bi = bf16_to_f32(biases[n * (K / 64) + g]);
  const uint32_t wd = w[i];
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = fmaf(sc, (float)((wd >> (8 * j)) & 0xFu), bi);
    const float hi = fmaf(sc, (float)((wd >> (8 * j + 4)) & 0xFu), bi);
    o[j] = pack_bf16x2(lo, hi);
  }
  u32x4 v;
  v.x = o[0]; v.y = o[1]; v.z = o[2]; v.w = o[3];
  *reinterpret_cast<u32x4*>(out + i * 8) = v;
}

}  // namespace

extern "C" int qvex_w4g64_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N, int K,
                                  uint16_t* out, void* stream) {
  QVEX_CHECK_ARG(w && scales && biases && out, "qvex_w4g64_dequant: null pointer");
  QVEX_CHECK_ARG(N >= 1 && K >= 64 && K % 64 == 0, "qvex_w4g64_dequant: N=%d K=%d (K a positive multiple of 64)", N,
                 K);
  QVEX_CHECK_ARG(qvex_aligned(out, 16) && qvex_aligned(w, 4), "qvex_w4g64_dequant: out must be 16-byte aligned");
  const long words = (long)N * (K / 8);
  QVEX_CHECK_ARG(words / 256 < 0x7fffffffL, "qvex_w4g64_dequant: too large");
  hipLaunchKernelGGL(dequant_w4g64_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     w, scales, biases, out, words, K);
  QVEX_CHECK_LAUNCH("qvex_w4g64_dequant");
  return QVEX_OK;
}

extern "C" int qvex_qmv_w4g64(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                              const uint16_t* biases, uint16_t* y, int M, int N, int K, void* stream) {
  int R = 4, KS = 1;
  if (M >= 1 && M <= 8 && K > 0) default_tile(M, N, K, &R, &KS);
  return launch(x, w, scales, biases, y, M, N, K, R, KS, (hipStream_t)stream);
}

extern "C" int qvex_qmv_w4g64_tiled(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                                    const uint16_t* biases, uint16_t* y, int M, int N, int K,
                                    int rows_per_wave, int k_split, void* stream) {
  return launch(x, w, scales, biases, y, M, N, K, rows_per_wave, k_split, (hipStream_t)stream);
}

extern "C" int qvex_qmv_w4g64_mfma(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                                   const uint16_t* biases, uint16_t* y, int M, int N, int K,
                                   int tiles_per_wave, int wave_ksplit, void* stream) {
  return launch_mfma(x, w, scales, biases, y, M, N, K, tiles_per_wave, wave_ksplit, (hipStream_t)stream);
}

template <int ITERS, bool LDS, int WPB>
int launch_read_probe(const void* buf, uint64_t bytes, uint32_t* sink, hipStream_t stream) {
  const uint64_t blocks = bytes / 1024 / ((uint64_t)ITERS * WPB);
  hipLaunchKernelGGL((read_probe_kernel<ITERS, LDS, WPB>), dim3((unsigned)blocks), dim3(64 * WPB), 0, stream,
                     reinterpret_cast<const u32x4*>(buf), sink);
  QVEX_CHECK_LAUNCH("qvex_read_probe");
  return QVEX_OK;
}

extern "C" int qvex_read_probe(const void* buf, uint64_t bytes, uint32_t* sink, int iters, int lds,
                               int waves_per_block, void* stream) {
  QVEX_CHECK_ARG(buf && sink && qvex_aligned(buf, 16), "qvex_read_probe: null or misaligned pointer");
  QVEX_CHECK_ARG((iters == 2 || iters == 4 || iters == 8 || iters == 16) && (waves_per_block == 4 ||
                 waves_per_block == 8) && (lds == 0 || lds == 1),
                 "qvex_read_probe: iters=%d (2, 4, 8, 16), waves_per_block=%d (4, 8), lds=%d", iters, waves_per_block,
                 lds);
  const uint64_t unit = 1024ull * iters * waves_per_block;
  QVEX_CHECK_ARG(bytes > 0 && bytes % unit == 0 && bytes / unit <= 0x7fffffffull,
                 "qvex_read_probe: bytes=%llu must be a positive multiple of %llu", (unsigned long long)bytes,
                 (unsigned long long)unit);
  hipStream_t st = (hipStream_t)stream;
#define QVEX_PROBE(I, Wp)                                                                        \
  if (iters == I && waves_per_block == Wp)                                                       \
    return lds ? launch_read_probe<I, true, Wp>(buf, bytes, sink, st) : launch_read_probe<I, false, Wp>(buf, bytes, sink, st);
  QVEX_PROBE(2, 4) QVEX_PROBE(2, 8) QVEX_PROBE(4, 4) QVEX_PROBE(4, 8)
  QVEX_PROBE(8, 4) QVEX_PROBE(8, 8) QVEX_PROBE(16, 4) QVEX_PROBE(16, 8)
#undef QVEX_PROBE
  return qvex::fail(QVEX_EINVAL, "qvex_read_probe: unreachable");
}

extern "C" int qvex_read_roof(const void* buf, uint64_t bytes, uint32_t* sink, int blocks, void* stream) {
  QVEX_CHECK_ARG(buf && sink, "qvex_read_roof: null pointer");
  QVEX_CHECK_ARG(bytes % 16 == 0 && qvex_aligned(buf, 16), "qvex_read_roof: bytes and buf must be 16-byte multiples");
  QVEX_CHECK_ARG(blocks >= 1 && blocks <= (1 << 20), "qvex_read_roof: blocks=%d", blocks);
  hipLaunchKernelGGL(read_roof_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const u32x4*>(buf), (uint64_t)(bytes / 16), sink);
  QVEX_CHECK_LAUNCH("qvex_read_roof");
  return QVEX_OK;
}
