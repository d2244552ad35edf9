// 4-bit group-64 skinny GEMM (M = 1..8 activation rows) on a tile-packed copy of
// the MLX weights, for the verify / draft matmuls of the decode cycle.
//
// Reference semantics: mx.quantized_matmul(transpose=True, group_size=64, bits=4)
// in QLinear.__call__ (engine/model.py:87-91); the weights are the QLinear
// triplet (engine/model.py:83-85), re-laid once when the layer is built.
//
// Why a second layout. The MFMA form of the product (block-diagonal activation
// operand, see the MFMA variant in qmv.hip) needs every lane of a wave to hold a
// different weight row; in the MLX row-major layout that makes each 16-byte load
// instruction touch 16 rows (16 cache lines per KiB), and the load path, not HBM,
// sets the speed. The packed layout stores each (16-row tile, 256-k set) as one
// record in exactly the order the lanes consume it:
//
//   record (tile t, set s), 2304 bytes, records ordered [t][s]:
//     bytes [0, 2048):    [q = 0..1][lane L = 0..63][4 words]; lane L = 16c + i
//                         holds words 4q .. 4q+3 of group 4s + c of row 16t + i
//     bytes [2048, 2304): [lane L] (scale, bias) bf16 pair of that row and group
//
//   Each word's nibbles are reordered so that (w >> 4j) & 0x000F000F yields the
//   codes of k = 2j and 2j + 1 (even k in the low half-word, odd k in the high
//   half-word); the activations then enter the MFMA in their natural order.
//   Rows past N are zero (weights, scale and bias) and never stored.
//
// A wave reads one record per (tile, set) with two fully coalesced 1 KiB loads
// plus one 256-byte load; the activation slice of the set (M x 256 bf16) comes in
// with two more coalesced loads, goes through a wave-private LDS slot and is read
// back per MFMA step by the 16 lanes whose A rows are live in that k-chunk (the
// other lanes read a zeroed area of the slot).
#include "qvex_common.h"
#include "w4_dequant.h"

namespace {

constexpr int PK_TILE = 16;
constexpr int PK_SET = 256;               // k per record = 4 groups
constexpr int PK_WBYTES = 2048;
constexpr int PK_RECORD = 2304;

// nibbles q0..q7 at bits 4k  ->  q_{2j} at bits 4j, q_{2j+1} at bits 16 + 4j
__device__ __forceinline__ uint32_t reorder_nibbles(uint32_t w) {
  uint32_t r = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r |= ((w >> (8 * j)) & 0xFu) << (4 * j);
    r |= ((w >> (8 * j + 4)) & 0xFu) << (16 + 4 * j);
  }
  return r;
}

// Source row of tile row i of tile t. Plain: 16t + i. SwiGLU interleave (the
// fused gate/up weight, gate rows [0, N/2), up rows [N/2, N)): tile t holds gate
// rows 8t..8t+7 in its first 8 rows and the matching up rows in its last 8, so
// one wave ends with both halves of 8 SwiGLU outputs. -1 = past the end (zero).
__device__ __forceinline__ int pack_src_row(int t, int i, int N, int swiglu) {
  if (!swiglu) {
    const int r = t * PK_TILE + i;
    return r < N ? r : -1;
  }
  const int half = N / 2;
  const int j = 8 * t + (i & 7);
  return j < half ? (i < 8 ? j : half + j) : -1;
}

// one 64-thread block per record
__global__ __launch_bounds__(64) void pack_kernel(const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases, int N, int K, int swiglu,
                                                  uint8_t* __restrict__ packed) {
  const int GS = K / PK_SET;
  const int t = blockIdx.x / GS, s = blockIdx.x % GS;
  const int L = threadIdx.x, c = L >> 4, i = L & 15;
  const int src = pack_src_row(t, i, N, swiglu);
  const int g = s * 4 + c;
  const int KW = K / 8, G = K / 64;
  uint8_t* rec = packed + (size_t)blockIdx.x * PK_RECORD;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (src >= 0) {
      const uint32_t* sp = w + (size_t)src * KW + g * 8 + 4 * q;
      v = u32x4{reorder_nibbles(sp[0]), reorder_nibbles(sp[1]), reorder_nibbles(sp[2]), reorder_nibbles(sp[3])};
    }
    *reinterpret_cast<u32x4*>(rec + q * 1024 + L * 16) = v;
  }
  uint32_t sb = 0;
  if (src >= 0) sb = (uint32_t)scales[(size_t)src * G + g] | ((uint32_t)biases[(size_t)src * G + g] << 16);
  *reinterpret_cast<uint32_t*>(rec + PK_WBYTES + L * 4) = sb;
}

// A 64-bit right shift as one v_lshrrev_b64 (the compiler would split it into
// v_alignbit_b32 + v_lshrrev_b32 when both halves are used separately).
template <int SH>
__device__ __forceinline__ uint64_t shr64(uint64_t v) {
  uint64_t r;
  asm("v_lshrrev_b64 %0, %1, %2" : "=v"(r) : "i"(SH), "v"(v));
  return r;
}

// Max / min over the 16 lanes of a DPP row, the same in all 16 lanes.
__device__ __forceinline__ float row16_allmax(float v) {
  v = fmaxf(v, dpp_row<0xB1>(v));
  v = fmaxf(v, dpp_row<0x4E>(v));
  v = fmaxf(v, dpp_row<0x124>(v));
  v = fmaxf(v, dpp_row<0x128>(v));
  return v;
}
template <int CTRL>
__device__ __forceinline__ int dpp_row_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ int row16_allmin(int v) {
  v = min(v, dpp_row_i<0xB1>(v));
  v = min(v, dpp_row_i<0x4E>(v));
  v = min(v, dpp_row_i<0x124>(v));
  v = min(v, dpp_row_i<0x128>(v));
  return v;
}

// Optional epilogues that take the residual RMSNorm out of its own launch
// (mx.fast.rms_norm after the residual add, engine/model.py:309-317). The norm's
// per-row scale rsqrt(mean(h^2) + eps) commutes with the product, so:
//   producer (resid != null): the layer output delta = bf16(x W^T) is added to
//     the residual stream, h = bf16(resid + delta), and the epilogue writes h,
//     u = bf16(h * norm_w) (the next norm's weight applied) and, per row and
//     16-row tile, the partial sum of h^2 (16-lane DPP sum) to sq_parts[r][tile];
//   consumer (rs_parts != null): x is such a u, and every output row r is scaled
//     by rsqrt(S_r / rs_dim + rs_eps) before rounding, S_r the sum of the row's
//     rs_nparts (<= 256, a multiple of 4) partials in a fixed order (lane l adds
//     parts 4l .. 4l+3, then an xor butterfly over the wave).
// The product itself is unchanged, so the rows stay independent of M.
// An argmax epilogue (greedy drafting on the lm_head) is below.
struct PkEpi {
  const float* rs_parts;
  int rs_nparts, rs_dim;
  float rs_eps;
  const uint16_t* resid;
  const uint16_t* norm_w;
  uint16_t* h_out;
  uint16_t* u_out;
  float* sq_parts;
  // argmax (am_parts != null): per row r and 16-row tile j, the largest
  // bf16-rounded output and its first index -> am_parts[(r * tiles + j) * 2 + {0, 1}]
  float* am_parts;
  // tile maxima (tm_out != null): per row r and 16-row tile j, the largest
  // bf16-rounded output -> tm_out[r * tiles + j] (bf16), what the sampler's
  // one-kernel list form starts from
  uint16_t* tm_out;
  // head-segment scale (seg_ss != null; the gated RMSNorm before out_proj,
  // engine/model.py:285-288): x is u = bf16(silu(z) * w * y) for K / 128 <= 64
  // heads of 128 columns, and the share of the product over head h of row r is
  // scaled by rsqrt(S_rh / 128 + seg_eps) in fp32, S_rh the sum of the seg_nb
  // (1, 2, 4 or 8) partials seg_ss[(r * K / 128 + h) * seg_nb + b] in order.
  // The block puts the scales in LDS once, while its first weights load; each
  // lane's 64-column group lies in one head.
  const float* seg_ss;
  int seg_nb;
  float seg_eps;
};

constexpr int pk_block(int WS) { return WS >= 4 ? 64 * WS : 256; }   // WS = 16: 1024 threads
// Waves per SIMD the register budget must allow: the lm_head-wide (2, 4)
// double-buffered product runs ~30 k waves in many rounds and needs 4 resident
// (at most 128 VGPRs: 84.9 against 91.8 us at M = 1 when the compiler takes 172);
// the others run one round of waves and keep the compiler's choice.
constexpr int pk_min_waves(int TN, int WS, int NP, int MH) { return TN == 2 && WS == 4 && NP == 0 && MH == 1 ? 4 : 1; }

// TN 16-row tiles per wave share each activation operand; WS waves of a block
// split the sets of the same tiles (set ws, ws + WS, ...) and combine through
// LDS in a fixed order; 4 / WS tile groups per block when WS < 4. Two register
// buffers: the records and activation slice of the next set are in flight while
// the current one is computed. NP > 0 instead issues the loads of all of a wave's
// sets (at most NP; indices past the last set are clamped and not computed) before
// computing any, so a wave with few sets keeps all its bytes in flight; the sets
// are still computed in the same order. Results depend on (N, K, TN, WS) only,
// never on M or NP.
// MODE 1 (SwiGLU): the weight was packed with the gate/up interleave; the
// epilogue rounds the gate and up products to bf16 (as the unfused pair of calls
// would) and writes bf16(silu(g) * u) to y [M, N/2]. MODE 2: the head-segment
// scale of PkEpi (a mode of its own so that the other kernels keep their
// registers). MODE 0: plain.
// The arguments read before the first weight loads - x, the packed weights and
// the shape, the consumer's partials (or the segment scales) with their count,
// the residual and the norm weight - are separate scalar arguments at the front,
// so that they fill the 14 dwords of kernel arguments preloaded into SGPRs (16
// user SGPRs less the argument pointer): an aggregate argument is never
// preloaded, and a wait for its fields held every first load back by a
// scalar-load round trip. y and PkEpi (which keeps all fields) are read later.
template <int TN, int WS, int NP, int MODE, int MH>
__global__ __launch_bounds__(pk_block(WS)) __attribute__((amdgpu_waves_per_eu(pk_min_waves(TN, WS, NP, MH)))) void qmv_packed_kernel(const uint16_t* __restrict__ x,
                                                                   const uint8_t* __restrict__ packed, int M,
                                                                   int N, int K, int pre_n,
                                                                   const float* __restrict__ pre_p,
                                                                   const uint16_t* __restrict__ pre_resid,
                                                                   const uint16_t* __restrict__ pre_norm_w,
                                                                   uint16_t* __restrict__ y, PkEpi e) {
  constexpr int NWAVE = pk_block(WS) / 64;
  constexpr int RG = NWAVE / WS;
  // the wave index is uniform: in an SGPR, the tile / set / record arithmetic is scalar
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave / WS, ws = wave % WS;
  const int GS = K / PK_SET;
  const int tiles = (N + PK_TILE - 1) / PK_TILE;
  const int c = lane >> 4, i16 = lane & 15;
  const int am = i16 & 3;
  constexpr int MR = 4 * MH;                     // activation rows: MH halves of 4
  const int tile0 = (blockIdx.x * RG + rg) * TN;

  // per wave: [activation row][32 chunks of 8 bf16], then 8 zero chunks that the
  // lanes outside the block diagonal read in place of x (no predicated reads).
  // Half h's A row i16 = (group slot i16/4, activation row 4h + i16%4).
  __shared__ u32x4 xslot[NWAVE][MR * 32 + 8];
  u32x4* slot = xslot[wave];
  if (lane < 8) slot[MR * 32 + lane] = u32x4{0u, 0u, 0u, 0u};
  const u32x4* arow[MH];
#pragma unroll
  for (int h = 0; h < MH; ++h) {
    const bool part = (i16 >> 2) == c && 4 * h + am < M;
    arow[h] = part ? slot + (4 * h + am) * 32 + c * 8 : slot + MR * 32;
  }

  const uint32_t magic = opaque_vgpr(kMagic);
  const uint32_t nib = opaque_sgpr(kNib);
  // four distinct registers (the compiler would otherwise keep one and copy it per step)
  const bf16x8_t ones = as_bf16x8(opaque_vgpr(kOnes), opaque_vgpr(kOnes), opaque_vgpr(kOnes), opaque_vgpr(kOnes));

  float acc[TN][MR];
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[t][r] = 0.0f;

  constexpr int NB = NP > 0 ? NP : 2;
  u32x4 wb[NB][TN][2];
  uint32_t sb[NB][TN];
  u32x4 xr[NB][2 * MH];
  int sgs[NB];

  // activation slice loader: lane L of load q covers row 2q + L/32, chunk L%32
  const int xm0 = lane >> 5, xch = lane & 31;
  constexpr bool SWIGLU = MODE == 1;
  constexpr bool seg = MODE == 2;

  // head-segment partials: thread i sums pair (head i / MR, row i % MR).
  // Epilogue inputs are loaded from clamped (always valid) addresses with no
  // condition, and the entries that do not exist are dropped where the values
  // are used: a conditional load makes the compiler wait for it at the end of
  // the condition, before the weight loads go out.
  __shared__ __align__(16) float seg_tab[seg ? 64 * MR : 4];
  const int H = K / 128;
  float segv[8];
  if constexpr (seg) {   // pre_p = e.seg_ss, pre_n = e.seg_nb
    const int sh = min((int)threadIdx.x / MR, H - 1), sr = min((int)threadIdx.x % MR, M - 1);
#pragma unroll
    for (int b = 0; b < 8; ++b) segv[b] = pre_p[((size_t)sr * H + sh) * pre_n + min(b, pre_n - 1)];
  }
  auto seg_table = [&]() {
    if constexpr (seg) {
      if ((int)threadIdx.x < MR * H) {
        float v = segv[0];
#pragma unroll
        for (int b = 1; b < 8; ++b)
          if (b < pre_n) v += segv[b];
        seg_tab[threadIdx.x] = (int)(threadIdx.x % MR) < M ? rsqrtf(v / 128.0f + e.seg_eps) : 1.0f;
      }
      __syncthreads();
    }
  };

  // epilogue inputs, requested before the weights so their latency hides
  // (MODE != 2: pre_p = e.rs_parts, pre_n = e.rs_nparts)
  const bool rs = !seg && pre_p != nullptr, prod = pre_resid != nullptr;
  u32x4 rsp[MR];
  if (rs && ws == 0) {
#pragma unroll
    for (int r = 0; r < MR; ++r)
      rsp[r] = load16(pre_p + (size_t)min(r, M - 1) * pre_n + min(4 * lane, pre_n - 4));
  }
  // the plain epilogue gives lane L row L / 16 and column L % 16 of each tile
  const int er = lane >> 4, ei = lane & 15;
  // (loaded by every wave, with x standing in when there is no residual: under a
  // branch the compiler converts them as soon as they arrive, which waits)
  uint16_t rsd[MH][TN], nw[TN];
  {
    const uint16_t* rp = prod ? pre_resid : x;
    const uint16_t* wp = prod ? pre_norm_w : x;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int nc = min((tile0 + t) * PK_TILE + ei, N - 1);   // columns past N and rows past M are never stored
      nw[t] = wp[prod ? nc : 0];
#pragma unroll
      for (int h = 0; h < MH; ++h) rsd[h][t] = rp[prod ? (size_t)min(4 * h + er, M - 1) * N + nc : 0];
    }
  }
  // consumer scale: summed as soon as the partials are in (they were requested
  // first), off the tail of the kernel; a DPP sum into lane 63, read back
  // rstd[r] for the SwiGLU epilogue, rs_row[mh] = rstd[4 mh + er] for the plain
  // one (selected as the sums complete: an index by the lane's row would make
  // the compiler keep the array in scratch)
  float rstd[MR], rs_row[MH];
#pragma unroll
  for (int r = 0; r < MR; ++r) rstd[r] = 1.0f;
#pragma unroll
  for (int mh = 0; mh < MH; ++mh) rs_row[mh] = 1.0f;
  auto compute_rstd = [&]() {
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      float v = ((__uint_as_float(rsp[r].x) + __uint_as_float(rsp[r].y)) + __uint_as_float(rsp[r].z)) +
                __uint_as_float(rsp[r].w);
      v = 4 * lane < pre_n ? v : 0.0f;   // lanes past the partials loaded a copy
      v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_to_lane63(v)), 63));
      rstd[r] = rsqrtf(v / (float)e.rs_dim + e.rs_eps);
      rs_row[r / 4] = (r % 4) == er ? rstd[r] : rs_row[r / 4];
    }
  };

  auto issue = [&](int buf, int gs) {
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int tile = min(tile0 + t, tiles - 1);   // tiles past the end re-read the last one, never stored
      const uint8_t* rec = packed + ((size_t)tile * GS + gs) * PK_RECORD;
      wb[buf][t][0] = load_nt16(rec + lane * 16);
      wb[buf][t][1] = load_nt16(rec + 1024 + lane * 16);
      sb[buf][t] = *reinterpret_cast<const uint32_t*>(rec + PK_WBYTES + lane * 4);
    }
    // rows m >= M re-read row M - 1: only the block-diagonal lanes of rows < M
    // ever read the slot, so no zero fill (and no predicated load) is needed
#pragma unroll
    for (int q = 0; q < 2 * MH; ++q) {
      const int m = min(2 * q + xm0, M - 1);
      xr[buf][q] = load16(x + (size_t)m * K + (size_t)gs * PK_SET + 8 * xch);
    }
    sgs[buf] = gs;
  };

  auto compute = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 2 * MH; ++q) slot[(2 * q + xm0) * 32 + xch] = xr[buf][q];
    f32x4_t C[MH][TN], CX[MH];
#pragma unroll
    for (int mh = 0; mh < MH; ++mh) {
      CX[mh] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < TN; ++t) C[mh][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
#pragma unroll
    for (int s = 0; s < 8; s += 2) {
      // steps s and s + 1 use adjacent words of a tile: one 64-bit shift moves
      // both (the bits a word takes from its neighbour fall outside the mask)
      bf16x8_t b[TN][2];
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const u32x4 wv = wb[buf][t][s / 4];
        const uint64_t pr = (s % 4 == 0) ? ((uint64_t)wv.y << 32 | wv.x) : ((uint64_t)wv.w << 32 | wv.z);
        const uint64_t p4 = shr64<4>(pr), p8 = shr64<8>(pr), p12 = shr64<12>(pr);
#pragma unroll
        for (int h = 0; h < 2; ++h)
          b[t][h] = as_bf16x8(and_or((uint32_t)(pr >> (32 * h)), nib, magic), and_or((uint32_t)(p4 >> (32 * h)), nib, magic),
                              and_or((uint32_t)(p8 >> (32 * h)), nib, magic), and_or((uint32_t)(p12 >> (32 * h)), nib, magic));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int mh = 0; mh < MH; ++mh) {   // both row halves share the dequantized weights
          const bf16x8_t a = __builtin_bit_cast(bf16x8_t, arow[mh][s + h]);
          CX[mh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, CX[mh], 0, 0, 0);
#pragma unroll
          for (int t = 0; t < TN; ++t) C[mh][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[t][h], C[mh][t], 0, 0, 0);
        }
    }
    if constexpr (seg) {
      // lane (c, i16) holds group slot c: head 2 gs + c / 2 of rows 4 mh .. 4 mh + 3
#pragma unroll
      for (int mh = 0; mh < MH; ++mh) {
        const float4 gt = reinterpret_cast<const float4*>(seg_tab)[(2 * sgs[buf] + (c >> 1)) * MH + mh];
        const float g[4] = {gt.x, gt.y, gt.z, gt.w};
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const float sc = bf16_to_f32((uint16_t)(sb[buf][t] & 0xffffu));
          const float bi = bf16_to_f32((uint16_t)(sb[buf][t] >> 16));
          const float bo = fmaf(-128.0f, sc, bi);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[t][4 * mh + r] = fmaf(g[r], fmaf(sc, C[mh][t][r], bo * CX[mh][r]), acc[t][4 * mh + r]);
        }
      }
      return;
    }
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const float sc = bf16_to_f32((uint16_t)(sb[buf][t] & 0xffffu));
      const float bi = bf16_to_f32((uint16_t)(sb[buf][t] >> 16));
      const float bo = fmaf(-128.0f, sc, bi);
#pragma unroll
      for (int mh = 0; mh < MH; ++mh)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[t][4 * mh + r] = fmaf(sc, C[mh][t][r], fmaf(bo, CX[mh][r], acc[t][4 * mh + r]));
    }
  };

  // this wave's sets ws, ws + WS, ... taken from a block-dependent start, so
  // the blocks' first activation loads spread over every slice of x instead of
  // all hitting the same few lines (fixed per tile, so rows stay M-independent;
  // every load pipeline uses the same order)
  const int nws = ws < GS ? (GS - ws + WS - 1) / WS : 0;
  const int rot = nws > 1 ? (int)(blockIdx.x % (unsigned)nws) : 0;
  auto set_of = [&](int j) { const int jj = j + rot; return ws + (jj >= nws ? jj - nws : jj) * WS; };
  if constexpr (NP == 0) {
    // Each step requests the next set, then computes the current one. The loop
    // body has no branch (a branch between a request and its use lets the
    // compiler sink the request past the compute before it, and a conditional
    // request makes its wait counts cover both paths, so that the wait for the
    // current set also waits for the next); the last one or two sets are
    // computed after it. Buffer 0 holds set j at the top of the loop.
    // unconditional (a wave without sets re-reads the last one, never used), so
    // that the folded norm's wait below counts only its own, earlier loads: a
    // conditional request made it wait for this set as well, before the next
    // set was requested
    issue(0, nws > 0 ? set_of(0) : GS - 1);
    seg_table();
    if (rs && ws == 0) compute_rstd();
    int j = 0;
    for (; j + 2 < nws; j += 2) {
      issue(1, set_of(j + 1));
      __builtin_amdgcn_sched_barrier(0);   // keep the request ahead of the compute
      compute(0);
      issue(0, set_of(j + 2));
      __builtin_amdgcn_sched_barrier(0);
      compute(1);
    }
    if (j + 1 < nws) {
      issue(1, set_of(j + 1));
      __builtin_amdgcn_sched_barrier(0);
      compute(0);
      compute(1);
    } else if (j < nws) {
      compute(0);
    }
  } else {
#pragma unroll
    for (int j = 0; j < NP; ++j) issue(j, j < nws ? set_of(j) : GS - 1);
    seg_table();
    if (rs && ws == 0) compute_rstd();
#pragma unroll
    for (int j = 0; j < NP; ++j)
      if (j < nws) compute(j);
  }

  // lane (c, i16) holds group slot c of row i16: sum the 4 slots
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      float v = acc[t][r];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc[t][r] = v;
    }
  if constexpr (WS > 1) {
    __shared__ float red[NWAVE][TN][MR][16];
    if (lane < 16) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < MR; ++r) red[wave][t][r][lane] = acc[t][r];
    }
    __syncthreads();
    if (ws != 0) return;
    if (lane < 16) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          float v = 0.0f;
#pragma unroll
          for (int j = 0; j < WS; ++j) v += red[rg * WS + j][t][r][lane];
          acc[t][r] = v;
        }
    }
  }
  if constexpr (SWIGLU) {
    // lanes 0-7 hold gate rows, lanes 8-15 the matching up rows. The TN*MR*8
    // outputs are spread over the wave through its (now idle) LDS slot so that
    // each lane evaluates at most TN*MR/8 of the exp/divide pairs.
    const int half = N / 2;
    float* ep = reinterpret_cast<float*>(slot);          // [TN][MR][16] floats <= 1 KiB per 4 rows of the slot
    if (lane < 16) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < MR; ++r) ep[(t * MR + r) * 16 + lane] = rs ? acc[t][r] * rstd[r] : acc[t][r];
    }
#pragma unroll
    for (int o = lane; o < TN * 8 * MR; o += 64) {
      const int t = o / (8 * MR), r = (o >> 3) % MR, i = o & 7;
      const float gv = bf16_to_f32(f32_to_bf16(ep[(t * MR + r) * 16 + i]));
      const float uv = bf16_to_f32(f32_to_bf16(ep[(t * MR + r) * 16 + 8 + i]));
      const int j = (tile0 + t) * 8 + i;
      if (j < half && r < M) y[(size_t)r * half + j] = f32_to_bf16(gv / (1.0f + expf(-gv)) * uv);
    }
  } else {
    // lanes 0-15 hold row r of tile t in acc[t][r]; spread through the wave's
    // (idle) LDS slot so that lane L finishes rows L / 16 + 4 mh, column L % 16
    float* ep = reinterpret_cast<float*>(slot);          // [TN][MR][16] floats <= 1 KiB per 4 rows of the slot
    if (lane < 16) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < MR; ++r) ep[(t * MR + r) * 16 + lane] = acc[t][r];
    }
#pragma unroll
    for (int mh = 0; mh < MH; ++mh) {
      const int row = 4 * mh + er;
      const float rs_r = rs_row[mh];
      if (row < M) {                    // whole 16-lane DPP rows
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const int n = (tile0 + t) * PK_TILE + ei;
          const int tile = tile0 + t;
          const float a = ep[(t * MR + row) * 16 + ei];
          const uint16_t d = f32_to_bf16(rs ? a * rs_r : a);
          if (prod) {
            const float hv = n < N ? bf16_to_f32(f32_to_bf16(bf16_to_f32(rsd[mh][t]) + bf16_to_f32(d))) : 0.0f;
            const float sq = row16_allsum(hv * hv);
            if (n < N) {
              e.h_out[(size_t)row * N + n] = f32_to_bf16(hv);
              e.u_out[(size_t)row * N + n] = f32_to_bf16(hv * bf16_to_f32(nw[t]));
            }
            if (ei == 0 && tile < tiles) e.sq_parts[(size_t)row * tiles + tile] = sq;
          }
          if (y && n < N) y[(size_t)row * N + n] = d;
          if (e.am_parts || e.tm_out) {
            // the tile's largest rounded output and its first column (whole DPP rows active)
            const float v = n < N ? bf16_to_f32(d) : -__builtin_inff();
            const float m = row16_allmax(v);
            if (e.am_parts) {
              const int j = row16_allmin(n < N && v == m ? n : 0x7fffffff);
              if (ei == 0 && tile < tiles) {
                e.am_parts[((size_t)row * tiles + tile) * 2] = m;
                e.am_parts[((size_t)row * tiles + tile) * 2 + 1] = __int_as_float(j);
              }
            }
            if (e.tm_out && ei == 0 && tile < tiles) e.tm_out[(size_t)row * tiles + tile] = f32_to_bf16(m);
          }
        }
      }
    }
  }
}

// Row r's first index of its largest output from the per-tile (max, first index)
// pairs, tiles in index order: thread t takes tiles t + AM_T * i (all its loads
// issued at once), keeps the largest value and, on a tie, the smaller index;
// the block then does the same over its threads.
constexpr int AM_T = 1024;
constexpr int AM_PER = 16;   // tiles per thread per round: 16384 tiles (262144 outputs) per round

__global__ __launch_bounds__(AM_T) void argmax_parts_kernel(const float* __restrict__ parts, int tiles,
                                                            int32_t* __restrict__ out) {
  __shared__ float bvs[AM_T / 64];
  __shared__ int bjs[AM_T / 64];
  const int r = blockIdx.x, t = threadIdx.x;
  const float2* p = reinterpret_cast<const float2*>(parts + (size_t)r * tiles * 2);
  float bv = -__builtin_inff();
  int bj = 0x7fffffff;
  for (int q0 = 0; q0 < tiles; q0 += AM_T * AM_PER) {
    float2 v[AM_PER];
#pragma unroll
    for (int i = 0; i < AM_PER; ++i) {
      const int q = q0 + t + AM_T * i;
      v[i] = q < tiles ? p[q] : make_float2(-__builtin_inff(), __int_as_float(0x7fffffff));
    }
#pragma unroll
    for (int i = 0; i < AM_PER; ++i) {
      const int j = __float_as_int(v[i].y);
      if (v[i].x > bv || (v[i].x == bv && j < bj)) { bv = v[i].x; bj = j; }
    }
  }
  const float m = wave_allmax(bv);
  int c = bv == m ? bj : 0x7fffffff;
  c = wave_allmin(c);
  if ((t & 63) == 0) { bvs[t >> 6] = m; bjs[t >> 6] = c; }
  __syncthreads();
  // the waves' pairs by wave 0: the largest value, then the smallest index holding it
  if (t < 64) {
    const float v = t < AM_T / 64 ? bvs[t] : -__builtin_inff();
    const int j = t < AM_T / 64 ? bjs[t] : 0x7fffffff;
    const float mm = wave_allmax(v);
    const int cc = wave_allmin(v == mm ? j : 0x7fffffff);
    if (t == 0) out[r] = cc == 0x7fffffff ? 0 : cc;
  }
}

// The producer epilogue's outputs for a residual row that no product made (the
// embedding, an MTP input): u = bf16(x * w) and the per-16-column sums of x^2,
// summed over the 16 lanes of a DPP row exactly as the epilogue does.
__global__ __launch_bounds__(256) void rms_parts_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                        uint16_t* __restrict__ u, float* __restrict__ parts, int D) {
  const int r = blockIdx.y;
  const int tiles = (D + PK_TILE - 1) / PK_TILE;
  const int tile = blockIdx.x * 16 + (threadIdx.x >> 4), i16 = threadIdx.x & 15;
  const int n = tile * PK_TILE + i16;
  const bool ok = tile < tiles && n < D;
  const float hv = ok ? bf16_to_f32(x[(size_t)r * D + n]) : 0.0f;
  const float sq = row16_allsum(hv * hv);
  if (ok) u[(size_t)r * D + n] = f32_to_bf16(hv * bf16_to_f32(w[n]));
  if (i16 == 0 && tile < tiles) parts[(size_t)r * tiles + tile] = sq;
}

typedef void (*qmv_packed_fn)(const uint16_t*, const uint8_t*, int, int, int, int, const float*, const uint16_t*,
                              const uint16_t*, uint16_t*, PkEpi);

template <int TN, int NP, int SW, int MH>
qmv_packed_fn pick_ws(int ws) {
  switch (ws) {
    case 1: return NP == 0 ? qmv_packed_kernel<TN, 1, 0, SW, MH> : nullptr;
    case 2: return qmv_packed_kernel<TN, 2, NP, SW, MH>;
    case 4: return qmv_packed_kernel<TN, 4, NP, SW, MH>;
    case 8: return qmv_packed_kernel<TN, 8, NP, SW, MH>;
    case 16: return TN == 1 ? qmv_packed_kernel<1, 16, NP, SW, MH> : nullptr;
  }
  return nullptr;
}

// 5..8 rows (MH = 2) for one or two tiles per wave (what the default tiles pick)
template <int NP, int SW, int MH>
qmv_packed_fn pick_tn(int tn, int ws) {
  switch (tn) {
    case 1: return pick_ws<1, NP, SW, MH>(ws);
    case 2: return NP <= 4 ? pick_ws<2, (NP <= 4 ? NP : 0), SW, MH>(ws) : nullptr;
    case 4: return NP <= 2 && MH == 1 ? pick_ws<4, (NP <= 2 ? NP : 0), SW, 1>(ws) : nullptr;
  }
  return nullptr;
}

template <int SW, int MH>
qmv_packed_fn pick_packed_np(int tn, int ws, int np) {
  switch (np) {
    case 0: return pick_tn<0, SW, MH>(tn, ws);
    case 2: return pick_tn<2, SW, MH>(tn, ws);
    case 4: return pick_tn<4, SW, MH>(tn, ws);
    case 6: return pick_tn<6, SW, MH>(tn, ws);
    case 8: return pick_tn<8, SW, MH>(tn, ws);
  }
  return nullptr;
}

template <int SW>
qmv_packed_fn pick_packed(int tn, int ws, int np, int mh) {
  return mh == 2 ? pick_packed_np<SW, 2>(tn, ws, np) : pick_packed_np<SW, 1>(tn, ws, np);
}

// Full prefetch when a wave's sets fit: the smallest NP in {2, 4, 6, 8} holding
// ceil(GS / WS) sets, with at most 4 records (TN * NP) of registers per wave
// (more costs occupancy: measured on gate_up (2,4), 13.3 us two-deep vs 13.8).
int packed_prefetch_depth(int K, int TN, int WS) {
  const int S = (K / PK_SET + WS - 1) / WS;
  if (WS < 2) return 0;
  for (int np = 2; np <= 8; np += 2)
    if (S <= np && TN * np <= 4) return np;
  return 0;
}

// Tile choice from (N, K) only, so a row's bits never depend on M. Two tiles per
// wave from ~700 tiles up; waves split K until the launch holds ~4096 waves
// (one tile per wave, up to 16 waves per tile) or ~3072 (two tiles), keeping at
// least 2 sets per wave; at most 8 waves per tile for K >= 12288 (the MLP down:
// 512-thread blocks, 9.3 against 9.5 us at (1,16), -9.7 us per decode cycle).
// Measured on the 9B shapes (M = 4 / 1, us): in_proj (2,8) 9.6 / 8.9, qkv (1,8)
// 8.4 / 7.5, o_proj (1,8) 5.2 / 4.8, gate_up (2,4) 13.3 / 12.9, mtp fc (1,16)
// 7.1 / 6.4, lm_head (2,4) 93.5 / 86.0. The fused gate/up + SwiGLU product takes
// the same tile: (2,4) two-deep 12.2 us against 13.2 for (1,4) with all four
// sets in flight, -24 us per decode cycle (3 of 3 alternations).
void packed_default_tile(int N, int K, int* TN, int* WS) {
  const long tiles = (N + PK_TILE - 1) / PK_TILE;
  const int GS = K / PK_SET;
  const int tn = tiles >= 704 ? 2 : 1;
  const long limit = tn == 1 ? 4096 : 3072;
  const int ws_max = tn == 1 ? 16 : 8;
  int ws = GS >= 8 ? 2 : 1;
  while (ws < ws_max && (tiles / tn) * ws < limit && GS >= 2 * (ws * 2)) ws *= 2;
  if (tiles / tn >= 4096 && GS >= 8 && ws < 4) ws = 4;   // lm_head-wide: 4 sets per wave (86 vs 89.5 us at M=1)
  if (GS >= 48 && ws > 8) ws = 8;                        // long K (the MLP down): 512-thread blocks
  *TN = tn;
  *WS = ws;
  // 704..1023 tiles (the DeltaNet in_proj, N = 12352): one tile per wave and 2
  // waves per tile, 8 sets each two-deep: -5 us per decode cycle against (2,8)
  // (5 of 5 alternations)
  if (tn == 2 && tiles < 1024 && GS >= 8) {
    *TN = 1;
    *WS = 2;
  }
}

int launch_packed(const uint16_t* x, const uint8_t* packed, uint16_t* y, int M, int N, int K, int TN, int WS,
                  bool swiglu, int prefetch_sets, const PkEpi& e, hipStream_t stream,
                  const char* fn_name_override = nullptr) {
  const char* fn_name =
      fn_name_override ? fn_name_override : swiglu ? "qvex_qmv_w4g64_packed_swiglu" : "qvex_qmv_w4g64_packed";
  QVEX_CHECK_ARG(x && packed && (y || e.resid || e.am_parts), "%s: null pointer", fn_name);
  QVEX_CHECK_ARG(M >= 1 && M <= 8, "%s: M=%d outside 1..8", fn_name, M);
  QVEX_CHECK_ARG(N >= 1 && K >= PK_SET && K % PK_SET == 0, "%s: N=%d K=%d (K must be a positive multiple of 256)",
                 fn_name, N, K);
  QVEX_CHECK_ARG(!swiglu || (N % 16 == 0), "%s: N=%d must be a multiple of 16 (gate and up halves of N/2 rows)",
                 fn_name, N);
  QVEX_CHECK_ARG(qvex_aligned(x, 16) && qvex_aligned(packed, 16) && qvex_aligned(y, 2),
                 "%s: x and packed must be 16-byte aligned", fn_name);
  const int NP = prefetch_sets < 0 ? packed_prefetch_depth(K, TN, WS) : prefetch_sets;
  QVEX_CHECK_ARG(NP == 0 || (WS >= 2 && (K / PK_SET + WS - 1) / WS <= NP),
                 "%s: prefetch_sets=%d must be 0 or hold all ceil(K/256 / WS) = %d sets of a wave", fn_name, NP,
                 (K / PK_SET + WS - 1) / WS);
  const int MH = M > 4 ? 2 : 1;           // 5..8 rows: two halves over one read of the weights
  QVEX_CHECK_ARG(!e.seg_ss || 4 * MH * (K / 128) <= pk_block(WS),
                 "%s: %d rows x %d heads of segment scales exceed the block's %d threads", fn_name, 4 * MH, K / 128,
                 pk_block(WS));
  qmv_packed_fn fn = swiglu   ? pick_packed<1>(TN, WS, NP, MH)
                     : e.seg_ss ? pick_packed<2>(TN, WS, NP, MH)
                                : pick_packed<0>(TN, WS, NP, MH);
  QVEX_CHECK_ARG(fn != nullptr, "%s: unsupported tile TN=%d WS=%d prefetch_sets=%d", fn_name, TN, WS, NP);
  const int threads = pk_block(WS);
  const int tiles = (N + PK_TILE - 1) / PK_TILE;
  const int tiles_per_block = TN * (threads / 64 / WS);
  const int blocks = (tiles + tiles_per_block - 1) / tiles_per_block;
  const bool segm = e.seg_ss != nullptr && !swiglu;
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(threads), 0, stream, x, packed, M, N, K, segm ? e.seg_nb : e.rs_nparts,
                     segm ? e.seg_ss : e.rs_parts, e.resid, e.norm_w, y, e);
  QVEX_CHECK_LAUNCH(fn_name);
  return QVEX_OK;
}

int pack(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N, int K, void* packed,
         uint64_t packed_bytes, int swiglu, hipStream_t stream) {
  const char* fn_name = swiglu ? "qvex_w4g64_pack_swiglu" : "qvex_w4g64_pack";
  QVEX_CHECK_ARG(w && scales && biases && packed, "%s: null pointer", fn_name);
  QVEX_CHECK_ARG(N >= 1 && K >= PK_SET && K % PK_SET == 0, "%s: N=%d K=%d (K must be a positive multiple of 256)",
                 fn_name, N, K);
  QVEX_CHECK_ARG(!swiglu || (N % 16 == 0), "%s: N=%d must be a multiple of 16", fn_name, N);
  const uint64_t need = (uint64_t)((N + PK_TILE - 1) / PK_TILE) * (uint64_t)(K / PK_SET) * PK_RECORD;
  QVEX_CHECK_ARG(packed_bytes >= need, "%s: packed buffer %llu < %llu bytes", fn_name,
                 (unsigned long long)packed_bytes, (unsigned long long)need);
  QVEX_CHECK_ARG(qvex_aligned(packed, 16) && qvex_aligned(w, 4) && qvex_aligned(scales, 2) && qvex_aligned(biases, 2),
                 "%s: packed must be 16-byte aligned", fn_name);
  const long records = (long)((N + PK_TILE - 1) / PK_TILE) * (K / PK_SET);
  QVEX_CHECK_ARG(records <= 0x7fffffffL, "%s: too many records", fn_name);
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)records), dim3(64), 0, stream, w, scales, biases, N, K, swiglu,
                     (uint8_t*)packed);
  QVEX_CHECK_LAUNCH(fn_name);
  return QVEX_OK;
}

}  // namespace

extern "C" uint64_t qvex_w4g64_packed_bytes(int N, int K) {
  if (N < 1 || K < PK_SET || K % PK_SET) return 0;
  return (uint64_t)((N + PK_TILE - 1) / PK_TILE) * (uint64_t)(K / PK_SET) * PK_RECORD;
}

extern "C" int qvex_w4g64_pack(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N, int K,
                               void* packed, uint64_t packed_bytes, void* stream) {
  return pack(w, scales, biases, N, K, packed, packed_bytes, 0, (hipStream_t)stream);
}

extern "C" int qvex_w4g64_pack_swiglu(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N,
                                      int K, void* packed, uint64_t packed_bytes, void* stream) {
  return pack(w, scales, biases, N, K, packed, packed_bytes, 1, (hipStream_t)stream);
}

extern "C" int qvex_qmv_w4g64_packed(const uint16_t* x, const void* packed, uint16_t* y, int M, int N, int K,
                                     void* stream) {
  int TN = 1, WS = 1;
  if (N >= 1 && K >= PK_SET) packed_default_tile(N, K, &TN, &WS);
  return launch_packed(x, (const uint8_t*)packed, y, M, N, K, TN, WS, false, -1, PkEpi{}, (hipStream_t)stream);
}

extern "C" int qvex_qmv_w4g64_packed_tiled(const uint16_t* x, const void* packed, uint16_t* y, int M, int N, int K,
                                           int tiles_per_wave, int wave_ksplit, int prefetch_sets, void* stream) {
  return launch_packed(x, (const uint8_t*)packed, y, M, N, K, tiles_per_wave, wave_ksplit, false, prefetch_sets,
                       PkEpi{}, (hipStream_t)stream);
}

extern "C" int qvex_qmv_w4g64_packed_swiglu(const uint16_t* x, const void* packed, uint16_t* y, int M, int N, int K,
                                            void* stream) {
  int TN = 1, WS = 1;
  if (N >= 1 && K >= PK_SET) packed_default_tile(N, K, &TN, &WS);
  return launch_packed(x, (const uint8_t*)packed, y, M, N, K, TN, WS, true, -1, PkEpi{}, (hipStream_t)stream);
}

extern "C" int qvex_qmv_w4g64_packed_resid(const uint16_t* x, const void* packed, int M, int N, int K,
                                           const uint16_t* resid, const uint16_t* norm_w, uint16_t* h_out,
                                           uint16_t* u_out, float* sq_parts, void* stream) {
  const char* fn = "qvex_qmv_w4g64_packed_resid";
  QVEX_CHECK_ARG(resid && norm_w && h_out && u_out && sq_parts, "%s: null pointer", fn);
  int TN = 1, WS = 1;
  if (N >= 1 && K >= PK_SET) packed_default_tile(N, K, &TN, &WS);
  PkEpi e{};
  e.resid = resid;
  e.norm_w = norm_w;
  e.h_out = h_out;
  e.u_out = u_out;
  e.sq_parts = sq_parts;
  return launch_packed(x, (const uint8_t*)packed, nullptr, M, N, K, TN, WS, false, -1, e, (hipStream_t)stream, fn);
}

extern "C" int qvex_qmv_w4g64_packed_gnorm_resid(const uint16_t* u, const void* packed, int M, int N, int K,
                                                 const float* seg_ss, int seg_nb, float seg_eps,
                                                 const uint16_t* resid, const uint16_t* norm_w, uint16_t* h_out,
                                                 uint16_t* u_out, float* sq_parts, void* stream) {
  const char* fn = "qvex_qmv_w4g64_packed_gnorm_resid";
  QVEX_CHECK_ARG(seg_ss && resid && norm_w && h_out && u_out && sq_parts, "%s: null pointer", fn);
  QVEX_CHECK_ARG(seg_nb == 1 || seg_nb == 2 || seg_nb == 4 || seg_nb == 8, "%s: seg_nb=%d must be 1, 2, 4 or 8", fn,
                 seg_nb);
  QVEX_CHECK_ARG(qvex_aligned(seg_ss, 4), "%s: seg_ss must be 4-byte aligned", fn);
  QVEX_CHECK_ARG(K <= 64 * 128, "%s: K=%d must be at most 8192 (64 heads of 128)", fn, K);
  int TN = 1, WS = 1;
  if (N >= 1 && K >= PK_SET) packed_default_tile(N, K, &TN, &WS);
  PkEpi e{};
  e.seg_ss = seg_ss;
  e.seg_nb = seg_nb;
  e.seg_eps = seg_eps;
  e.resid = resid;
  e.norm_w = norm_w;
  e.h_out = h_out;
  e.u_out = u_out;
  e.sq_parts = sq_parts;
  return launch_packed(u, (const uint8_t*)packed, nullptr, M, N, K, TN, WS, false, -1, e, (hipStream_t)stream, fn);
}

extern "C" int qvex_qmv_w4g64_packed_rstd(const uint16_t* u, const void* packed, uint16_t* y, int M, int N, int K,
                                          const float* sq_parts, int nparts, int dim, float eps, int swiglu,
                                          void* stream) {
  const char* fn = "qvex_qmv_w4g64_packed_rstd";
  QVEX_CHECK_ARG(sq_parts && y, "%s: null pointer", fn);
  QVEX_CHECK_ARG(nparts >= 1 && nparts <= 256 && nparts % 4 == 0 && dim >= 1 && nparts == (dim + PK_TILE - 1) / PK_TILE,
                 "%s: nparts=%d must be ceil(dim/16) for dim=%d, a multiple of 4 and <= 256", fn, nparts, dim);
  QVEX_CHECK_ARG(qvex_aligned(sq_parts, 16), "%s: sq_parts must be 16-byte aligned", fn);
  int TN = 1, WS = 1;
  if (N >= 1 && K >= PK_SET) packed_default_tile(N, K, &TN, &WS);
  PkEpi e{};
  e.rs_parts = sq_parts;
  e.rs_nparts = nparts;
  e.rs_dim = dim;
  e.rs_eps = eps;
  return launch_packed(u, (const uint8_t*)packed, y, M, N, K, TN, WS, swiglu != 0, -1, e, (hipStream_t)stream, fn);
}

extern "C" int qvex_rms_parts(const uint16_t* x, const uint16_t* norm_w, uint16_t* u_out, float* sq_parts, int M,
                              int D, void* stream) {
  QVEX_CHECK_ARG(x && norm_w && u_out && sq_parts, "qvex_rms_parts: null pointer");
  QVEX_CHECK_ARG(M >= 1 && D >= 1, "qvex_rms_parts: M=%d D=%d", M, D);
  const int tiles = (D + PK_TILE - 1) / PK_TILE;
  hipLaunchKernelGGL(rms_parts_kernel, dim3((tiles + 15) / 16, M), dim3(256), 0, (hipStream_t)stream, x, norm_w,
                     u_out, sq_parts, D);
  QVEX_CHECK_LAUNCH("qvex_rms_parts");
  return QVEX_OK;
}

extern "C" int qvex_qmv_w4g64_packed_rstd_tilemax(const uint16_t* u, const void* packed, uint16_t* y, int M, int N,
                                                  int K, const float* sq_parts, int nparts, int dim, float eps,
                                                  uint16_t* tile_max, void* stream) {
  const char* fn = "qvex_qmv_w4g64_packed_rstd_tilemax";
  QVEX_CHECK_ARG(sq_parts && y && tile_max, "%s: null pointer", fn);
  QVEX_CHECK_ARG(nparts >= 1 && nparts <= 256 && nparts % 4 == 0 && dim >= 1 && nparts == (dim + PK_TILE - 1) / PK_TILE,
                 "%s: nparts=%d must be ceil(dim/16) for dim=%d, a multiple of 4 and <= 256", fn, nparts, dim);
  QVEX_CHECK_ARG(qvex_aligned(sq_parts, 16) && qvex_aligned(tile_max, 16),
                 "%s: sq_parts and tile_max must be 16-byte aligned", fn);
  int TN = 1, WS = 1;
  if (N >= 1 && K >= PK_SET) packed_default_tile(N, K, &TN, &WS);
  PkEpi e{};
  e.rs_parts = sq_parts;
  e.rs_nparts = nparts;
  e.rs_dim = dim;
  e.rs_eps = eps;
  e.tm_out = tile_max;
  return launch_packed(u, (const uint8_t*)packed, y, M, N, K, TN, WS, false, -1, e, (hipStream_t)stream, fn);
}

extern "C" uint64_t qvex_qmv_w4g64_argmax_workspace_bytes(int M, int N) {
  if (M < 1 || N < 1) return 0;
  return (uint64_t)M * ((N + PK_TILE - 1) / PK_TILE) * 2 * sizeof(float);
}

extern "C" int qvex_qmv_w4g64_packed_argmax(const uint16_t* x, const void* packed, int M, int N, int K,
                                            const float* sq_parts, int nparts, int dim, float eps, int32_t* out_token,
                                            void* workspace, uint64_t workspace_bytes, void* stream) {
  const char* fn = "qvex_qmv_w4g64_packed_argmax";
  QVEX_CHECK_ARG(workspace, "%s: null pointer", fn);
  QVEX_CHECK_ARG(workspace_bytes >= qvex_qmv_w4g64_argmax_workspace_bytes(M, N),
                 "%s: workspace %llu bytes < %llu", fn, (unsigned long long)workspace_bytes,
                 (unsigned long long)qvex_qmv_w4g64_argmax_workspace_bytes(M, N));
  if (sq_parts) {
    QVEX_CHECK_ARG(nparts >= 1 && nparts <= 256 && nparts % 4 == 0 && nparts == (dim + PK_TILE - 1) / PK_TILE,
                   "%s: nparts=%d must be ceil(dim/16) for dim=%d, a multiple of 4 and <= 256", fn, nparts, dim);
    QVEX_CHECK_ARG(qvex_aligned(sq_parts, 16), "%s: sq_parts must be 16-byte aligned", fn);
  }
  int TN = 1, WS = 1;
  if (N >= 1 && K >= PK_SET) packed_default_tile(N, K, &TN, &WS);
  PkEpi e{};
  e.rs_parts = sq_parts;
  e.rs_nparts = nparts;
  e.rs_dim = dim;
  e.rs_eps = eps;
  e.am_parts = (float*)workspace;
  // the product itself is launch_packed's; y is not written
  e.resid = nullptr;
  if (int rc = launch_packed(x, (const uint8_t*)packed, nullptr, M, N, K, TN, WS, false, -1, e,
                             (hipStream_t)stream, fn))
    return rc;
  if (!out_token) return QVEX_OK;   // the caller reduces the per-tile pairs (qvex_mtp_input, qvex_embed_rms_parts)
  hipLaunchKernelGGL(argmax_parts_kernel, dim3(M), dim3(AM_T), 0, (hipStream_t)stream, (const float*)workspace,
                     (N + PK_TILE - 1) / PK_TILE, out_token);
  QVEX_CHECK_LAUNCH(fn);
  return QVEX_OK;
}
