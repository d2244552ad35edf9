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

namespace {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

constexpr uint32_t kMagic = 0x43004300u;   // bf16 pair (128.0, 128.0)
constexpr uint32_t kNib = 0x000F000Fu;
constexpr uint32_t kOnes = 0x3f803f80u;    // bf16 pair (1.0, 1.0)

// (a & mask) | magic as one VOP3 op. gfx9 VOP3 takes no literal operand, so the
// compiler would otherwise split it into two VOP2 ops with literals; the mask
// rides in an SGPR and the magic in a VGPR (one constant-bus read).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(magic));
  return r;
}

// Chunk = 32 consecutive k of one row = 4 uint32 words = 16 bytes.
// Block = 256 threads = 4 waves; KS waves share one row group of R rows and
// split the chunk sequence between them; 4/KS row groups per block.
template <int M, int R, int KS>
__global__ __launch_bounds__(256) void qmv_w4g64_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ w,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ biases,
    uint16_t* __restrict__ y, int N, int K) {
  constexpr int RG = 4 / KS;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rg = wave / KS;
  const int ws = wave % KS;
  const int row0 = (blockIdx.x * RG + rg) * R;

  const int nchunk = K >> 5;
  const int KW = K >> 3;   // words per row
  uint32_t magic = kMagic;
  asm volatile("" : "+v"(magic));   // keep the magic constant in a VGPR
  const int G = K >> 6;    // groups per row

  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

  for (int cbase = ws * 64; cbase < nchunk; cbase += 64 * KS) {
    const int c = cbase + lane;
    if (c < nchunk) {
      // weights first: they are the long-latency stream
      u32x4 wv[R];
      uint32_t sb[R][2];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row < N) {
          wv[r] = load_nt16(w + (size_t)row * KW + (size_t)c * 4);
          sb[r][0] = scales[(size_t)row * G + (c >> 1)];
          sb[r][1] = biases[(size_t)row * G + (c >> 1)];
        } else {
          wv[r] = u32x4{0, 0, 0, 0};
          sb[r][0] = sb[r][1] = 0;
        }
      }
      // x chunk of every activation row, permuted into (x_j, x_{j+4}) pairs
      uint32_t xp[M][16];
      float xs[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (size_t)m * K + (size_t)c * 32;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = load16(xr + 8 * i);
          xp[m][4 * i + 0] = (v.x & 0xffffu) | (v.z << 16);
          xp[m][4 * i + 1] = (v.x >> 16) | (v.z & 0xffff0000u);
          xp[m][4 * i + 2] = (v.y & 0xffffu) | (v.w << 16);
          xp[m][4 * i + 3] = (v.y >> 16) | (v.w & 0xffff0000u);
          s = dot2(v.x, kOnes, s);
          s = dot2(v.y, kOnes, s);
          s = dot2(v.z, kOnes, s);
          s = dot2(v.w, kOnes, s);
        }
        xs[m] = s;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t ws4[4] = {wv[r].x, wv[r].y, wv[r].z, wv[r].w};
        float d[M];
#pragma unroll
        for (int m = 0; m < M; ++m) d[m] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t wd = ws4[i];
          const uint32_t p0 = and_or(wd, kNib, magic);
          const uint32_t p1 = and_or(wd >> 4, kNib, magic);
          const uint32_t p2 = and_or(wd >> 8, kNib, magic);
          const uint32_t p3 = and_or(wd >> 12, kNib, magic);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            d[m] = dot2(p0, xp[m][4 * i + 0], d[m]);
            d[m] = dot2(p1, xp[m][4 * i + 1], d[m]);
            d[m] = dot2(p2, xp[m][4 * i + 2], d[m]);
            d[m] = dot2(p3, xp[m][4 * i + 3], d[m]);
          }
        }
        const float sc = bf16_to_f32((uint16_t)sb[r][0]);
        const float bi = bf16_to_f32((uint16_t)sb[r][1]);
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

// Default tile: rows per wave shrink as M grows (x pairs cost 16*M VGPRs);
// K is split across waves when the row groups alone cannot fill 256 CUs.
void default_tile(int M, int N, int K, int* R, int* KS) {
  int r = M <= 2 ? 4 : (M <= 4 ? 4 : 2);
  const int nchunk = K / 32;
  int ks = 1;
  const long target_waves = 4096;  // 16 waves per CU on 256 CUs
  while (ks < 4 && (long)((N + r - 1) / r) * ks < target_waves && nchunk >= 64 * ks * 2) ks *= 2;
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

}  // namespace

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

extern "C" int qvex_read_roof(const void* buf, uint64_t bytes, uint32_t* sink, int blocks, void* stream) {
  QVEX_CHECK_ARG(buf && sink, "qvex_read_roof: null pointer");
  QVEX_CHECK_ARG(bytes % 16 == 0 && qvex_aligned(buf, 16), "qvex_read_roof: bytes and buf must be 16-byte multiples");
  QVEX_CHECK_ARG(blocks >= 1 && blocks <= (1 << 20), "qvex_read_roof: blocks=%d", blocks);
  hipLaunchKernelGGL(read_roof_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const u32x4*>(buf), (uint64_t)(bytes / 16), sink);
  QVEX_CHECK_LAUNCH("qvex_read_roof");
  return QVEX_OK;
}
