// MLX affine quantization of any supported width: bits 2, 3, 4, 5, 6, 8 and
// groups of 32, 64 or 128 codes (the per-module overrides of Config.qparams,
// engine/model.py:68-71, fed to mx.quantized_matmul / mx.dequantize at
// engine/model.py:87-91, 127-130).
//
// Layout (quant/quantize.py:71-75): each weight row is one little-endian bit
// stream, code k at stream bits [k*bits, (k+1)*bits), read as uint32 words; a
// row of K codes is K*bits/32 words. Per (row, group): a bf16 scale s and bias
// b, w = s*q + b.
//
// Three kernels:
//   * qmv_affine_kernel: y = x W^T for 1..8 activation rows, VALU only. A chunk
//     is 32 consecutive codes of one row = `bits` words (K % 32 == 0 and the
//     group is a multiple of 32, so a chunk lies in one group). Each lane
//     extracts its chunk's 32 codes once per weight row (compile-time bit
//     offsets: one v_bfe per code, an alignbit first where a code straddles two
//     words), then accumulates d = sum q*x and X = sum x per activation row in
//     fp32 and folds acc += s*d + b*X. R weight rows per wave share the
//     activation chunk; lanes stride over the chunks; one wave sum per output.
//   * embed_affine_kernel: the rows of an embedding table, bf16(s*q + b).
//   * widen_w4_kernel: lossless re-encoding of a width <= 4, group % 64 == 0
//     weight as 4-bit group-64 (codes widened to nibbles, a group-128 scale and
//     bias repeated for both 64-code halves), so such layers run the packed
//     MFMA products and every fused epilogue of the 4-bit path unchanged.
#include "qvex_common.h"

namespace {

// Code j (0..31) of a chunk held as BITS words: compile-time offsets after unrolling.
template <int BITS>
__device__ __forceinline__ uint32_t chunk_code(const uint32_t (&wv)[BITS], int j) {
  const int o = j * BITS;
  const int wi = o >> 5, sh = o & 31;
  const uint32_t mask = (1u << BITS) - 1u;
  if (sh + BITS <= 32) return (wv[wi] >> sh) & mask;
  return __builtin_amdgcn_alignbit(wv[wi + 1], wv[wi], sh) & mask;
}

// The BITS words of one chunk: the widest vector load the chunk's alignment
// allows (a chunk starts at a multiple of 4*BITS bytes of a 16-byte aligned row
// stream): x4 for 4 and 8 bits, x2 for 2 and 6, single words for 3 and 5.
template <int BITS>
__device__ __forceinline__ void load_chunk(const uint32_t* __restrict__ p, uint32_t (&wv)[BITS]) {
  if constexpr (BITS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < BITS / 4; ++i) {
      const u32x4 v = load_nt16(p + 4 * i);
      wv[4 * i] = v.x; wv[4 * i + 1] = v.y; wv[4 * i + 2] = v.z; wv[4 * i + 3] = v.w;
    }
  } else if constexpr (BITS % 2 == 0) {
#pragma unroll
    for (int i = 0; i < BITS / 2; ++i) {
      const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p + 2 * i));
      wv[2 * i] = v.x; wv[2 * i + 1] = v.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) wv[i] = __builtin_nontemporal_load(p + i);
  }
}

constexpr int AFF_MAXM = 8;    // activation rows per launch

// AFF_R weight rows per wave share each activation chunk: 1 for one or two
// activation rows (81 VGPRs, more waves in flight: 12.6 against 13.6 us for a
// 5-bit 12,288 x 4,096 product at one row), 2 above (the dequantized codes serve
// twice as many products: 25 against 28.5 us at four rows).
template <int BITS, int AFF_R>
__global__ __launch_bounds__(256) void qmv_affine_kernel(const uint16_t* __restrict__ x,
                                                         const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         uint16_t* __restrict__ y, int M, int N, int K,
                                                         int gshift) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * AFF_R;
  const int nchunk = K >> 5;
  const int KW = nchunk * BITS;        // words per row
  const int G = K >> gshift;           // groups per row

  float acc[AFF_R][AFF_MAXM];
#pragma unroll
  for (int r = 0; r < AFF_R; ++r)
#pragma unroll
    for (int m = 0; m < AFF_MAXM; ++m) acc[r][m] = 0.0f;

  for (int c = lane; c < nchunk; c += 64) {
    // rows past N re-read row N-1 (never stored)
    float q[AFF_R][32];
    float s[AFF_R], b[AFF_R];
#pragma unroll
    for (int r = 0; r < AFF_R; ++r) {
      const int row = min(row0 + r, N - 1);
      uint32_t wv[BITS];
      load_chunk<BITS>(w + (size_t)row * KW + (size_t)c * BITS, wv);
      const int g = (c << 5) >> gshift;
      s[r] = bf16_to_f32(scales[(size_t)row * G + g]);
      b[r] = bf16_to_f32(biases[(size_t)row * G + g]);
#pragma unroll
      for (int j = 0; j < 32; ++j) q[r][j] = (float)chunk_code<BITS>(wv, j);
    }
#pragma unroll
    for (int m = 0; m < AFF_MAXM; ++m) {
      if (m >= M) break;
      const uint16_t* xr = x + (size_t)m * K + (size_t)c * 32;
      float xs = 0.0f;
      float d[AFF_R];
#pragma unroll
      for (int r = 0; r < AFF_R; ++r) d[r] = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 v = load16(xr + 8 * i);
        const uint32_t pr[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float x0 = bf16_lo(pr[h]), x1 = bf16_hi(pr[h]);
          xs += x0;
          xs += x1;
#pragma unroll
          for (int r = 0; r < AFF_R; ++r) {
            d[r] = fmaf(q[r][8 * i + 2 * h], x0, d[r]);
            d[r] = fmaf(q[r][8 * i + 2 * h + 1], x1, d[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < AFF_R; ++r) acc[r][m] = fmaf(s[r], d[r], fmaf(b[r], xs, acc[r][m]));
    }
  }

#pragma unroll
  for (int r = 0; r < AFF_R; ++r)
#pragma unroll
    for (int m = 0; m < AFF_MAXM; ++m)
      if (m < M) acc[r][m] = wave_sum_to_lane63(acc[r][m]);
  if (lane == 63) {
#pragma unroll
    for (int r = 0; r < AFF_R; ++r) {
      const int row = row0 + r;
      if (row >= N) continue;
#pragma unroll
      for (int m = 0; m < AFF_MAXM; ++m)
        if (m < M) y[(size_t)m * N + row] = f32_to_bf16(acc[r][m]);
    }
  }
}

// One block per gathered row; a thread per 32-code chunk writes 64 bytes.
template <int BITS>
__global__ __launch_bounds__(256) void embed_affine_kernel(const int32_t* __restrict__ ids,
                                                           const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ sc,
                                                           const uint16_t* __restrict__ bi,
                                                           uint16_t* __restrict__ out, int V, int H, int gshift) {
  const int l = blockIdx.x;
  int id = ids[l];
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);          // clamped like the 4-bit gather
  const int nchunk = H >> 5, G = H >> gshift;
  const uint32_t* wr = w + (size_t)id * nchunk * BITS;
  for (int c = threadIdx.x; c < nchunk; c += blockDim.x) {
    uint32_t wv[BITS];
    load_chunk<BITS>(wr + (size_t)c * BITS, wv);
    const int g = (c << 5) >> gshift;
    const float s = bf16_to_f32(sc[(size_t)id * G + g]);
    const float b = bf16_to_f32(bi[(size_t)id * G + g]);
    uint16_t* o = out + (size_t)l * H + (size_t)c * 32;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t pk[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int j = 8 * i + 2 * h;
        pk[h] = pack_bf16x2(fmaf(s, (float)chunk_code<BITS>(wv, j), b),
                            fmaf(s, (float)chunk_code<BITS>(wv, j + 1), b));
      }
      u32x4 v;
      v.x = pk[0]; v.y = pk[1]; v.z = pk[2]; v.w = pk[3];
      *reinterpret_cast<u32x4*>(o + 8 * i) = v;
    }
  }
}

// One thread per 32-code chunk: four nibble words out; the first chunk of each
// 64-code group also writes that group's scale and bias.
template <int BITS>
__global__ __launch_bounds__(256) void widen_w4_kernel(const uint32_t* __restrict__ w,
                                                       const uint16_t* __restrict__ sc,
                                                       const uint16_t* __restrict__ bi, uint32_t* __restrict__ w4,
                                                       uint16_t* __restrict__ sc4, uint16_t* __restrict__ bi4,
                                                       long chunks, int K, int gshift) {
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= chunks) return;
  const int nchunk = K >> 5;
  const long n = t / nchunk;
  const int c = (int)(t - n * nchunk);
  uint32_t wv[BITS];
  load_chunk<BITS>(w + (size_t)t * BITS, wv);
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t v = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) v |= chunk_code<BITS>(wv, 8 * i + j) << (4 * j);
    o[i] = v;
  }
  u32x4 v;
  v.x = o[0]; v.y = o[1]; v.z = o[2]; v.w = o[3];
  *reinterpret_cast<u32x4*>(w4 + (size_t)t * 4) = v;
  if ((c & 1) == 0) {
    const int g = (c << 5) >> gshift;
    sc4[n * (K >> 6) + (c >> 1)] = sc[n * (K >> gshift) + g];
    bi4[n * (K >> 6) + (c >> 1)] = bi[n * (K >> gshift) + g];
  }
}

int group_shift(int group_size) {
  switch (group_size) {
    case 32: return 5;
    case 64: return 6;
    case 128: return 7;
  }
  return -1;
}

bool width_ok(int bits) { return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8; }

#define AFFINE_BITS_SWITCH(bits, KERNEL, ...)          \
  switch (bits) {                                      \
    case 2: KERNEL<2>(__VA_ARGS__); break;             \
    case 3: KERNEL<3>(__VA_ARGS__); break;             \
    case 4: KERNEL<4>(__VA_ARGS__); break;             \
    case 5: KERNEL<5>(__VA_ARGS__); break;             \
    case 6: KERNEL<6>(__VA_ARGS__); break;             \
    case 8: KERNEL<8>(__VA_ARGS__); break;             \
  }

template <int BITS>
void launch_qmv(hipStream_t st, const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                uint16_t* y, int M, int N, int K, int gs) {
  if (M <= 2)
    hipLaunchKernelGGL((qmv_affine_kernel<BITS, 1>), dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, x, w, s, b, y,
                       M, N, K, gs);
  else
    hipLaunchKernelGGL((qmv_affine_kernel<BITS, 2>), dim3((unsigned)((N + 7) / 8)), dim3(256), 0, st, x, w, s, b, y,
                       M, N, K, gs);
}

template <int BITS>
void launch_embed(dim3 grid, hipStream_t st, const int32_t* ids, const uint32_t* w, const uint16_t* s,
                  const uint16_t* b, uint16_t* out, int V, int H, int gs) {
  hipLaunchKernelGGL(embed_affine_kernel<BITS>, grid, dim3(256), 0, st, ids, w, s, b, out, V, H, gs);
}

template <int BITS>
void launch_widen(dim3 grid, hipStream_t st, const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t* w4,
                  uint16_t* s4, uint16_t* b4, long chunks, int K, int gs) {
  hipLaunchKernelGGL(widen_w4_kernel<BITS>, grid, dim3(256), 0, st, w, s, b, w4, s4, b4, chunks, K, gs);
}

}  // namespace

extern "C" int qvex_qmv_affine(const uint16_t* x, const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                               uint16_t* y, int M, int N, int K, int bits, int group_size, void* stream) {
  QVEX_CHECK_ARG(x && w && scales && biases && y, "qvex_qmv_affine: null pointer");
  const int gs = group_shift(group_size);
  QVEX_CHECK_ARG(width_ok(bits) && gs > 0, "qvex_qmv_affine: bits=%d group_size=%d (bits 2,3,4,5,6,8; groups 32,64,128)",
                 bits, group_size);
  QVEX_CHECK_ARG(M >= 1 && M <= AFF_MAXM && N >= 1 && K >= group_size && K % group_size == 0,
                 "qvex_qmv_affine: M=%d N=%d K=%d (1 <= M <= 8, K a positive multiple of the group size %d)", M, N,
                 K, group_size);
  QVEX_CHECK_ARG(qvex_aligned(x, 16) && qvex_aligned(w, 16), "qvex_qmv_affine: x and w must be 16-byte aligned");
  AFFINE_BITS_SWITCH(bits, launch_qmv, (hipStream_t)stream, x, w, scales, biases, y, M, N, K, gs);
  QVEX_CHECK_LAUNCH("qvex_qmv_affine");
  return QVEX_OK;
}

extern "C" int qvex_embed_affine(const int32_t* ids, int L, const uint32_t* w, const uint16_t* scales,
                                 const uint16_t* biases, int V, int H, int bits, int group_size, uint16_t* out,
                                 void* stream) {
  QVEX_CHECK_ARG(ids && w && scales && biases && out, "qvex_embed_affine: null pointer");
  const int gs = group_shift(group_size);
  QVEX_CHECK_ARG(width_ok(bits) && gs > 0,
                 "qvex_embed_affine: bits=%d group_size=%d (bits 2,3,4,5,6,8; groups 32,64,128)", bits, group_size);
  QVEX_CHECK_ARG(L >= 1 && V >= 1 && H >= group_size && H % group_size == 0,
                 "qvex_embed_affine: L=%d V=%d H=%d (H a positive multiple of the group size)", L, V, H);
  QVEX_CHECK_ARG(qvex_aligned(out, 16) && qvex_aligned(w, 16), "qvex_embed_affine: w and out must be 16-byte aligned");
  AFFINE_BITS_SWITCH(bits, launch_embed, dim3(L), (hipStream_t)stream, ids, w, scales, biases, out, V, H, gs);
  QVEX_CHECK_LAUNCH("qvex_embed_affine");
  return QVEX_OK;
}

extern "C" int qvex_affine_widen_w4g64(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N,
                                       int K, int bits, int group_size, uint32_t* w4, uint16_t* scales4,
                                       uint16_t* biases4, void* stream) {
  QVEX_CHECK_ARG(w && scales && biases && w4 && scales4 && biases4, "qvex_affine_widen_w4g64: null pointer");
  const int gs = group_shift(group_size);
  QVEX_CHECK_ARG((bits == 2 || bits == 3 || bits == 4) && (group_size == 64 || group_size == 128),
                 "qvex_affine_widen_w4g64: bits=%d group_size=%d (bits 2..4, groups 64 or 128 widen losslessly)",
                 bits, group_size);
  QVEX_CHECK_ARG(N >= 1 && K >= group_size && K % group_size == 0,
                 "qvex_affine_widen_w4g64: N=%d K=%d (K a positive multiple of the group size)", N, K);
  QVEX_CHECK_ARG(qvex_aligned(w, 16) && qvex_aligned(w4, 16), "qvex_affine_widen_w4g64: w and w4 must be 16-byte aligned");
  const long chunks = (long)N * (K / 32);
  QVEX_CHECK_ARG(chunks / 256 < 0x7fffffffL, "qvex_affine_widen_w4g64: too large");
  const dim3 grid((unsigned)((chunks + 255) / 256));
  if (bits == 2) launch_widen<2>(grid, (hipStream_t)stream, w, scales, biases, w4, scales4, biases4, chunks, K, gs);
  if (bits == 3) launch_widen<3>(grid, (hipStream_t)stream, w, scales, biases, w4, scales4, biases4, chunks, K, gs);
  if (bits == 4) launch_widen<4>(grid, (hipStream_t)stream, w, scales, biases, w4, scales4, biases4, chunks, K, gs);
  QVEX_CHECK_LAUNCH("qvex_affine_widen_w4g64");
  return QVEX_OK;
}
