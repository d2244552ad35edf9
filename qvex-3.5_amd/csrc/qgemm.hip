// Prefill products: y[M, N] = x[M, K] @ W^T for prompt chunks (M >= 16 rows),
// read straight from the tile-packed 4-bit copy of the weight.
//
// Reference semantics: mx.quantized_matmul(transpose=True, group_size=64,
// bits=4) in QLinear.__call__ (engine/model.py:87-91) on a prefill chunk
// (engine/engine.py:232-248). Each weight is dequantized in registers to
// bf16(s * q + b) (the value an fp32 fma gives, rounded once to bf16) and the
// products accumulate in fp32 on the matrix cores, so the result equals a bf16
// GEMM on the dequantized weight up to the summation order.
//
// Layout. The packed record (tile t of 16 rows, set s of 256 k; see
// qmv_packed.hip) gives lane L = 16c + i the 64 codes of row 16t + i, group
// 4s + c, plus that group's (scale, bias). For v_mfma_f32_16x16x32_bf16 the B
// operand of lane (c, i) is 8 consecutive k of column i from k-chunk c: taking
// chunk c of step j (0..7) as k = (4s + c) * 64 + 8j .. + 7 makes every lane's
// B operand a slice of its own record words, and the A operand of lane (c, m)
// the same 8 k of activation row m. The 32 k of one MFMA therefore span four
// quantization groups, which is harmless here: the weights are already scaled.
//
// Blocking. A 256-thread block owns 64 rows x 128 outputs: wave w computes
// tiles 8 bn + 2w, 8 bn + 2w + 1 for all 64 rows (4 x 2 MFMA tiles). The 64 x 256
// activation slice of a set sits in LDS (rows padded to 528 bytes so that the
// 16 lanes of a k-chunk group read 16 different bank groups), double-buffered:
// the next set's activations and records are requested before the current set
// is computed.
#include "qvex_common.h"
#include "w4_dequant.h"

namespace {

constexpr int QG_TILE = 16;
constexpr int QG_SET = 256;                 // k per record
constexpr int QG_RECORD = 2304;             // bytes per (tile, set) record
constexpr int QG_WBYTES = 2048;
constexpr int QG_BM = 64;                   // rows per block
constexpr int QG_TPW = 2;                   // 16-row weight tiles per wave
constexpr int QG_BN = 4 * QG_TPW * QG_TILE; // outputs per block
constexpr int QG_LDS_ROW = QG_SET + 8;      // bf16 per LDS row (528 bytes)
constexpr int QG_XLOADS = QG_BM * QG_SET / 8 / 256;   // 16-byte activation loads per thread per set

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// bf16(s * v + bo) for the bf16 pair v = (128 + q0, 128 + q1), bo = b - 128 s
__device__ __forceinline__ uint32_t dq_pair(uint32_t v, float s, float bo) {
  const float lo = fmaf(s, bf16_lo(v), bo), hi = fmaf(s, bf16_hi(v), bo);
  const bf16x2v r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}

template <bool SWIGLU>
__global__ __launch_bounds__(256) void packed_gemm_kernel(const uint16_t* __restrict__ x,
                                                          const uint8_t* __restrict__ packed,
                                                          uint16_t* __restrict__ y, int M, int N, int K) {
  __shared__ __align__(16) uint16_t xs[2][QG_BM][QG_LDS_ROW];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int c = lane >> 4, i16 = lane & 15;
  const int tiles = (N + QG_TILE - 1) / QG_TILE;
  const int GS = K / QG_SET;
  const int m0 = blockIdx.y * QG_BM;
  const int tile0 = blockIdx.x * (QG_BN / QG_TILE) + wave * QG_TPW;

  const uint32_t magic = opaque_vgpr(kMagic);
  const uint32_t nib = opaque_sgpr(kNib);

  // activation slice loader: thread t, load j covers row (t + 256 j) / 32, chunk (t + 256 j) % 32
  u32x4 xr[QG_XLOADS];
  auto load_x = [&](int s) {
#pragma unroll
    for (int j = 0; j < QG_XLOADS; ++j) {
      const int q = t + 256 * j, row = q >> 5, ch = q & 31;
      const int m = m0 + row;
      xr[j] = m < M ? load16(x + (size_t)m * K + (size_t)s * QG_SET + 8 * ch) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int j = 0; j < QG_XLOADS; ++j) {
      const int q = t + 256 * j, row = q >> 5, ch = q & 31;
      *reinterpret_cast<u32x4*>(&xs[buf][row][8 * ch]) = xr[j];
    }
  };
  u32x4 wb[2][QG_TPW][2];
  uint32_t sb[2][QG_TPW];
  auto load_w = [&](int buf, int s) {
#pragma unroll
    for (int p = 0; p < QG_TPW; ++p) {
      const int tile = min(tile0 + p, tiles - 1);     // tiles past the end re-read the last one, never stored
      const uint8_t* rec = packed + ((size_t)tile * GS + s) * QG_RECORD;
      wb[buf][p][0] = load_nt16(rec + lane * 16);
      wb[buf][p][1] = load_nt16(rec + 1024 + lane * 16);
      sb[buf][p] = *reinterpret_cast<const uint32_t*>(rec + QG_WBYTES + lane * 4);
    }
  };

  f32x4_t acc[4][QG_TPW];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int p = 0; p < QG_TPW; ++p) acc[mt][p] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int xb, int wbuf) {
    float sc[QG_TPW], bo[QG_TPW];
#pragma unroll
    for (int p = 0; p < QG_TPW; ++p) {
      sc[p] = bf16_to_f32((uint16_t)(sb[wbuf][p] & 0xffffu));
      bo[p] = fmaf(-128.0f, sc[p], bf16_to_f32((uint16_t)(sb[wbuf][p] >> 16)));
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bf16x8_t b[QG_TPW];
#pragma unroll
      for (int p = 0; p < QG_TPW; ++p) {
        const uint32_t w = j < 4 ? wb[wbuf][p][0][j] : wb[wbuf][p][1][j - 4];
        b[p] = as_bf16x8(dq_pair(and_or(w, nib, magic), sc[p], bo[p]),
                         dq_pair(and_or(w >> 4, nib, magic), sc[p], bo[p]),
                         dq_pair(and_or(w >> 8, nib, magic), sc[p], bo[p]),
                         dq_pair(and_or(w >> 12, nib, magic), sc[p], bo[p]));
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const bf16x8_t a =
            __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4*>(&xs[xb][mt * 16 + i16][c * 64 + 8 * j]));
#pragma unroll
        for (int p = 0; p < QG_TPW; ++p) acc[mt][p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[p], acc[mt][p], 0, 0, 0);
      }
    }
  };

  load_x(0);
  load_w(0, 0);
  store_x(0);
  __syncthreads();
  for (int s = 0; s < GS; ++s) {
    const int cur = s & 1;
    if (s + 1 < GS) {
      load_x(s + 1);
      load_w(cur ^ 1, s + 1);
    }
    compute(cur, cur);
    if (s + 1 < GS) store_x(cur ^ 1);
    __syncthreads();
  }

  // lane (c, i16) of tile p holds rows 4c + r of each 16-row slab, column i16
#pragma unroll
  for (int p = 0; p < QG_TPW; ++p) {
    const int tile = tile0 + p;
    if (tile >= tiles) continue;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + mt * 16 + 4 * c + r;
        const float v = acc[mt][p][r];
        if constexpr (SWIGLU) {
          // interleaved tile: columns 0-7 gate rows 8 tile + i, 8-15 the matching up rows
          const float u = __shfl_xor(v, 8, 64);
          const int half = N / 2, jj = 8 * tile + i16;
          if (i16 < 8 && m < M && jj < half) {
            const float gv = bf16_to_f32(f32_to_bf16(v)), uv = bf16_to_f32(f32_to_bf16(u));
            y[(size_t)m * half + jj] = f32_to_bf16(gv / (1.0f + expf(-gv)) * uv);
          }
        } else {
          const int n = tile * QG_TILE + i16;
          if (m < M && n < N) y[(size_t)m * N + n] = f32_to_bf16(v);
        }
      }
  }
}

int launch_gemm(const uint16_t* x, const void* packed, uint16_t* y, int M, int N, int K, bool swiglu,
                void* stream, const char* name) {
  QVEX_CHECK_ARG(x && packed && y, "%s: null pointer", name);
  QVEX_CHECK_ARG(M >= 1 && N >= 1 && K >= QG_SET && K % QG_SET == 0, "%s: M=%d N=%d K=%d (K a multiple of 256)",
                 name, M, N, K);
  QVEX_CHECK_ARG(!swiglu || N % 16 == 0, "%s: N=%d must be a multiple of 16 for the gate/up interleave", name, N);
  QVEX_CHECK_ARG(qvex_aligned(x, 16) && qvex_aligned(packed, 16), "%s: x and packed must be 16-byte aligned", name);
  const int tiles = (N + QG_TILE - 1) / QG_TILE;
  const int nb = (tiles + QG_BN / QG_TILE - 1) / (QG_BN / QG_TILE);
  const int mb = (M + QG_BM - 1) / QG_BM;
  QVEX_CHECK_ARG(mb <= 65535, "%s: M=%d too large", name, M);
  if (swiglu)
    hipLaunchKernelGGL(packed_gemm_kernel<true>, dim3(nb, mb), dim3(256), 0, (hipStream_t)stream, x,
                       (const uint8_t*)packed, y, M, N, K);
  else
    hipLaunchKernelGGL(packed_gemm_kernel<false>, dim3(nb, mb), dim3(256), 0, (hipStream_t)stream, x,
                       (const uint8_t*)packed, y, M, N, K);
  QVEX_CHECK_LAUNCH(name);
  return QVEX_OK;
}

}  // namespace

extern "C" int qvex_w4g64_packed_gemm(const uint16_t* x, const void* packed, uint16_t* y, int M, int N, int K,
                                      void* stream) {
  return launch_gemm(x, packed, y, M, N, K, false, stream, "qvex_w4g64_packed_gemm");
}

extern "C" int qvex_w4g64_packed_gemm_swiglu(const uint16_t* x, const void* packed, uint16_t* y, int M, int N,
                                             int K, void* stream) {
  return launch_gemm(x, packed, y, M, N, K, true, stream, "qvex_w4g64_packed_gemm_swiglu");
}
