// One RMSNorm row on the first 256 threads of a block: thread t holds the
// 8-element chunks t, t+256, ... of the row in registers (16-byte loads), so the
// row is read once and the reduction is one wave butterfly plus 4 LDS slots in a
// fixed order. y = w * (x * rsqrt(mean(x^2) + eps)) * scale (w optional); with
// ADD the row is first h = bf16(x + delta), stored to h_out, and normalised.
// Every thread of the block must call it (it holds a barrier); threads past 255
// only pass the barrier, so any block size gives the same bits. `red` holds 4
// floats of LDS; callers that reuse it for another row barrier in between.
// mx.fast.rms_norm as used by the layer stack (engine/model.py:309-317, 335).
#pragma once
#include "qvex_common.h"

namespace {

constexpr int RMS_MAXC = 4;   // chunks of 8 per thread: D <= 8192

__device__ __forceinline__ void unpack8(const u32x4 v, float* f) {
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x); f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z); f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
  v.x = pack_bf16x2(f[0], f[1]); v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]); v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

// The normalisation of a row whose values thread t already holds as v[c][e] =
// element 8 (t + 256 c) + e (what rms_row256 loads): y = w * (v * inv) * scale.
__device__ __forceinline__ void rms_vals256(float (&v)[RMS_MAXC][8], const uint16_t* __restrict__ w,
                                            uint16_t* __restrict__ outr, int D, float eps, float scale, float* red) {
  const int t = threadIdx.x;
  const bool act = t < 256;
  // the weight chunks requested before the reduction (chunks past D re-read
  // chunk 0, never used): loaded where they are used, each chunk would wait
  // for its own round trip after the barrier
  u32x4 wq[RMS_MAXC];
  if (w && act) {
#pragma unroll
    for (int c = 0; c < RMS_MAXC; ++c) {
      const int i = (t + 256 * c) * 8;
      wq[c] = load16(w + (i < D ? i : 0));
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < RMS_MAXC; ++c) {
    const int i = (t + 256 * c) * 8;
    if (act && i < D) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[c][e], v[c][e], ss);
    }
  }
  ss = wave_allsum(ss);
  if (act && (t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
  for (int c = 0; c < RMS_MAXC; ++c) {
    const int i = (t + 256 * c) * 8;
    if (act && i < D) {
      float o[8];
      if (w) {
        float wf[8];
        unpack8(wq[c], wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = wf[e] * (v[c][e] * inv) * scale;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (v[c][e] * inv) * scale;
      }
      *reinterpret_cast<u32x4*>(outr + i) = pack8(o);
    }
  }
}

template <bool ADD>
__device__ __forceinline__ void rms_row256(const uint16_t* __restrict__ xr, const uint16_t* __restrict__ dr,
                                           uint16_t* __restrict__ hr, const uint16_t* __restrict__ w,
                                           uint16_t* __restrict__ outr, int D, float eps, float scale, float* red) {
  const int t = threadIdx.x;
  const bool act = t < 256;
  float v[RMS_MAXC][8];
  // every chunk's loads first (chunks past D re-read chunk 0, never used), then
  // the arithmetic: a load used inside its own chunk's branch is waited for
  // there, one round trip per chunk
  u32x4 xq[RMS_MAXC], dq[RMS_MAXC];
  if (act) {
#pragma unroll
    for (int c = 0; c < RMS_MAXC; ++c) {
      const int i = (t + 256 * c) * 8, ic = i < D ? i : 0;
      xq[c] = load16(xr + ic);
      if constexpr (ADD) dq[c] = load16(dr + ic);
    }
  }
#pragma unroll
  for (int c = 0; c < RMS_MAXC; ++c) {
    const int i = (t + 256 * c) * 8;
    if (act && i < D) {
      unpack8(xq[c], v[c]);
      if constexpr (ADD) {
        float d[8];
        unpack8(dq[c], d);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[c][e] = bf16_to_f32(f32_to_bf16(v[c][e] + d[e]));
        *reinterpret_cast<u32x4*>(hr + i) = pack8(v[c]);
      }
    }
  }
  rms_vals256(v, w, outr, D, eps, scale, red);
}

}  // namespace
