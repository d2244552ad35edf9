// Shared device/host helpers for the qvex HIP kernels (gfx950, wave64).
//
// bf16 values cross the C ABI as raw uint16_t bit patterns; kernels widen them
// to fp32 with a shift and narrow with round-to-nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/qvex.h"

#define QVEX_WAVE 64

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16-byte streaming load (nontemporal: the data is used once).
__device__ __forceinline__ u32x4 load_nt16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// ---------------------------------------------------------------- bf16

__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// fp32 -> bf16, round to nearest even; NaN stays NaN (quiet). Written as a
// select, not a branch, so that it compiles to a few VALU instructions with no
// exec-mask changes.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t nan = (u >> 16) | 0x40u;
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? nan : rne);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// ---------------------------------------------------------------- wave reductions (DPP)
//
// Sum over the 64 lanes of a wave. Row (16-lane) sums use row_shr, then
// row_bcast15/31 carry partials across rows; the full sum lands in lane 63.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, bool BOUND_CTRL = false>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, BOUND_CTRL));
}

// DPP control codes (GCN3+ encoding).
#define DPP_ROW_SHR(n) (0x110 + (n))
#define DPP_ROW_BCAST15 0x142
#define DPP_ROW_BCAST31 0x143

// After this, lane 63 holds the wave total (other lanes hold partials).
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_f<DPP_ROW_SHR(1), 0xf, 0xf, true>(v);   // bound_ctrl: out-of-row source reads 0
  v += dpp_f<DPP_ROW_SHR(2), 0xf, 0xf, true>(v);
  v += dpp_f<DPP_ROW_SHR(4), 0xf, 0xf, true>(v);
  v += dpp_f<DPP_ROW_SHR(8), 0xf, 0xf, true>(v);
  v += dpp_f<DPP_ROW_BCAST15, 0xa, 0xf, false>(v);  // rows 1,3 get lane 15 of rows 0,2
  v += dpp_f<DPP_ROW_BCAST31, 0xc, 0xf, false>(v);  // rows 2,3 get lane 31
  return v;
}

// Sum over the 16 lanes of a DPP row in every lane of it (quad swaps, then row
// rotations by 4 and 8). The lanes pair the four quad sums differently, so they
// can differ in the last bit: where that matters, one lane's value is used.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_allsum(float v) {
  v += dpp_row<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_row<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_row<0x124>(v);  // row_ror 4
  v += dpp_row<0x128>(v);  // row_ror 8
  return v;
}

// Lane i of each DPP row gets lane i - n of the same row (n in 0..8, a
// constant after unrolling; lanes i < n read 0).
__device__ __forceinline__ float row_shr_n(float v, int n) {
  switch (n) {
    case 1: return dpp_row<DPP_ROW_SHR(1)>(v);
    case 2: return dpp_row<DPP_ROW_SHR(2)>(v);
    case 3: return dpp_row<DPP_ROW_SHR(3)>(v);
    case 4: return dpp_row<DPP_ROW_SHR(4)>(v);
    case 5: return dpp_row<DPP_ROW_SHR(5)>(v);
    case 6: return dpp_row<DPP_ROW_SHR(6)>(v);
    case 7: return dpp_row<DPP_ROW_SHR(7)>(v);
    case 8: return dpp_row<DPP_ROW_SHR(8)>(v);
    default: return v;
  }
}

// Minimum over the wave in every lane (all 64 lanes active): each DPP row's
// minimum, then the four row minima read into scalars (a minimum is order-free).
__device__ __forceinline__ int wave_allmin(int v) {
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false));  // row_ror 4
  v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false));  // row_ror 8
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Sum over the wave broadcast to every lane (all 64 lanes active): each DPP
// row's sum, then the four row sums read into scalars and added as
// (r0 + r1) + (r2 + r3). Four DPP steps and four readlanes instead of six
// dependent LDS-permute round trips of an xor butterfly.
__device__ __forceinline__ float wave_allsum(float v) {
  v = row16_allsum(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// DPP move whose disabled or out-of-range lanes keep their own value.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_keep(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Maximum broadcast to every lane: quad swaps, half-row and row mirrors give
// every lane its row maximum, row_bcast15/31 fold the rows into lane 63, which
// is read back. A maximum is order-free, so the result equals any other
// reduction order's (up to the sign of a zero).
__device__ __forceinline__ float wave_allmax(float v) {
  v = fmaxf(v, dpp_keep<0xB1>(v));                     // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_keep<0x4E>(v));                     // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_keep<0x141>(v));                    // row_half_mirror
  v = fmaxf(v, dpp_keep<0x140>(v));                    // row_mirror
  v = fmaxf(v, dpp_keep<DPP_ROW_BCAST15, 0xa>(v));     // rows 1,3 take rows 0,2
  v = fmaxf(v, dpp_keep<DPP_ROW_BCAST31, 0xc>(v));     // rows 2,3 take row 1
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}


// ---------------------------------------------------------------- host-side error plumbing

namespace qvex {

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

}  // namespace qvex

#define QVEX_CHECK_ARG(cond, ...)                                  \
  do {                                                             \
    if (!(cond)) return qvex::fail(QVEX_EINVAL, __VA_ARGS__);      \
  } while (0)

#define QVEX_CHECK_LAUNCH(name)                                                      \
  do {                                                                               \
    hipError_t _e = hipGetLastError();                                               \
    if (_e != hipSuccess)                                                            \
      return qvex::fail(QVEX_EHIP, "%s: launch failed: %s", name, hipGetErrorString(_e)); \
  } while (0)

#define QVEX_HIP(call, name)                                                         \
  do {                                                                               \
    hipError_t _e = (call);                                                          \
    if (_e != hipSuccess)                                                            \
      return qvex::fail(QVEX_EHIP, "%s: %s", name, hipGetErrorString(_e));           \
  } while (0)

static inline bool qvex_aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }
