// Device helpers shared by the 4-bit group-64 kernels: the bf16 "magic 128"
// nibble unpack and the fp32 dot products / MFMA operand casts around it.
//
// A 4-bit code q sits in the low mantissa bits of the bf16 number 128 + q
// (0x4300 | q), so (word >> 4j) & 0x000F000F | 0x43004300 turns two codes of a
// packed word into an exact bf16 pair in one v_and_or_b32; the +128 offset is
// folded into the group bias afterwards (s*(D - 128*X) + b*X).
#pragma once
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

// (a & mask) | magic. gfx9 VOP3 takes no literal operand, so with both constants
// as literals the compiler splits this into two VOP2 ops; callers make the mask
// an opaque SGPR value and the magic an opaque VGPR value (see opaque_sgpr /
// opaque_vgpr), which lets it select one v_and_or_b32 (one constant-bus read)
// while the hazard recognizer still sees every instruction.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
  return (a & mask) | magic;
}
__device__ __forceinline__ uint32_t opaque_sgpr(uint32_t v) {
  asm volatile("" : "+s"(v));
  return v;
}
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_t as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(bf16x8_t, v);
}

}  // namespace
