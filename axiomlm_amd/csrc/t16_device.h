// Device helpers shared by the tile16 GEMV kernels (stand-alone launches and
// the persistent decode-step kernel).
#pragma once
#include "axm_common.h"

// Nibble expansion: (w & mask) | magic as one v_and_or_b32.  gfx950 VOP3 takes
// neither literals nor two scalar operands, so the masks must sit in VGPRs and
// the magic exponents in SGPRs for instruction selection to fuse the pair.
// The masks are moved into VGPRs once, through an opaque move the compiler
// cannot fold back into a constant; the AND-OR itself stays compiler-generated
// so the MFMA hazard recognizer sees every VALU write that feeds a B operand
// (a VALU write read by an MFMA source needs two wait states, and the
// recognizer does not model inline-asm producers).
struct Unpack {
  uint32_t m_lo, m_hi, g_lo, g_hi;  // 0x000F000F, 0x00F000F0, 0x64006400, 0x54005400
};

__device__ __forceinline__ uint32_t to_vgpr(uint32_t s) {
  uint32_t v;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "s"(s));
  return v;
}

// A VGPR copy the compiler cannot see through (keeps a loaded uniform value out of
// SGPRs until here, so the wait for it lands here).
__device__ __forceinline__ uint32_t t16_vgpr(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(v));
  return r;
}

// A value the compiler cannot fold into a literal operand, kept in an SGPR.
__device__ __forceinline__ uint32_t to_sgpr(uint32_t s) {
  uint32_t v;
  asm volatile("s_mov_b32 %0, %1" : "=s"(v) : "s"(s));
  return v;
}

__device__ __forceinline__ uint32_t and_or(uint32_t w, uint32_t mask_v, uint32_t magic_s) {
  return (w & mask_v) | magic_s;
}

__device__ __forceinline__ f16x8 unpack_word(uint32_t w, const Unpack& u) {
  const uint32_t w8 = w >> 8;
  const u32x4 h = {and_or(w, u.m_lo, u.g_lo), and_or(w, u.m_hi, u.g_hi), and_or(w8, u.m_lo, u.g_lo),
                   and_or(w8, u.m_hi, u.g_hi)};
  return __builtin_bit_cast(f16x8, h);
}

__device__ __forceinline__ float t16_silu(float g) { return g / (1.0f + expf(-g)); }

