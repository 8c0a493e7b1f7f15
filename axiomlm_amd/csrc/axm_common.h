// Shared device/host helpers for the AxiomLM MI355X (gfx950) decode kernels.
//
// Everything here is CDNA4-specific: wave64, 64 KB..160 KB LDS per CU, fp16
// activations with fp32 accumulation.  No CUDA / Metal code paths exist.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define AXM_WAVE 64

// ----------------------------------------------------------------------------
// Error reporting shared by every C-ABI entry point (thread-local message).
// ----------------------------------------------------------------------------
#ifdef __cplusplus
extern "C" void axm_set_error(const char* fmt, ...);
#endif

#define AXM_CHECK_ARG(cond, code, ...)      \
  do {                                      \
    if (!(cond)) {                          \
      axm_set_error(__VA_ARGS__);           \
      return (code);                        \
    }                                       \
  } while (0)

#define AXM_LAUNCH_CHECK(what)                                                  \
  do {                                                                          \
    hipError_t _e = hipGetLastError();                                          \
    if (_e != hipSuccess) {                                                     \
      axm_set_error("%s: launch failed: %s", what, hipGetErrorString(_e));      \
      return -3;                                                                \
    }                                                                           \
  } while (0)

// ----------------------------------------------------------------------------
// Bit casts / conversions.  _Float16 conversions are round-to-nearest-even,
// matching torch's CPU fp16 semantics (compute in fp32, round once).
// ----------------------------------------------------------------------------
__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ float h2f(f16 h) { return (float)h; }
__device__ __forceinline__ f16 f2h(float f) { return (f16)f; }
__device__ __forceinline__ f16 u16_as_h(uint16_t u) { return __builtin_bit_cast(f16, u); }
__device__ __forceinline__ uint16_t h_as_u16(f16 h) { return __builtin_bit_cast(uint16_t, h); }

// fp32 operations rounded one at a time: never fused into a multiply-add, so
// sequences of them reproduce the CPU reference's rounding step for step.
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

// fp16 op emulation of torch CPU kernels: every elementwise op rounds to fp16.
__device__ __forceinline__ f16 hadd(f16 a, f16 b) { return f2h(add_rn(h2f(a), h2f(b))); }
__device__ __forceinline__ f16 hmul(f16 a, f16 b) { return f2h(mul_rn(h2f(a), h2f(b))); }

// One output of the interleaved-pair RoPE rotation (x0, x1) by (c, s) as the
// reference CPU path evaluates it (quant.py:970-980, modules.py:111-121): fp32
// products and sum each rounded (no fused multiply-add), then one fp16 rounding.
__device__ __forceinline__ f16 rope_out(f16 x0, f16 x1, float c, float s, bool even) {
  const float a = h2f(x0), b = h2f(x1);
  return even ? f2h(sub_rn(mul_rn(a, c), mul_rn(b, s))) : f2h(add_rn(mul_rn(a, s), mul_rn(b, c)));
}

// Torch-CPU fp16 RMSNorm scale (axiomlm/models/modules.py:41-43 evaluated on a
// half model): mean of the fp16-rounded squares accumulated in fp32 and
// rounded once, + eps (a Python float, applied in fp32), rsqrt rounded to fp16.
__device__ __forceinline__ float rms_inv_fp16(float sumsq_of_rounded_sq, int D, float eps) {
  f16 mean = (f16)(sumsq_of_rounded_sq / (float)D);
  f16 t = (f16)((float)mean + eps);
  return (float)(f16)(1.0f / __builtin_sqrtf((float)t));
}

// ----------------------------------------------------------------------------
// Wave64 reductions.
// ----------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
// Lane reductions on DPP lane moves (no LDS round trip):
// within a 16-lane row, lane pairs (xor 1, xor 2), then the two quads of each half
// row (row_half_mirror sends lane i to 7 - i), then the two halves (row_mirror,
// i to 15 - i).  Every lane ends with the sum of its group; wave_sum_dpp returns
// the wave's total (a wave-uniform value).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float group8_sum_dpp(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  return v;
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = group8_sum_dpp(v);
  v += dpp_move<0x140>(v);  // row_mirror
  // The four row sums, read out to scalars (the staging needs the total once per wave).
  const int iv = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48)));
}

// Sum over a group of 2^k lanes (aligned), width must be a power of two <= 64.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ----------------------------------------------------------------------------
// OCP FP8 E4M3FN (the torch.float8_e4m3fn format).
//  encode: round-to-nearest-even on the 3-bit mantissa; |x| >= 480 (and NaN)
//  -> 0x7F|sign; |x| in (464, 480) rounds up into the NaN code 0x7F; 464 is a
//  tie and rounds to even (448, 0x7E); subnormals use RNE on the 2^-9 grid.
//  These are torch's CPU cast semantics (c10 fp8e4m3fn_from_fp32_value).
// ----------------------------------------------------------------------------
__device__ __forceinline__ uint8_t fp8e4m3fn_from_f32(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  // Overflow threshold: 480 = 0x43F00000 (also catches inf / NaN inputs).
  if (a >= 0x43F00000u) return (uint8_t)(sign | 0x7Fu);
  // Normal range of the result starts at 2^-6 (0x3C800000).
  if (a >= 0x3C800000u) {
    // Re-bias exponent from 127 to 7 (subtract 120 << 23) and round mantissa
    // from 23 to 3 bits with round-to-nearest-even.
    uint32_t mant_odd = (a >> 20) & 1u;
    a += 0x0007FFFFu + mant_odd;  // RNE on bit 20
    a -= (120u << 23);
    return (uint8_t)(sign | (a >> 20));
  }
  // Subnormal result: value = m * 2^-9, m in [0, 8].  Compute RNE of |f| * 512.
  float af = __builtin_bit_cast(float, a);
  float m = __builtin_rintf(af * 512.0f);  // exact scaling by power of two; rint = RNE
  return (uint8_t)(sign | (uint32_t)m);
}

__device__ __forceinline__ float fp8e4m3fn_to_f32(uint32_t b) {
  uint32_t sign = (b & 0x80u) << 24;
  uint32_t e = (b >> 3) & 0xFu;
  uint32_t m = b & 7u;
  if ((b & 0x7Fu) == 0x7Fu) return __builtin_bit_cast(float, sign | 0x7FC00000u);
  if (e == 0) {
    float v = (float)m * 0.001953125f;  // m * 2^-9
    return sign ? -v : v;
  }
  return __builtin_bit_cast(float, sign | ((e + 120u) << 23) | (m << 20));
}

// ----------------------------------------------------------------------------
// Host-side helpers.
// ----------------------------------------------------------------------------
static inline int axm_ceil_div(int a, int b) { return (a + b - 1) / b; }

// Number of compute units on the current device (cached per device).
int axm_num_cus();
