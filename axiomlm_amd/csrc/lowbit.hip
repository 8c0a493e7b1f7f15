// Packers for the group-64 row formats (Q8_G64, BitNet ternary, reference
// "Q2_K" affine 2-bit) and the row-wise KV quantizers, gfx950.
//
// One wave per (row, 64-column group), one lane per column.  Arithmetic is the
// reference's torch CPU op sequence with explicit rounding (no contraction):
// fp16 sources round every elementwise op to fp16, fp32 sources stay fp32.
#include "kernels.h"

namespace {

__device__ __forceinline__ float load_src(const void* w, bool fp16, size_t i) {
  return fp16 ? h2f(reinterpret_cast<const f16*>(w)[i]) : reinterpret_cast<const float*>(w)[i];
}

// Affine min/max formats: Q8 (qmax 255, quant.py:72-111) and Q2 (qmax 3, quant.py:339-378).
__global__ void pack_affine_kernel(const void* __restrict__ w, int src_fp16, int N, int K, float qmax,
                                   uint8_t* __restrict__ codes, f16* __restrict__ sb) {
  const int KG = K / 64;
  const long rg = (long)blockIdx.x;
  const int row = (int)(rg / KG), g = (int)(rg % KG);
  const int lane = threadIdx.x;
  const size_t idx = (size_t)row * K + 64 * g + lane;
  const float x = load_src(w, src_fp16, idx);
  const float mn = -wave_max(-x);
  const float mx = wave_max(x);
  float denom;
  if (src_fp16) {
    denom = h2f(f2h(sub_rn(mx, mn)));  // fp16 subtraction; the 1e-8 clamp bound rounds to 0 in fp16
  } else {
    denom = fmaxf(sub_rn(mx, mn), 1e-8f);
  }
  const f16 sc = f2h(__fdiv_rn(denom, qmax));
  const f16 bi = f2h(mn);
  float q = __builtin_rintf(__fdiv_rn(sub_rn(x, h2f(bi)), fmaxf(h2f(sc), 1e-8f)));
  q = fminf(fmaxf(q, 0.f), qmax);
  if (qmax > 3.5f) {
    codes[idx] = (uint8_t)q;
  } else {
    // four 2-bit codes per byte, element 4b+j at bits 2j
    const uint32_t qi = (uint32_t)q;
    uint32_t byte = qi;
    byte |= (uint32_t)__shfl_down((int)qi, 1, 64) << 2;
    byte |= (uint32_t)__shfl_down((int)qi, 2, 64) << 4;
    byte |= (uint32_t)__shfl_down((int)qi, 3, 64) << 6;
    if ((lane & 3) == 0) codes[((size_t)row * K + 64 * g + lane) / 4] = (uint8_t)byte;
  }
  if (lane == 0) {
    sb[((size_t)row * KG + g) * 2 + 0] = sc;
    sb[((size_t)row * KG + g) * 2 + 1] = bi;
  }
}

// BitNet 1.58 ternary, per-(row, group) absmean scale (quant.py:236-276).
__global__ void pack_ternary_kernel(const void* __restrict__ w, int src_fp16, int N, int K,
                                    uint8_t* __restrict__ codes, f16* __restrict__ scales) {
  const int KG = K / 64;
  const long rg = (long)blockIdx.x;
  const int row = (int)(rg / KG), g = (int)(rg % KG);
  const int lane = threadIdx.x;
  const size_t idx = (size_t)row * K + 64 * g + lane;
  const float x = load_src(w, src_fp16, idx);
  const float mean = __fdiv_rn(wave_sum(fabsf(x)), 64.f);
  f16 sc;
  if (src_fp16) {
    sc = f2h(mean);                           // mean rounded to fp16
    const f16 lo = f2h(1e-5f);                // clamp bound cast to fp16
    if (h2f(sc) < h2f(lo)) sc = lo;
  } else {
    sc = f2h(fmaxf(mean, 1e-5f));
  }
  float q = __builtin_rintf(__fdiv_rn(x, fmaxf(h2f(sc), 1e-5f)));
  q = fminf(fmaxf(q, -1.f), 1.f);
  const uint32_t code = q > 0.5f ? 1u : (q < -0.5f ? 2u : 0u);
  uint32_t byte = code;
  byte |= (uint32_t)__shfl_down((int)code, 1, 64) << 2;
  byte |= (uint32_t)__shfl_down((int)code, 2, 64) << 4;
  byte |= (uint32_t)__shfl_down((int)code, 3, 64) << 6;
  if ((lane & 3) == 0) codes[idx / 4] = (uint8_t)byte;
  if (lane == 0) scales[(size_t)row * KG + g] = sc;
}

}  // namespace

extern "C" int axm_pack_q8_g64(const void* w, int src_is_fp16, int N, int K, void* packed_u8, void* sb,
                               void* stream) {
  AXM_CHECK_ARG(w && packed_u8 && sb && N > 0 && K > 0 && K % 64 == 0, -1, "pack_q8_g64: bad arguments");
  hipLaunchKernelGGL(pack_affine_kernel, dim3((unsigned)((long)N * (K / 64))), dim3(64), 0, (hipStream_t)stream, w,
                     src_is_fp16, N, K, 255.0f, (uint8_t*)packed_u8, (f16*)sb);
  AXM_LAUNCH_CHECK("pack_q8_g64");
  return 0;
}

extern "C" int axm_pack_q2_k(const void* w, int src_is_fp16, int N, int K, void* packed_u8, void* sb,
                             void* stream) {
  AXM_CHECK_ARG(w && packed_u8 && sb && N > 0 && K > 0 && K % 64 == 0, -1, "pack_q2_k: bad arguments");
  hipLaunchKernelGGL(pack_affine_kernel, dim3((unsigned)((long)N * (K / 64))), dim3(64), 0, (hipStream_t)stream, w,
                     src_is_fp16, N, K, 3.0f, (uint8_t*)packed_u8, (f16*)sb);
  AXM_LAUNCH_CHECK("pack_q2_k");
  return 0;
}

extern "C" int axm_pack_ternary(const void* w, int src_is_fp16, int N, int K, void* packed_u8, void* scales,
                                void* stream) {
  AXM_CHECK_ARG(w && packed_u8 && scales && N > 0 && K > 0 && K % 64 == 0, -1, "pack_ternary: bad arguments");
  hipLaunchKernelGGL(pack_ternary_kernel, dim3((unsigned)((long)N * (K / 64))), dim3(64), 0, (hipStream_t)stream, w,
                     src_is_fp16, N, K, (uint8_t*)packed_u8, (f16*)scales);
  AXM_LAUNCH_CHECK("pack_ternary");
  return 0;
}
