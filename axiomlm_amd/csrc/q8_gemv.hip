// Q8_G64 GEMV / small-M GEMM on gfx950 (quant.py:72-129; qmv_q8_g64_half_kernel /
// qmm_q8_g64_half_kernel, metal_kernels.metal:1941-2110): y[n] = sum_g scale * (sum q x)
// + bias * (sum x) over 64-column groups, codes uint8 [N][K], (scale, bias) fp16 [N][K/64][2].
//
// The activations (RMS-normalized when asked, with the fp16 op order of the other GEMVs)
// are staged once per workgroup in LDS as fp16, with the sum of every 16 consecutive
// values.  A wave owns R rows; lane l takes the 16 codes at 16 l + 1024 s of each of them
// in step s (one 16-byte load per row), so every activation value it reads from LDS
// serves R rows.  One v_perm_b32 turns two code bytes into the fp16 pair
// (1024 + b0, 1024 + b1) (byte next to the exponent byte 0x64), consumed with the matching
// activation pair by one v_dot2_f32_f16; sum q x = acc - 1024 * (sum x) is applied per
// 16 codes with the group's scale and bias.  The next step's codes are requested before
// the current ones are consumed.
#include "kernels.h"

namespace {

constexpr int kQ8vThreads = 256;
constexpr int kQ8vWaves = kQ8vThreads / 64;
constexpr int kOOB = 0x7FFFFFF0;

// fp16 pair (1024 + b_lo, 1024 + b_hi) of two bytes of a code word: selector bytes 0-3
// pick bytes of the code word, 4 the exponent byte 0x64 of the constant.
__device__ __forceinline__ uint32_t q8_pair(uint32_t c, uint32_t sel) { return __builtin_amdgcn_perm(0x64646464u, c, sel); }
constexpr uint32_t kSelLo = 0x04010400u;  // bytes 0, 1
constexpr uint32_t kSelHi = 0x04030402u;  // bytes 2, 3

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

template <int M, int R>
__global__ void __launch_bounds__(kQ8vThreads)
    q8v_kernel(const f16* __restrict__ x, int K, int N, const uint8_t* __restrict__ w, const f16* __restrict__ sb,
               const f16* __restrict__ bias, f16* __restrict__ y, const f16* __restrict__ ln_w, float eps) {
  extern __shared__ __align__(16) unsigned char smem[];
  f16* xs = reinterpret_cast<f16*>(smem);                       // [M][K]
  float* s16 = reinterpret_cast<float*>(xs + (size_t)M * K);    // [M][K / 16]
  __shared__ float red[kQ8vWaves];
  __shared__ float rinv_m[M];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // Codes and (scale, bias) of step 0, requested before the staging.
  const int row0 = (blockIdx.x * kQ8vWaves + wave) * R;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, N * K, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)sb, (short)0, N * (K / 64) * 4, 0x00020000);
  const int steps = (K + 1023) / 1024;
  u32x4 cw[R];
  uint32_t sv[R];
  auto load = [&](int s) {
    const int k0 = 1024 * s + 16 * lane;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = row0 + i;
      const bool ok = row < N && k0 < K;
      cw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? row * K + k0 : kOOB, 0, 0));
      sv[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (row * (K / 64) + k0 / 64) * 4 : kOOB, 0, 0);
    }
  };
  load(0);

  // RMSNorm scale per token (fp16 op order of the other normed GEMVs).
  if (ln_w != nullptr) {
    for (int m = 0; m < M; ++m) {
      float s = 0.f;
      for (int k = tid; k < K; k += kQ8vThreads) {
        const float v = h2f(x[(size_t)m * K + k]);
        s += h2f(f2h(v * v));
      }
      s = wave_sum(s);
      if (lane == 0) red[wave] = s;
      __syncthreads();
      if (tid == 0) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < kQ8vWaves; ++i) t += red[i];
        rinv_m[m] = rms_inv_fp16(t, K, eps);
      }
      __syncthreads();
    }
  }
  // Stage x (fp16) and the 16-element sums: thread -> 8 consecutive elements.
  for (int v = tid; v < M * K / 8; v += kQ8vThreads) {
    const int m = v / (K / 8), c = v % (K / 8);
    f16x8 h = *reinterpret_cast<const f16x8*>(x + (size_t)m * K + 8 * c);
    if (ln_w != nullptr) {
      const f16x8 lw = *reinterpret_cast<const f16x8*>(ln_w + 8 * c);
      const float ri = rinv_m[m];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = f2h(h2f(f2h(h2f(h[e]) * ri)) * h2f(lw[e]));
    }
    *reinterpret_cast<f16x8*>(xs + (size_t)m * K + 8 * c) = h;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s = add_rn(s, h2f(h[e]));
    s = add_rn(s, __shfl_xor(s, 1, 64));  // c and c ^ 1 are adjacent lanes (K / 8 is even)
    if ((c & 1) == 0) s16[(size_t)m * (K / 16) + c / 2] = s;
  }
  __syncthreads();

  float r[R][M];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) r[i][m] = 0.f;
  for (int s = 0; s < steps; ++s) {
    u32x4 c0[R];
    uint32_t s0[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      c0[i] = cw[i];
      s0[i] = sv[i];
    }
    if (s + 1 < steps) load(s + 1);
    const int k0 = 1024 * s + 16 * lane;
    if (k0 < K) {
      u32x4 xa[M], xb[M];
      float sx[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        xa[m] = *reinterpret_cast<const u32x4*>(xs + (size_t)m * K + k0);
        xb[m] = *reinterpret_cast<const u32x4*>(xs + (size_t)m * K + k0 + 8);
        sx[m] = s16[(size_t)m * (K / 16) + k0 / 16];
      }
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const f16x2 scb = as_h2(s0[i]);
        const float sc = h2f(scb.x), bi = h2f(scb.y);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          float acc = 0.f;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const uint32_t cwd = c0[i][g];
            const u32x4& xv = g < 2 ? xa[m] : xb[m];
            acc = dot2(xv[2 * (g & 1)], q8_pair(cwd, kSelLo), acc);
            acc = dot2(xv[2 * (g & 1) + 1], q8_pair(cwd, kSelHi), acc);
          }
          r[i][m] += sc * (acc - 1024.f * sx[m]) + bi * sx[m];
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) r[i][m] = wave_sum(r[i][m]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = row0 + i;
      if (row >= N) continue;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        f16 h = f2h(r[i][m]);
        if (bias != nullptr) h = f2h(h2f(h) + h2f(bias[row]));
        y[(size_t)m * N + row] = h;
      }
    }
  }
}

template <int M, int R>
int q8v_launch(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int K, int N,
               const f16* ln_w, float eps, hipStream_t s) {
  const size_t smem = (size_t)M * K * sizeof(f16) + (size_t)M * (K / 16) * sizeof(float);
  static bool attr_set = false;
  if (smem > 48 * 1024 && !attr_set) {
    if (hipFuncSetAttribute((const void*)q8v_kernel<M, R>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            150 * 1024) != hipSuccess) {
      (void)hipGetLastError();
      axm_set_error("q8 gemv: cannot reserve %zu bytes of LDS", smem);
      return -2;
    }
    attr_set = true;
  }
  const int rows = kQ8vWaves * R;
  hipLaunchKernelGGL((q8v_kernel<M, R>), dim3((N + rows - 1) / rows), dim3(kQ8vThreads), smem, s, x, K, N, w, sb,
                     bias, y, ln_w, eps);
  return 0;
}

// Rows per wave: four while that leaves two workgroups per CU, else two, else one.
template <int M>
int q8v_launch_m(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int K, int N,
                 const f16* ln_w, float eps, hipStream_t s) {
  const int cus = axm_num_cus();
  if (N >= 2 * cus * kQ8vWaves * 4) return q8v_launch<M, 4>(x, w, sb, bias, y, K, N, ln_w, eps, s);
  if (N >= cus * kQ8vWaves * 2) return q8v_launch<M, 2>(x, w, sb, bias, y, K, N, ln_w, eps, s);
  return q8v_launch<M, 1>(x, w, sb, bias, y, K, N, ln_w, eps, s);
}

}  // namespace

int launch_q8_gemv(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int M, int K, int N,
                   const f16* ln_w, float eps, hipStream_t s) {
  if (K % 64 != 0 || (long)N * K >= 0x7FFFFFF0L) {
    axm_set_error("q8 gemv: K=%d must be a multiple of 64 and the codes under 2 GiB (N=%d)", K, N);
    return -2;
  }
  // Up to four rows per launch, fewer when their LDS staging would not fit.
  auto lds = [K](int rows) { return (size_t)rows * K * sizeof(f16) + (size_t)rows * (K / 16) * sizeof(float); };
  int rows_max = 4;
  while (rows_max > 1 && lds(rows_max) > 150 * 1024) --rows_max;
  if (lds(1) > 150 * 1024) {
    axm_set_error("q8 gemv: K=%d too large for LDS staging", K);
    return -2;
  }
  for (int m0 = 0; m0 < M; m0 += rows_max) {
    const int mc = (M - m0) < rows_max ? (M - m0) : rows_max;
    const f16* xm = x + (size_t)m0 * K;
    f16* ym = y + (size_t)m0 * N;
    int rc;
    switch (mc) {
      case 1: rc = q8v_launch_m<1>(xm, w, sb, bias, ym, K, N, ln_w, eps, s); break;
      case 2: rc = q8v_launch_m<2>(xm, w, sb, bias, ym, K, N, ln_w, eps, s); break;
      case 3: rc = q8v_launch_m<3>(xm, w, sb, bias, ym, K, N, ln_w, eps, s); break;
      default: rc = q8v_launch_m<4>(xm, w, sb, bias, ym, K, N, ln_w, eps, s); break;
    }
    if (rc) return rc;
  }
  return 0;
}
