// GEMV / small-M GEMM on the 2-bit row formats, gfx950:
//   BitNet 1.58 ternary  (quant.py:236-296; qmv/qmm_ternary_half_kernel,
//                         metal_kernels.metal:3990-4160)
//   reference "Q2_K"     (affine 2-bit, quant.py:339-403; qmv/qmm_q2_k_half_kernel,
//                         metal_kernels.metal:4167-4334)
// Both store uint8 [N][K/4], element 4b+j of a row at bits 2j of byte b, and one
// (scale) or (scale, bias) fp16 entry per row and 64-column group.
//
// Mapping: 4 waves per workgroup, ROWS rows per wave (four when the grid still
// holds two workgroups per CU, else two: fewer workgroups re-stage the activation
// row); lane l handles groups
// g = l, l + 64, ... (ITERS of them, K <= ITERS * 4096).  One 16-byte load per
// (row, group) brings all 64 codes of the group; a lane requests the codes and
// scales of all its groups before the workgroup stages the activations, so the
// weight stream and the staging overlap.  Each 32-bit word holds the codes of columns 16d .. 16d+15 and is
// expanded in pairs: pair p takes the fields at bits 2p and 16 + 2p (columns
// 16d + p and 16d + p + 8), moves them into bits 8-9 of each half and ORs the
// fp16 exponent of 4.0, giving the exact halves (4 + v, 4 + v').  The
// activations are staged in LDS in the same pair order, so each pair is one
// v_dot2_f32_f16 with fp32 accumulation; the 4.0 offset is removed once per
// group with the group's activation sum.
//   ternary: the 2-bit code c = (lo, hi) decodes to q = lo - hi (quant.py:287-293);
//            a bitwise pass turns every field into v = 1 + q in [0, 2], so
//            sum w x = scale * (sum x v - sum x).
//   Q2     : v = c, sum w x = scale * sum x c + bias * sum x.
#include "kernels.h"

namespace {

constexpr int kLbThreads = 256;

__device__ __forceinline__ uint32_t ternary_to_offset(uint32_t w) {
  const uint32_t lo = w & 0x55555555u;
  const uint32_t hi = (w >> 1) & 0x55555555u;
  const uint32_t t_lo = ~(lo ^ hi) & 0x55555555u;  // v bit 0: lo == hi
  const uint32_t t_hi = (lo & ~hi) << 1;            // v bit 1: lo && !hi
  return t_lo | t_hi;
}

__device__ __forceinline__ f16x2 code_pair(uint32_t w, int p) {
  const uint32_t t = p < 4 ? (w << (8 - 2 * p)) : (w >> (2 * p - 8));
  return __builtin_bit_cast(f16x2, (t & 0x03000300u) | 0x44004400u);
}

// LDS slot of activation quad q (8 staged values, 16 bytes) within its row: bits 4-6
// of q are XORed onto bits 0-2.  Lane g reads quads 8 g .. 8 g + 7 of a row, so
// without it the 16 lanes of one LDS cycle hit two 16-byte bank groups (8-way
// conflicts); with it they hit 16 distinct ones.  A bijection on aligned 8-quad
// blocks: a lane's eight quads stay its own, in another order.
__device__ __forceinline__ int lb_lds_quad(int q) { return q ^ ((q >> 4) & 7); }

// xs: [M][K] fp16, each 16-column block stored as pairs (k, k+8), k = 0..7, quad q
// of a row at slot lb_lds_quad(q).
// gs: [M][K/64] fp32 group sums of x.
template <int FMT, int M, int ITERS, int kLbRows>
__global__ void __launch_bounds__(kLbThreads) lowbit_gemv_kernel(const f16* __restrict__ x, int K, int N,
                                                                const uint8_t* __restrict__ w,
                                                                const f16* __restrict__ s, const f16* __restrict__ bias,
                                                                f16* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  f16* xs = reinterpret_cast<f16*>(smem);
  float* gs = reinterpret_cast<float*>(xs + (size_t)M * K);
  const int tid = threadIdx.x;
  const int KG = K / 64;
  const int nblk = K / 16;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row0 = (blockIdx.x * (kLbThreads / 64) + wave) * kLbRows;
  const size_t row_bytes = (size_t)K / 4;

  // Activation vectors of this thread (blocks tid + 256 i, i < ITERS: K / 16
  // blocks of 16 columns), requested first: a wave's loads complete in issue
  // order, so the staging below then waits only for these.  Blocks past the row
  // are clamped and masked.
  f16x8 xlo[M][ITERS], xhi[M][ITERS];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int i = 0; i < ITERS; ++i) {
      const int b = min(tid + kLbThreads * i, nblk - 1);
      xlo[m][i] = *reinterpret_cast<const f16x8*>(x + (size_t)m * K + 16 * b);
      xhi[m][i] = *reinterpret_cast<const f16x8*>(x + (size_t)m * K + 16 * b + 8);
    }
  // Then the codes and scales of every (row, group) of this lane (groups past
  // the row are clamped to the last one and skipped below).
  u32x4 cw[ITERS][kLbRows];
  float sc[ITERS][kLbRows], bi[ITERS][kLbRows];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int g = min(lane + 64 * it, KG - 1);
#pragma unroll
    for (int r = 0; r < kLbRows; ++r) {
      const int row = min(row0 + r, N - 1);
      cw[it][r] = *reinterpret_cast<const u32x4*>(w + (size_t)row * row_bytes + 16 * g);
      if (FMT == 0) {
        sc[it][r] = h2f(s[(size_t)row * KG + g]);
        bi[it][r] = 0.f;
      } else {
        const f16x2 v = *reinterpret_cast<const f16x2*>(s + ((size_t)row * KG + g) * 2);
        sc[it][r] = h2f(v.x);
        bi[it][r] = h2f(v.y);
      }
    }
  }
  // Stage the activations in pair order with their group sums.
#pragma unroll
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int i = 0; i < ITERS; ++i) {
      const int b = tid + kLbThreads * i;
      const f16x8 lo = xlo[m][i], hi = xhi[m][i];
      f16x8 p0, p1;
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p0[2 * j] = lo[j];
        p0[2 * j + 1] = hi[j];
        p1[2 * j] = lo[4 + j];
        p1[2 * j + 1] = hi[4 + j];
        part += h2f(lo[j]) + h2f(hi[j]) + h2f(lo[4 + j]) + h2f(hi[4 + j]);
      }
      // Four consecutive blocks form one group (nblk is a multiple of 4): a quad
      // of lanes, summed with DPP lane moves.
      part += dpp_move<0xB1>(part);  // quad_perm [1,0,3,2]
      part += dpp_move<0x4E>(part);  // quad_perm [2,3,0,1]
      if (b < nblk) {
        f16x8* xq = reinterpret_cast<f16x8*>(xs + (size_t)m * K);
        xq[lb_lds_quad(2 * b)] = p0;
        xq[lb_lds_quad(2 * b + 1)] = p1;
        if ((b & 3) == 0) gs[m * KG + b / 4] = part;
      }
    }
  }
  __syncthreads();

  float yacc[kLbRows][M];
#pragma unroll
  for (int r = 0; r < kLbRows; ++r)
#pragma unroll
    for (int m = 0; m < M; ++m) yacc[r][m] = 0.f;

#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int g = lane + 64 * it;
    if (g >= KG) break;
    if (FMT == 0) {
#pragma unroll
      for (int r = 0; r < kLbRows; ++r)
#pragma unroll
        for (int d = 0; d < 4; ++d) cw[it][r][d] = ternary_to_offset(cw[it][r][d]);
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u32x4* xp = reinterpret_cast<const u32x4*>(xs + (size_t)m * K);
      u32x4 xv[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) xv[q] = xp[lb_lds_quad(8 * g + q)];
      const float gsum = gs[m * KG + g];
#pragma unroll
      for (int r = 0; r < kLbRows; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
#pragma unroll
          for (int p = 0; p < 8; ++p) {
            // Copy the element out first: a bit_cast applied directly to an
            // ext_vector element expression reads element 0 with this compiler.
            const uint32_t xw = xv[2 * d + p / 4][p % 4];
            const f16x2 xpair = as_h2(xw);
            acc = __builtin_amdgcn_fdot2(xpair, code_pair(cw[it][r][d], p), acc, false);
          }
        }
        if (FMT == 0)
          yacc[r][m] = __builtin_fmaf(sc[it][r], acc - 5.f * gsum, yacc[r][m]);
        else
          yacc[r][m] = __builtin_fmaf(sc[it][r], acc - 4.f * gsum, __builtin_fmaf(bi[it][r], gsum, yacc[r][m]));
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kLbRows; ++r) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum_dpp(yacc[r][m]);
      const int row = row0 + r;
      if (lane == 0 && row < N) {
        const float b = bias != nullptr ? h2f(bias[row]) : 0.f;
        y[(size_t)m * N + row] = f2h(v + b);
      }
    }
  }
}

template <int FMT, int M, int ITERS, int ROWS>
int lowbit_launch_rows(const f16* x, int K, int N, const uint8_t* w, const f16* s, const f16* bias, f16* y,
                       hipStream_t st) {
  const size_t smem = (size_t)M * K * sizeof(f16) + (size_t)M * (K / 64) * sizeof(float);
  if (smem > 160 * 1024) {
    axm_set_error("lowbit gemv: K=%d needs %zu B of LDS", K, smem);
    return -2;
  }
  if (smem > 64 * 1024 &&
      hipFuncSetAttribute((const void*)lowbit_gemv_kernel<FMT, M, ITERS, ROWS>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess) {
    (void)hipGetLastError();
    axm_set_error("lowbit gemv: cannot reserve %zu B of LDS", smem);
    return -2;
  }
  const int rows_per_block = (kLbThreads / 64) * ROWS;
  const int grid = (N + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((lowbit_gemv_kernel<FMT, M, ITERS, ROWS>), dim3(grid), dim3(kLbThreads), smem, st, x, K, N, w,
                     s, bias, y);
  return 0;
}

template <int FMT, int M, int ITERS>
int lowbit_launch_iters(const f16* x, int K, int N, const uint8_t* w, const f16* s, const f16* bias, f16* y,
                        hipStream_t st) {
  const int wg4 = (N + 4 * (kLbThreads / 64) - 1) / (4 * (kLbThreads / 64));
  if (wg4 >= 2 * axm_num_cus()) return lowbit_launch_rows<FMT, M, ITERS, 4>(x, K, N, w, s, bias, y, st);
  return lowbit_launch_rows<FMT, M, ITERS, 2>(x, K, N, w, s, bias, y, st);
}

// Groups per lane: K / 64 groups over 64 lanes, up to 8 (K <= 32768).
template <int FMT, int M>
int lowbit_launch(const f16* x, int K, int N, const uint8_t* w, const f16* s, const f16* bias, f16* y,
                  hipStream_t st) {
  const int iters = (K / 64 + 63) / 64;
  switch (iters) {
    case 1: return lowbit_launch_iters<FMT, M, 1>(x, K, N, w, s, bias, y, st);
    case 2: return lowbit_launch_iters<FMT, M, 2>(x, K, N, w, s, bias, y, st);
    case 3: return lowbit_launch_iters<FMT, M, 3>(x, K, N, w, s, bias, y, st);
    case 4: return lowbit_launch_iters<FMT, M, 4>(x, K, N, w, s, bias, y, st);
  }
  if (iters <= 8) return lowbit_launch_iters<FMT, M, 8>(x, K, N, w, s, bias, y, st);
  axm_set_error("lowbit gemv: K=%d above 32768", K);
  return -2;
}

template <int FMT>
int lowbit_gemv(const void* x, const void* w, const void* s, const void* bias, void* y, int M, int K, int N,
                hipStream_t st) {
  for (int m0 = 0; m0 < M; m0 += 4) {
    const int mc = (M - m0) < 4 ? (M - m0) : 4;
    const f16* xm = (const f16*)x + (size_t)m0 * K;
    f16* ym = (f16*)y + (size_t)m0 * N;
    int rc = 0;
    switch (mc) {
      case 1: rc = lowbit_launch<FMT, 1>(xm, K, N, (const uint8_t*)w, (const f16*)s, (const f16*)bias, ym, st); break;
      case 2: rc = lowbit_launch<FMT, 2>(xm, K, N, (const uint8_t*)w, (const f16*)s, (const f16*)bias, ym, st); break;
      case 3: rc = lowbit_launch<FMT, 3>(xm, K, N, (const uint8_t*)w, (const f16*)s, (const f16*)bias, ym, st); break;
      default: rc = lowbit_launch<FMT, 4>(xm, K, N, (const uint8_t*)w, (const f16*)s, (const f16*)bias, ym, st); break;
    }
    if (rc) return rc;
  }
  return 0;
}

}  // namespace

extern "C" int axm_qmv_ternary(const void* x, const void* w_packed, const void* scales, const void* bias, void* y,
                               int M, int K, int N, void* stream) {
  AXM_CHECK_ARG(x && w_packed && scales && y, -1, "qmv_ternary: null pointer");
  AXM_CHECK_ARG(M >= 1 && N >= 1 && K >= 64 && K % 64 == 0, -1, "qmv_ternary: bad shape M=%d K=%d N=%d", M, K, N);
  const int rc = lowbit_gemv<0>(x, w_packed, scales, bias, y, M, K, N, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmv_ternary");
  return 0;
}

extern "C" int axm_qmv_q2_k(const void* x, const void* w_packed, const void* scales_biases, const void* bias, void* y,
                            int M, int K, int N, void* stream) {
  AXM_CHECK_ARG(x && w_packed && scales_biases && y, -1, "qmv_q2_k: null pointer");
  AXM_CHECK_ARG(M >= 1 && N >= 1 && K >= 64 && K % 64 == 0, -1, "qmv_q2_k: bad shape M=%d K=%d N=%d", M, K, N);
  const int rc = lowbit_gemv<1>(x, w_packed, scales_biases, bias, y, M, K, N, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmv_q2_k");
  return 0;
}
