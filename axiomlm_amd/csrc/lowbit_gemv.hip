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
// That kernel runs one or two tokens (and the shapes below); three to sixteen tokens per
// launch run lb_mfma_kernel, which expands each code word once for all of them on MFMA.
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

// LDS bytes of lb_mfma_kernel (below) for M tokens: padded pair rows and group sums of
// 16 token slots, reused at the end for the waves' partial sums.
size_t lb_mfma_smem(int M, int K, int W) {
  const size_t staged = (size_t)M * (K / 2 + 4) * sizeof(uint32_t) + (size_t)(K / 64) * 16 * sizeof(float);
  const size_t partial = (size_t)W * 16 * 16 * sizeof(float);
  return staged > partial ? staged : partial;
}

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

// Several tokens (3 to 16 per launch) on MFMA: each 16-column code word is expanded
// once and the tokens are the A rows of v_mfma_f32_16x16x32_f16, so the VALU work per
// weight does not grow with the token count (the kernel above spends one
// v_dot2_f32_f16 per two weights and token).  A workgroup owns 16 weight rows, the B
// columns: lane l takes row n = l & 15 and word t = l >> 4 of every 64-column group
// (columns 16 t .. 16 t + 15), whose pairs 0-3 and 4-7 are the lane's 8-value MFMA
// k-groups of the group's two MFMAs, in the staged pair order.  The W waves take
// contiguous ranges of four-group chunks and add their partial products through LDS.
// Codes arrive as one 16-byte load per lane and chunk (lane row t loads group 4 c + t,
// 64 contiguous bytes per weight row and instruction) and a 4 x 4 transpose across the
// four 16-lane rows (two v_permlane32_swap, two v_permlane16_swap) leaves word t of
// each of the four groups in the lane; the same transpose of a lane's own group scale,
// copied into four registers, gives every lane the four scales.  One 4-byte load per
// group and lane (and one scale load per group and lane) made every
// load instruction touch 16 cache lines for 16 bytes each (C4 shapes at two to four
// tokens: 13.5-15 us).
// Exact up to fp32 accumulation: B holds the integers q (ternary: 4 + v - 5, v = 1 + q)
// or v (affine: 4 + v - 4); the two-MFMA chain of a group is scaled by the group's
// scale in fp32, and the affine bias term b sum x comes from staged group sums.  Lane
// l holds C rows 4 (l / 16) .. + 3, the tokens of those numbers, for row n; the staged
// activation rows are padded by 16 bytes so that the A reads of 16 tokens hit
// distinct LDS banks.
constexpr int kLbOOB = 0x7FFFFFF0;  // buffer offset past every descriptor: the load returns zeros
constexpr int kLbChunks = 4;        // four-group chunks per wave (K <= 4 W * 4 * 64)

__device__ __forceinline__ void lb_transpose4(u32x4& v) {
  typedef unsigned u32p __attribute__((ext_vector_type(2)));
  u32p a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
  u32p b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
  u32p c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  u32p d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  v[0] = c[0];
  v[1] = c[1];
  v[2] = d[0];
  v[3] = d[1];
}

template <int FMT, int W>
__global__ void __launch_bounds__(W * 64) lb_mfma_kernel(const f16* __restrict__ x, int M, int K, int N,
                                                         const uint8_t* __restrict__ w, const f16* __restrict__ s,
                                                         const f16* __restrict__ bias, f16* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int TH = W * 64;
  constexpr int kU = 4;  // staged 16-column blocks per thread and round
  const int KG = K / 64, nblk = K / 16;
  const int row_dw = K / 2 + 4;
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem);               // [M][row_dw] pairs
  float* gs = reinterpret_cast<float*>(xs + (size_t)M * row_dw);  // [KG][16] group sums
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, t = lane >> 4;
  const int row = blockIdx.x * 16 + n;
  const int nch = (KG + 3) / 4;
  const int cpw = (nch + W - 1) / W;  // chunks per wave, <= kLbChunks (checked by the host)
  const int c0 = wave * cpw, c1 = min(c0 + cpw, nch);
  const int nitems = M * nblk;  // (token, 16-column block) items of the staging

  // Staging: item i = (token i / nblk, block i % nblk), 16 columns stored as the pairs
  // (k, k + 8), with the sum of every group of four blocks (four adjacent threads).
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, nitems * 32, 0x00020000);
  u32x4 lo[kU], hi[kU];
  auto fetch = [&](int base) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = base + u * TH + tid;
      lo[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, i < nitems ? 32 * i : kLbOOB, 0, 0));
      hi[u] = __builtin_bit_cast(u32x4,
                                 __builtin_amdgcn_raw_buffer_load_b128(rx, i < nitems ? 32 * i + 16 : kLbOOB, 0, 0));
    }
  };
  auto store = [&](int base) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = base + u * TH + tid;
      const f16x8 l8 = __builtin_bit_cast(f16x8, lo[u]), h8 = __builtin_bit_cast(f16x8, hi[u]);
      f16x8 p0, p1;
      float part = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p0[2 * j] = l8[j];
        p0[2 * j + 1] = h8[j];
        p1[2 * j] = l8[4 + j];
        p1[2 * j + 1] = h8[4 + j];
        part += h2f(l8[j]) + h2f(h8[j]) + h2f(l8[4 + j]) + h2f(h8[4 + j]);
      }
      part += dpp_move<0xB1>(part);  // the group's four blocks: items 4 k .. 4 k + 3
      part += dpp_move<0x4E>(part);
      if (i < nitems) {
        const int m = i / nblk, b = i % nblk;
        f16x8* xq = reinterpret_cast<f16x8*>(xs + (size_t)m * row_dw + 8 * b);
        xq[0] = p0;
        xq[1] = p1;
        if ((b & 3) == 0) gs[(b >> 2) * 16 + m] = part;
      }
    }
  };
  fetch(0);
  // Keep those loads ahead of the codes: loads complete in issue order, so staging
  // then waits for the activations only (the scheduler otherwise sank three of the
  // four behind the code loads).
  __builtin_amdgcn_sched_barrier(0);

  // This lane's codes and scale of group 4 c + t of each chunk c (zeros past the
  // matrix, the row or the wave's range).
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)((size_t)N * K / 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)s, (short)0, (int)((size_t)N * KG * (FMT == 0 ? 2 : 4)), 0x00020000);
  u32x4 cq[kLbChunks];
  uint32_t sq[kLbChunks];
#pragma unroll
  for (int c = 0; c < kLbChunks; ++c) {
    const int ch = c0 + c;
    const int g = 4 * ch + t;
    const bool ok = row < N && ch < c1 && g < KG;
    cq[c] = __builtin_bit_cast(u32x4,
                               __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? 16 * (row * KG + g) : kLbOOB, 0, 0));
    if (FMT == 0)
      sq[c] = __builtin_amdgcn_raw_buffer_load_b16(rs, ok ? 2 * (row * KG + g) : kLbOOB, 0, 0);
    else
      sq[c] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? 4 * (row * KG + g) : kLbOOB, 0, 0);
  }
  store(0);
  for (int base = kU * TH; base < nitems; base += kU * TH) {
    fetch(base);
    store(base);
  }
  __syncthreads();

  // A row n: token n; rows past M repeat token M - 1 and only reach C rows never stored.
  const uint32_t* xa = xs + (size_t)min(n, M - 1) * row_dw;
  const f16 off = (f16)(FMT == 0 ? 5.f : 4.f);
  const f16x2 offv = {off, off};
  f32x4 tot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < kLbChunks; ++c) {
    const int ch = c0 + c;
    if (ch >= c1) break;  // wave-uniform
    u32x4 words = cq[c];
    lb_transpose4(words);  // words[i]: word t of group 4 ch + i
    u32x4 scales = {sq[c], sq[c], sq[c], sq[c]};
    lb_transpose4(scales);  // scales[i]: the scale (and bias) of group 4 ch + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = 4 * ch + i;
      if (g >= KG) break;  // wave-uniform
      const uint32_t word = FMT == 0 ? ternary_to_offset(words[i]) : words[i];
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        f16x8 B;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const f16x2 v = code_pair(word, 4 * f + p) - offv;
          B[2 * p] = v.x;
          B[2 * p + 1] = v.y;
        }
        const f16x8 A = *reinterpret_cast<const f16x8*>(xa + 4 * (2 * (4 * g + t) + f));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc, 0, 0, 0);
      }
      if (FMT == 0) {
        const float sc = h2f(u16_as_h((uint16_t)scales[i]));
#pragma unroll
        for (int k = 0; k < 4; ++k) tot[k] = __builtin_fmaf(sc, acc[k], tot[k]);
      } else {
        const f16x2 sv = as_h2(scales[i]);
        const float sc = h2f(sv.x), bi = h2f(sv.y);
        const f32x4 gsum = *reinterpret_cast<const f32x4*>(gs + g * 16 + 4 * t);
#pragma unroll
        for (int k = 0; k < 4; ++k) tot[k] = __builtin_fmaf(sc, acc[k], __builtin_fmaf(bi, gsum[k], tot[k]));
      }
    }
  }
  __syncthreads();  // every wave is done with the staged rows, which the partial sums reuse
  float* red = reinterpret_cast<float*>(smem);  // [W][16 tokens][16 rows]
#pragma unroll
  for (int i = 0; i < 4; ++i) red[(wave * 16 + 4 * t + i) * 16 + n] = tot[i];
  __syncthreads();
  if (tid < 16 * M) {
    const int m = tid >> 4, nn = tid & 15;
    float v = 0.f;
#pragma unroll
    for (int ww = 0; ww < W; ++ww) v += red[(ww * 16 + m) * 16 + nn];
    const int r = blockIdx.x * 16 + nn;
    if (r < N) y[(size_t)m * N + r] = f2h(v + (bias != nullptr ? h2f(bias[r]) : 0.f));
  }
}

template <int FMT, int W>
int lb_mfma_launch_w(const f16* x, int M, int K, int N, const uint8_t* w, const f16* s, const f16* bias, f16* y,
                     hipStream_t st) {
  const size_t smem = lb_mfma_smem(M, K, W);
  if (smem > 64 * 1024 && hipFuncSetAttribute((const void*)lb_mfma_kernel<FMT, W>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess) {
    (void)hipGetLastError();
    axm_set_error("lowbit gemv: cannot reserve %zu B of LDS", smem);
    return -2;
  }
  hipLaunchKernelGGL((lb_mfma_kernel<FMT, W>), dim3((N + 15) / 16), dim3(W * 64), smem, st, x, M, K, N, w, s, bias,
                     y);
  return 0;
}

// Waves per 16-row workgroup: four while the grid holds two workgroups per CU and the
// four waves' chunk ranges cover K, else sixteen (K <= kLbMfmaMaxK; larger K take the
// other kernel).
constexpr int kLbMfmaMaxK = 16 * kLbChunks * 4 * 64;
template <int FMT>
int lb_mfma_launch(const f16* x, int M, int K, int N, const uint8_t* w, const f16* s, const f16* bias, f16* y,
                   hipStream_t st) {
  const long wgs = (N + 15) / 16;
  if (wgs >= 2L * axm_num_cus() && K <= 4 * kLbChunks * 4 * 64)
    return lb_mfma_launch_w<FMT, 4>(x, M, K, N, w, s, bias, y, st);
  return lb_mfma_launch_w<FMT, 16>(x, M, K, N, w, s, bias, y, st);
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

// Tokens per lb_mfma_kernel launch at this K: as many as LDS holds, up to 16.
int lb_mfma_max_tokens(int K) {
  const size_t per_token = (size_t)(K / 2 + 4) * sizeof(uint32_t);
  const size_t fixed = (size_t)(K / 64) * 16 * sizeof(float);
  const size_t cap = 160 * 1024;
  const int m = fixed >= cap ? 0 : (int)((cap - fixed) / per_token);
  return m < 16 ? m : 16;
}

template <int FMT>
int lowbit_gemv(const void* x, const void* w, const void* s, const void* bias, void* y, int M, int K, int N,
                hipStream_t st) {
  // MFMA launches of up to lb_mfma_max_tokens(K) tokens while at least three remain;
  // one or two tokens, K above kLbMfmaMaxK, codes beyond 31-bit buffer offsets and
  // shapes whose staged rows leave room for fewer than three tokens take the
  // dot-product kernel (C4 shapes, dot-product / MFMA: one token 6.6 / -, two 8.1 /
  // 9.4 us, three 10.0 / 9.5, four 11.2 / 9.6; at 11008 -> 4096 four tokens 17.5 /
  // 10.3 us).
  constexpr int kMinTokens = 3;
  const int mt = (size_t)N * K / 4 < (size_t)kLbOOB && K <= kLbMfmaMaxK ? lb_mfma_max_tokens(K) : 0;
  int m0 = 0;
  while (mt >= kMinTokens && M - m0 >= kMinTokens) {
    const int mc = (M - m0) < mt ? (M - m0) : mt;
    const int rc = lb_mfma_launch<FMT>((const f16*)x + (size_t)m0 * K, mc, K, N, (const uint8_t*)w, (const f16*)s,
                                       (const f16*)bias, (f16*)y + (size_t)m0 * N, st);
    if (rc) return rc;
    m0 += mc;
  }
  for (; m0 < M; m0 += 4) {
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
