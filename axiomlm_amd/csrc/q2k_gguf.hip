// GGUF Q2_K super-blocks on gfx950: packer, dequantization and GEMV.
//
// Format (ggml block_q2_K, QK_K = 256; 84 bytes per 256 weights = 0.328125 B/w):
//   bytes  0..15  scales[16]: sub-block s (elements 16s .. 16s+15) has a 4-bit
//                 scale (low nibble) and a 4-bit min (high nibble)
//   bytes 16..79  qs[64]: element e = 128h + 32j + l (h < 2, j < 4, l < 32) is the
//                 2-bit field at bits 2j of qs[32h + l]
//   bytes 80..83  d, dmin (fp16): super-block scale of the scales and of the mins
//   w[e] = d * (scales[e / 16] & 15) * q[e] - dmin * (scales[e / 16] >> 4)
// A row of K weights is K / 256 consecutive blocks; a matrix is N such rows, so
// the tensor data of a GGUF Q2_K tensor is read as it is stored.
//
// GEMV mapping: four lanes per block (lane t of the four takes half h = t / 2 and
// the 16-byte run qs[32h + 16 (t % 2) ..], i.e. 64 weights in four sub-blocks
// j = 0..3), sixteen blocks per wave and pass, R rows per wave sharing each
// activation value held in registers.  The activations are staged once per
// workgroup in LDS with every group of four (e0, e1, e2, e3) stored as the pairs
// (e0, e2), (e1, e3), the order in which a 32-bit word of codes expands: the
// fields of sub-block j sit at bits 2j of bytes 0 and 2 (and of bytes 1 and 3
// after a shift by 8), and OR-ing the fp16 exponent of 64.0 makes the exact halves
// 64 + q 4^j / 16, one AND-OR per pair, consumed by one v_dot2_f32_f16.  Per
// sub-block, sum x w = d sc (16 / 4^j) (acc - 64 S) - dmin m S with S the
// sub-block's activation sum (staged with the activations).  That kernel runs one
// token; two to sixteen tokens per launch run q2k_mfma_kernel, which expands each
// weight's codes once and multiplies the tokens on MFMA.
#include "kernels.h"

namespace {

constexpr int kQ2kBlockBytes = 84;
// Workgroup size of the one-token dot-product kernel.
constexpr int kQ2kThreads = 512;
constexpr int kQ2kMaxK = 16384;
constexpr int kQ2kStageU = 8;  // activation vectors requested per thread and staging round

__device__ __forceinline__ float q2k_src(const void* w, bool fp16, size_t i) {
  return fp16 ? h2f(reinterpret_cast<const f16*>(w)[i]) : reinterpret_cast<const float*>(w)[i];
}

// One wave per (row, block), lane l holding elements 4l .. 4l+3 (sub-block l / 4).
// Round to nearest: per sub-block min m = min(0, min w) and scale (max w - m) / 3;
// d = fp16(max scale / 15), dmin = fp16(max(-m) / 15); 4-bit codes of scale / d and
// -m / dmin rounded to nearest even and clamped to [0, 15]; then the 2-bit codes
// rint((w + dmin mc) / (d sc)) clamped to [0, 3] with the quantized values
// (0 where d sc == 0).  fp32 arithmetic, one rounding per operation.
__global__ void q2k_pack_kernel(const void* __restrict__ w, int src_fp16, int K, uint8_t* __restrict__ out) {
  const int NB = K / 256;
  const long rb = (long)blockIdx.x;
  const int row = (int)(rb / NB), b = (int)(rb % NB);
  const int lane = threadIdx.x;
  const size_t base = (size_t)row * K + 256 * b + 4 * lane;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = q2k_src(w, src_fp16, base + i);
  float mn = fminf(fminf(v[0], v[1]), fminf(v[2], v[3]));
  float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
  for (int o = 1; o < 4; o <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  mn = fminf(mn, 0.f);
  const float sub_scale = __fdiv_rn(sub_rn(mx, mn), 3.f);
  const float sub_min = -mn;
  const float d = h2f(f2h(__fdiv_rn(wave_max(sub_scale), 15.f)));
  const float dmin = h2f(f2h(__fdiv_rn(wave_max(sub_min), 15.f)));
  const float sc = d > 0.f ? fminf(fmaxf(__builtin_rintf(__fdiv_rn(sub_scale, d)), 0.f), 15.f) : 0.f;
  const float mc = dmin > 0.f ? fminf(fmaxf(__builtin_rintf(__fdiv_rn(sub_min, dmin)), 0.f), 15.f) : 0.f;
  const float dl = mul_rn(d, sc), dm = mul_rn(dmin, mc);
  uint32_t codes = 0;  // four 2-bit codes of this lane's elements, element i at bits 2i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float q = dl > 0.f ? __builtin_rintf(__fdiv_rn(add_rn(v[i], dm), dl)) : 0.f;
    q = fminf(fmaxf(q, 0.f), 3.f);
    codes |= (uint32_t)q << (2 * i);
  }
  uint8_t* blk = out + ((size_t)row * NB + b) * kQ2kBlockBytes;
  // qs byte lane (0..63): element 128h + 32j + l of the byte sits in lane (128h + 32j + l) / 4
  const int h = lane >> 5, l = lane & 31;
  uint32_t byte = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 128 * h + 32 * j + l;
    const uint32_t c = (uint32_t)__shfl((int)codes, e >> 2, 64);
    byte |= ((c >> (2 * (e & 3))) & 3u) << (2 * j);
  }
  blk[16 + lane] = (uint8_t)byte;
  if ((lane & 3) == 0) blk[lane >> 2] = (uint8_t)((uint32_t)sc | ((uint32_t)mc << 4));
  if (lane == 0) {
    const f16 dh = f2h(d), mh = f2h(dmin);
    blk[80] = (uint8_t)(h_as_u16(dh) & 0xFF);
    blk[81] = (uint8_t)(h_as_u16(dh) >> 8);
    blk[82] = (uint8_t)(h_as_u16(mh) & 0xFF);
    blk[83] = (uint8_t)(h_as_u16(mh) >> 8);
  }
}

// One thread per element: fp16(d sc q - dmin m) computed in fp32.
__global__ void q2k_dequant_kernel(const uint8_t* __restrict__ wq, int K, long total, f16* __restrict__ out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int NB = K / 256;
  const long row = i / K;
  const int k = (int)(i % K);
  const int b = k >> 8, e = k & 255;
  const uint8_t* blk = wq + ((size_t)row * NB + b) * kQ2kBlockBytes;
  const int h = e >> 7, j = (e >> 5) & 3, l = e & 31;
  const uint32_t q = (blk[16 + 32 * h + l] >> (2 * j)) & 3u;
  const uint32_t s = blk[e >> 4];
  const float d = h2f(u16_as_h((uint16_t)(blk[80] | (blk[81] << 8))));
  const float dmin = h2f(u16_as_h((uint16_t)(blk[82] | (blk[83] << 8))));
  const float dl = mul_rn(d, (float)(s & 15u)), ml = mul_rn(dmin, (float)(s >> 4));
  out[i] = f2h(sub_rn(mul_rn(dl, (float)q), ml));
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
}

// LDS slot of activation quad q (8 staged values, 16 bytes) within its row: bits 4-6
// of q are XORed onto bits 0, 2 and 3.  A GEMV read instruction has lane 4 bs + t
// fetch quad 32 bs + 16 (t / 2) + 2 (t % 2) + c (c the same for every lane), so
// without it the 16 lanes of one LDS cycle hit two 16-byte bank groups (8-way
// conflicts); with it they hit 16 distinct ones.  A bijection on aligned 16-quad
// blocks, so a row's quads stay inside the row.
__device__ __forceinline__ int q2k_lds_quad(int q) {
  const int s = (q >> 4) & 7;
  return q ^ ((s & 1) | ((s & 6) << 1));
}

constexpr int kOOB = 0x7FFFFFF0;  // buffer offset past every descriptor: the load returns zeros

// Stage x ([M][K] fp16, rows contiguous) in LDS in pair order, 8 elements (one quad of
// four pairs) per thread and vector.  MODE 0 (dot-product kernel): quad c of row m at
// xs + m row_dw + 4 q2k_lds_quad(c), and the 16-element sums into ss [M][K / 16].
// MODE 1 (MFMA kernel): quad c at 4 c, no sums.  Rounds of kQ2kStageU vectors per
// thread, all requested before any is used (a loop of one load each waited a full
// round trip per vector: M = 4 at K = 11008 is 22 vectors per thread).  Vectors past
// the end read zeros through a bounded descriptor (no memory traffic).
template <int TH, int MODE>
__device__ __forceinline__ void q2k_stage_x(const f16* x, int M, int K, uint32_t* xs, int row_dw, float* ss,
                                            int tid) {
  const int nvec = M * K / 8;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, nvec * 16, 0x00020000);
  for (int v0 = tid; v0 < nvec; v0 += kQ2kStageU * TH) {
    // Slices u whose first vector (thread 0's) is past the end are skipped by every
    // thread alike (a workgroup-uniform bound).
    const int base = v0 - tid;
    u32x4 av[kQ2kStageU];
#pragma unroll
    for (int u = 0; u < kQ2kStageU; ++u) {
      if (base + u * TH >= nvec) break;
      const int v = v0 + u * TH;  // x rows are contiguous: vector v is x + 8 v
      av[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, v < nvec ? 16 * v : kOOB, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < kQ2kStageU; ++u) {
      if (base + u * TH >= nvec) break;
      // Lanes past the end hold zeros and store nothing.  Vectors c and
      // c ^ 1 of a 16-element sub-block sit in adjacent lanes, and nvec is even, so
      // both lanes of a pair are on the same side of the end.
      const int v = v0 + u * TH;
      const int m = min(v, nvec - 1) / (K / 8), c = min(v, nvec - 1) % (K / 8);
      const u32x4 a = av[u];
      u32x4 p;
      p[0] = (a[0] & 0xFFFFu) | (a[1] << 16);
      p[1] = (a[0] >> 16) | (a[1] & 0xFFFF0000u);
      p[2] = (a[2] & 0xFFFFu) | (a[3] << 16);
      p[3] = (a[2] >> 16) | (a[3] & 0xFFFF0000u);
      float s = 0.f;
      if (MODE == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f16x2 hv = as_h2(a[q]);
          s = add_rn(s, add_rn(h2f(hv.x), h2f(hv.y)));
        }
        s = add_rn(s, dpp_move<0xB1>(s));  // elements 16(c/2) .. +15: the pair (c, c ^ 1)
      }
      if (v < nvec) {
        *reinterpret_cast<u32x4*>(xs + (size_t)m * row_dw + 4 * (MODE == 0 ? q2k_lds_quad(c) : c)) = p;
        if (MODE == 0 && (c & 1) == 0) ss[(size_t)m * (K / 16) + c / 2] = s;
      }
    }
  }
}

// Two to sixteen tokens per launch on MFMA: the codes of each weight are expanded once
// and the tokens are the A rows of v_mfma_f32_16x16x32_f16, so the VALU work per
// weight does not grow with the token count (the dot-product kernel below spends two
// v_dot2_f32_f16 per four weights and token).  A workgroup owns 16 weight rows, the B
// columns: lane l takes row n = l & 15 and block part t = l >> 4 (half h = t / 2 and
// the 16-byte run hx = t % 2 of the codes, as in the dot-product kernel), which is
// also the MFMA k-group of 8 values that the lane supplies.  Its W waves take blocks
// w, w + W, ... and add their partial products through LDS at the end.  Lane l holds
// C rows 4 (l / 16) .. + 3, the tokens of those numbers, for row n.
// The product is exact up to fp32 accumulation, as in the dot-product kernel: B holds
// the integer sc q, made from the exact halves 64 + q 4^j / 16 of the exponent OR by
// one fp16 fma with sc 16 / 4^j and -64 sc 16 / 4^j (both exact), and a second chain
// multiplies the same A by the sub-block's min code m (sum_k x_k m = sum_s m_s S_s);
// the two chains of a block are scaled by its d and dmin in fp32.  The x rows are
// staged with 16 bytes of padding, so the A reads of 16 token rows hit distinct banks.
template <int W>
__global__ void __launch_bounds__(W * 64) q2k_mfma_kernel(const f16* __restrict__ x, int M, int K, int N,
                                                          const uint8_t* __restrict__ wq, size_t w_bytes,
                                                          const f16* __restrict__ bias, f16* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int row_dw = K / 2 + 4;
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem);  // [M][row_dw] pairs
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NB = K / 256;
  const int n = lane & 15, t = lane >> 4, h = t >> 1, hx = t & 1;
  const int row = blockIdx.x * 16 + n;
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)wq, (short)0, (int)w_bytes, 0x00020000);
  u32x4 cw;
  u32x2 sc;
  uint32_t dd;
  auto load = [&](int b) {
    const bool ok = row < N && b < NB;
    const int base = ok ? (row * NB + b) * kQ2kBlockBytes : 0;
    cw = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? base + 16 + 32 * h + 16 * hx : kOOB, 0, 0));
    sc = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, ok ? base + 8 * h : kOOB, 0, 0));
    dd = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? base + 80 : kOOB, 0, 0);
  };
  load(wave);  // the first block's codes before the staging (loads complete in issue order)
  q2k_stage_x<W * 64, 1>(x, M, K, xs, row_dw, nullptr, tid);
  __syncthreads();

  // A row n: token n; rows past M repeat token M - 1 and only reach C rows never stored.
  const uint32_t* xa = xs + (size_t)min(n, M - 1) * row_dw;
  f32x4 tot = {0.f, 0.f, 0.f, 0.f};
  for (int b = wave; b < NB; b += W) {
    const u32x4 c0 = cw;
    const u32x2 s0 = sc;
    const f16x2 dm = as_h2(dd);
    if (b + W < NB) load(b + W);
    const int q0 = 32 * b + 16 * h + 2 * hx;  // quad of element 256 b + 128 h + 16 hx
    f32x4 acc = {0.f, 0.f, 0.f, 0.f}, accm = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // scale byte of sub-block 8 h + 2 j + hx: byte 2 j + hx of the half's eight
      const uint32_t sbyte = (s0[j >> 1] >> (16 * (j & 1) + 8 * hx)) & 0xFFu;
      // sc 16 / 4^j and -64 sc 16 / 4^j, both exact in fp16: (v - 64) sc 16 / 4^j = sc q
      const f16 scf = (f16)((float)(sbyte & 15u) * (16.f / (float)(1 << (2 * j))));
      const f16x2 sv = {scf, scf};
      const f16x2 ov = -(f16x2){(f16)64.f, (f16)64.f} * sv;
      const f16 mf = (f16)(float)(sbyte >> 4);
      const f16x8 Bm = {mf, mf, mf, mf, mf, mf, mf, mf};
      const uint32_t mask = 0x00030003u << (2 * j);
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        // B: words 2 gp and 2 gp + 1 of the run (elements 8 gp .. 8 gp + 7 of sub-block j),
        // in the staged pair order (e0, e2), (e1, e3), (e4, e6), (e5, e7)
        f16x8 B;
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
          const uint32_t cword = c0[2 * gp + gg];
          const f16x2 lo = as_h2((cword & mask) | 0x54005400u);
          const f16x2 hi = as_h2(((cword >> 8) & mask) | 0x54005400u);
          const f16x2 wl = __builtin_elementwise_fma(lo, sv, ov);
          const f16x2 wh = __builtin_elementwise_fma(hi, sv, ov);
          B[4 * gg + 0] = wl.x;
          B[4 * gg + 1] = wl.y;
          B[4 * gg + 2] = wh.x;
          B[4 * gg + 3] = wh.y;
        }
        const f16x8 A = *reinterpret_cast<const f16x8*>(xa + 4 * (q0 + 4 * j + gp));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc, 0, 0, 0);
        accm = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bm, accm, 0, 0, 0);
      }
    }
    const float d = h2f(dm.x), dmin = h2f(dm.y);
#pragma unroll
    for (int i = 0; i < 4; ++i) tot[i] = __builtin_fmaf(d, acc[i], __builtin_fmaf(-dmin, accm[i], tot[i]));
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
    for (int w = 0; w < W; ++w) v = add_rn(v, red[(w * 16 + m) * 16 + nn]);
    const int r = blockIdx.x * 16 + nn;
    if (r < N) {
      if (bias != nullptr) v = add_rn(v, h2f(bias[r]));
      y[(size_t)m * N + r] = f2h(v);
    }
  }
}

// xs: [M][K] fp16 in pair order; ss: [M][K / 16] fp32 sub-block sums.
template <int M, int R, int TH>
__global__ void __launch_bounds__(TH) q2k_gemv_kernel(const f16* __restrict__ x, int K, int N,
                                                              const uint8_t* __restrict__ wq, size_t w_bytes,
                                                              const f16* __restrict__ bias, f16* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* xs = reinterpret_cast<uint32_t*>(smem);            // [M][K / 2] pairs
  float* ss = reinterpret_cast<float*>(xs + (size_t)M * K / 2);  // [M][K / 16]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int NB = K / 256;
  const int row0 = (blockIdx.x * (TH / 64) + wave) * R;
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)wq, (short)0, (int)w_bytes, 0x00020000);
  const int t = lane & 3, bs = lane >> 2;  // sub-lane of the block, block slot
  const int h = t >> 1, hx = t & 1;

  // First pass's weights before the staging (loads complete in issue order).
  u32x4 cw[R];
  u32x2 sc[R];
  uint32_t dd[R];
  auto load = [&](int b) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = row0 + i;
      const bool ok = row < N && b < NB;
      const int base = ok ? (row * NB + b) * kQ2kBlockBytes : kOOB;
      cw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? base + 16 + 32 * h + 16 * hx : kOOB, 0, 0));
      sc[i] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, ok ? base + 8 * h : kOOB, 0, 0));
      dd[i] = __builtin_amdgcn_raw_buffer_load_b32(rw, ok ? base + 80 : kOOB, 0, 0);
    }
  };
  load(bs);

  q2k_stage_x<TH, 0>(x, M, K, xs, K / 2, ss, tid);
  __syncthreads();

  float r[R][M];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) r[i][m] = 0.f;

  const int passes = (NB + 15) / 16;
  for (int p = 0; p < passes; ++p) {
    const int b = 16 * p + bs;
    u32x4 c0[R];
    u32x2 s0[R];
    uint32_t d0[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      c0[i] = cw[i];
      s0[i] = sc[i];
      d0[i] = dd[i];
    }
    if (p + 1 < passes) load(b + 16);
    if (b < NB) {
      // element offset of this lane's run in a block: 128h + 16hx (+ 32j + 4g + {0,1,2,3})
      const int e0 = 256 * b + 128 * h + 16 * hx;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t mask = 0x00030003u << (2 * j);
        u32x4 xp[M][2];
#pragma unroll
        for (int m = 0; m < M; ++m) {
          // quads (e0 + 32 j) / 8 (even) and the next one, which differs in bit 0 only
          const int pq = q2k_lds_quad((e0 + 32 * j) / 8);
          const uint32_t* xr = xs + (size_t)m * K / 2;
          xp[m][0] = *reinterpret_cast<const u32x4*>(xr + 4 * pq);
          xp[m][1] = *reinterpret_cast<const u32x4*>(xr + 4 * (pq ^ 1));
        }
        float sx[M];
#pragma unroll
        for (int m = 0; m < M; ++m) sx[m] = ss[(size_t)m * (K / 16) + (e0 + 32 * j) / 16];
#pragma unroll
        for (int i = 0; i < R; ++i) {
          float acc[M];
#pragma unroll
          for (int m = 0; m < M; ++m) acc[m] = 0.f;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const uint32_t cword = c0[i][g];
            const uint32_t lo = (cword & mask) | 0x54005400u;
            const uint32_t hi = ((cword >> 8) & mask) | 0x54005400u;
#pragma unroll
            for (int m = 0; m < M; ++m) {
              const u32x4& xv = xp[m][g >> 1];
              acc[m] = dot2(xv[2 * (g & 1)], lo, acc[m]);
              acc[m] = dot2(xv[2 * (g & 1) + 1], hi, acc[m]);
            }
          }
          const uint32_t sbyte = ((hx + 2 * j) < 4 ? (s0[i][0] >> (8 * (hx + 2 * j))) : (s0[i][1] >> (8 * (hx + 2 * j - 4)))) & 0xFFu;
          const f16x2 dm = as_h2(d0[i]);
          const float a = h2f(dm.x) * (float)(sbyte & 15u) * (16.f / (float)(1 << (2 * j)));
          const float bm = h2f(dm.y) * (float)(sbyte >> 4);
#pragma unroll
          for (int m = 0; m < M; ++m) r[i][m] += a * (acc[m] - 64.f * sx[m]) - bm * sx[m];
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) r[i][m] = wave_sum_dpp(r[i][m]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = row0 + i;
      if (row >= N) continue;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float v = r[i][m];
        if (bias != nullptr) v = add_rn(v, h2f(bias[row]));
        y[(size_t)m * N + row] = f2h(v);
      }
    }
  }
}

template <int M, int R, int TH>
int q2k_launch_mr(const f16* x, int K, int N, const uint8_t* w, const f16* bias, f16* y, hipStream_t st) {
  const size_t smem = (size_t)M * K * sizeof(f16) + (size_t)M * (K / 16) * sizeof(float);
  if (smem > 160 * 1024) {
    axm_set_error("qmv_q2_k_gguf: K=%d with %d rows needs %zu B of LDS", K, M, smem);
    return -2;
  }
  if (smem > 64 * 1024 && hipFuncSetAttribute((const void*)q2k_gemv_kernel<M, R, TH>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess) {
    (void)hipGetLastError();
    axm_set_error("qmv_q2_k_gguf: cannot reserve %zu B of LDS", smem);
    return -2;
  }
  const int rows = (TH / 64) * R;
  const size_t w_bytes = (size_t)N * (K / 256) * kQ2kBlockBytes;
  hipLaunchKernelGGL((q2k_gemv_kernel<M, R, TH>), dim3((N + rows - 1) / rows), dim3(TH), smem, st, x, K, N, w,
                     w_bytes, bias, y);
  return 0;
}

// LDS bytes of q2k_mfma_kernel for M tokens: padded pair rows, reused at the end for
// the waves' partial sums.
size_t q2k_mfma_smem(int M, int K, int W) {
  const size_t staged = (size_t)M * (K / 2 + 4) * sizeof(uint32_t);
  const size_t partial = (size_t)W * 16 * 16 * sizeof(float);
  return staged > partial ? staged : partial;
}

// Tokens per q2k_mfma_kernel launch at this K: as many as LDS holds, up to 16.
int q2k_mfma_max_tokens(int K) {
  const int m = (int)((size_t)160 * 1024 / ((size_t)(K / 2 + 4) * sizeof(uint32_t)));
  return m < 16 ? m : 16;
}

template <int W>
int q2k_mfma_launch_w(const f16* x, int M, int K, int N, const uint8_t* w, const f16* bias, f16* y, hipStream_t st) {
  const size_t smem = q2k_mfma_smem(M, K, W);
  if (smem > 64 * 1024 && hipFuncSetAttribute((const void*)q2k_mfma_kernel<W>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess) {
    (void)hipGetLastError();
    axm_set_error("qmv_q2_k_gguf: cannot reserve %zu B of LDS", smem);
    return -2;
  }
  const size_t w_bytes = (size_t)N * (K / 256) * kQ2kBlockBytes;
  hipLaunchKernelGGL((q2k_mfma_kernel<W>), dim3((N + 15) / 16), dim3(W * 64), smem, st, x, M, K, N, w, w_bytes, bias,
                     y);
  return 0;
}

// Several tokens: the MFMA kernel with four waves per 16-row workgroup while the grid
// holds two workgroups per CU, else sixteen (C4 shapes at four tokens: 4096 -> 11008
// 11.3 us with four waves, 11.4 with eight, 12.2 with sixteen; 11008 -> 4096, 256
// workgroups, 10.7 with four or eight, 10.3 with sixteen).  One token stays on the
// dot-product kernel (the MFMA form: 8.7 / 8.0 against 8.4 / 7.8 us).
int q2k_mfma_launch(const f16* x, int M, int K, int N, const uint8_t* w, const f16* bias, f16* y, hipStream_t st) {
  const long groups = (N + 15) / 16;
  if (groups >= 2L * axm_num_cus()) return q2k_mfma_launch_w<4>(x, M, K, N, w, bias, y, st);
  return q2k_mfma_launch_w<16>(x, M, K, N, w, bias, y, st);
}

// One token: the dot-product kernel with two rows per wave while the grid keeps at
// least one workgroup per CU (measured best at the C4 shapes: 8.1 / 8.4 us against
// 9.9 / 8.4 with four), else one.
int q2k_launch1(const f16* x, int K, int N, const uint8_t* w, const f16* bias, f16* y, hipStream_t st) {
  constexpr int W = kQ2kThreads / 64;
  if ((N + 2 * W - 1) / (2 * W) >= axm_num_cus()) return q2k_launch_mr<1, 2, kQ2kThreads>(x, K, N, w, bias, y, st);
  return q2k_launch_mr<1, 1, kQ2kThreads>(x, K, N, w, bias, y, st);
}

}  // namespace

extern "C" int axm_pack_q2_k_gguf(const void* w, int src_is_fp16, int N, int K, void* blocks, void* stream) {
  AXM_CHECK_ARG(w && blocks && N > 0 && K > 0 && K % 256 == 0, -1, "pack_q2_k_gguf: bad arguments N=%d K=%d", N, K);
  hipLaunchKernelGGL(q2k_pack_kernel, dim3((unsigned)((long)N * (K / 256))), dim3(64), 0, (hipStream_t)stream, w,
                     src_is_fp16, K, (uint8_t*)blocks);
  AXM_LAUNCH_CHECK("pack_q2_k_gguf");
  return 0;
}

extern "C" int axm_dequantize_q2_k_gguf(const void* blocks, int N, int K, void* out, void* stream) {
  AXM_CHECK_ARG(blocks && out && N > 0 && K > 0 && K % 256 == 0, -1, "dequantize_q2_k_gguf: bad arguments");
  const long total = (long)N * K;
  hipLaunchKernelGGL(q2k_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t*)blocks, K, total, (f16*)out);
  AXM_LAUNCH_CHECK("dequantize_q2_k_gguf");
  return 0;
}

extern "C" int axm_qmv_q2_k_gguf(const void* x, const void* blocks, const void* bias, void* y, int M, int K, int N,
                                 void* stream) {
  AXM_CHECK_ARG(x && blocks && y, -1, "qmv_q2_k_gguf: null pointer");
  AXM_CHECK_ARG(M >= 1 && N >= 1 && K >= 256 && K % 256 == 0 && K <= kQ2kMaxK, -1,
                "qmv_q2_k_gguf: bad shape M=%d K=%d N=%d (K %% 256 == 0, K <= %d)", M, K, N, kQ2kMaxK);
  AXM_CHECK_ARG((size_t)N * (K / 256) * kQ2kBlockBytes < (size_t)0x7FFFFFF0, -1,
                "qmv_q2_k_gguf: weight tensor above 2 GiB");
  hipStream_t st = (hipStream_t)stream;
  // MFMA launches of up to q2k_mfma_max_tokens(K) tokens (16 at K <= 4096, 4 at the
  // largest K) while at least two remain, the dot-product kernel for a single token.
  const int mt = q2k_mfma_max_tokens(K);
  int m0 = 0;
  while (m0 < M) {
    const int left = M - m0;
    const int mc = left < 2 ? 1 : (left < mt ? left : mt);
    const f16* xm = (const f16*)x + (size_t)m0 * K;
    f16* ym = (f16*)y + (size_t)m0 * N;
    const int rc = mc == 1 ? q2k_launch1(xm, K, N, (const uint8_t*)blocks, (const f16*)bias, ym, st)
                           : q2k_mfma_launch(xm, mc, K, N, (const uint8_t*)blocks, (const f16*)bias, ym, st);
    if (rc) return rc;
    m0 += mc;
  }
  AXM_LAUNCH_CHECK("qmv_q2_k_gguf");
  return 0;
}
