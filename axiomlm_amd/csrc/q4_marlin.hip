// MARLIN-interleaved Q4 (group 64, fp16 scale + fp16 bias) kernels for gfx950.
//
// Weight format (the reference's packed layout, axiomlm/kernels/quant.py:447-594):
//   w_marlin  [n_tiles][KG][32 lanes][2 words]  u32,  n_tiles = ceil(N/8), KG = K/64
//   sb_marlin [n_tiles][KG][8 rows][2]          f16  (scale, bias)
// Lane l of an 8-row tile, word j, nibble s (bits 4s and 16+4s) holds the code of
//   row c0 = ((l&8)>>1)|((l&1)<<1) (low half) / c0+1 (high half) at
//   column k = 64g + 32j + 8s + r,  r = ((l&16)>>2)|((l&6)>>1).
//
// GEMV mapping on CDNA4: one dwordx4 per lane covers the 16-byte pair of
// reference lanes (2m, 2m+1); a wave64 therefore streams 1 KB = four
// consecutive 64-column groups of one tile per load, fully coalesced.  Lane
// (gs = l>>4, m = l&15) owns rows cb..cb+3 (cb = m&4) and columns
// {64g + 32j + 8s + r} with r = ((m&8)>>1)|(m&3).
//
// Codes are expanded with the fp16 magic-exponent trick ((w & 0x000F000F) |
// 0x64006400 = 1024+q, (w & 0x00F000F0) | 0x54005400 = 64+q) and consumed by
// mixed-precision FMAs (fp16 code x fp32 activation -> fp32 accumulator); the
// magic offsets are removed once per (group, lane) with a precomputed
// correction sum, so each weight costs one FMA plus half an AND-OR.
#include "axm_common.h"
#include "q4_marlin.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / AXM_WAVE;

// ---------------------------------------------------------------------------
// LDS staging of activations in the lane-permuted order.
//   xh  : f16  [KG*8 (g,r)][8] = x[64g + 32j + 8s + r] at slot j*4+s
//   cx  : f32x2[KG*8]          = (1024*(s even) + 64*(s odd) weighted sum, plain sum)
// ---------------------------------------------------------------------------
struct XStage {
  f16* xh;
  f32x2* cx;
};


template <int M>
__device__ void stage_x(const Q4GemvArgs& a, XStage* st, float* red) {
  const int tid = threadIdx.x;
  const int K = a.K;
  float rinv[M];
  if (a.ln_w != nullptr) {
    // Pass 1: sum of fp16-rounded squares per token.
    for (int mi = 0; mi < M; ++mi) {
      const f16* xr = a.x + (size_t)mi * a.ldx;
      float s = 0.f;
      for (int k = tid; k < K; k += kThreads) {
        float v = h2f(xr[k]);
        s += h2f(f2h(v * v));
      }
      s = wave_sum(s);
      if ((tid & 63) == 0) red[mi * kWaves + (tid >> 6)] = s;
    }
    __syncthreads();
    for (int mi = 0; mi < M; ++mi) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += red[mi * kWaves + w];
      rinv[mi] = rms_inv_fp16(s, K, a.eps);
    }
    __syncthreads();
  }
  const int n_gr = a.KG * 8;
  for (int mi = 0; mi < M; ++mi) {
    const f16* xr = a.x + (size_t)mi * a.ldx;
    for (int p = tid; p < n_gr; p += kThreads) {
      const int g = p >> 3, r = p & 7;
      f16x8 v;
      float corr = 0.f, sum = 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int k = 64 * g + 32 * j + 8 * s + r;
          f16 h = xr[k];
          if (a.ln_w != nullptr) {
            f16 t = f2h(h2f(h) * rinv[mi]);
            h = f2h(h2f(t) * h2f(a.ln_w[k]));
          }
          v[j * 4 + s] = h;
          float f = h2f(h);
          sum += f;
          corr += f * ((s & 1) ? 64.f : 1024.f);
        }
      }
      *reinterpret_cast<f16x8*>(st[mi].xh + (size_t)p * 8) = v;
      st[mi].cx[p] = f32x2{corr, sum};
      if (a.x_norm_out != nullptr) {
        // Optional export of the normalized activations (row-major).
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int s = 0; s < 4; ++s)
            a.x_norm_out[(size_t)mi * K + 64 * g + 32 * j + 8 * s + r] = v[j * 4 + s];
      }
    }
  }
  __syncthreads();
}

// Accumulate one 64-column group for the lane's 4 rows.
// wv = (A, B, C, D) words: A/B rows cb,cb+1 (j=0/1), C/D rows cb+2,cb+3.
__device__ __forceinline__ void q4_group_fma(u32x4 wv, u32x4 sv, f16x8 xv, f32x2 cx, float acc[4]) {
  float d[4] = {0.f, 0.f, 0.f, 0.f};
  const uint32_t words[4] = {wv[0], wv[1], wv[2], wv[3]};
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
    const uint32_t w = words[wi];
    const int j = wi & 1;         // k half
    const int rp = (wi >> 1) * 2; // row pair offset 0 or 2
    const uint32_t w8 = w >> 8;
    f16x2 h0 = as_h2((w & 0x000F000Fu) | 0x64006400u);
    f16x2 h1 = as_h2((w & 0x00F000F0u) | 0x54005400u);
    f16x2 h2 = as_h2((w8 & 0x000F000Fu) | 0x64006400u);
    f16x2 h3 = as_h2((w8 & 0x00F000F0u) | 0x54005400u);
    const float x0 = h2f(xv[j * 4 + 0]), x1 = h2f(xv[j * 4 + 1]);
    const float x2 = h2f(xv[j * 4 + 2]), x3 = h2f(xv[j * 4 + 3]);
    d[rp] = __builtin_fmaf(h2f(h0.x), x0, d[rp]);
    d[rp] = __builtin_fmaf(h2f(h1.x), x1, d[rp]);
    d[rp] = __builtin_fmaf(h2f(h2.x), x2, d[rp]);
    d[rp] = __builtin_fmaf(h2f(h3.x), x3, d[rp]);
    d[rp + 1] = __builtin_fmaf(h2f(h0.y), x0, d[rp + 1]);
    d[rp + 1] = __builtin_fmaf(h2f(h1.y), x1, d[rp + 1]);
    d[rp + 1] = __builtin_fmaf(h2f(h2.y), x2, d[rp + 1]);
    d[rp + 1] = __builtin_fmaf(h2f(h3.y), x3, d[rp + 1]);
  }
  const uint32_t sbw[4] = {sv[0], sv[1], sv[2], sv[3]};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f16x2 sb = as_h2(sbw[i]);
    acc[i] = __builtin_fmaf(h2f(sb.x), d[i] - cx.x, acc[i]);
    acc[i] = __builtin_fmaf(h2f(sb.y), cx.y, acc[i]);
  }
}

// Reduce the 4 row partials of every lane over the 32 lanes that share cb.
// Returns, in lane L, the full sum for tile row  (L&4) + 2*(L&1) + ((L>>1)&1).
__device__ __forceinline__ float wave_reduce_rows(const float v[4], int lane) {
  const bool b0 = lane & 1, b1 = lane & 2;
  float s0 = b0 ? v[0] : v[2], s1 = b0 ? v[1] : v[3];
  float k0 = b0 ? v[2] : v[0], k1 = b0 ? v[3] : v[1];
  k0 += __shfl_xor(s0, 1, 64);
  k1 += __shfl_xor(s1, 1, 64);
  float send = b1 ? k0 : k1;
  float keep = b1 ? k1 : k0;
  keep += __shfl_xor(send, 2, 64);
  keep += __shfl_xor(keep, 8, 64);
  keep += __shfl_xor(keep, 16, 64);
  keep += __shfl_xor(keep, 32, 64);
  return keep;
}
__device__ __forceinline__ int reduced_row_of_lane(int lane) {
  return (lane & 4) + 2 * (lane & 1) + ((lane >> 1) & 1);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// Main GEMV kernel.  NT = tiles per work unit (2 for the SwiGLU gate/up pair).
// ---------------------------------------------------------------------------
template <int M, int NT, int EPI>
__global__ void __launch_bounds__(kThreads) q4m_gemv_kernel(Q4GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  // Layout: [M] xh (K halves) | [M] cx (K/8 float2) | red (kWaves*NT*M*8 f32) | fin (NT*M*8 f32)
  XStage st[M];
  unsigned char* p = smem;
  for (int mi = 0; mi < M; ++mi) {
    st[mi].xh = reinterpret_cast<f16*>(p);
    p += (size_t)a.K * sizeof(f16);
  }
  for (int mi = 0; mi < M; ++mi) {
    st[mi].cx = reinterpret_cast<f32x2*>(p);
    p += (size_t)(a.K / 8) * sizeof(f32x2);
  }
  float* red = reinterpret_cast<float*>(p);
  float* fin = red + kWaves * NT * M * 8;

  stage_x<M>(a, st, red);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int gs = lane >> 4;
  const int m = lane & 15;
  const int r = ((m & 8) >> 1) | (m & 3);
  const int cb = m & 4;
  const int n_chunks = (a.KG + 3) >> 2;
  const u32x4* __restrict__ w4 = a.w;
  const u32x4* __restrict__ sb4 = a.sb;

  for (int unit = blockIdx.x; unit < a.n_units; unit += gridDim.x) {
    int tiles[NT];
    tiles[0] = unit;
    if (NT == 2) tiles[NT - 1] = unit + a.pair_offset;
    float acc[NT][M][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mi = 0; mi < M; ++mi)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][mi][i] = 0.f;

    constexpr int U = (NT == 2) ? 2 : 4;  // chunks in flight per wave
    for (int c0 = wave; c0 < n_chunks; c0 += kWaves * U) {
      u32x4 wv[U][NT], sv[U][NT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * kWaves;
        const int g = c * 4 + gs;
        const bool ok = (c < n_chunks) && (g < a.KG);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const size_t base = (size_t)tiles[t] * a.KG + g;
          wv[u][t] = ok ? __builtin_nontemporal_load(w4 + base * 16 + m) : u32x4{0u, 0u, 0u, 0u};
          sv[u][t] = ok ? sb4[base * 2 + (cb >> 2)] : u32x4{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * kWaves;
        const int g = c * 4 + gs;
        if (c < n_chunks && g < a.KG) {
          const int pidx = g * 8 + r;
#pragma unroll
          for (int mi = 0; mi < M; ++mi) {
            const f16x8 xv = *reinterpret_cast<const f16x8*>(st[mi].xh + (size_t)pidx * 8);
            const f32x2 cx = st[mi].cx[pidx];
#pragma unroll
            for (int t = 0; t < NT; ++t) q4_group_fma(wv[u][t], sv[u][t], xv, cx, acc[t][mi]);
          }
        }
      }
    }

    // Wave reduction then cross-wave reduction through LDS.
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mi = 0; mi < M; ++mi) {
        float v = wave_reduce_rows(acc[t][mi], lane);
        if (lane < 8) red[((wave * NT + t) * M + mi) * 8 + reduced_row_of_lane(lane)] = v;
      }
    __syncthreads();
    if (tid < NT * M * 8) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += red[w * NT * M * 8 + tid];
      fin[tid] = s;
    }
    __syncthreads();

    if (EPI == Q4_EPI_STORE || EPI == Q4_EPI_RESID) {
      if (tid < M * 8) {
        const int mi = tid >> 3, row = tiles[0] * 8 + (tid & 7);
        if (row < a.N) {
          float v = fin[tid];
          f16 h = f2h(v);
          if (a.bias != nullptr) h = f2h(h2f(h) + h2f(a.bias[row]));
          if (EPI == Q4_EPI_STORE) {
            a.y[(size_t)mi * a.ldy + row] = h;
          } else {
            f16* xr = a.resid + (size_t)mi * a.ldr + row;
            *xr = f2h(h2f(*xr) + h2f(h));
          }
        }
      }
    } else if (EPI == Q4_EPI_SWIGLU) {
      // fin layout [t][mi][8]; t=0 gate rows, t=1 up rows.  Torch-CPU fp16
      // semantics: gu rounded to fp16, silu(g) rounded, product rounded.
      if (tid < M * 8) {
        const int mi = tid >> 3, row = tiles[0] * 8 + (tid & 7);
        if (row < a.N) {
          f16 g = f2h(fin[(0 * M + mi) * 8 + (tid & 7)]);
          f16 u = f2h(fin[(1 * M + mi) * 8 + (tid & 7)]);
          f16 sg = f2h(silu_f(h2f(g)));
          a.y[(size_t)mi * a.ldy + row] = f2h(h2f(sg) * h2f(u));
        }
      }
    } else if (EPI == Q4_EPI_QKV_ROPE) {
      // Rows [0, q_dim): rotated q -> y;  [q_dim, q_dim+kv_dim): rotated k ->
      // k_out slot;  [q_dim+kv_dim, N): v -> v_out slot.  Pairs (2i, 2i+1)
      // share a tile, so each thread owns one pair.
      if (tid < M * 4) {
        const int mi = tid >> 2, pr = tid & 3;
        const int row0 = tiles[0] * 8 + 2 * pr;
        if (row0 < a.N) {
          f16 h0 = f2h(fin[mi * 8 + 2 * pr]);
          f16 h1 = f2h(fin[mi * 8 + 2 * pr + 1]);
          if (a.bias != nullptr) {
            h0 = f2h(h2f(h0) + h2f(a.bias[row0]));
            h1 = f2h(h2f(h1) + h2f(a.bias[row0 + 1]));
          }
          const int hd = a.head_dim, half_hd = hd >> 1;
          const int pos_mi = a.rope_pos_dev ? a.rope_pos_dev[0] + mi : a.rope_pos + mi;
          if (row0 < a.q_dim + a.kv_dim) {
            const int within = row0 < a.q_dim ? row0 : row0 - a.q_dim;
            const int fi = (within % hd) >> 1;
            const int rp = pos_mi % a.rope_len;
            const float c = a.freqs[((size_t)rp * half_hd + fi) * 2 + 0];
            const float sn = a.freqs[((size_t)rp * half_hd + fi) * 2 + 1];
            const float x0 = h2f(h0), x1 = h2f(h1);
            h0 = f2h(x0 * c - x1 * sn);
            h1 = f2h(x0 * sn + x1 * c);
          }
          if (row0 < a.q_dim) {
            a.y[(size_t)mi * a.ldy + row0] = h0;
            a.y[(size_t)mi * a.ldy + row0 + 1] = h1;
          } else {
            const bool is_k = row0 < a.q_dim + a.kv_dim;
            const int within = is_k ? row0 - a.q_dim : row0 - a.q_dim - a.kv_dim;
            const int kvh = within / hd, e = within % hd;
            const int wp = a.write_pos_dev ? a.write_pos_dev[0] + mi : a.write_pos + mi;
            f16* dst = (is_k ? a.k_out : a.v_out) + ((size_t)kvh * a.kv_stride_h + (size_t)(wp % a.max_seq) * hd + e);
            dst[0] = h0;
            dst[1] = h1;
          }
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Dequantization (row-major fp16 output), fp32 math then one fp16 rounding,
// quant.py:597-634.
// ---------------------------------------------------------------------------
__global__ void q4m_dequant_kernel(const uint32_t* __restrict__ w, const f16x2* __restrict__ sb,
                                   f16* __restrict__ out, int n_tiles, int KG, int N) {
  // One thread per (tile, g, ref lane); writes 16 values.
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)n_tiles * KG * 32;
  if (idx >= total) return;
  const int l = (int)(idx & 31);
  const long tg = idx >> 5;
  const int g = (int)(tg % KG);
  const int tile = (int)(tg / KG);
  const int r = ((l & 16) >> 2) | ((l & 6) >> 1);
  const int c0 = ((l & 8) >> 1) | ((l & 1) << 1);
  const int K = KG * 64;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t word = w[idx * 2 + j];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int row = tile * 8 + c0 + half;
      if (row >= N) continue;
      const f16x2 s_b = sb[((size_t)tile * KG + g) * 8 + c0 + half];
      const float sc = h2f(s_b.x), bi = h2f(s_b.y);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t q = (word >> (16 * half + 4 * s)) & 0xFu;
        out[(size_t)row * K + 64 * g + 32 * j + 8 * s + r] = f2h(__fadd_rn(__fmul_rn((float)q, sc), bi));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Round-to-nearest packer, quant.py:482-494 + the lane interleave :573-593.
// One 64-thread block per (tile, group).  SRC_FP16 selects torch's fp16 op
// semantics for (max - min) and the /15 (each rounded to fp16).
// ---------------------------------------------------------------------------
template <bool SRC_FP16>
__global__ void __launch_bounds__(64) q4m_pack_rtn_kernel(const void* __restrict__ wsrc, int N, int K,
                                                          uint32_t* __restrict__ w_out, f16x2* __restrict__ sb_out) {
  const int KG = K / 64;
  const int tile = blockIdx.x / KG;
  const int g = blockIdx.x % KG;
  const int t = threadIdx.x;
  const int c = t >> 3;     // row within tile
  const int sub = t & 7;    // 8-element slice
  const int row = tile * 8 + c;
  __shared__ uint8_t qs[8][64];
  float vals[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = 64 * g + 8 * sub + i;
    if (row < N) {
      vals[i] = SRC_FP16 ? h2f(reinterpret_cast<const f16*>(wsrc)[(size_t)row * K + k])
                         : reinterpret_cast<const float*>(wsrc)[(size_t)row * K + k];
    } else {
      vals[i] = 0.f;  // zero-padded rows (quant.py:474-478)
    }
  }
  float mn = vals[0], mx = vals[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    mn = fminf(mn, vals[i]);
    mx = fmaxf(mx, vals[i]);
  }
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  float denom;
  f16 sc_h;
  if (SRC_FP16) {
    f16 d = f2h(__fsub_rn(mx, mn));  // fp16 subtraction; clamp(min=1e-8) is a no-op in fp16
    denom = h2f(d);
    sc_h = f2h(__fdiv_rn(denom, 15.0f));
  } else {
    denom = fmaxf(__fsub_rn(mx, mn), 1e-8f);
    sc_h = f2h(__fdiv_rn(denom, 15.0f));
  }
  const f16 bi_h = f2h(mn);
  const float scf = fmaxf(h2f(sc_h), 1e-8f);
  const float bif = h2f(bi_h);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float q = __builtin_rintf(__fdiv_rn(__fsub_rn(vals[i], bif), scf));
    q = fminf(fmaxf(q, 0.f), 15.f);
    qs[c][8 * sub + i] = (uint8_t)q;
  }
  if (sub == 0) sb_out[((size_t)tile * KG + g) * 8 + c] = f16x2{sc_h, bi_h};
  __syncthreads();
  if (t < 32) {
    const int l = t;
    const int r = ((l & 16) >> 2) | ((l & 6) >> 1);
    const int c0 = ((l & 8) >> 1) | ((l & 1) << 1);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t word = 0;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int kk = 32 * j + 8 * s + r;
        word |= (uint32_t)qs[c0][kk] << (4 * s);
        word |= (uint32_t)qs[c0 + 1][kk] << (16 + 4 * s);
      }
      w_out[(((size_t)tile * KG + g) * 32 + l) * 2 + j] = word;
    }
  }
}


// ---------------------------------------------------------------------------
// Importance-weighted MSE clip search, quant.py:495-571.  One 8-wave block per
// (tile, group): wave c searches row 8*tile+c, lane = column within the group.
// All fp32 ops are explicitly rounded (no contraction) in the reference's op
// order; only the 64-term error sums use a different (tree) summation order.
// alphas: the fp32 values of torch.linspace(1.0, min_shrink, steps).
// ---------------------------------------------------------------------------
template <bool SRC_FP16>
__global__ void __launch_bounds__(512) q4m_pack_mse_kernel(const void* __restrict__ wsrc, int N, int K,
                                                           const float* __restrict__ col_imp,
                                                           const float* __restrict__ alphas, int n_alpha,
                                                           uint32_t* __restrict__ w_out, f16x2* __restrict__ sb_out) {
  const int KG = K / 64;
  const int tile = blockIdx.x / KG;
  const int g = blockIdx.x % KG;
  const int c = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = tile * 8 + c;
  const int k = 64 * g + lane;
  __shared__ uint8_t qs[8][64];
  float w = 0.f;
  if (row < N) w = SRC_FP16 ? h2f(reinterpret_cast<const f16*>(wsrc)[(size_t)row * K + k])
                            : reinterpret_cast<const float*>(wsrc)[(size_t)row * K + k];
  float ig = 1.f;
  const bool has_ig = col_imp != nullptr;
  if (has_ig) {
    const float imp = col_imp[k];
    const float ig2 = __fmul_rn(imp, imp);
    const float mean = __fdiv_rn(wave_sum(ig2), 64.f);
    ig = __fdiv_rn(ig2, fmaxf(mean, 1e-8f));
  }
  const float mn0 = -wave_max(-w);
  const float mx0 = wave_max(w);
  const float mu = __fdiv_rn(wave_sum(has_ig ? __fmul_rn(w, ig) : w), 64.f);

  auto err_of = [&](float sc, float bi) {
    float q = __builtin_rintf(__fdiv_rn(__fsub_rn(w, bi), fmaxf(sc, 1e-8f)));
    q = fminf(fmaxf(q, 0.f), 15.f);
    const float diff = __fsub_rn(w, __fadd_rn(__fmul_rn(q, sc), bi));
    const float e = __fmul_rn(diff, diff);
    return wave_sum(has_ig ? __fmul_rn(ig, e) : e);
  };

  float best = INFINITY;
  float cur_mn = mn0;
  for (int i = 0; i < n_alpha; ++i) {
    const float a = alphas[i];
    const float cand_mn = __fadd_rn(mu, __fmul_rn(a, __fsub_rn(mn0, mu)));
    const float sc = h2f(f2h(__fdiv_rn(fmaxf(__fsub_rn(mx0, cand_mn), 1e-8f), 15.f)));
    const float bi = h2f(f2h(cand_mn));
    const float e = err_of(sc, bi);
    if (e < best) {
      best = e;
      cur_mn = cand_mn;
    }
  }
  best = INFINITY;
  f16 best_sc = f2h(__fdiv_rn(fmaxf(__fsub_rn(mx0, cur_mn), 1e-8f), 15.f));
  f16 best_bi = f2h(cur_mn);
  for (int i = 0; i < n_alpha; ++i) {
    const float a = alphas[i];
    const float cand_mx = __fadd_rn(mu, __fmul_rn(a, __fsub_rn(mx0, mu)));
    const f16 sc_h = f2h(__fdiv_rn(fmaxf(__fsub_rn(cand_mx, cur_mn), 1e-8f), 15.f));
    const f16 bi_h = f2h(cur_mn);
    const float e = err_of(h2f(sc_h), h2f(bi_h));
    if (e < best) {
      best = e;
      best_sc = sc_h;
      best_bi = bi_h;
    }
  }
  float q = __builtin_rintf(__fdiv_rn(__fsub_rn(w, h2f(best_bi)), fmaxf(h2f(best_sc), 1e-8f)));
  q = fminf(fmaxf(q, 0.f), 15.f);
  qs[c][lane] = (uint8_t)q;
  if (lane == 0) sb_out[((size_t)tile * KG + g) * 8 + c] = f16x2{best_sc, best_bi};
  __syncthreads();
  if (threadIdx.x < 32) {
    const int l = threadIdx.x;
    const int r = ((l & 16) >> 2) | ((l & 6) >> 1);
    const int c0 = ((l & 8) >> 1) | ((l & 1) << 1);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t word = 0;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int kk = 32 * j + 8 * s + r;
        word |= (uint32_t)qs[c0][kk] << (4 * s);
        word |= (uint32_t)qs[c0 + 1][kk] << (16 + 4 * s);
      }
      w_out[(((size_t)tile * KG + g) * 32 + l) * 2 + j] = word;
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
size_t q4m_gemv_smem_bytes(int M, int NT, int K) {
  return (size_t)M * K * sizeof(f16) + (size_t)M * (K / 8) * sizeof(f32x2) +
         (size_t)kWaves * NT * M * 8 * sizeof(float) + (size_t)NT * M * 8 * sizeof(float);
}

template <int M, int NT, int EPI>
static void set_attr_one() {
  if (hipFuncSetAttribute((const void*)q4m_gemv_kernel<M, NT, EPI>, hipFuncAttributeMaxDynamicSharedMemorySize,
                          160 * 1024) != hipSuccess)
    (void)hipGetLastError();  // keep the sticky error slot clean; launches re-check sizes
}

// Raise the dynamic-LDS limit of every GEMV instantiation once per process
// (must happen before any stream capture).
void q4m_prepare_attributes() {
  static bool done = false;
  if (done) return;
  done = true;
#define AXM_Q4_ATTR(MM)                      \
  set_attr_one<MM, 1, Q4_EPI_STORE>();       \
  set_attr_one<MM, 1, Q4_EPI_RESID>();       \
  set_attr_one<MM, 2, Q4_EPI_SWIGLU>();      \
  set_attr_one<MM, 1, Q4_EPI_QKV_ROPE>();
  AXM_Q4_ATTR(1)
  AXM_Q4_ATTR(2)
  AXM_Q4_ATTR(3)
  AXM_Q4_ATTR(4)
#undef AXM_Q4_ATTR
}

template <int M, int NT, int EPI>
static int launch_one(const Q4GemvArgs& a, int grid, hipStream_t s) {
  const size_t smem = q4m_gemv_smem_bytes(M, NT, a.K);
  hipLaunchKernelGGL((q4m_gemv_kernel<M, NT, EPI>), dim3(grid), dim3(kThreads), smem, s, a);
  return 0;
}

int q4m_gemv_launch(const Q4GemvArgs& a, int M, int epi, int grid, hipStream_t s) {
  q4m_prepare_attributes();
  const int NT = (epi == Q4_EPI_SWIGLU) ? 2 : 1;
  if (q4m_gemv_smem_bytes(M, NT, a.K) > 160 * 1024) {
    axm_set_error("q4 gemv: K=%d with M=%d needs %zu B of LDS (> 160 KiB)", a.K, M, q4m_gemv_smem_bytes(M, NT, a.K));
    return -2;
  }
#define AXM_Q4_CASE(MM)                                                              \
  case MM:                                                                           \
    switch (epi) {                                                                   \
      case Q4_EPI_STORE: return launch_one<MM, 1, Q4_EPI_STORE>(a, grid, s);         \
      case Q4_EPI_RESID: return launch_one<MM, 1, Q4_EPI_RESID>(a, grid, s);         \
      case Q4_EPI_SWIGLU: return launch_one<MM, 2, Q4_EPI_SWIGLU>(a, grid, s);       \
      case Q4_EPI_QKV_ROPE: return launch_one<MM, 1, Q4_EPI_QKV_ROPE>(a, grid, s);   \
    }                                                                                \
    break;
  switch (M) {
    AXM_Q4_CASE(1)
    AXM_Q4_CASE(2)
    AXM_Q4_CASE(3)
    AXM_Q4_CASE(4)
  }
#undef AXM_Q4_CASE
  axm_set_error("q4 gemv: unsupported M=%d / epilogue=%d", M, epi);
  return -2;
}

int q4m_default_grid(int n_units) {
  const int cap = axm_num_cus() * 4;
  return n_units < cap ? n_units : cap;
}

extern "C" int axm_qmv_q4_marlin(const void* x, const void* w_marlin, const void* sb_marlin, const void* bias,
                                 void* y, int M, int K, int N, void* stream) {
  AXM_CHECK_ARG(x && w_marlin && sb_marlin && y, -1, "qmv_q4_marlin: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0, -1, "qmv_q4_marlin: K=%d must be a positive multiple of 64", K);
  AXM_CHECK_ARG(N > 0 && M >= 1, -1, "qmv_q4_marlin: bad shape M=%d N=%d", M, N);
  hipStream_t s = (hipStream_t)stream;
  const int n_tiles = (N + 7) / 8;
  for (int m0 = 0; m0 < M; m0 += 4) {
    const int mc = (M - m0) < 4 ? (M - m0) : 4;
    // Tokens that do not fit the LDS budget are processed one at a time.
    int mstep = mc;
    while (mstep > 1 && q4m_gemv_smem_bytes(mstep, 1, K) > 160 * 1024) --mstep;
    for (int mm = m0; mm < m0 + mc; mm += mstep) {
      const int cnt = (m0 + mc - mm) < mstep ? (m0 + mc - mm) : mstep;
      Q4GemvArgs a{};
      a.x = (const f16*)x + (size_t)mm * K;
      a.ldx = K;
      a.w = (const u32x4*)w_marlin;
      a.sb = (const u32x4*)sb_marlin;
      a.K = K;
      a.KG = K / 64;
      a.N = N;
      a.n_units = n_tiles;
      a.y = (f16*)y + (size_t)mm * N;
      a.ldy = N;
      a.bias = (const f16*)bias;
      int rc = q4m_gemv_launch(a, cnt, Q4_EPI_STORE, q4m_default_grid(n_tiles), s);
      if (rc) return rc;
    }
  }
  AXM_LAUNCH_CHECK("qmv_q4_marlin");
  return 0;
}

extern "C" int axm_dequantize_q4_marlin(const void* w_marlin, const void* sb_marlin, void* out, int K, int N,
                                        void* stream) {
  AXM_CHECK_ARG(w_marlin && sb_marlin && out, -1, "dequantize_q4_marlin: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0, -1, "dequantize_q4_marlin: bad shape K=%d N=%d", K, N);
  const int n_tiles = (N + 7) / 8, KG = K / 64;
  const long total = (long)n_tiles * KG * 32;
  hipLaunchKernelGGL(q4m_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)w_marlin, (const f16x2*)sb_marlin, (f16*)out, n_tiles, KG, N);
  AXM_LAUNCH_CHECK("dequantize_q4_marlin");
  return 0;
}

extern "C" int axm_pack_q4_marlin_rtn(const void* w, int src_is_fp16, int N, int K, void* w_marlin, void* sb_marlin,
                                      void* stream) {
  AXM_CHECK_ARG(w && w_marlin && sb_marlin, -1, "pack_q4_marlin: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0, -1, "pack_q4_marlin: K=%d must be a multiple of 64", K);
  const int n_tiles = (N + 7) / 8, KG = K / 64;
  const unsigned blocks = (unsigned)n_tiles * KG;
  if (src_is_fp16)
    hipLaunchKernelGGL(q4m_pack_rtn_kernel<true>, dim3(blocks), dim3(64), 0, (hipStream_t)stream, w, N, K,
                       (uint32_t*)w_marlin, (f16x2*)sb_marlin);
  else
    hipLaunchKernelGGL(q4m_pack_rtn_kernel<false>, dim3(blocks), dim3(64), 0, (hipStream_t)stream, w, N, K,
                       (uint32_t*)w_marlin, (f16x2*)sb_marlin);
  AXM_LAUNCH_CHECK("pack_q4_marlin_rtn");
  return 0;
}

extern "C" int axm_pack_q4_marlin_mse(const void* w, int src_is_fp16, int N, int K, const float* col_importance,
                                      const float* alphas, int n_alpha, void* w_marlin, void* sb_marlin,
                                      void* stream) {
  AXM_CHECK_ARG(w && w_marlin && sb_marlin && alphas, -1, "pack_q4_marlin_mse: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0, -1, "pack_q4_marlin_mse: K=%d must be a multiple of 64", K);
  AXM_CHECK_ARG(n_alpha >= 1 && n_alpha <= 1024, -1, "pack_q4_marlin_mse: bad grid size %d", n_alpha);
  const int n_tiles = (N + 7) / 8, KG = K / 64;
  const unsigned blocks = (unsigned)n_tiles * KG;
  if (src_is_fp16)
    hipLaunchKernelGGL(q4m_pack_mse_kernel<true>, dim3(blocks), dim3(512), 0, (hipStream_t)stream, w, N, K,
                       col_importance, alphas, n_alpha, (uint32_t*)w_marlin, (f16x2*)sb_marlin);
  else
    hipLaunchKernelGGL(q4m_pack_mse_kernel<false>, dim3(blocks), dim3(512), 0, (hipStream_t)stream, w, N, K,
                       col_importance, alphas, n_alpha, (uint32_t*)w_marlin, (f16x2*)sb_marlin);
  AXM_LAUNCH_CHECK("pack_q4_marlin_mse");
  return 0;
}

// Fused RMSNorm -> gate/up MARLIN GEMV -> SwiGLU for M tokens (the MLP input
// half of a decoder layer; transformer.py:1178-1189).  gu_w/gu_sb pack the
// concatenated [W_gate; W_up] rows (transformer.py:959-963), H % 8 == 0.
extern "C" int axm_qmv_q4_marlin_swiglu(const void* x, const void* ln_w, float eps, const void* gu_w,
                                        const void* gu_sb, void* y, int M, int K, int H, void* stream) {
  AXM_CHECK_ARG(x && gu_w && gu_sb && y, -1, "qmv_q4_marlin_swiglu: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && H > 0 && H % 8 == 0, -1,
                "qmv_q4_marlin_swiglu: K=%d must be a multiple of 64 and H=%d of 8", K, H);
  AXM_CHECK_ARG(M >= 1 && M <= 4, -1, "qmv_q4_marlin_swiglu: M=%d must be in [1, 4]", M);
  Q4GemvArgs a{};
  a.x = (const f16*)x;
  a.ldx = K;
  a.w = (const u32x4*)gu_w;
  a.sb = (const u32x4*)gu_sb;
  a.K = K;
  a.KG = K / 64;
  a.N = H;
  a.n_units = H / 8;
  a.pair_offset = H / 8;
  a.y = (f16*)y;
  a.ldy = H;
  a.ln_w = (const f16*)ln_w;
  a.eps = eps;
  int rc = q4m_gemv_launch(a, M, Q4_EPI_SWIGLU, q4m_default_grid(a.n_units), (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmv_q4_marlin_swiglu");
  return 0;
}
