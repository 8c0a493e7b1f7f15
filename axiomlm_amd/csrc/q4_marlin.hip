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
//   cx  : f32x2[KG*8]          = (sum with magic weights 1024 (s even) / 64 (s odd), plain sum)
// ---------------------------------------------------------------------------
struct XStage {
  f16* xh;
  f32x2* cx;
};

template <int M>
__device__ void stage_x(const Q4GemvArgs& a, XStage* st, float* red) {
  const int tid = threadIdx.x;
  const int K = a.K;
  const int nv = K >> 3;  // 8-element vectors
  float rinv[M];
#pragma unroll
  for (int mi = 0; mi < M; ++mi) rinv[mi] = 1.f;
  if (a.ln_w != nullptr) {
    // Sum of fp16-rounded squares per token (vectorized loads).
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
      const f16x8* xr = reinterpret_cast<const f16x8*>(a.x + (size_t)mi * a.ldx);
      float s = 0.f;
      for (int i = tid; i < nv; i += kThreads) {
        const f16x8 v = xr[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = h2f(v[e]);
          s += h2f(f2h(f * f));
        }
      }
      s = wave_sum(s);
      if ((tid & 63) == 0) red[mi * kWaves + (tid >> 6)] = s;
    }
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += red[mi * kWaves + w];
      rinv[mi] = rms_inv_fp16(s, K, a.eps);
    }
  }
  // Vector i holds k = 8i..8i+7: g = i>>3, j = (i>>2)&1, s = i&3, r = 0..7.
#pragma unroll
  for (int mi = 0; mi < M; ++mi) {
    const f16x8* xr = reinterpret_cast<const f16x8*>(a.x + (size_t)mi * a.ldx);
    const f16x8* wr = reinterpret_cast<const f16x8*>(a.ln_w);
    for (int i = tid; i < nv; i += kThreads) {
      f16x8 v = xr[i];
      if (a.ln_w != nullptr) {
        const f16x8 w = wr[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = f2h(h2f(f2h(h2f(v[e]) * rinv[mi])) * h2f(w[e]));
      }
      if (a.x_norm_out != nullptr) reinterpret_cast<f16x8*>(a.x_norm_out + (size_t)mi * K)[i] = v;
      const int g = i >> 3, js = ((i >> 2) & 1) * 4 + (i & 3);
      f16* dst = st[mi].xh + (size_t)g * 64 + js;
#pragma unroll
      for (int r = 0; r < 8; ++r) dst[r * 8] = v[r];
    }
  }
  __syncthreads();
  const int n_gr = a.KG * 8;
#pragma unroll
  for (int mi = 0; mi < M; ++mi) {
    for (int p = tid; p < n_gr; p += kThreads) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(st[mi].xh + (size_t)p * 8);
      float corr = 0.f, sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = h2f(v[e]);
        sum += f;
        corr += f * ((e & 1) ? 64.f : 1024.f);
      }
      st[mi].cx[p] = f32x2{corr, sum};
    }
  }
  __syncthreads();
}

// Accumulate one 64-column group for the lane's 4 rows.
// wv = (A, B, C, D) words: A/B rows cb,cb+1 (j=0/1), C/D rows cb+2,cb+3.
__device__ __forceinline__ void q4_group_fma(u32x4 wv, u32x4 sv, f16x8 xv, f32x2 cx, float acc[4]) {
  float d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int wi = 0; wi < 4; ++wi) {
    const uint32_t w = wv[wi];
    const int j = wi & 1;          // k half
    const int rp = (wi >> 1) * 2;  // row pair offset 0 or 2
    const uint32_t w8 = w >> 8;
    const f16x2 h0 = as_h2((w & 0x000F000Fu) | 0x64006400u);
    const f16x2 h1 = as_h2((w & 0x00F000F0u) | 0x54005400u);
    const f16x2 h2 = as_h2((w8 & 0x000F000Fu) | 0x64006400u);
    const f16x2 h3 = as_h2((w8 & 0x00F000F0u) | 0x54005400u);
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
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 sb = as_h2(sv[i]);
    acc[i] = __builtin_fmaf(h2f(sb.x), d[i] - cx.x, acc[i]);
    acc[i] = __builtin_fmaf(h2f(sb.y), cx.y, acc[i]);
  }
}

// Reduce the 4 row partials of every lane over the lanes that share cb.
// Returns, in lane L < 8, the full sum for tile row (L&4) + 2*(L&1) + ((L>>1)&1);
// the rows of a RoPE pair (2i, 2i+1) sit in lanes L and L^2.
__device__ __forceinline__ float wave_reduce_rows(const float v[4], int lane) {
  const bool b0 = lane & 1, b1 = lane & 2;
  const float s0 = b0 ? v[0] : v[2], s1 = b0 ? v[1] : v[3];
  float k0 = b0 ? v[2] : v[0], k1 = b0 ? v[3] : v[1];
  k0 += __shfl_xor(s0, 1, 64);
  k1 += __shfl_xor(s1, 1, 64);
  const float send = b1 ? k0 : k1;
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

// Epilogue run by lanes 0..7 of one wave; v[t][mi] is the row sum of tile t
// for row `row` of token mi (t = 0: the unit's tile / gate tile, t = 1: up tile).
template <int M, int NT, int EPI>
__device__ __forceinline__ void q4_epilogue(const Q4GemvArgs& a, int unit, int lane, const float (&v)[NT][M]) {
  const int row = unit * 8 + reduced_row_of_lane(lane);
  if (EPI == Q4_EPI_QKV_ROPE) {
    // Pair partner (row ^ 1) lives in lane ^ 2; every lane of the pair needs it.
    float pv[M];
#pragma unroll
    for (int mi = 0; mi < M; ++mi) pv[mi] = __shfl_xor(v[0][mi], 2, 64);
    if (lane >= 8 || row >= a.N) return;
    const bool even = (row & 1) == 0;
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
      f16 h_self = f2h(v[0][mi]);
      f16 h_part = f2h(pv[mi]);
      const int row0 = row & ~1;
      if (a.bias != nullptr) {
        h_self = f2h(h2f(h_self) + h2f(a.bias[row]));
        h_part = f2h(h2f(h_part) + h2f(a.bias[row ^ 1]));
      }
      const f16 h0 = even ? h_self : h_part;
      const f16 h1 = even ? h_part : h_self;
      const int hd = a.head_dim, half_hd = hd >> 1;
      f16 out = even ? h0 : h1;
      if (row0 < a.q_dim + a.kv_dim) {
        const int pos = (a.rope_pos_dev ? a.rope_pos_dev[0] : a.rope_pos) + mi;
        const int within = row0 < a.q_dim ? row0 : row0 - a.q_dim;
        const int fi = (within % hd) >> 1;
        const int rp = pos % a.rope_len;
        const float c = a.freqs[((size_t)rp * half_hd + fi) * 2 + 0];
        const float sn = a.freqs[((size_t)rp * half_hd + fi) * 2 + 1];
        out = rope_out(h0, h1, c, sn, even);
      }
      if (row < a.q_dim) {
        a.y[(size_t)mi * a.ldy + row] = out;
      } else {
        const bool is_k = row < a.q_dim + a.kv_dim;
        const int within = is_k ? row - a.q_dim : row - a.q_dim - a.kv_dim;
        const int kvh = within / hd, e = within % hd;
        const int wp = (a.write_pos_dev ? a.write_pos_dev[0] : a.write_pos) + mi;
        f16* dst = (is_k ? a.k_out : a.v_out) + ((size_t)kvh * a.kv_stride_h + (size_t)(wp % a.max_seq) * hd + e);
        *dst = out;
      }
    }
    return;
  }
  if (EPI == Q4_EPI_STORE && M == 1 && a.argmax_keys != nullptr) {
    // Ordered key: fp16 value (sign-folded) in the high word, ~index in the low
    // word, so the max is the largest logit with the lowest index on ties.
    unsigned long long key = 0ull;
    if (lane < 8 && row < a.N) {
      const f16 h = f2h(v[0][0]);
      const uint32_t u = __builtin_bit_cast(uint32_t, h2f(h));
      const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
      key = ((unsigned long long)ord << 32) | (0xFFFFFFFFu - (uint32_t)row);
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
      const unsigned long long other = __shfl_xor(key, o, 64);
      key = other > key ? other : key;
    }
    if (lane == 0) a.argmax_keys[unit] = key;
  }
  if (lane >= 8 || row >= a.N) return;
#pragma unroll
  for (int mi = 0; mi < M; ++mi) {
    if (EPI == Q4_EPI_SWIGLU) {
      const f16 g = f2h(v[0][mi]);
      const f16 u = f2h(v[NT - 1][mi]);
      const f16 sg = f2h(silu_f(h2f(g)));
      a.y[(size_t)mi * a.ldy + row] = f2h(h2f(sg) * h2f(u));
    } else {
      f16 h = f2h(v[0][mi]);
      if (a.bias != nullptr) h = f2h(h2f(h) + h2f(a.bias[row]));
      if (EPI == Q4_EPI_STORE) {
        a.y[(size_t)mi * a.ldy + row] = h;
      } else {
        f16* xr = a.resid + (size_t)mi * a.ldr + row;
        *xr = f2h(h2f(*xr) + h2f(h));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Main GEMV kernel.
//   NT = tiles per work unit (2 for the SwiGLU gate/up pair).
//   a.split (S in {1, 2, 4}) = waves that share one unit (split-K); the 4 waves of
//   a workgroup therefore cover 4/S units at a time.  S == 1 runs a persistent
//   loop over units; S > 1 requires one unit group per workgroup (grid covers all).
//   P = chunk loads in flight per wave (rolling pipeline, 1 KB per chunk and tile).
// The first P chunks of a wave are requested before the activations are staged,
// so the staging latency hides under the weight stream.
// ---------------------------------------------------------------------------
template <int M, int NT, int EPI, int P>
__global__ void __launch_bounds__(kThreads) q4m_gemv_kernel(Q4GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  // Layout: [M] xh (K halves) | [M] cx (K/8 float2) | red (kWaves*NT*M*8 f32)
  XStage st[M];
  unsigned char* p = smem;
#pragma unroll
  for (int mi = 0; mi < M; ++mi) {
    st[mi].xh = reinterpret_cast<f16*>(p);
    p += (size_t)a.K * sizeof(f16);
  }
#pragma unroll
  for (int mi = 0; mi < M; ++mi) {
    st[mi].cx = reinterpret_cast<f32x2*>(p);
    p += (size_t)(a.K / 8) * sizeof(f32x2);
  }
  float* red = reinterpret_cast<float*>(p);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int gs = lane >> 4;
  const int m = lane & 15;
  const int r = ((m & 8) >> 1) | (m & 3);
  const int cb = m & 4;
  const int S = a.split;
  const int upw = kWaves / S;
  const int sub = wave % S;
  const int slot = wave / S;
  const int n_chunks = (a.KG + 3) >> 2;
  const int my = (n_chunks - sub + S - 1) / S;  // chunks of this wave per unit (host keeps S <= n_chunks)
  const u32x4* __restrict__ w4 = a.w;
  const u32x4* __restrict__ sb4 = a.sb;

  u32x4 wr[P][NT], sr[P][NT];
  auto load = [&](int unit, int ci, int j) {
    const int g = (sub + ci * S) * 4 + gs;
    const bool ok = unit < a.n_units && ci < my && g < a.KG;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const size_t base = (size_t)(unit + t * a.pair_offset) * a.KG + g;
      wr[j][t] = ok ? __builtin_nontemporal_load(w4 + base * 16 + m) : u32x4{0u, 0u, 0u, 0u};
      sr[j][t] = ok ? sb4[base * 2 + (cb >> 2)] : u32x4{0u, 0u, 0u, 0u};
    }
  };

  int it = 0;
  int unit = blockIdx.x * upw + slot;
#pragma unroll
  for (int j = 0; j < P; ++j) load(unit, j, j);
  stage_x<M>(a, st, red);

  while (true) {
    float acc[NT][M][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mi = 0; mi < M; ++mi)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][mi][i] = 0.f;

    for (int ci0 = 0; ci0 < my; ci0 += P) {
#pragma unroll
      for (int j = 0; j < P; ++j) {
        const int ci = ci0 + j;
        if (ci < my) {
          const int g = (sub + ci * S) * 4 + gs;
          if (g < a.KG) {
            const int pidx = g * 8 + r;
#pragma unroll
            for (int mi = 0; mi < M; ++mi) {
              const f16x8 xv = *reinterpret_cast<const f16x8*>(st[mi].xh + (size_t)pidx * 8);
              const f32x2 cx = st[mi].cx[pidx];
#pragma unroll
              for (int t = 0; t < NT; ++t) q4_group_fma(wr[j][t], sr[j][t], xv, cx, acc[t][mi]);
            }
          }
          if (ci + P < my) load(unit, ci + P, j);
        }
      }
    }

    // Request the next unit's first chunks before the reduction / epilogue.
    const int next_unit = (blockIdx.x + (it + 1) * gridDim.x) * upw + slot;
    const bool more = (S == 1) && ((blockIdx.x + (it + 1) * gridDim.x) * upw < a.n_units);
    if (more) {
#pragma unroll
      for (int j = 0; j < P; ++j) load(next_unit, j, j);
    }

    float v[NT][M];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mi = 0; mi < M; ++mi) v[t][mi] = wave_reduce_rows(acc[t][mi], lane);
    if (S > 1) {
      // Split-K partials of the S waves of a unit meet in LDS.
      if (lane < 8) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int mi = 0; mi < M; ++mi) red[((wave * NT + t) * M + mi) * 8 + lane] = v[t][mi];
      }
      __syncthreads();
      if (sub == 0 && lane < 8) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int mi = 0; mi < M; ++mi) {
            float s = 0.f;
            for (int w = wave; w < wave + S; ++w) s += red[((w * NT + t) * M + mi) * 8 + lane];
            v[t][mi] = s;
          }
      }
    }
    if (sub == 0 && unit < a.n_units) q4_epilogue<M, NT, EPI>(a, unit, lane, v);
    if (!more) break;
    ++it;
    unit = next_unit;
  }
}

// ---------------------------------------------------------------------------
// Dequantization (row-major fp16 output), fp32 math then one fp16 rounding,
// quant.py:597-634.
// ---------------------------------------------------------------------------
__global__ void q4m_dequant_kernel(const uint32_t* __restrict__ w, const f16x2* __restrict__ sb,
                                   f16* __restrict__ out, int n_tiles, int KG, int N, int g_shift) {
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
      // (scale, bias) of group g >> g_shift: g_shift 1 for one pair per 128 columns
      const f16x2 s_b = sb[((size_t)tile * (KG >> g_shift) + (g >> g_shift)) * 8 + c0 + half];
      const float sc = h2f(s_b.x), bi = h2f(s_b.y);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t q = (word >> (16 * half + 4 * s)) & 0xFu;
        out[(size_t)row * K + 64 * g + 32 * j + 8 * s + r] = f2h(add_rn(mul_rn((float)q, sc), bi));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Round-to-nearest packer, quant.py:482-494 + the lane interleave :573-593.
// One 64-thread block per (tile, group).  SRC_FP16 selects torch's fp16 op
// semantics for (max - min) and the /15 (each rounded to fp16).
// ---------------------------------------------------------------------------
// One block per (8-row tile, GS-column group), GS = 64 (the reference layout) or
// 128 (the group-128 variant: same code layout per 64-column block, one
// (scale, bias) per 128 columns in sb [N/8][K/GS][8]).  Thread t holds row t / (GS/8)
// of the tile and the 8-column slice t % (GS/8).
template <bool SRC_FP16, int GS>
__global__ void __launch_bounds__(GS) q4m_pack_rtn_kernel(const void* __restrict__ wsrc, int N, int K,
                                                          uint32_t* __restrict__ w_out, f16x2* __restrict__ sb_out) {
  constexpr int SL = GS / 8;  // slices per row
  const int KG = K / GS;
  const int tile = blockIdx.x / KG;
  const int g = blockIdx.x % KG;
  const int t = threadIdx.x;
  const int c = t / SL;     // row within tile
  const int sub = t % SL;   // 8-element slice
  const int row = tile * 8 + c;
  __shared__ uint8_t qs[8][GS];
  float vals[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int k = GS * g + 8 * sub + i;
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
  for (int o = 1; o < SL; o <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  float denom;
  f16 sc_h;
  if (SRC_FP16) {
    f16 d = f2h(sub_rn(mx, mn));  // fp16 subtraction; clamp(min=1e-8) is a no-op in fp16
    denom = h2f(d);
    sc_h = f2h(__fdiv_rn(denom, 15.0f));
  } else {
    denom = fmaxf(sub_rn(mx, mn), 1e-8f);
    sc_h = f2h(__fdiv_rn(denom, 15.0f));
  }
  const f16 bi_h = f2h(mn);
  const float scf = fmaxf(h2f(sc_h), 1e-8f);
  const float bif = h2f(bi_h);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float q = __builtin_rintf(__fdiv_rn(sub_rn(vals[i], bif), scf));
    q = fminf(fmaxf(q, 0.f), 15.f);
    qs[c][8 * sub + i] = (uint8_t)q;
  }
  if (sub == 0) sb_out[((size_t)tile * KG + g) * 8 + c] = f16x2{sc_h, bi_h};
  __syncthreads();
  // One 32-lane set per 64-column block of the group.
  if (t < 32 * (GS / 64)) {
    const int l = t & 31;
    const int blk = t >> 5;
    const int r = ((l & 16) >> 2) | ((l & 6) >> 1);
    const int c0 = ((l & 8) >> 1) | ((l & 1) << 1);
    const int KG64 = K / 64;
    const int g64 = g * (GS / 64) + blk;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t word = 0;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int kk = 64 * blk + 32 * j + 8 * s + r;
        word |= (uint32_t)qs[c0][kk] << (4 * s);
        word |= (uint32_t)qs[c0 + 1][kk] << (16 + 4 * s);
      }
      w_out[(((size_t)tile * KG64 + g64) * 32 + l) * 2 + j] = word;
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
    const float ig2 = mul_rn(imp, imp);
    const float mean = __fdiv_rn(wave_sum(ig2), 64.f);
    ig = __fdiv_rn(ig2, fmaxf(mean, 1e-8f));
  }
  const float mn0 = -wave_max(-w);
  const float mx0 = wave_max(w);
  const float mu = __fdiv_rn(wave_sum(has_ig ? mul_rn(w, ig) : w), 64.f);

  auto err_of = [&](float sc, float bi) {
    float q = __builtin_rintf(__fdiv_rn(sub_rn(w, bi), fmaxf(sc, 1e-8f)));
    q = fminf(fmaxf(q, 0.f), 15.f);
    const float diff = sub_rn(w, add_rn(mul_rn(q, sc), bi));
    const float e = mul_rn(diff, diff);
    return wave_sum(has_ig ? mul_rn(ig, e) : e);
  };

  float best = INFINITY;
  float cur_mn = mn0;
  for (int i = 0; i < n_alpha; ++i) {
    const float a = alphas[i];
    const float cand_mn = add_rn(mu, mul_rn(a, sub_rn(mn0, mu)));
    const float sc = h2f(f2h(__fdiv_rn(fmaxf(sub_rn(mx0, cand_mn), 1e-8f), 15.f)));
    const float bi = h2f(f2h(cand_mn));
    const float e = err_of(sc, bi);
    if (e < best) {
      best = e;
      cur_mn = cand_mn;
    }
  }
  best = INFINITY;
  f16 best_sc = f2h(__fdiv_rn(fmaxf(sub_rn(mx0, cur_mn), 1e-8f), 15.f));
  f16 best_bi = f2h(cur_mn);
  for (int i = 0; i < n_alpha; ++i) {
    const float a = alphas[i];
    const float cand_mx = add_rn(mu, mul_rn(a, sub_rn(mx0, mu)));
    const f16 sc_h = f2h(__fdiv_rn(fmaxf(sub_rn(cand_mx, cur_mn), 1e-8f), 15.f));
    const f16 bi_h = f2h(cur_mn);
    const float e = err_of(h2f(sc_h), h2f(bi_h));
    if (e < best) {
      best = e;
      best_sc = sc_h;
      best_bi = bi_h;
    }
  }
  float q = __builtin_rintf(__fdiv_rn(sub_rn(w, h2f(best_bi)), fmaxf(h2f(best_sc), 1e-8f)));
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
         (size_t)kWaves * NT * M * 8 * sizeof(float);
}

// Chunk loads in flight per wave: 8 KB per wave for one tile, 2 x 4 KB for pairs.
template <int NT>
struct PipeDepth {
  static constexpr int value = NT == 2 ? 4 : 8;
};

template <int M, int NT, int EPI>
static void set_attr_one() {
  if (hipFuncSetAttribute((const void*)q4m_gemv_kernel<M, NT, EPI, PipeDepth<NT>::value>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
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
  hipLaunchKernelGGL((q4m_gemv_kernel<M, NT, EPI, PipeDepth<NT>::value>), dim3(grid), dim3(kThreads), smem, s, a);
  return 0;
}

// Work decomposition: S waves per unit (split-K inside a workgroup) so that the
// launch has about 8 waves per CU; S == 1 launches a persistent grid.
static void choose_split(Q4GemvArgs& a, int* grid) {
  const int cus = axm_num_cus();
  const int target_waves = 8 * cus;
  const int n_chunks = (a.KG + 3) / 4;
  int S = 1;
  while (S < kWaves && a.n_units * S < target_waves && n_chunks >= 2 * S * 2) S *= 2;
  a.split = S;
  const int upw = kWaves / S;
  int g = (a.n_units + upw - 1) / upw;
  if (S == 1) {
    const int cap = cus * 4;
    if (g > cap) g = cap;
  }
  *grid = g;
}

int q4m_gemv_launch(Q4GemvArgs a, int M, int epi, hipStream_t s) {
  q4m_prepare_attributes();
  const int NT = (epi == Q4_EPI_SWIGLU) ? 2 : 1;
  if (q4m_gemv_smem_bytes(M, NT, a.K) > 160 * 1024) {
    axm_set_error("q4 gemv: K=%d with M=%d needs %zu B of LDS (> 160 KiB)", a.K, M, q4m_gemv_smem_bytes(M, NT, a.K));
    return -2;
  }
  if (a.K % 64 != 0 || a.KG != a.K / 64 || a.n_units <= 0) {
    axm_set_error("q4 gemv: bad shape K=%d units=%d", a.K, a.n_units);
    return -2;
  }
  int grid = 0;
  choose_split(a, &grid);
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
      int rc = q4m_gemv_launch(a, cnt, Q4_EPI_STORE, s);
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
                     (const uint32_t*)w_marlin, (const f16x2*)sb_marlin, (f16*)out, n_tiles, KG, N, 0);
  AXM_LAUNCH_CHECK("dequantize_q4_marlin");
  return 0;
}

extern "C" int axm_dequantize_q4_marlin_g128(const void* w_marlin, const void* sb128, void* out, int K, int N,
                                             void* stream) {
  AXM_CHECK_ARG(w_marlin && sb128 && out, -1, "dequantize_q4_marlin_g128: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0, -1, "dequantize_q4_marlin_g128: bad shape K=%d N=%d", K, N);
  const int n_tiles = (N + 7) / 8, KG = K / 64;
  const long total = (long)n_tiles * KG * 32;
  hipLaunchKernelGGL(q4m_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)w_marlin, (const f16x2*)sb128, (f16*)out, n_tiles, KG, N, 1);
  AXM_LAUNCH_CHECK("dequantize_q4_marlin_g128");
  return 0;
}

extern "C" int axm_pack_q4_marlin_rtn(const void* w, int src_is_fp16, int N, int K, void* w_marlin, void* sb_marlin,
                                      void* stream) {
  AXM_CHECK_ARG(w && w_marlin && sb_marlin, -1, "pack_q4_marlin: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0, -1, "pack_q4_marlin: K=%d must be a multiple of 64", K);
  const int n_tiles = (N + 7) / 8, KG = K / 64;
  const unsigned blocks = (unsigned)n_tiles * KG;
  if (src_is_fp16)
    hipLaunchKernelGGL((q4m_pack_rtn_kernel<true, 64>), dim3(blocks), dim3(64), 0, (hipStream_t)stream, w, N, K,
                       (uint32_t*)w_marlin, (f16x2*)sb_marlin);
  else
    hipLaunchKernelGGL((q4m_pack_rtn_kernel<false, 64>), dim3(blocks), dim3(64), 0, (hipStream_t)stream, w, N, K,
                       (uint32_t*)w_marlin, (f16x2*)sb_marlin);
  AXM_LAUNCH_CHECK("pack_q4_marlin_rtn");
  return 0;
}

extern "C" int axm_pack_q4_marlin_rtn_g128(const void* w, int src_is_fp16, int N, int K, void* w_marlin,
                                           void* sb128, void* stream) {
  AXM_CHECK_ARG(w && w_marlin && sb128, -1, "pack_q4_marlin_g128: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 128 == 0 && N > 0, -1, "pack_q4_marlin_g128: K=%d must be a multiple of 128", K);
  const unsigned blocks = (unsigned)((N + 7) / 8) * (K / 128);
  if (src_is_fp16)
    hipLaunchKernelGGL((q4m_pack_rtn_kernel<true, 128>), dim3(blocks), dim3(128), 0, (hipStream_t)stream, w, N, K,
                       (uint32_t*)w_marlin, (f16x2*)sb128);
  else
    hipLaunchKernelGGL((q4m_pack_rtn_kernel<false, 128>), dim3(blocks), dim3(128), 0, (hipStream_t)stream, w, N, K,
                       (uint32_t*)w_marlin, (f16x2*)sb128);
  AXM_LAUNCH_CHECK("pack_q4_marlin_rtn_g128");
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
  int rc = q4m_gemv_launch(a, M, Q4_EPI_SWIGLU, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmv_q4_marlin_swiglu");
  return 0;
}
