// Runner-native MARLIN Q4 layout and its MFMA GEMV for gfx950.
//
// The reference MARLIN layout (8-row tiles, quant.py:573-593) pairs two rows in
// every 16-bit half, which suits a SIMD-group FMA but not a matrix core.  The
// decode runner therefore re-tiles the codes once, bit-exactly, into "tile16":
//
//   w16  [N16][KB][64 lanes][4 words] u32     N16 = ceil(N/16), KB = ceil(K/128)
//        lane l, word c  ->  row j = l % 16 of the tile,
//                            k = 128 kb + 32 c + 8 (l / 16) + i,  i = 0..7
//        slot i sits at bits  i0:0-3  i1:16-19  i2:4-7  i3:20-23
//                             i4:8-11 i5:24-27  i6:12-15 i7:28-31
//   sb16 [N16][KB][16 rows][2 groups] (f16 scale, f16 bias), groups 2kb, 2kb+1
//
// so one dwordx4 per lane (1 KB per wave) is exactly the B operand of four
// v_mfma_f32_16x16x32_f16 (16 rows x 128 k).  Each word expands with four
// AND-ORs into fp16 (1024 + q | 64 + q) pairs; the magic offsets are removed
// once per group with a precomputed sum of the activations, and the per-group
// (scale, bias) are applied to the 16 x 16 accumulator tile after the two MFMAs
// of that group.  Padding rows / columns carry code 0 with scale 0 and bias 0.
//
// The activation tile (A operand: token = lane % 16, k = 8 (lane / 16) + i)
// is read from LDS; tokens >= M read a zero block.
#include "kernels.h"
#include "q4_tile16.h"
#include "t16_device.h"

namespace {

// GEMV workgroups have TH = 512 threads (8 waves) or, where a 512-thread grid
// would leave most CUs with a single workgroup, 256 (t16_gemv_launch).
constexpr int kT16Threads = 512;
constexpr int kT16ThreadsSmall = 256;

// Reference lane holding (r, even column c0) of an 8-row MARLIN tile
// (inverse of quant.py:573-576).
__device__ __forceinline__ int marlin_lane_of(int r, int c0) {
  return ((r >> 2) << 4) | ((c0 >> 2) << 3) | ((r & 3) << 1) | ((c0 >> 1) & 1);
}

// One thread per (tile16, kb, lane): the four words of that lane.
// g128: sbm holds one (scale, bias) per 128 columns ([N/8][K/128][8]) and sb16
// one per (row, kb) ([N16][KB][16 rows]); otherwise two per kb as above.
__global__ void repack_tile16_kernel(const uint32_t* __restrict__ wm, const f16x2* __restrict__ sbm, int N_pad8,
                                     int K, uint32_t* __restrict__ w16, f16x2* __restrict__ sb16, int N16, int KB,
                                     int g128) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)N16 * KB * 64) return;
  const int l = (int)(idx & 63);
  const long tk = idx >> 6;
  const int kb = (int)(tk % KB);
  const int t16 = (int)(tk / KB);
  const int KG = K / 64;
  const int row = t16 * 16 + (l & 15);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = 128 * kb + 32 * c + 8 * (l >> 4) + i;
      uint32_t q = 0;
      if (row < N_pad8 && k < K) {
        const int tile = row >> 3, cin = row & 7, g = k >> 6, kk = k & 63;
        const int j = kk >> 5, s = (kk >> 3) & 3, r = kk & 7;
        const int lane = marlin_lane_of(r, cin & ~1);
        const uint32_t rw = wm[(((size_t)tile * KG + g) * 32 + lane) * 2 + j];
        q = (rw >> (16 * (cin & 1) + 4 * s)) & 0xFu;
      }
      const int pos = (i & 1) ? 16 + 4 * (i >> 1) : 4 * (i >> 1);
      word |= q << pos;
    }
    w16[idx * 4 + c] = word;
  }
  if (l < 16 && g128) {
    f16x2 v = f16x2{f16(0), f16(0)};
    if (row < N_pad8 && kb < KB) v = sbm[((size_t)(row >> 3) * KB + kb) * 8 + (row & 7)];
    sb16[((size_t)t16 * KB + kb) * 16 + l] = v;
  } else if (l < 16) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int g = 2 * kb + h;
      f16x2 v = f16x2{f16(0), f16(0)};
      if (row < N_pad8 && g < KG) v = sbm[((size_t)(row >> 3) * KG + g) * 8 + (row & 7)];
      sb16[(((size_t)t16 * KB + kb) * 16 + l) * 2 + h] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Activation staging: xs [M][K_pad] f16 (normalized if ln_w), zero block,
// cx [M][2 KB] float2 (magic-offset-weighted sum, plain sum) per 64-group.
//
// Thread tid owns the 8-element vectors i = tid + r * TH of every row.
// t16_load_x issues the activation (and norm weight) loads into registers
// before the kernel issues its weight loads: a wave's loads complete in issue
// order, so staging that loaded x only after the weight loads would first wait
// for every weight chunk of the wave to arrive.
// ---------------------------------------------------------------------------
constexpr int kT16MaxK = kTile16MaxK;
// Vectors per thread and row: K <= XV * TH * 8 = kT16MaxK.
template <int TH>
struct T16XV {
  static constexpr int value = kT16MaxK / (8 * TH);
};

template <int M, int TH>
struct T16X {
  static constexpr int XV = T16XV<TH>::value;
  f16x8 x[M][XV];
  f16x8 w[XV];
};

template <int M, int TH>
__device__ __forceinline__ void t16_load_x(const T16Args& a, T16X<M, TH>& r) {
  constexpr int XV = T16XV<TH>::value;
  const int tid = threadIdx.x;
  const int nv = a.K >> 3;
  const int nv_pad = (a.KB * 128) >> 3;
#pragma unroll
  for (int v = 0; v < XV; ++v) {
    // Vectors past the padded row are never staged (workgroup-uniform bound).
    if (v * TH >= nv_pad) break;
    const int i = tid + v * TH;
    const bool ok = i < nv;
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
      const f16x8* xr = reinterpret_cast<const f16x8*>(a.x + (size_t)mi * a.ldx);
      f16x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = f16(0);
      if (ok) t = xr[i];
      r.x[mi][v] = t;
    }
    f16x8 t;
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = f16(0);
    if (ok && a.ln_w != nullptr) t = reinterpret_cast<const f16x8*>(a.ln_w)[i];
    r.w[v] = t;
  }
}

// Split-partial activation source (Q4_EPI_RESID, M == 1): thread tid owns the
// 8 elements 8 tid.. of x.  Every partial slot is loaded unconditionally through
// a bounded buffer descriptor (slots past n_parts read as zero) so that the
// number of loads in flight before the weight loads is static.
// (512-thread workgroups only.)
static_assert(kTile16PartsMaxK == kT16Threads * 8, "one partial vector per thread");
struct T16Parts {
  u32x4 o[kTile16MaxParts];
  u32x2 ml[kTile16MaxParts];
};

__device__ __forceinline__ void t16_load_parts(const T16Args& a, T16Parts& pp) {
  const int i = threadIdx.x;
  const int heads = a.K / a.parts_hd;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.x_parts, (short)0, a.n_parts * a.K * (int)sizeof(f16), 0x00020000);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.x_ml, (short)0, a.n_parts * heads * (int)sizeof(f32x2), 0x00020000);
  const bool ok = i < (a.K >> 3);
  const int h = (8 * i) / a.parts_hd;
#pragma unroll
  for (int sp = 0; sp < kTile16MaxParts; ++sp) {
    const int oo = ok ? (sp * a.K + 8 * i) * (int)sizeof(f16) : 0x7FFFFFF0;
    const int mo = ok ? (sp * heads + h) * (int)sizeof(f32x2) : 0x7FFFFFF0;
    pp.o[sp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, oo, 0, 0));
    pp.ml[sp] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rm, mo, 0, 0));
  }
}

template <int M, int TH>
__device__ __forceinline__ void t16_merge_parts(const T16Args& a, const T16Parts& pp, T16X<M, TH>& r) {
  static_assert(TH == kT16Threads, "partial merge with 512-thread workgroups");
  constexpr float kNoScore = -1e30f;
  // The (m, l) words are copied to scalars before the bit casts: a bit cast of an
  // ext_vector element expression reads element 0.
  float m[kTile16MaxParts], l[kTile16MaxParts];
#pragma unroll
  for (int sp = 0; sp < kTile16MaxParts; ++sp) {
    const uint32_t mu = pp.ml[sp][0];
    const uint32_t lu = pp.ml[sp][1];
    m[sp] = __builtin_bit_cast(float, mu);
    l[sp] = __builtin_bit_cast(float, lu);
  }
  float mx = kNoScore;
#pragma unroll
  for (int sp = 0; sp < kTile16MaxParts; ++sp)
    if (sp < a.n_parts) mx = fmaxf(mx, m[sp]);
  float wsum = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int sp = 0; sp < kTile16MaxParts; ++sp) {
    if (sp < a.n_parts) {
      const float w = l[sp] * exp2f(m[sp] - mx);
      wsum += w;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f16x2 h2 = as_h2(pp.o[sp][c]);
        acc[2 * c] = __builtin_fmaf(w, h2f(h2.x), acc[2 * c]);
        acc[2 * c + 1] = __builtin_fmaf(w, h2f(h2.y), acc[2 * c + 1]);
      }
    }
  }
  f16x8 x;
#pragma unroll
  // One reciprocal instead of eight divisions on the O launch's staging path.
  for (int e = 0; e < 8; ++e) x[e] = f2h(acc[e] * (wsum > 0.f ? 1.f / wsum : 0.f));
  const bool ok = (int)threadIdx.x < (a.K >> 3);
#pragma unroll
  for (int v = 0; v < T16XV<TH>::value; ++v) {
#pragma unroll
    for (int e = 0; e < 8; ++e) r.x[0][v][e] = f16(0);
    r.w[v] = r.x[0][v];
  }
  if (ok) r.x[0][0] = x;
}

template <int M, int TH>
__device__ void t16_stage_x(const T16Args& a, const T16X<M, TH>& r, f16* xs, f32x2* cx, float* red) {
  constexpr int XV = T16XV<TH>::value;
  constexpr int W = TH / 64;
  const int tid = threadIdx.x;
  const int K = a.K;
  const int nv = K >> 3;
  const int nv_pad = (a.KB * 128) >> 3;
  float rinv[M];
#pragma unroll
  for (int mi = 0; mi < M; ++mi) rinv[mi] = 1.f;
  if (a.ln_w != nullptr) {
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
      float s = 0.f;
#pragma unroll
      for (int v = 0; v < XV; ++v) {
        // Vectors past nv hold zeros and add nothing: the loop stops at the last
        // vector any thread loaded (a uniform bound; K = 4096 needs one or two of
        // the XV vectors that K = 16384 would).
        if (v * TH >= nv) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = h2f(r.x[mi][v][e]);
          s += h2f(f2h(f * f));
        }
      }
      s = wave_sum_dpp(s);
      if ((tid & 63) == 0) red[mi * W + (tid >> 6)] = s;
    }
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < M; ++mi) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) s += red[mi * W + w];
      rinv[mi] = rms_inv_fp16(s, K, a.eps);
    }
  }
#pragma unroll
  for (int mi = 0; mi < M; ++mi) {
    // nv_pad is a multiple of 16 (KB*128/8) and the same for every thread, so
    // the 8-lane group reduction below always runs with full wave participation.
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      if (v * TH >= nv_pad) break;
      const int i = tid + v * TH;
      f16x8 x = r.x[mi][v];
      if (i < nv) {
        if (a.ln_w != nullptr) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = f2h(h2f(f2h(h2f(x[e]) * rinv[mi])) * h2f(r.w[v][e]));
        }
        if (a.x_norm_out != nullptr) reinterpret_cast<f16x8*>(a.x_norm_out + (size_t)mi * K)[i] = x;
      }
      float corr = 0.f, sum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = h2f(x[e]);
        sum += f;
        corr += f * (((e >> 1) & 1) ? 64.f : 1024.f);
      }
      // 8 consecutive vectors form one 64-group.
      corr = group8_sum_dpp(corr);
      sum = group8_sum_dpp(sum);
      if (i < nv_pad) {
        reinterpret_cast<f16x8*>(xs + (size_t)mi * a.KB * 128)[i] = x;
        if ((tid & 7) == 0) cx[(size_t)mi * 2 * a.KB + (i >> 3)] = f32x2{corr, sum};
      }
    }
  }
  __syncthreads();
}

// Epilogue operands of a one-token, one-pass launch, requested after the first
// weight chunks instead of after the last: at the end of the weight stream they
// would add a dependent round trip (two for RoPE: position, then its cos / sin)
// to the launch's tail.  QKV: RoPE cos / sin, the bias pair and the cache slot;
// residual epilogues: the residual value.  Lanes 0..15 hold rows unit*16 + lane.
struct T16EpiPre {
  float c, sn;
  f16 b_self, b_part, resid;
  int wp;
};

template <int EPI>
__device__ __forceinline__ T16EpiPre t16_epi_prefetch(const T16Args& a, int unit, int lane, int pos, int wp) {
  T16EpiPre e{1.f, 0.f, f16(0), f16(0), f16(0), wp};
  const int row = unit * 16 + (lane & 15);
  if (lane >= 16 || unit >= a.n_units || row >= a.N) return e;
  if (EPI == Q4_EPI_QKV_ROPE) {
    if (a.bias != nullptr) {
      e.b_self = a.bias[row];
      e.b_part = a.bias[row ^ 1];
    }
    const int row0 = row & ~1;
    if (row0 < a.q_dim + a.kv_dim) {
      const int hd = a.head_dim, half_hd = hd >> 1;
      const int within = row0 < a.q_dim ? row0 : row0 - a.q_dim;
      const int fi = (within % hd) >> 1;
      const int rp = pos % a.rope_len;
      e.c = a.freqs[((size_t)rp * half_hd + fi) * 2 + 0];
      e.sn = a.freqs[((size_t)rp * half_hd + fi) * 2 + 1];
    }
  } else if (EPI == Q4_EPI_RESID) {
    e.resid = a.resid[row];
  }
  return e;
}

// Epilogue for lane l: row = unit*16 + l%16, token = 4*(l/16) + v.  PRE: the
// operands come from t16_epi_prefetch (M == 1).
template <int M, int NT, int EPI, bool PRE>
__device__ __forceinline__ void t16_epilogue(const T16Args& a, int unit, int lane, const float (&v)[NT][4],
                                             const T16EpiPre& pre) {
  static_assert(!PRE || M == 1, "prefetched epilogue operands: one token");
  const int j = lane & 15;
  const int row = unit * 16 + j;
  if (EPI == Q4_EPI_STORE && M == 1 && a.argmax_keys != nullptr) {
    unsigned long long key = 0ull;
    if (lane < 16 && row < a.N) {
      const uint32_t u = __builtin_bit_cast(uint32_t, h2f(f2h(v[0][0])));
      const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
      key = ((unsigned long long)ord << 32) | (0xFFFFFFFFu - (uint32_t)row);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const unsigned long long other = __shfl_xor(key, o, 64);
      key = other > key ? other : key;
    }
    if (lane == 0) a.argmax_keys[unit] = key;
  }
#pragma unroll
  for (int vi = 0; vi < 4; ++vi) {
    const int tok = 4 * (lane >> 4) + vi;
    if (EPI == Q4_EPI_QKV_ROPE) {
      const float partner = __shfl_xor(v[0][vi], 1, 64);
      if (tok >= M || row >= a.N) continue;
      const bool even = (row & 1) == 0;
      f16 h_self = f2h(v[0][vi]);
      f16 h_part = f2h(partner);
      if (a.bias != nullptr) {
        h_self = f2h(h2f(h_self) + h2f(PRE ? pre.b_self : a.bias[row]));
        h_part = f2h(h2f(h_part) + h2f(PRE ? pre.b_part : a.bias[row ^ 1]));
      }
      const f16 h0 = even ? h_self : h_part;
      const f16 h1 = even ? h_part : h_self;
      const int row0 = row & ~1;
      const int hd = a.head_dim, half_hd = hd >> 1;
      f16 out = h_self;
      if (row0 < a.q_dim + a.kv_dim) {
        if (PRE) {
          out = rope_out(h0, h1, pre.c, pre.sn, even);
        } else {
          const int pos = (a.rope_pos_dev ? a.rope_pos_dev[0] : a.rope_pos) + tok;
          const int within = row0 < a.q_dim ? row0 : row0 - a.q_dim;
          const int fi = (within % hd) >> 1;
          const int rp = pos % a.rope_len;
          const float c = a.freqs[((size_t)rp * half_hd + fi) * 2 + 0];
          const float sn = a.freqs[((size_t)rp * half_hd + fi) * 2 + 1];
          out = rope_out(h0, h1, c, sn, even);
        }
      }
      if (row < a.q_dim) {
        a.y[(size_t)tok * a.ldy + row] = out;
      } else {
        const bool is_k = row < a.q_dim + a.kv_dim;
        const int within = is_k ? row - a.q_dim : row - a.q_dim - a.kv_dim;
        const int kvh = within / hd, e = within % hd;
        const int wp = (PRE ? pre.wp : (a.write_pos_dev ? a.write_pos_dev[0] : a.write_pos)) + tok;
        f16* dst = (is_k ? a.k_out : a.v_out) + ((size_t)kvh * a.kv_stride_h + (size_t)(wp % a.max_seq) * hd + e);
        *dst = out;
      }
      continue;
    }
    if (tok >= M || row >= a.N) continue;
    if (EPI == Q4_EPI_SWIGLU) {
      const f16 g = f2h(v[0][vi]);
      const f16 u = f2h(v[NT - 1][vi]);
      const f16 sg = f2h(t16_silu(h2f(g)));
      a.y[(size_t)tok * a.ldy + row] = f2h(h2f(sg) * h2f(u));
    } else {
      f16 h = f2h(v[0][vi]);
      if (a.bias != nullptr) h = f2h(h2f(h) + h2f(a.bias[row]));
      if (EPI == Q4_EPI_STORE) {
        a.y[(size_t)tok * a.ldy + row] = h;
      } else {
        f16* xr = a.resid + (size_t)tok * a.ldr + row;
        *xr = f2h(h2f(PRE ? pre.resid : *xr) + h2f(h));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA GEMV.  Unit = one tile16 (or a gate/up pair, NT = 2).  S = a.split
// waves share a unit (split-K over kb); 8 / S units per workgroup pass.
// MODE kT16Loop (S == 1): waves loop over units, prefetching the next unit's
// chunks.  Otherwise (S > 1) the grid covers all units in one pass with a
// straight-line body; the modes are separate instantiations so that the
// one-pass body has no loop back edge carrying loads in flight, which would
// make the compiler wait for every outstanding load before the first chunk is
// consumed.
// kT16Wave (one pass over at most kT16WaveMaxChunks chunks per wave, loads
// kept in flight through a ring of P register slots): a wave's (scale, bias)
// pairs for its my chunks are one contiguous my * 128-byte run, fetched with
// two 16-byte loads per lane into a wave-private LDS slot instead of one
// 8-byte load per chunk.
// kT16OnePass: one pass with per-chunk scale loads and in-loop refills.
// P kb-loads (1 KB per tile each) stay in flight per wave.
// ---------------------------------------------------------------------------
// Residual epilogue whose activations are merged from attention split partials
// (an instantiation of its own, M == 1 only, so that the plain residual GEMV
// keeps its smaller register footprint).
constexpr int kT16EpiResidParts = 16;

constexpr int kT16Loop = 0;
constexpr int kT16OnePass = 1;
constexpr int kT16Wave = 2;
// Chunk register slots per wave in kT16Wave (a ring; 7B decode step: 6 / 8 / 12 /
// 16 slots gave 727 / 726 / 730.5 / 729 tok/s).
constexpr int kT16WaveDepth = 12;
// Chunks issued before the activation staging (7B decode step on one MI355X:
// 1 / 2 / 3 / 4 / 8 gave 698 / 721 / 725 / 713 / 529 tok/s).
constexpr int kT16WavePre = 3;
// The same PRE chunks stay requested ahead of the one being consumed after the
// staging (keeping 5 / 7 / 9 / 11 ahead instead, topped up right after the staging
// barrier, gave 728 / 720 / 722 / 725 against 756 tok/s).
// Chunk jj + PRE is requested into the slot of chunk jj + PRE - P before chunk jj is
// consumed, so PRE must stay below the ring size.
static_assert(kT16WavePre < kT16WaveDepth, "kT16Wave ring");
constexpr int kT16WaveMaxChunks = 16;  // chunks per wave kT16Wave handles

// G128: one (scale, bias) word per row and chunk (group-128 packs) instead of two;
// it is applied to both 64-column halves of the chunk.
template <int M, int NT, int EPI, int P, int MODE, bool G128, int TH>
//
// The fields the first loads need come as leading scalar arguments, which the
// hardware preloads into SGPRs (-mllvm -amdgpu-kernarg-preload-count): the weight,
// scale and activation requests then issue without waiting for a scalar load of the
// argument struct.
__global__ void __launch_bounds__(TH)
    t16_gemv_kernel(const f16* x_p, const f16* ln_w_p, const u32x4* w16_p, const u32x2* sb16_p, int K_p,
                    int n_units_p, int split_p, int pair_offset_p, int w16_bytes_p, int sb16_bytes_p, T16Args a) {
  // (At most 14 argument dwords are preloaded; KB follows from K.)
  a.x = x_p;
  a.ln_w = ln_w_p;
  a.w16 = w16_p;
  a.sb16 = sb16_p;
  a.K = K_p;
  a.KB = (K_p + 127) >> 7;
  a.n_units = n_units_p;
  a.split = split_p;
  a.pair_offset = pair_offset_p;
  a.w16_bytes = (size_t)w16_bytes_p;
  a.sb16_bytes = (size_t)sb16_bytes_p;
  constexpr int W = TH / 64;  // waves per workgroup
  constexpr bool ONE = MODE != kT16Loop;
  constexpr bool SBW = MODE == kT16Wave;
  constexpr int VPC = G128 ? 4 : 8;  // 16-byte scale vectors per chunk and tile
  constexpr int QS = SBW ? kT16WaveMaxChunks * VPC / 64 : 1;  // 16-byte scale loads per lane and tile (kT16Wave)
  constexpr int NJ = SBW ? kT16WaveMaxChunks : P;        // unrolled chunk slots per pass
  extern __shared__ __align__(16) unsigned char smem[];
  f16* xs = reinterpret_cast<f16*>(smem);                                   // [M][KB*128]
  f16* zero = xs + (size_t)M * a.KB * 128;                                   // 16 halves of zeros
  f32x2* cx = reinterpret_cast<f32x2*>(zero + 16);                           // [M][2 KB]
  float* red = reinterpret_cast<float*>(cx + (size_t)M * 2 * a.KB);          // [waves][NT][4][64]
  u32x2* sbw = reinterpret_cast<u32x2*>(red + W * NT * 4 * 64);              // kT16Wave: [waves][NT][per][16]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int S = a.split;
  const int upw = W / S;
  const int sub = wave % S;
  const int slot = wave / S;
  // Contiguous kb range [kb0, kb0 + my) of this wave within a unit.
  const int per = (a.KB + S - 1) / S;
  const int kb0 = sub * per;
  const int my = max(0, min(per, a.KB - kb0));
  const int tokA = lane & 15;  // A-operand token of this lane
  const int kq = lane >> 4;    // 8-wide k sub-block of this lane
  // The nibble masks and magic exponents as constants (no argument load ahead of the
  // first requests); the opaque moves keep the masks in VGPRs.
  const Unpack U{to_vgpr(0x000F000Fu), to_vgpr(0x00F000F0u), to_sgpr(0x64006400u), to_sgpr(0x54005400u)};

  // Raw buffer descriptors: out-of-range offsets read as zero, so every chunk
  // load is issued unconditionally and the load pipeline stays static.
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w16, (short)0, (int)a.w16_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.sb16, (short)0, (int)a.sb16_bytes, 0x00020000);
  constexpr int kOOB = 0x7FFFFFF0;

  if (tid < 8) reinterpret_cast<uint32_t*>(zero)[tid] = 0u;

  u32x4 wr[P][NT];
  u32x2 sr[P][NT];
  // Byte offsets of (unit, ci) for this lane, OOB when outside the wave's range.
  auto load = [&](int unit, int ci, int j) {
    // Branch-free select of the offsets: the condition is wave-uniform, and as a
    // conditional the compiler split the requests into branches whose register
    // reuse forced a wait for every load in flight.
    const int m = -((int)(unit < a.n_units) & (int)(ci < my));
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int base = (unit + t * a.pair_offset) * a.KB + kb0 + ci;
      const int wo = (((base * 64 + lane) * 16) & m) | (kOOB & ~m);
      const int so = (((base * 16 + (lane & 15)) * (G128 ? 4 : 8)) & m) | (kOOB & ~m);
      wr[j][t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, 2));
      if (!SBW && G128) {
        const uint32_t v = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(rs, so, 0, 0));
        sr[j][t] = u32x2{v, v};
      } else if (!SBW) {
        sr[j][t] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0));
      }
    }
  };

  int it = 0;
  int unit = blockIdx.x * upw + slot;
  // Prefetched epilogue operands (one token, one pass); the RoPE / cache positions
  // are requested first (uniform, scalar loads) so that the cos / sin loads issued
  // after the first weight chunks find them arrived.
  constexpr int EPI_BASE = EPI == kT16EpiResidParts ? Q4_EPI_RESID : EPI;
  constexpr bool EPI_PRE = M == 1 && ONE && (EPI_BASE == Q4_EPI_QKV_ROPE || EPI_BASE == Q4_EPI_RESID);
  // The positions are vector loads left in VGPRs until the operands are requested
  // (t16_vgpr there): a scalar copy of a loaded value made the compiler wait for it
  // right away, before any other request of the launch was issued.  A null device
  // pointer gives a zero-sized descriptor (the load reads 0) and the host value.
  uint32_t pre_pos_raw = 0, pre_wp_raw = 0;
  if constexpr (EPI_PRE && EPI_BASE == Q4_EPI_QKV_ROPE) {
    const __amdgpu_buffer_rsrc_t rpp = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.rope_pos_dev, (short)0, a.rope_pos_dev ? 4 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rwp = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.write_pos_dev, (short)0, a.write_pos_dev ? 4 : 0, 0x00020000);
    pre_pos_raw = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(rpp, 0, 0, 0));
    pre_wp_raw = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(rwp, 0, 0, 0));
  }
  T16EpiPre epre{1.f, 0.f, f16(0), f16(0), f16(0), 0};
  T16X<M, TH> xr;
  // Q4_EPI_RESID with one token may take its activations from attention split
  // partials (merged after the weight loads are issued).
  constexpr bool from_parts = EPI == kT16EpiResidParts;
  T16Parts pp;
  if (from_parts)
    t16_load_parts(a, pp);
  else
    t16_load_x<M, TH>(a, xr);
  // kT16Wave: the wave's (scale, bias) run; 16-byte vector v holds chunk v / 8,
  // rows 2 (v % 8) and 2 (v % 8) + 1 (G128: chunk v / 4, rows 4 (v % 4) ..
  // 4 (v % 4) + 3).  Issued before the weight loads so that storing it to LDS
  // waits only for itself.
  u32x4 sbv[NT][QS];
  u32x2* my_sb = sbw + (size_t)wave * NT * per * 16;
  if (SBW) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int q = 0; q < QS; ++q) {
        const int v = q * 64 + lane;
        const bool ok = unit < a.n_units && v < my * VPC;
        const int bo = ok ? (((unit + t * a.pair_offset) * a.KB + kb0) * VPC + v) * 16 : kOOB;
        sbv[t][q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, bo, 0, 0));
      }
  }
  // kT16Wave issues only the first PRE chunks before the staging barrier: a
  // wave that blocks on a full memory queue while issuing its later loads
  // would hold the whole workgroup at the barrier.  The rest are issued while
  // the first chunks are consumed.
  constexpr int PRE = SBW ? kT16WavePre : P;
#pragma unroll
  for (int j = 0; j < PRE; ++j) load(unit, j, j);
  if constexpr (EPI_PRE) {
    if (sub == 0) {
      int pre_pos = 0, pre_wp = 0;
      if constexpr (EPI_BASE == Q4_EPI_QKV_ROPE) {
        pre_pos = (int)t16_vgpr(pre_pos_raw) + (a.rope_pos_dev ? 0 : a.rope_pos);
        pre_wp = (int)t16_vgpr(pre_wp_raw) + (a.write_pos_dev ? 0 : a.write_pos);
      }
      epre = t16_epi_prefetch<EPI_BASE>(a, unit, lane, pre_pos, pre_wp);
    }
  }
  if (SBW) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int q = 0; q < QS; ++q) {
        // Every lane stores (lanes past the run into a dummy slot after the
        // per-wave runs): with a conditional store the compiler moved the scale
        // loads into it, behind the weight requests, and waited for all of them.
        const int v = q * 64 + lane;
        u32x4* dst = v < my * VPC ? reinterpret_cast<u32x4*>(my_sb + (size_t)t * per * 16 + 2 * v)
                                  : reinterpret_cast<u32x4*>(sbw + (size_t)W * NT * per * 16);
        *dst = sbv[t][q];
      }
  }
  if constexpr (from_parts) t16_merge_parts<M, TH>(a, pp, xr);
  t16_stage_x<M, TH>(a, xr, xs, cx, red);  // ends with a workgroup barrier

  // LDS addresses: A operand of this lane and (corr, sum) of its D tokens.
  const f16* xa = (tokA < M) ? xs + (size_t)tokA * a.KB * 128 + 8 * kq : zero;
  const int a_kb = (tokA < M) ? 128 : 0;
  const int a_c = (tokA < M) ? 32 : 0;

  while (true) {
    float acc[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int vi = 0; vi < 4; ++vi) acc[t][vi] = 0.f;

    // kT16Wave: a single pass over its my <= kT16WaveMaxChunks chunks.
    const int n_pass = SBW ? 1 : (my + P - 1) / P;
    for (int pass = 0; pass < n_pass; ++pass) {
      const int ci0 = pass * P;
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        // kT16Wave: chunk jj lives in ring slot jj % P; chunk jj + PRE is
        // requested into the slot chunk jj + PRE - P freed.
        const int j = jj % P;
        const int ci = ci0 + jj;
        if (SBW && jj + PRE < NJ && jj + PRE < my) load(unit, jj + PRE, (jj + PRE) % P);
        if (SBW && ci >= my) break;  // wave-uniform
        // Chunks past the range carry zero codes and zero scales: clamp the LDS
        // reads to a valid kb so they only ever multiply finite values by zero.
        const int kb = kb0 + min(ci, my - 1);
        const f16* xk = xa + kb * a_kb;
        f16x8 A[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) A[c] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(xk + c * a_c));
        f32x4 cxv[4];
#pragma unroll
        for (int vi = 0; vi < 4; ++vi) {
          if (vi < M) {
            const int tok = min(4 * kq + vi, M - 1);
            cxv[vi] = *reinterpret_cast<const f32x4*>(cx + (size_t)tok * 2 * a.KB + 2 * kb);
          }
        }
        if (SBW && G128) {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const uint32_t v = reinterpret_cast<const uint32_t*>(my_sb + (size_t)t * per * 16)[ci * 16 + (lane & 15)];
            sr[j][t] = u32x2{v, v};
          }
        } else if (SBW) {
#pragma unroll
          for (int t = 0; t < NT; ++t) sr[j][t] = my_sb[(size_t)t * per * 16 + ci * 16 + (lane & 15)];
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
          f32x4 d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], unpack_word(wr[j][t][0], U), z4, 0, 0, 0);
          f32x4 d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[2], unpack_word(wr[j][t][2], U), z4, 0, 0, 0);
          d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1], unpack_word(wr[j][t][1], U), d0, 0, 0, 0);
          d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[3], unpack_word(wr[j][t][3], U), d1, 0, 0, 0);
          const f16x2 sb0 = as_h2(sr[j][t][0]);
          const f16x2 sb1 = as_h2(sr[j][t][1]);
#pragma unroll
          for (int vi = 0; vi < 4; ++vi) {
            if (vi < M) {
              float r = acc[t][vi];
              r = __builtin_fmaf(h2f(sb0.x), d0[vi] - cxv[vi][0], r);
              r = __builtin_fmaf(h2f(sb0.y), cxv[vi][1], r);
              r = __builtin_fmaf(h2f(sb1.x), d1[vi] - cxv[vi][2], r);
              r = __builtin_fmaf(h2f(sb1.y), cxv[vi][3], r);
              acc[t][vi] = r;
            }
          }
        }
        // kT16Wave has every chunk in flight already (my <= P).
        if (!SBW) load(unit, ci + P, j);
      }
    }

    const int next_unit = (blockIdx.x + (it + 1) * gridDim.x) * upw + slot;
    const bool more = !ONE && ((blockIdx.x + (it + 1) * gridDim.x) * upw < a.n_units);
    if (more) {
#pragma unroll
      for (int j = 0; j < P; ++j) load(next_unit, j, j);
    }
    if (ONE) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int vi = 0; vi < 4; ++vi)
          if (vi < M) red[((wave * NT + t) * 4 + vi) * 64 + lane] = acc[t][vi];
      __syncthreads();
      if (sub == 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int vi = 0; vi < 4; ++vi)
            if (vi < M) {
              float s = 0.f;
              for (int w = wave; w < wave + S; ++w) s += red[((w * NT + t) * 4 + vi) * 64 + lane];
              acc[t][vi] = s;
            }
      }
    }
    if (sub == 0 && unit < a.n_units) t16_epilogue<M, NT, EPI_BASE, EPI_PRE>(a, unit, lane, acc, epre);
    if (ONE || !more) break;
    ++it;
    unit = next_unit;
  }
}

template <int NT>
struct T16Depth {
  static constexpr int value = NT == 2 ? 4 : 8;
};

template <int M, int NT, int EPI, int P, int MODE, int TH>
void t16_set_attr_mode() {
  if (hipFuncSetAttribute((const void*)t16_gemv_kernel<M, NT, EPI, P, MODE, false, TH>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
    (void)hipGetLastError();
  if (hipFuncSetAttribute((const void*)t16_gemv_kernel<M, NT, EPI, P, MODE, true, TH>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
    (void)hipGetLastError();
}

template <int M, int NT, int EPI, int TH>
void t16_set_attr_th() {
  t16_set_attr_mode<M, NT, EPI, T16Depth<NT>::value, kT16Loop, TH>();
  t16_set_attr_mode<M, NT, EPI, T16Depth<NT>::value, kT16OnePass, TH>();
  t16_set_attr_mode<M, NT, EPI, kT16WaveDepth, kT16Wave, TH>();
}

template <int M, int NT, int EPI>
void t16_set_attr() {
  t16_set_attr_th<M, NT, EPI, kT16Threads>();
  if constexpr (M == 1 && EPI != kT16EpiResidParts) t16_set_attr_th<M, NT, EPI, kT16ThreadsSmall>();
}

#define T16_HOT(a)                                                                                  \
  (a).x, (a).ln_w, (a).w16, (a).sb16, (a).K, (a).n_units, (a).split, (a).pair_offset, (int)(a).w16_bytes, \
      (int)(a).sb16_bytes

template <int M, int NT, int EPI, bool G128, int TH>
void t16_launch_g(const T16Args& a, int mode, int grid, size_t smem, hipStream_t s) {
  const dim3 g(grid), b(TH);
  if (mode == kT16Wave)
    hipLaunchKernelGGL((t16_gemv_kernel<M, NT, EPI, kT16WaveDepth, kT16Wave, G128, TH>), g, b, smem, s, T16_HOT(a), a);
  else if (mode == kT16OnePass)
    hipLaunchKernelGGL((t16_gemv_kernel<M, NT, EPI, T16Depth<NT>::value, kT16OnePass, G128, TH>), g, b, smem, s, T16_HOT(a), a);
  else
    hipLaunchKernelGGL((t16_gemv_kernel<M, NT, EPI, T16Depth<NT>::value, kT16Loop, G128, TH>), g, b, smem, s, T16_HOT(a), a);
}

template <int M, int NT, int EPI>
int t16_launch_one(const T16Args& a, int mode, int grid, size_t smem, int th, hipStream_t s) {
  if constexpr (M == 1 && EPI != kT16EpiResidParts) {
    if (th == kT16ThreadsSmall) {
      if (a.g128)
        t16_launch_g<M, NT, EPI, true, kT16ThreadsSmall>(a, mode, grid, smem, s);
      else
        t16_launch_g<M, NT, EPI, false, kT16ThreadsSmall>(a, mode, grid, smem, s);
      return 0;
    }
  }
  if (a.g128)
    t16_launch_g<M, NT, EPI, true, kT16Threads>(a, mode, grid, smem, s);
  else
    t16_launch_g<M, NT, EPI, false, kT16Threads>(a, mode, grid, smem, s);
  return 0;
}

}  // namespace

size_t t16_smem_bytes(int M, int NT, int K, int waves) {
  const int KB = (K + 127) / 128;
  return (size_t)M * KB * 128 * sizeof(f16) + 32 + (size_t)M * 2 * KB * sizeof(f32x2) +
         (size_t)waves * NT * 4 * 64 * sizeof(float);
}

void t16_prepare_attributes() {
  static bool done = false;
  if (done) return;
  done = true;
#define AXM_T16_ATTR(MM)                      \
  t16_set_attr<MM, 1, Q4_EPI_STORE>();        \
  t16_set_attr<MM, 1, Q4_EPI_RESID>();        \
  t16_set_attr<MM, 2, Q4_EPI_SWIGLU>();       \
  t16_set_attr<MM, 1, Q4_EPI_QKV_ROPE>();
  AXM_T16_ATTR(1)
  AXM_T16_ATTR(2)
  AXM_T16_ATTR(3)
  AXM_T16_ATTR(4)
#undef AXM_T16_ATTR
  t16_set_attr<1, 1, kT16EpiResidParts>();
}

int t16_gemv_launch(T16Args a, int M, int epi, hipStream_t s) {
  t16_prepare_attributes();
  const int NT = (epi == Q4_EPI_SWIGLU) ? 2 : 1;
  if (M < 1 || M > 4 || a.K > kT16MaxK) {
    axm_set_error("tile16 gemv: M=%d K=%d unsupported (M in [1, 4], K <= %d)", M, a.K, kT16MaxK);
    return -2;
  }
  if (a.x_parts != nullptr &&
      (M != 1 || epi != Q4_EPI_RESID || a.ln_w != nullptr || a.K > kTile16PartsMaxK || a.n_parts < 2 ||
       a.n_parts > kTile16MaxParts || a.parts_hd <= 0 || a.parts_hd % 8 != 0 || a.K % a.parts_hd != 0 ||
       a.x_ml == nullptr)) {
    axm_set_error("tile16 gemv: split-partial activations need M=1, the residual epilogue, no norm, K <= %d, "
                  "2..%d parts, head size %% 8 == 0 (M=%d K=%d parts=%d hd=%d)",
                  kTile16PartsMaxK, kTile16MaxParts, M, a.K, a.n_parts, a.parts_hd);
    return -2;
  }
  // Waves per unit: aim for ~8 waves per CU with >= 2 kb-loads per wave; the S
  // waves of a unit belong to one workgroup.
  const int cus = axm_num_cus();
  // (Aiming at 16 or 32 waves per CU instead left a second round of gate|up
  // workgroups: 764 -> 670 tok/s.)
  auto split_for = [&](int waves) {
    int S = 1;
    while (S < waves && a.n_units * S < 8 * cus && a.KB >= 4 * S) S *= 2;
    return S;
  };
  int th = kT16Threads;
  int S = split_for(kT16Threads / 64);
  // Above one and up to 1.5 512-thread workgroups per CU, some CUs would hold
  // two and the rest one (workgroups of one launch all resident): 256-thread
  // workgroups spread the same waves evenly (7B decode on one MI355X: gate|up
  // 13.3 -> 12.3 us; QKV, exactly 1.5 per CU, 790 -> 796 tok/s once the staging
  // reductions moved to DPP).  With exactly one per CU (the down projection)
  // and beyond 1.5 per CU (the lm_head) 512 threads were as fast or faster
  // (down with 256 threads: 742 -> 731 tok/s).  One token only: with more,
  // the activation registers of 256 threads covering K <= 16384 (eight vectors
  // per thread and token) cost more than the balance gains (two-token verify
  // 1.33 -> 1.47 decode steps).  The split-partial source needs one thread per
  // 8 activations of a 4096-wide row, i.e. 512 threads.  Only split-K launches
  // (S > 1, the measured one-pass forms) switch: with S == 1 the 256-thread grid
  // would run the looping form, which was never measured against 512 threads.
  if (M == 1 && a.x_parts == nullptr && S > 1) {
    const int grid512 = (a.n_units + kT16Threads / 64 / S - 1) / (kT16Threads / 64 / S);
    if (grid512 > cus && 2 * grid512 <= 3 * cus) {
      th = kT16ThreadsSmall;
      S = split_for(kT16ThreadsSmall / 64);
    }
  }
  const int waves = th / 64;
  size_t smem = t16_smem_bytes(M, NT, a.K, waves);
  if (smem > 160 * 1024) {
    axm_set_error("tile16 gemv: M=%d K=%d needs %zu B of LDS", M, a.K, smem);
    return -2;
  }
  a.split = S;
  a.w16_bytes = t16_weight_bytes(a.N_rows_alloc, a.K);
  a.sb16_bytes = t16_sb_bytes(a.N_rows_alloc, a.K, a.g128);
  a.unpack[0] = 0x000F000Fu;
  a.unpack[1] = 0x00F000F0u;
  a.unpack[2] = 0x64006400u;
  a.unpack[3] = 0x54005400u;
  const int upw = waves / S;
  int grid = (a.n_units + upw - 1) / upw;
  if (S == 1 && grid > 2 * cus) grid = 2 * cus;
  // Chunks per wave; kT16Wave keeps all of them in flight (per <= depth).
  const int per = (a.KB + S - 1) / S;
  int mode = S == 1 ? kT16Loop : kT16OnePass;
  if (S > 1 && per <= kT16WaveMaxChunks) {
    const size_t sb_lds = (size_t)waves * NT * per * 128 + 16;  // + the dummy slot
    if (smem + sb_lds <= 160 * 1024) {
      mode = kT16Wave;
      smem += sb_lds;
    }
  }
#define AXM_T16_CASE(MM)                                                                 \
  case MM:                                                                               \
    switch (epi) {                                                                       \
      case Q4_EPI_STORE: return t16_launch_one<MM, 1, Q4_EPI_STORE>(a, mode, grid, smem, th, s);   \
      case Q4_EPI_RESID: return t16_launch_one<MM, 1, Q4_EPI_RESID>(a, mode, grid, smem, th, s);   \
      case Q4_EPI_SWIGLU: return t16_launch_one<MM, 2, Q4_EPI_SWIGLU>(a, mode, grid, smem, th, s); \
      case Q4_EPI_QKV_ROPE: return t16_launch_one<MM, 1, Q4_EPI_QKV_ROPE>(a, mode, grid, smem, th, s); \
    }                                                                                    \
    break;
  if (a.x_parts != nullptr) return t16_launch_one<1, 1, kT16EpiResidParts>(a, mode, grid, smem, th, s);
  switch (M) {
    AXM_T16_CASE(1)
    AXM_T16_CASE(2)
    AXM_T16_CASE(3)
    AXM_T16_CASE(4)
  }
#undef AXM_T16_CASE
  axm_set_error("tile16 gemv: unsupported epilogue %d", epi);  // unreachable for valid codes
  return -2;
}

int t16_repack(const void* w_marlin, const void* sb_marlin, int N, int K, void* w16, void* sb16, hipStream_t s,
               int g128) {
  const int n_tiles8 = (N + 7) / 8;
  const int N16 = (N + 15) / 16;
  const int KB = (K + 127) / 128;
  const long total = (long)N16 * KB * 64;
  hipLaunchKernelGGL(repack_tile16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     (const uint32_t*)w_marlin, (const f16x2*)sb_marlin, n_tiles8 * 8, K, (uint32_t*)w16,
                     (f16x2*)sb16, N16, KB, g128);
  return 0;
}

size_t t16_weight_bytes(int N, int K) { return (size_t)((N + 15) / 16) * ((K + 127) / 128) * 64 * 16; }
size_t t16_sb_bytes(int N, int K, int g128) {
  return (size_t)((N + 15) / 16) * ((K + 127) / 128) * 16 * (g128 ? 4 : 8);
}

// ---------------------------------------------------------------------------
// C ABI: repack + GEMV on the tile16 layout (the runner uses the same code).
// ---------------------------------------------------------------------------
extern "C" size_t axm_tile16_bytes(int N, int K, int which) {
  return which == 0 ? t16_weight_bytes(N, K) : t16_sb_bytes(N, K, which == 2);
}

extern "C" int axm_repack_q4_marlin_tile16(const void* w_marlin, const void* sb_marlin, int N, int K, void* w16,
                                           void* sb16, void* stream) {
  AXM_CHECK_ARG(w_marlin && sb_marlin && w16 && sb16, -1, "repack_tile16: null pointer");
  AXM_CHECK_ARG(N > 0 && K > 0 && K % 64 == 0, -1, "repack_tile16: bad shape N=%d K=%d", N, K);
  t16_repack(w_marlin, sb_marlin, N, K, w16, sb16, (hipStream_t)stream, 0);
  AXM_LAUNCH_CHECK("repack_tile16");
  return 0;
}

extern "C" int axm_repack_q4_marlin_g128_tile16(const void* w_marlin, const void* sb128, int N, int K, void* w16,
                                                void* sb16, void* stream) {
  AXM_CHECK_ARG(w_marlin && sb128 && w16 && sb16, -1, "repack_g128_tile16: null pointer");
  AXM_CHECK_ARG(N > 0 && K > 0 && K % 128 == 0, -1, "repack_g128_tile16: bad shape N=%d K=%d", N, K);
  t16_repack(w_marlin, sb128, N, K, w16, sb16, (hipStream_t)stream, 1);
  AXM_LAUNCH_CHECK("repack_g128_tile16");
  return 0;
}

extern "C" int axm_qmv_q4_tile16(const void* x, const void* w16, const void* sb16, const void* bias, void* y, int M,
                                 int K, int N, int group_size, void* stream) {
  AXM_CHECK_ARG(x && w16 && sb16 && y, -1, "qmv_q4_tile16: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0 && M >= 1, -1, "qmv_q4_tile16: bad shape M=%d K=%d N=%d", M, K, N);
  AXM_CHECK_ARG(group_size == 64 || (group_size == 128 && K % 128 == 0), -1,
                "qmv_q4_tile16: group_size %d (64, or 128 with K %% 128 == 0)", group_size);
  for (int m0 = 0; m0 < M; m0 += 4) {
    const int mc = (M - m0) < 4 ? (M - m0) : 4;
    T16Args a{};
    a.x = (const f16*)x + (size_t)m0 * K;
    a.ldx = K;
    a.w16 = (const u32x4*)w16;
    a.sb16 = (const u32x2*)sb16;
    a.g128 = group_size == 128;
    a.K = K;
    a.KB = (K + 127) / 128;
    a.N = N;
    a.n_units = (N + 15) / 16;
    a.N_rows_alloc = N;
    a.y = (f16*)y + (size_t)m0 * N;
    a.ldy = N;
    a.bias = (const f16*)bias;
    int rc = t16_gemv_launch(a, mc, Q4_EPI_STORE, (hipStream_t)stream);
    if (rc) return rc;
  }
  AXM_LAUNCH_CHECK("qmv_q4_tile16");
  return 0;
}

extern "C" int axm_qmv_q4_tile16_swiglu(const void* x, const void* ln_w, float eps, const void* gu16,
                                        const void* gusb16, void* y, int M, int K, int H, int group_size,
                                        void* stream) {
  AXM_CHECK_ARG(x && gu16 && gusb16 && y, -1, "qmv_q4_tile16_swiglu: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && H > 0 && H % 16 == 0 && M >= 1 && M <= 4, -1,
                "qmv_q4_tile16_swiglu: bad shape M=%d K=%d H=%d (H %% 16 == 0, M <= 4)", M, K, H);
  AXM_CHECK_ARG(group_size == 64 || (group_size == 128 && K % 128 == 0), -1,
                "qmv_q4_tile16_swiglu: group_size %d (64, or 128 with K %% 128 == 0)", group_size);
  T16Args a{};
  a.x = (const f16*)x;
  a.ldx = K;
  a.w16 = (const u32x4*)gu16;
  a.sb16 = (const u32x2*)gusb16;
  a.g128 = group_size == 128;
  a.K = K;
  a.KB = (K + 127) / 128;
  a.N = H;
  a.n_units = H / 16;
  a.N_rows_alloc = 2 * H;
  a.pair_offset = H / 16;
  a.y = (f16*)y;
  a.ldy = H;
  a.ln_w = (const f16*)ln_w;
  a.eps = eps;
  int rc = t16_gemv_launch(a, M, Q4_EPI_SWIGLU, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmv_q4_tile16_swiglu");
  return 0;
}
