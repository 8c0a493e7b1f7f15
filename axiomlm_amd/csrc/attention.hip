// KV-cache writes (fp16 / FP8-E4M3FN / INT4, group 64 scales) and split-KV
// decode / tree-verification attention for gfx950.
//
// Cache layouts are the reference StaticKVCache ones (axiomlm/engine/paged_cache.py:158-198):
//   fp16 : [B][Hkv][S][hd]            f16
//   fp8  : [B][Hkv][S][hd]            u8  + scales [B][Hkv][S][hd/64] f16
//   int4 : [B][Hkv][S][hd/2]          u8  + scales [B][Hkv][S][hd/64] f16
//
// Attention mapping: one workgroup (4 waves) per (batch, kv head, key split)
// and up to QR query rows that share the kv head (GQA replicas and/or tree
// nodes).  A key row is spread over hd/8 lanes (8 elements = 16 B of fp16,
// 8 B of fp8, 4 B of int4 per lane), so a wave walks 512/hd keys at once and
// every key/value byte is read exactly once per workgroup.  Softmax is online
// in the exp2 domain with fp32 state; partial (m, l, o) per split are merged by
// a second kernel (or written directly when there is a single split).
#include <mutex>
#include <type_traits>

#include "kernels.h"

namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1e30f;

// ---------------------------------------------------------------------------
// KV quantization + write.  One wave per (token, kv head, 64-group, k|v).
// CPU semantics of quantize_kv_fp8 / quantize_kv_int4 (quant.py:692-807):
//   scale = fp16(amax / 448 | 7)            (clamp(min=1e-8) is a no-op in fp16)
//   xs    = fp16(x / scale)                 (fp16 division)
//   fp8   = e4m3fn(float(xs));   int4 = clamp(rne(xs), -8, 7)
// ---------------------------------------------------------------------------
// Lane `lane` of one wave stores element g*64 + lane of the key (which = 0) or
// value (which = 1) row of kv head h at `slot` (batch 0).  Quantized caches
// need all 64 lanes of the wave on the same (row, group).
__device__ __forceinline__ void kv_store_lane(const KvView& kv, int which, int h, int slot, int g, int lane, f16 x) {
  const int G = kv.hd / 64;
  const size_t row = (size_t)h * kv.S + slot;  // batch 0
  if (kv.kv_dtype == AXM_KV_FP16) {
    f16* dst = (f16*)(which == 0 ? kv.k : kv.v);
    dst[row * kv.hd + g * 64 + lane] = x;
    return;
  }
  const float ax = fabsf(h2f(x));
  const float amax = wave_max(ax);
  const float div = kv.kv_dtype == AXM_KV_FP8 ? 448.0f : 7.0f;
  const f16 sc = f2h(__fdiv_rn(amax, div));
  const float scf = h2f(sc);
  f16* sdst = which == 0 ? kv.ks : kv.vs;
  if (lane == 0) sdst[row * G + g] = sc;
  // fp16 division of x by the scale; 0/0 follows x86 (negative quiet NaN).
  float q;
  if (scf == 0.f) {
    q = (h2f(x) == 0.f) ? __builtin_bit_cast(float, 0xFFC00000u) : h2f(x) / scf;
  } else {
    q = h2f(f2h(__fdiv_rn(h2f(x), scf)));
  }
  uint8_t* dst = (uint8_t*)(which == 0 ? kv.k : kv.v);
  if (kv.kv_dtype == AXM_KV_FP8) {
    dst[row * kv.hd + g * 64 + lane] = fp8e4m3fn_from_f32(q);
  } else {
    int qi;
    if (q != q) {
      qi = 0;  // NaN -> int8 conversion yields 0 on the reference CPU path
    } else {
      float r = __builtin_rintf(q);
      r = fminf(fmaxf(r, -8.f), 7.f);
      qi = (int)r;
    }
    const int partner = __shfl_xor(qi, 1, 64);
    if ((lane & 1) == 0) {
      dst[row * (kv.hd / 2) + g * 32 + lane / 2] = (uint8_t)((qi & 0xF) | ((partner & 0xF) << 4));
    }
  }
}

// Four waves per workgroup, one (token, k|v, kv head, 64-group) per wave.
constexpr int kKvWriteWaves = 4;
__global__ void __launch_bounds__(kKvWriteWaves * 64)
    kv_write_kernel(KvView kv, const f16* __restrict__ k_rows, const f16* __restrict__ v_rows, int ld, int write_pos,
                    const int* __restrict__ write_pos_dev, int n_items) {
  const int lane = threadIdx.x & 63;
  const int G = kv.hd / 64;
  int idx = blockIdx.x * kKvWriteWaves + (threadIdx.x >> 6);
  if (idx >= n_items) return;
  const int g = idx % G;
  idx /= G;
  const int h = idx % kv.Hkv;
  idx /= kv.Hkv;
  const int which = idx % 2;  // 0 = k, 1 = v
  const int t = idx / 2;
  const int wp0 = write_pos_dev ? write_pos_dev[0] : write_pos;
  const int slot = (wp0 + t) % kv.S;
  const f16* src = (which == 0 ? k_rows : v_rows) + (size_t)t * ld + h * kv.hd + g * 64;
  kv_store_lane(kv, which, h, slot, g, lane, src[lane]);
}

// Row form of the KV write: one wave per (token, k|v, kv head); lane l holds the
// EPL = hd / 64 consecutive elements EPL l .. EPL l + EPL - 1 (one vector load),
// so a 64-group spans 64 / EPL lanes and its maximum is taken by shuffles within
// them.  Per element the arithmetic is kv_store_lane's.
template <int EPL>
using kv_hvec = _Float16 __attribute__((ext_vector_type(EPL)));

template <int EPL>
__device__ __forceinline__ void kv_row_store(const KvView& kv, int which, int h, int slot, int lane,
                                             kv_hvec<EPL> xv) {
  constexpr int LPG = 64 / EPL;  // lanes per 64-group
  const size_t row = (size_t)h * kv.S + slot;  // batch 0
  if (kv.kv_dtype == AXM_KV_FP16) {
    *reinterpret_cast<kv_hvec<EPL>*>((f16*)(which == 0 ? kv.k : kv.v) + row * kv.hd + EPL * lane) = xv;
    return;
  }
  float ax = fabsf(h2f(xv[0]));  // seeded like wave_max (an all-NaN group keeps a NaN maximum)
#pragma unroll
  for (int e = 1; e < EPL; ++e) ax = fmaxf(ax, fabsf(h2f(xv[e])));
#pragma unroll
  for (int off = LPG / 2; off > 0; off >>= 1) ax = fmaxf(ax, __shfl_xor(ax, off, 64));
  const float div = kv.kv_dtype == AXM_KV_FP8 ? 448.0f : 7.0f;
  const f16 sc = f2h(__fdiv_rn(ax, div));
  const float scf = h2f(sc);
  if (lane % LPG == 0) (which == 0 ? kv.ks : kv.vs)[row * (kv.hd / 64) + lane / LPG] = sc;
  float q[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float xf = h2f(xv[e]);
    if (scf == 0.f)
      q[e] = (xf == 0.f) ? __builtin_bit_cast(float, 0xFFC00000u) : xf / scf;
    else
      q[e] = h2f(f2h(__fdiv_rn(xf, scf)));
  }
  uint8_t* dst = (uint8_t*)(which == 0 ? kv.k : kv.v);
  if (kv.kv_dtype == AXM_KV_FP8) {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < EPL; ++e) packed |= (uint32_t)fp8e4m3fn_from_f32(q[e]) << (8 * e);
    uint8_t* d = dst + row * kv.hd + EPL * lane;
    if (EPL == 1) *d = (uint8_t)packed;
    else if (EPL == 2) *reinterpret_cast<uint16_t*>(d) = (uint16_t)packed;
    else *reinterpret_cast<uint32_t*>(d) = packed;
    return;
  }
  int qi[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    if (q[e] != q[e]) {
      qi[e] = 0;  // NaN -> int8 conversion yields 0 on the reference CPU path
    } else {
      const float r = fminf(fmaxf(__builtin_rintf(q[e]), -8.f), 7.f);
      qi[e] = (int)r;
    }
  }
  if (EPL == 1) {
    const int partner = __shfl_xor(qi[0], 1, 64);
    if ((lane & 1) == 0) dst[row * (kv.hd / 2) + lane / 2] = (uint8_t)((qi[0] & 0xF) | ((partner & 0xF) << 4));
  } else {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < EPL / 2; ++e)
      packed |= (uint32_t)((qi[2 * e] & 0xF) | ((qi[2 * e + 1] & 0xF) << 4)) << (8 * e);
    uint8_t* d = dst + row * (kv.hd / 2) + EPL / 2 * lane;
    if (EPL == 2) *d = (uint8_t)packed;
    else *reinterpret_cast<uint16_t*>(d) = (uint16_t)packed;
  }
}

template <int EPL>
__global__ void __launch_bounds__(kKvWriteWaves * 64)
    kv_write_row_kernel(KvView kv, const f16* __restrict__ k_rows, const f16* __restrict__ v_rows, int ld,
                        int write_pos, const int* __restrict__ write_pos_dev, int n_items) {
  const int lane = threadIdx.x & 63;
  int idx = blockIdx.x * kKvWriteWaves + (threadIdx.x >> 6);
  if (idx >= n_items) return;
  const int h = idx % kv.Hkv;
  idx /= kv.Hkv;
  const int which = idx & 1;
  const int t = idx >> 1;
  const int wp0 = write_pos_dev ? write_pos_dev[0] : write_pos;
  const int slot = (wp0 + t) % kv.S;
  const kv_hvec<EPL> xv = *reinterpret_cast<const kv_hvec<EPL>*>((which == 0 ? k_rows : v_rows) + (size_t)t * ld +
                                                                 h * kv.hd + EPL * lane);
  kv_row_store<EPL>(kv, which, h, slot, lane, xv);
}

// RoPE + KV write of T tokens in one launch (head size 128): one wave per
// (token, head row) of qkv [T][q_dim + 2 kv_dim] (bias already added); lane l
// holds rotation pair l.  Query rows are rotated at pos_dev[t] into q
// [T][q_dim], key rows rotated and value rows as they are go to slot
// (write_pos + t) % S (the arithmetic of the RoPE kernel and of kv_row_store).
__device__ __forceinline__ void rope_kv_row(const KvView& kv, int Hq, int t, int r, int lane, f16x2 v,
                                            const float* __restrict__ freqs, const int* __restrict__ pos_dev,
                                            f16* __restrict__ q, int write_pos) {
  constexpr int HD = 128;
  const int q_dim = Hq * HD;
  kv_hvec<2> out;
  if (r < Hq + kv.Hkv) {
    const float* f = freqs + ((size_t)pos_dev[t] * (HD / 2) + lane) * 2;
    out[0] = rope_out(v[0], v[1], f[0], f[1], true);
    out[1] = rope_out(v[0], v[1], f[0], f[1], false);
  } else {
    out[0] = v[0];
    out[1] = v[1];
  }
  if (r < Hq) {
    *reinterpret_cast<kv_hvec<2>*>(q + (size_t)t * q_dim + (size_t)r * HD + 2 * lane) = out;
    return;
  }
  const int which = r < Hq + kv.Hkv ? 0 : 1;
  const int h = r - Hq - which * kv.Hkv;
  kv_row_store<2>(kv, which, h, (write_pos + t) % kv.S, lane, out);
}

__global__ void __launch_bounds__(kKvWriteWaves * 64)
    rope_kv_row_kernel(KvView kv, const f16* __restrict__ qkv, int Hq, int T, const float* __restrict__ freqs,
                       const int* __restrict__ pos_dev, f16* __restrict__ q, int write_pos) {
  constexpr int HD = 128;
  const int lane = threadIdx.x & 63;
  const int rows = Hq + 2 * kv.Hkv;
  const int idx = blockIdx.x * kKvWriteWaves + (threadIdx.x >> 6);
  if (idx >= T * rows) return;
  const int t = idx / rows, r = idx % rows;
  const int qkv_dim = (Hq + 2 * kv.Hkv) * HD;
  const f16x2 v = *reinterpret_cast<const f16x2*>(qkv + (size_t)t * qkv_dim + (size_t)r * HD + 2 * lane);
  rope_kv_row(kv, Hq, t, r, lane, v, freqs, pos_dev, q, write_pos);
}

// The same, with the row taken from the K-split partial sums of the multi-token
// QKV GEMM (part [split][token (stride tok_stride)][part_cols] fp32): the splits
// are summed in order and rounded with the GEMM store epilogue's arithmetic (fp16
// of the sum, then fp16 of that plus the bias), so the row equals the one the split
// reduce would have stored; the reduce launch is saved.
__global__ void __launch_bounds__(kKvWriteWaves * 64)
    reduce_rope_kv_row_kernel(KvView kv, const float* __restrict__ part, int n_splits, int tok_stride,
                              int part_cols, const f16* __restrict__ bias, int Hq, int T,
                              const float* __restrict__ freqs, const int* __restrict__ pos_dev, f16* __restrict__ q,
                              int write_pos) {
  constexpr int HD = 128;
  const int lane = threadIdx.x & 63;
  const int rows = Hq + 2 * kv.Hkv;
  const int idx = blockIdx.x * kKvWriteWaves + (threadIdx.x >> 6);
  if (idx >= T * rows) return;
  const int t = idx / rows, r = idx % rows;
  const int col = r * HD + 2 * lane;
  float v0 = 0.f, v1 = 0.f;
  for (int sp = 0; sp < n_splits; ++sp) {
    const float2 pv = *reinterpret_cast<const float2*>(part + ((size_t)sp * tok_stride + t) * part_cols + col);
    v0 += pv.x;
    v1 += pv.y;
  }
  f16 h0 = f2h(v0), h1 = f2h(v1);
  if (bias != nullptr) {
    h0 = f2h(h2f(h0) + h2f(bias[col]));
    h1 = f2h(h2f(h1) + h2f(bias[col + 1]));
  }
  rope_kv_row(kv, Hq, t, r, lane, f16x2{h0, h1}, freqs, pos_dev, q, write_pos);
}

// Fused bias + RoPE + KV-cache write of T tokens (rope_kv_cache_write_half_kernel,
// metal_kernels.metal:991-1036; fp8/int4 :1110-1279; tree variants :2862-2918,
// :1282-1473).  qkv [T][q_dim + 2 kv_dim] fp16, updated in place for the query
// part: token t is rotated at pos[t]; its rotated key and its value go to slot
// (write_pos + t) % S.  One wave per (token, 64-element chunk of the row).
struct RopePositions {
  int pos[64];
};

__global__ void __launch_bounds__(64) rope_kv_write_kernel(f16* __restrict__ qkv, const f16* __restrict__ bias,
                                                           const float* __restrict__ freqs, RopePositions rp,
                                                           int q_dim, int kv_dim, KvView kv, int write_pos) {
  const int lane = threadIdx.x;
  const int t = blockIdx.y;
  const int qkv_dim = q_dim + 2 * kv_dim;
  const int e = blockIdx.x * 64 + lane;
  const int hd = kv.hd;
  f16* row = qkv + (size_t)t * qkv_dim;
  const int slot = (write_pos + t) % kv.S;
  const bool quant = kv.kv_dtype != AXM_KV_FP16;
  if (e >= qkv_dim) return;  // only the fp16 cache allows a partial last chunk
  f16 x = row[e];
  f16 xp = row[e ^ 1];
  if (bias != nullptr) {
    x = hadd(x, bias[e]);
    xp = hadd(xp, bias[e ^ 1]);
  }
  if (e < q_dim + kv_dim) {
    const int within = e < q_dim ? e : e - q_dim;
    const int fi = (within % hd) >> 1;
    const float* f = freqs + ((size_t)rp.pos[t] * (hd / 2) + fi) * 2;
    const bool even = (e & 1) == 0;
    x = even ? rope_out(x, xp, f[0], f[1], true) : rope_out(xp, x, f[0], f[1], false);
  }
  if (e < q_dim) {
    row[e] = x;
    return;
  }
  const int which = e < q_dim + kv_dim ? 0 : 1;
  const int within = e - q_dim - which * kv_dim;
  const int h = within / hd, c = within % hd;
  if (!quant) {
    f16* dst = (f16*)(which == 0 ? kv.k : kv.v);
    dst[((size_t)h * kv.S + slot) * hd + c] = x;
    return;
  }
  kv_store_lane(kv, which, h, slot, c / 64, lane, x);
}

// Dequantized key/value chunk: 8 consecutive elements starting at e0 of slot `slot`.
// Values are rounded to fp16 exactly as the reference CPU dequantizers do
// (fp8 -> fp16 exact, then fp16 * fp16 scale rounded; int4 q * scale rounded).
template <int KVT>
__device__ __forceinline__ void load_kv8(const void* base, const f16* scales, size_t row, int hd, int e0,
                                         float out[8]) {
  if (KVT == AXM_KV_FP16) {
    const f16x8 v = *reinterpret_cast<const f16x8*>((const f16*)base + row * hd + e0);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = h2f(v[i]);
  } else if (KVT == AXM_KV_FP8) {
    const u32x2 v = *reinterpret_cast<const u32x2*>((const uint8_t*)base + row * hd + e0);
    const float sc = h2f(scales[row * (hd / 64) + e0 / 64]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t b = (v[i >> 2] >> (8 * (i & 3))) & 0xFFu;
      out[i] = h2f(f2h(fp8e4m3fn_to_f32(b) * sc));
    }
  } else {
    const uint32_t v = *reinterpret_cast<const uint32_t*>((const uint8_t*)base + row * (hd / 2) + e0 / 2);
    const float sc = h2f(scales[row * (hd / 64) + e0 / 64]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = (int)(((v >> (4 * i)) & 0xFu) ^ 0x8u) - 8;
      out[i] = h2f(f2h((float)q * sc));
    }
  }
}

// A raw 8-element key/value chunk (fp16: 16 B, fp8: 8 B, int4: 4 B) and its fp16
// group scale become eight fp32 values with the rounding of load_kv8.
// HW: fp8 codes through v_cvt_pk_f32_fp8 (OCP E4M3FN on gfx950; every finite
// code converts exactly, so the result equals the table-free decode below for
// all non-NaN codes).  The attention kernels use it; the dequantization entry
// point keeps the bitwise decode so that NaN codes keep their exact pattern.
typedef float f32x2_hw __attribute__((ext_vector_type(2)));
template <int KVT, bool HW = false>
__device__ __forceinline__ void kv8_convert(u32x4 r, float sc, float out[8]) {
  if (KVT == AXM_KV_FP8 && HW) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t word = r[w];
      const f32x2_hw lo = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
      const f32x2_hw hi = __builtin_amdgcn_cvt_pk_f32_fp8(word, true);
      out[4 * w + 0] = h2f(f2h(lo.x * sc));
      out[4 * w + 1] = h2f(f2h(lo.y * sc));
      out[4 * w + 2] = h2f(f2h(hi.x * sc));
      out[4 * w + 3] = h2f(f2h(hi.y * sc));
    }
    return;
  }
  if (KVT == AXM_KV_FP16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = r[i];
      const f16x2 h = as_h2(w);
      out[2 * i] = h2f(h.x);
      out[2 * i + 1] = h2f(h.y);
    }
  } else if (KVT == AXM_KV_FP8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = r[i >> 2];
      out[i] = h2f(f2h(fp8e4m3fn_to_f32((w >> (8 * (i & 3))) & 0xFFu) * sc));
    }
  } else {
    const uint32_t w = r.x;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = (int)(((w >> (4 * i)) & 0xFu) ^ 0x8u) - 8;
      out[i] = h2f(f2h((float)q * sc));
    }
  }
}

// 8 consecutive elements [e0, e0 + 8) of a cache row: raw codes and the raw
// fp16 group scale, fetched ahead of use through bounded buffer descriptors
// over one head's slots (an out-of-range offset reads zeros, so fetches of keys
// past the range need no branch), converted to fp16 with the reference
// rounding only when consumed.  A conditional fetch, or converting the scale
// at the fetch, made the compiler wait for each load right after issuing it.
struct KvRaw8 {
  u32x4 r;
  uint32_t sc;  // fp16 bits in the low half
};
struct KvHead {
  __amdgpu_buffer_rsrc_t codes, scales;
};
template <int KVT>
__device__ __forceinline__ int kv_row_bytes(int hd) {
  return KVT == AXM_KV_FP16 ? hd * 2 : (KVT == AXM_KV_FP8 ? hd : hd / 2);
}
template <int KVT>
__device__ __forceinline__ KvHead kv_head(const void* base, const f16* scales, size_t head_row0, int S, int hd) {
  KvHead h;
  const int rb = kv_row_bytes<KVT>(hd);
  h.codes = __builtin_amdgcn_make_buffer_rsrc((void*)((const uint8_t*)base + head_row0 * rb), (short)0, S * rb,
                                              0x00020000);
  h.scales = h.codes;
  if (KVT != AXM_KV_FP16)
    h.scales = __builtin_amdgcn_make_buffer_rsrc((void*)(scales + head_row0 * (hd / 64)), (short)0,
                                                 S * (hd / 64) * 2, 0x00020000);
  return h;
}
template <int KVT>
__device__ __forceinline__ KvRaw8 kv_fetch8(const KvHead& h, int slot, int hd, int e0, bool ok) {
  constexpr int kOff = 0x7FFFFFF0;
  const int rb = kv_row_bytes<KVT>(hd);
  KvRaw8 f;
  f.r = u32x4{0u, 0u, 0u, 0u};
  f.sc = 0u;
  if (KVT == AXM_KV_FP16) {
    f.r = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(h.codes, ok ? slot * rb + e0 * 2 : kOff, 0, 0));
  } else if (KVT == AXM_KV_FP8) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(h.codes, ok ? slot * rb + e0 : kOff, 0, 0));
    f.r.x = v.x;
    f.r.y = v.y;
  } else {
    f.r.x = __builtin_amdgcn_raw_buffer_load_b32(h.codes, ok ? slot * rb + e0 / 2 : kOff, 0, 0);
  }
  if (KVT != AXM_KV_FP16)
    f.sc = __builtin_amdgcn_raw_buffer_load_b16(h.scales, ok ? (slot * (hd / 64) + e0 / 64) * 2 : kOff, 0, 0);
  return f;
}
// NC consecutive 8-element chunks [e0, e0 + 8 NC) of a cache row (all inside one
// 64-element scale group) in as few loads as their bytes allow (int4 with NC 4:
// one 16-byte load and one scale load instead of four of each).
template <int KVT, int NC>
struct KvRun {
  static constexpr int kDw8 = KVT == AXM_KV_FP16 ? 4 : (KVT == AXM_KV_FP8 ? 2 : 1);  // dwords per chunk
  static constexpr int kDw = NC * kDw8;
  uint32_t w[kDw];
  uint32_t sc;  // fp16 bits in the low half
  __device__ __forceinline__ KvRaw8 chunk(int c) const {
    KvRaw8 f;
    f.r = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int d = 0; d < kDw8; ++d) f.r[d] = w[c * kDw8 + d];
    f.sc = sc;
    return f;
  }
};
template <int KVT, int NC>
__device__ __forceinline__ KvRun<KVT, NC> kv_fetch_run(const KvHead& h, int slot, int hd, int e0, bool ok = true) {
  using Run = KvRun<KVT, NC>;
  constexpr int kOff = 0x7FFFFFF0;
  const int eb = KVT == AXM_KV_FP16 ? 2 * e0 : (KVT == AXM_KV_FP8 ? e0 : e0 / 2);
  const int off = ok ? slot * kv_row_bytes<KVT>(hd) + eb : kOff;
  Run r;
  if constexpr (Run::kDw % 4 == 0) {
#pragma unroll
    for (int i = 0; i < Run::kDw / 4; ++i) {
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(h.codes, off + 16 * i, 0, 0));
      r.w[4 * i + 0] = v.x;
      r.w[4 * i + 1] = v.y;
      r.w[4 * i + 2] = v.z;
      r.w[4 * i + 3] = v.w;
    }
  } else if constexpr (Run::kDw == 2) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(h.codes, off, 0, 0));
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else {
    r.w[0] = __builtin_amdgcn_raw_buffer_load_b32(h.codes, off, 0, 0);
  }
  r.sc = 0u;
  if (KVT != AXM_KV_FP16)
    r.sc = __builtin_amdgcn_raw_buffer_load_b16(h.scales, ok ? (slot * (hd / 64) + e0 / 64) * 2 : kOff, 0, 0);
  return r;
}

// Position e of an f16x8 from kv_half8 holds element kv_dim_of<KVT>(e) of the chunk:
// the int4 form delivers the even elements 0, 2, 4, 6, then the odd ones.
template <int KVT>
__device__ __forceinline__ constexpr int kv_dim_of(int e) {
  return KVT == AXM_KV_INT4 ? ((e & 3) << 1) | (e >> 2) : e;
}

// Eight consecutive query elements in the order kv_half8 delivers the chunk's
// elements (the MFMA k index then pairs each query element with its key element).
template <int KVT>
__device__ __forceinline__ f16x8 kv_order8(f16x8 v) {
  f16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = v[kv_dim_of<KVT>(e)];
  return r;
}

template <int KVT>
__device__ __forceinline__ f16x8 kv_half8(const KvRaw8& f) {
  if (KVT == AXM_KV_FP16) return __builtin_bit_cast(f16x8, f.r);
  if (KVT == AXM_KV_INT4) {
    // u = nibble ^ 8 = q + 8 in [0, 15].  The even nibbles (one per byte of lo) and
    // the odd ones (hi) become, by one byte permute per pair with the exponent byte
    // 0x64, the exact halves 1024 + u; minus 1032 gives q exactly, and one fp16
    // multiply by the scale rounds q * scale once (the fp32 product of a 4-bit
    // integer and an fp16 scale is exact, so this equals fp16(float(q) * scale)).
    const uint32_t u = f.r.x ^ 0x88888888u;
    const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
    const f16 sc = u16_as_h((uint16_t)f.sc);
    const f16x2 s2 = {sc, sc};
    const f16x2 off = {(f16)1032.f, (f16)1032.f};
    const uint32_t pr[4] = {__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u),
                            __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u),
                            __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u),
                            __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)};
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = as_u32((as_h2(pr[i]) - off) * s2);
    return __builtin_bit_cast(f16x8, o);
  }
  if (KVT == AXM_KV_FP8) {
    // Two E4M3FN codes -> two fp16 per conversion (scale 1.0: every finite code is
    // an exact fp16), then one fp16 multiply rounds code * scale once, as the fp32
    // product (exact: 4 x 11 significant bits) rounded to fp16 does.
    const f16 sc = u16_as_h((uint16_t)f.sc);
    const f16x2 s2 = {sc, sc};
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      o[2 * w] = as_u32(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(f.r[w], 1.0f, false) * s2);
      o[2 * w + 1] = as_u32(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(f.r[w], 1.0f, true) * s2);
    }
    return __builtin_bit_cast(f16x8, o);
  }
  float x[8];
  kv8_convert<KVT, true>(f.r, h2f(u16_as_h((uint16_t)f.sc)), x);
  f16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = f2h(x[i]);
  return h;
}

// Sum over the LPT lanes that hold one key row (aligned groups of 8 or 16
// lanes; hd = 64 or 128) with DPP lane permutes instead of LDS-routed
// shuffles: xor 1 and xor 2 within each quad, then the 8-lane and 16-lane
// mirrors pair each lane with the complementary half.
template <int CTRL>
__device__ __forceinline__ float dpp_sum_step(float v) {
  const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
  return v + __builtin_bit_cast(float, o);
}
// Packed halves in the operand type of v_dot2_f32_f16 (products exact in fp32,
// accumulated in fp32).
typedef __fp16 dot_h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ dot_h2 as_dot_h2(uint32_t u) { return __builtin_bit_cast(dot_h2, u); }

// 2^x with the bare v_exp_f32: softmax weights below 2^-126 of the running
// maximum are flushed to zero instead of kept as denormals, which changes no
// fp16 output.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float key_row_sum(float v, int lpt) {
  if (lpt == 16 || lpt == 8) {
    v = dpp_sum_step<0xB1>(v);   // quad_perm [1,0,3,2]
    v = dpp_sum_step<0x4E>(v);   // quad_perm [2,3,0,1]
    v = dpp_sum_step<0x141>(v);  // row_half_mirror
    if (lpt == 16) v = dpp_sum_step<0x140>(v);  // row_mirror
    return v;
  }
  for (int off = lpt / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

struct AttnParams {
  const f16* q;           // query rows, row r at q + r_off(r)
  KvView kv;
  f16* out;
  float* ws;              // partials [n_rows_total][n_splits][2 + hd]
  f16* parts_o;           // decode, merged by the consumer: o / l per split [n_splits][rows][hd]
  f32x2* parts_ml;        //   and (running max m, sum l) per split [n_splits][rows]
  int Hq, n_rep;
  int n_splits;
  int prefix_len;         // keys [0, prefix_len) (decode: active_len)
  const int* prefix_dev;  // overrides prefix_len when non-null
  int T;                  // tree nodes (0 for decode)
  int short_splits;       // decode: <= 64 keys per split (4-wave workgroups)
  int write_pos;          // slot of tree node 0
  const uint64_t* masks;  // [T] ancestor bitmasks (tree mode)
  float scale_log2;       // log2(e) / sqrt(hd)
};

// Rows of one workgroup: decode -> (b, kv head, replica r) with r < n_rep;
// tree -> (node u, kv head, replica) flattened, QR rows per workgroup.
// NW waves per workgroup; each wave fetches the keys / values of U steps
// (U * 64 / (hd / 8) keys) before consuming them, so a workgroup keeps
// NW * U loads per lane pair in flight.
template <int KVT, int QR, bool TREE, int NW, int U>
__global__ void __launch_bounds__(NW * 64) attn_split_kernel(AttnParams p) {
  constexpr int kThreads = NW * 64;
  const int hd = p.kv.hd;
  const int LPT = hd / 8;        // lanes per key
  const int KPW = 64 / LPT;      // keys per wave step
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / LPT;    // key sub-slot within the wave
  const int e0 = (lane % LPT) * 8;

  // Work decomposition.
  const int split = blockIdx.y;
  const int kvh_all = blockIdx.x;  // (b, kv head) or (row chunk, kv head) in tree mode
  int b, kvh, row_base, n_rows;
  if (!TREE) {
    b = kvh_all / p.kv.Hkv;
    kvh = kvh_all % p.kv.Hkv;
    row_base = blockIdx.z * QR;  // replica chunk
    n_rows = min(QR, p.n_rep - row_base);
  } else {
    b = 0;
    kvh = kvh_all % p.kv.Hkv;
    const int chunk = kvh_all / p.kv.Hkv;  // chunk over (node, replica) pairs
    row_base = chunk * QR;
    n_rows = min(QR, p.T * p.n_rep - row_base);
  }
  if (n_rows <= 0) return;

  const int prefix = p.prefix_dev ? p.prefix_dev[0] : p.prefix_len;
  const int n_keys = prefix + (TREE ? p.T : 0);
  const int per = (n_keys + p.n_splits - 1) / p.n_splits;
  const int k_begin = min(split * per, n_keys);
  const int k_end = min(k_begin + per, n_keys);
  const size_t head_row0 = ((size_t)b * p.kv.Hkv + kvh) * p.kv.S;

  // Keys / values of U steps; the first batch is requested before the query
  // rows so that the two latencies overlap.
  u32x4 kr[U], vr[U];
  uint32_t ksc[U], vsc[U];  // raw fp16 group scales
  const KvHead kh = kv_head<KVT>(p.kv.k, p.kv.ks, head_row0, p.kv.S, hd);
  const KvHead vh = kv_head<KVT>(p.kv.v, p.kv.vs, head_row0, p.kv.S, hd);
  auto fetch = [&](int kb0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int key = kb0 + u * NW * KPW + sub;
      int slot = key;
      if (TREE && key >= prefix) slot = (p.write_pos + (key - prefix)) % p.kv.S;
      const KvRaw8 fk = kv_fetch8<KVT>(kh, slot, hd, e0, key < k_end);
      const KvRaw8 fv = kv_fetch8<KVT>(vh, slot, hd, e0, key < k_end);
      kr[u] = fk.r;
      ksc[u] = fk.sc;
      vr[u] = fv.r;
      vsc[u] = fv.sc;
    }
  };
  int kb0 = k_begin + wave * KPW;
  if (kb0 < k_end) fetch(kb0);

  // Global query-row index and query pointers.
  float q[QR][8];
  dot_h2 qh[QR][4];  // the same query halves packed for v_dot2_f32_f16 (fp16 KV)
  int qrow[QR];
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    int hq, tok;
    if (!TREE) {
      tok = b;
      hq = kvh * p.n_rep + row_base + r;
    } else {
      const int rr = row_base + r;
      tok = rr / p.n_rep;
      hq = kvh * p.n_rep + rr % p.n_rep;
    }
    qrow[r] = tok * p.Hq + hq;
    if (r < n_rows) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(p.q + (size_t)qrow[r] * hd + e0);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[r][i] = h2f(v[i]);
#pragma unroll
      for (int i = 0; i < 4; ++i) qh[r][i] = dot_h2{(__fp16)v[2 * i], (__fp16)v[2 * i + 1]};
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) q[r][i] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) qh[r][i] = dot_h2{(__fp16)0.f, (__fp16)0.f};
    }
  }

  float m[QR], l[QR], o[QR][8];
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    m[r] = kNegBig;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[r][i] = 0.f;
  }

  uint64_t node_mask[QR];
  if (TREE) {
#pragma unroll
    for (int r = 0; r < QR; ++r) node_mask[r] = r < n_rows ? p.masks[(row_base + r) / p.n_rep] : 0ull;
  }

  for (; kb0 < k_end; kb0 += NW * KPW * U) {
    // This batch's keys / values; the next batch is requested before they are
    // consumed, so one batch of loads is always in flight.
    u32x4 kcur[U], vcur[U];
    uint32_t kscur[U], vscur[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      kcur[u] = kr[u];
      vcur[u] = vr[u];
      kscur[u] = ksc[u];
      vscur[u] = vsc[u];
    }
    if (kb0 + NW * KPW * U < k_end) fetch(kb0 + NW * KPW * U);
    // Steps of this batch that hold at least one key of the range (wave-uniform);
    // the scores of the batch are taken first so that the running maximum and
    // the rescaling of (l, o) happen once per batch instead of once per key.
    const int n_steps = min(U, (k_end - kb0 + NW * KPW - 1) / (NW * KPW));
    float sc[QR][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u < n_steps) {
        const int key = kb0 + u * NW * KPW + sub;
        const bool valid = key < k_end;
        float kf[8];
        if constexpr (KVT != AXM_KV_FP16) kv8_convert<KVT, true>(kcur[u], h2f(u16_as_h((uint16_t)kscur[u])), kf);
#pragma unroll
        for (int r = 0; r < QR; ++r) {
          float d = 0.f;
          if constexpr (KVT == AXM_KV_FP16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) d = __builtin_amdgcn_fdot2(qh[r][i], as_dot_h2(kcur[u][i]), d, false);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) d = __builtin_fmaf(q[r][i], kf[i], d);
          }
          d = key_row_sum(d, LPT);
          bool vis = valid && r < n_rows;
          if (TREE && key >= prefix) vis = vis && ((node_mask[r] >> (key - prefix)) & 1ull);
          sc[r][u] = vis ? d * p.scale_log2 : kNegBig;
        }
      }
    }
    float vf[U][8];
    if constexpr (KVT != AXM_KV_FP16) {
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u < n_steps) kv8_convert<KVT, true>(vcur[u], h2f(u16_as_h((uint16_t)vscur[u])), vf[u]);
    }
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      float m_new = m[r];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u < n_steps) m_new = fmaxf(m_new, sc[r][u]);
      const float alpha = fast_exp2(m[r] - m_new);
      float lsum = l[r] * alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[r][i] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (u < n_steps) {
          const float pr = sc[r][u] == kNegBig ? 0.f : fast_exp2(sc[r][u] - m_new);
          lsum += pr;
          if constexpr (KVT == AXM_KV_FP16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f16x2 vh = as_h2(vcur[u][i]);
              o[r][2 * i] = __builtin_fmaf(pr, h2f(vh.x), o[r][2 * i]);
              o[r][2 * i + 1] = __builtin_fmaf(pr, h2f(vh.y), o[r][2 * i + 1]);
            }
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) o[r][i] = __builtin_fmaf(pr, vf[u][i], o[r][i]);
          }
        }
      }
      l[r] = lsum;
      m[r] = m_new;
    }
  }

  // Merge the KPW key sub-slots of the wave (lanes with equal e0).
#pragma unroll
  for (int r = 0; r < QR; ++r) {
    for (int off = LPT; off < 64; off <<= 1) {
      const float m2 = __shfl_xor(m[r], off, 64);
      const float l2 = __shfl_xor(l[r], off, 64);
      const float mn = fmaxf(m[r], m2);
      const float a1 = exp2f(m[r] - mn), a2 = exp2f(m2 - mn);
      l[r] = l[r] * a1 + l2 * a2;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float o2 = __shfl_xor(o[r][i], off, 64);
        o[r][i] = o[r][i] * a1 + o2 * a2;
      }
      m[r] = mn;
    }
  }

  // Merge the waves through LDS: [wave][r][2 + hd].
  __shared__ float sm[NW][QR][2 + 128];
  if (lane < LPT) {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      if (lane == 0) {
        sm[wave][r][0] = m[r];
        sm[wave][r][1] = l[r];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) sm[wave][r][2 + e0 + i] = o[r][i];
    }
  }
  __syncthreads();
  // Thread t handles (r, e) pairs.
  for (int idx = threadIdx.x; idx < QR * hd; idx += kThreads) {
    const int r = idx / hd, e = idx % hd;
    if (r >= n_rows) continue;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < NW; ++w) mm = fmaxf(mm, sm[w][r][0]);
    float ll = 0.f, oo = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = exp2f(sm[w][r][0] - mm);
      ll += sm[w][r][1] * a;
      oo += sm[w][r][2 + e] * a;
    }
    if (p.n_splits == 1) {
      const int gr = (!TREE) ? (b * p.Hq + kvh * p.n_rep + row_base + r)
                             : (((row_base + r) / p.n_rep) * p.Hq + kvh * p.n_rep + (row_base + r) % p.n_rep);
      p.out[(size_t)gr * hd + e] = f2h(ll > 0.f ? oo / ll : 0.f);
    } else if (!TREE && p.parts_o != nullptr) {
      const int gr = b * p.Hq + kvh * p.n_rep + row_base + r;
      const size_t rows_total = (size_t)p.kv.B * p.Hq;
      p.parts_o[((size_t)split * rows_total + gr) * hd + e] = f2h(ll > 0.f ? oo / ll : 0.f);
      if (e == 0) p.parts_ml[(size_t)split * rows_total + gr] = f32x2{mm, ll};
    } else {
      const int gr = (!TREE) ? (b * p.Hq + kvh * p.n_rep + row_base + r)
                             : (((row_base + r) / p.n_rep) * p.Hq + kvh * p.n_rep + (row_base + r) % p.n_rep);
      float* dst = p.ws + ((size_t)gr * p.n_splits + split) * (2 + hd);
      if (e == 0) {
        dst[0] = mm;
        dst[1] = ll;
      }
      dst[2 + e] = oo;
    }
  }
}

// Merges the split partials of one query row: wave 0 takes the splits' (m, l)
// (one split per lane, in steps of 64), forms the global max, the weights
// 2^(m_s - max) (kept in LDS) and the total l; then thread e sums its output
// element over the splits in order, all split loads independent.
// Launch: max(hd, 64) threads rounded to whole waves, (n_splits + 1) floats of LDS.
__global__ void attn_reduce_kernel(const float* __restrict__ ws, f16* __restrict__ out, int n_splits, int hd) {
  extern __shared__ float a_sh[];
  const int row = blockIdx.x;
  const int e = threadIdx.x;
  const size_t st = 2 + hd;
  const float* base = ws + (size_t)row * n_splits * st;
  if (e < 64) {
    float mm = kNegBig;
    for (int sp = e; sp < n_splits; sp += 64) mm = fmaxf(mm, base[sp * st]);
    mm = wave_max(mm);
    float ll = 0.f;
    for (int sp = e; sp < n_splits; sp += 64) {
      const float a = exp2f(base[sp * st] - mm);
      a_sh[sp] = a;
      ll += base[sp * st + 1] * a;
    }
    ll = wave_sum(ll);
    if (e == 0) a_sh[n_splits] = ll;
  }
  __syncthreads();
  if (e >= hd) return;
  const float ll = a_sh[n_splits];
  float oo = 0.f;
#pragma unroll 8
  for (int sp = 0; sp < n_splits; ++sp) oo += base[sp * st + 2 + e] * a_sh[sp];
  out[(size_t)row * hd + e] = f2h(ll > 0.f ? oo / ll : 0.f);
}

// Up to kReduceRegSplits splits: every thread requests the (m, l) of all splits
// and its output element of each at once, one round of loads with no barrier,
// and sums in split order.
constexpr int kReduceRegSplits = 16;
__global__ void attn_reduce_reg_kernel(const float* __restrict__ ws, f16* __restrict__ out, int n_splits, int hd) {
  const int row = blockIdx.x;
  const int e = threadIdx.x;
  if (e >= hd) return;
  const size_t st = 2 + hd;
  const float* base = ws + (size_t)row * n_splits * st;
  float mv[kReduceRegSplits], lv[kReduceRegSplits], ov[kReduceRegSplits];
#pragma unroll
  for (int sp = 0; sp < kReduceRegSplits; ++sp) {
    // Splits past n_splits load the last one (always in range) and are masked.
    const bool in = sp < n_splits;
    const float* src = base + (size_t)min(sp, n_splits - 1) * st;
    const float m0 = src[0], l0 = src[1], o0 = src[2 + e];
    mv[sp] = in ? m0 : kNegBig;
    lv[sp] = in ? l0 : 0.f;
    ov[sp] = in ? o0 : 0.f;
  }
  float mm = kNegBig;
#pragma unroll
  for (int sp = 0; sp < kReduceRegSplits; ++sp) mm = fmaxf(mm, mv[sp]);
  float ll = 0.f, oo = 0.f;
#pragma unroll
  for (int sp = 0; sp < kReduceRegSplits; ++sp) {
    if (sp < n_splits) {
      const float a = exp2f(mv[sp] - mm);
      ll += lv[sp] * a;
      oo += ov[sp] * a;
    }
  }
  out[(size_t)row * hd + e] = f2h(ll > 0.f ? oo / ll : 0.f);
}

void launch_attn_reduce(const float* ws, f16* out, int rows, int n_splits, int hd, hipStream_t s) {
  const int threads = ((hd > 64 ? hd : 64) + 63) / 64 * 64;
  if (n_splits <= kReduceRegSplits) {
    hipLaunchKernelGGL(attn_reduce_reg_kernel, dim3(rows), dim3(threads), 0, s, ws, out, n_splits, hd);
    return;
  }
  hipLaunchKernelGGL(attn_reduce_kernel, dim3(rows), dim3(threads), (n_splits + 1) * sizeof(float), s, ws, out,
                     n_splits, hd);
}

// Decode uses 16 waves (8 for more than 2 rows per workgroup, which need the
// registers) with 4 steps of loads in flight; tree verification keeps 4 waves,
// one step.
template <int KVT, int QR, bool TREE>
void launch_attn_t(const AttnParams& p, dim3 grid, hipStream_t s) {
  if constexpr (TREE) {
    hipLaunchKernelGGL((attn_split_kernel<KVT, QR, TREE, kAttnWaves, 1>), grid, dim3(kAttnThreads), 0, s, p);
  } else {
    // 16 waves (8 for more than 2 rows, which need the registers); splits of at
    // most 64 keys (one batch of four 4-wave key steps) take 4-wave workgroups,
    // whose merge is cheaper (7B decode at 250 keys: 1.514 -> 1.498 ms/token;
    // 16 waves stay faster from 1k keys).
    constexpr int nw = QR <= 2 ? 16 : 8;
    if (QR <= 2 && p.short_splits)
      hipLaunchKernelGGL((attn_split_kernel<KVT, QR, TREE, 4, 4>), grid, dim3(4 * 64), 0, s, p);
    else
      hipLaunchKernelGGL((attn_split_kernel<KVT, QR, TREE, nw, 4>), grid, dim3(nw * 64), 0, s, p);
  }
}

template <bool TREE>
int launch_attn_dispatch(const AttnParams& p, int qr, dim3 grid, hipStream_t s) {
#define AXM_ATTN_QR(KVT)                                              \
  switch (qr) {                                                       \
    case 1: launch_attn_t<KVT, 1, TREE>(p, grid, s); return 0;        \
    case 2: launch_attn_t<KVT, 2, TREE>(p, grid, s); return 0;        \
    case 4: launch_attn_t<KVT, 4, TREE>(p, grid, s); return 0;        \
    case 8: launch_attn_t<KVT, 8, TREE>(p, grid, s); return 0;        \
  }                                                                   \
  break;
  switch (p.kv.kv_dtype) {
    case AXM_KV_FP16: AXM_ATTN_QR(AXM_KV_FP16)
    case AXM_KV_FP8: AXM_ATTN_QR(AXM_KV_FP8)
    case AXM_KV_INT4: AXM_ATTN_QR(AXM_KV_INT4)
  }
#undef AXM_ATTN_QR
  axm_set_error("attention: unsupported kv dtype %d / rows %d", p.kv.kv_dtype, qr);
  return -2;
}

int pick_qr(int rows) {
  if (rows <= 1) return 1;
  if (rows <= 2) return 2;
  if (rows <= 4) return 4;
  return 8;
}

}  // namespace

int launch_kv_write(const KvView& kv, const f16* k_rows, const f16* v_rows, int ld_rows, int T, int write_pos,
                    const int* write_pos_dev, hipStream_t s) {
  const int G = kv.hd / 64;
  const int epl = G;  // elements per lane of the row form
  const uintptr_t al = (uintptr_t)k_rows | (uintptr_t)v_rows;
  if ((epl == 1 || epl == 2 || epl == 4) && ld_rows % epl == 0 && al % (2 * epl) == 0) {
    const int items = T * 2 * kv.Hkv;
    const unsigned blocks = (unsigned)((items + kKvWriteWaves - 1) / kKvWriteWaves);
    const dim3 b(kKvWriteWaves * 64);
    if (epl == 1)
      hipLaunchKernelGGL(kv_write_row_kernel<1>, dim3(blocks), b, 0, s, kv, k_rows, v_rows, ld_rows, write_pos,
                         write_pos_dev, items);
    else if (epl == 2)
      hipLaunchKernelGGL(kv_write_row_kernel<2>, dim3(blocks), b, 0, s, kv, k_rows, v_rows, ld_rows, write_pos,
                         write_pos_dev, items);
    else
      hipLaunchKernelGGL(kv_write_row_kernel<4>, dim3(blocks), b, 0, s, kv, k_rows, v_rows, ld_rows, write_pos,
                         write_pos_dev, items);
    return 0;
  }
  const int items = T * 2 * kv.Hkv * G;
  const unsigned blocks = (unsigned)((items + kKvWriteWaves - 1) / kKvWriteWaves);
  hipLaunchKernelGGL(kv_write_kernel, dim3(blocks), dim3(kKvWriteWaves * 64), 0, s, kv, k_rows, v_rows, ld_rows,
                     write_pos, write_pos_dev, items);
  return 0;
}

int launch_rope_kv_write(const KvView& kv, const f16* qkv, int Hq, int T, const float* freqs, const int* pos_dev,
                         f16* q, int write_pos, hipStream_t s) {
  if (kv.hd != 128 || ((uintptr_t)qkv & 3) != 0 || ((uintptr_t)q & 3) != 0) {
    axm_set_error("rope_kv_write: head size %d (128) or misaligned rows", kv.hd);
    return -2;
  }
  const int items = T * (Hq + 2 * kv.Hkv);
  hipLaunchKernelGGL(rope_kv_row_kernel, dim3((unsigned)((items + kKvWriteWaves - 1) / kKvWriteWaves)),
                     dim3(kKvWriteWaves * 64), 0, s, kv, qkv, Hq, T, freqs, pos_dev, q, write_pos);
  return 0;
}

int launch_reduce_rope_kv_write(const KvView& kv, const float* part, int n_splits, int tok_stride, int part_cols,
                                const f16* bias, int Hq, int T, const float* freqs, const int* pos_dev, f16* q,
                                int write_pos, hipStream_t s) {
  const int qkv_dim = (Hq + 2 * kv.Hkv) * kv.hd;
  if (kv.hd != 128 || ((uintptr_t)q & 3) != 0 || n_splits < 1 || tok_stride < T || part_cols < qkv_dim ||
      (part_cols & 1) != 0 || ((uintptr_t)part & 7) != 0) {
    axm_set_error("reduce_rope_kv_write: head size %d (128), %d splits, token stride %d, %d partial columns",
                  kv.hd, n_splits, tok_stride, part_cols);
    return -2;
  }
  const int items = T * (Hq + 2 * kv.Hkv);
  hipLaunchKernelGGL(reduce_rope_kv_row_kernel, dim3((unsigned)((items + kKvWriteWaves - 1) / kKvWriteWaves)),
                     dim3(kKvWriteWaves * 64), 0, s, kv, part, n_splits, tok_stride, part_cols, bias, Hq, T, freqs,
                     pos_dev, q, write_pos);
  return 0;
}

size_t attn_workspace_bytes(int B, int Hq, int hd, int n_splits) {
  return n_splits <= 1 ? 0 : (size_t)B * Hq * n_splits * (2 + hd) * sizeof(float);
}

int attn_choose_splits(int B, int Hkv, int active_len) {
  // Measured with 16-wave decode workgroups (32 KV heads, hd 128): one
  // workgroup per head is fastest up to 512 keys; beyond that a four-way split
  // (128 workgroups) is fastest from 1k to 4k keys.  Fewer (batch x head) rows
  // take proportionally more splits; every split keeps >= 128 keys.
  // Long contexts take about four workgroups per CU (>= 256 keys each) so that
  // enough key batches are in flight.
  const int rows = B * Hkv;
  const int want_wg = active_len <= 512 ? 32 : (active_len <= 4096 ? 128 : 4 * axm_num_cus());
  int splits = (want_wg + rows - 1) / rows;
  const int by_len = active_len <= 4096 ? (active_len + 127) / 128 : (active_len + 255) / 256;
  if (splits > by_len) splits = by_len;
  if (splits > 64) splits = 64;
  if (splits < 1) splits = 1;
  return splits;
}

int attn_flash_splits(int B, int Hq, int Hkv, int hd, int kv_dtype, int active_len) {
  const int n_rep = Hkv > 0 ? Hq / Hkv : 0;
  if (!(n_rep >= 2 && n_rep <= 16 && (hd == 64 || hd == 128))) return attn_choose_splits(B, Hkv, active_len);
  // Matrix-core decode (4-wave workgroups, 32-key blocks).  Measured on the C3
  // shape (batch 8, 32 query / 8 KV heads of 128, 1k-32k keys): fastest at
  // about two workgroups per CU for int4 / fp16 caches and one per CU for fp8
  // (whose two-block prefetch holds more registers), with every split keeping
  // >= 256 keys, two 32-key blocks per wave (1k int4 keys: 4 splits 9.4 us,
  // 8 splits 9.9 us; half or a quarter of the chosen splits were slower at every C3
  // length, e.g. 1k int4 keys 11.1 / 12.6 us, 32k fp8 137 / 237 against 101 us).
  const int rows = B * Hkv;
  const int target = (kv_dtype == AXM_KV_FP8 ? 1 : 2) * axm_num_cus();
  int splits = (target + rows - 1) / rows;
  const int by_len = (active_len + 255) / 256;
  if (splits > by_len) splits = by_len;
  if (splits > 64) splits = 64;
  if (splits < 1) splits = 1;
  return splits;
}

int attn_parts_splits(int B, int Hkv, int active_len) {
  // Split partials merged by the consumer cost no reduce launch, so the split
  // count aims at one workgroup per CU (measured on 32 heads x 128: eight
  // splits fastest from 250 to 1k keys) with >= 16 keys per split.
  const int rows = B * Hkv;
  int splits = 1;
  while (splits < kAttnMaxParts && rows * splits < 256) splits <<= 1;
  while (splits > 1 && active_len < 16 * splits) splits >>= 1;
  return splits;
}

size_t attn_parts_bytes(int B, int Hq, int hd) {
  return (size_t)kAttnMaxParts * B * Hq * (hd * sizeof(f16) + sizeof(f32x2));
}

int launch_flash_decode_parts(const f16* q, const KvView& kv, int Hq, int active_len, const int* active_len_dev,
                              int n_splits, f16* parts_o, f32x2* parts_ml, bool short_splits, hipStream_t s) {
  if (n_splits < 2 || n_splits > kAttnMaxParts || parts_o == nullptr || parts_ml == nullptr) {
    axm_set_error("flash_decode_parts: %d splits (2..%d) or null partial buffers", n_splits, kAttnMaxParts);
    return -1;
  }
  AttnParams p{};
  p.q = q;
  p.kv = kv;
  p.parts_o = parts_o;
  p.parts_ml = parts_ml;
  p.Hq = Hq;
  p.n_rep = Hq / kv.Hkv;
  p.n_splits = n_splits;
  p.prefix_len = active_len;
  p.prefix_dev = active_len_dev;
  p.T = 0;
  p.short_splits = short_splits;
  p.scale_log2 = kLog2e / sqrtf((float)kv.hd);
  const int qr = pick_qr(p.n_rep);
  dim3 grid(kv.B * kv.Hkv, n_splits, (p.n_rep + qr - 1) / qr);
  return launch_attn_dispatch<false>(p, qr, grid, s);
}

int launch_decode_mfma(const AttnParams& p, dim3 grid, hipStream_t s);

int launch_flash_decode(const f16* q, const KvView& kv, f16* out, int Hq, int active_len, const int* active_len_dev,
                        int n_splits, float* ws, hipStream_t s) {
  AttnParams p{};
  p.q = q;
  p.kv = kv;
  p.out = out;
  p.ws = ws;
  p.Hq = Hq;
  p.n_rep = Hq / kv.Hkv;
  p.n_splits = n_splits;
  p.prefix_len = active_len;
  p.prefix_dev = active_len_dev;
  p.T = 0;
  p.scale_log2 = kLog2e / sqrtf((float)kv.hd);
  int rc;
  if (p.n_rep >= 2 && p.n_rep <= 16 && (kv.hd == 64 || kv.hd == 128)) {
    rc = launch_decode_mfma(p, dim3(kv.B * kv.Hkv, n_splits), s);
  } else {
    const int qr = pick_qr(p.n_rep);
    dim3 grid(kv.B * kv.Hkv, n_splits, (p.n_rep + qr - 1) / qr);
    rc = launch_attn_dispatch<false>(p, qr, grid, s);
  }
  if (rc) return rc;
  if (n_splits > 1)
    launch_attn_reduce(ws, out, kv.B * Hq, n_splits, kv.hd, s);
  return 0;
}

size_t tree_workspace_bytes(int T, int Hq, int hd, int n_splits) {
  return n_splits <= 1 ? 0 : (size_t)T * Hq * n_splits * (2 + hd) * sizeof(float);
}

// ---------------------------------------------------------------------------
// Tree verification attention on the matrix cores.  The query rows of one KV
// head (tree node u x replica r, up to 64 per workgroup, 16 per wave) attend
// over 32-key blocks of [prefix keys | tree slots]:
//   S = Q K^T   v_mfma_f32_16x16x32_f16, A = the wave's 16 query rows (loaded
//               once), B = 16 keys x 32 dims straight from the cache rows
//               (dequantized to fp16 with the reference rounding),
//   masked online softmax on the D tile (a query row's 16 keys sit in the 16
//               lanes of one DPP row, so row max / sum are DPP reductions),
//   O += P V    A = P (fp16, through a wave-private LDS tile), B = the block's
//               V staged transposed (dim-major) in LDS by the workgroup.
// A key block is loaded once per workgroup for all its rows, instead of once
// per few rows.  Partials over key splits use the decode layout
// ([row][split][m, l, o]) and attn_reduce_kernel.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_max_step(float v) {
  const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false);
  return fmaxf(v, __builtin_bit_cast(float, o));
}
__device__ __forceinline__ float row16_max(float v) {
  v = dpp_max_step<0xB1>(v);
  v = dpp_max_step<0x4E>(v);
  v = dpp_max_step<0x141>(v);
  return dpp_max_step<0x140>(v);
}
__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_sum_step<0xB1>(v);
  v = dpp_sum_step<0x4E>(v);
  v = dpp_sum_step<0x141>(v);
  return dpp_sum_step<0x140>(v);
}

constexpr int kTreeKeys = 32;    // keys per block (the k extent of one P V MFMA)

// P tile of the matrix-core attention kernels, [row][key] with 32 keys per row:
// written 4 rows x 16 keys at a time, read 8 keys per row; the 8-key groups of
// row r are XOR-swizzled by bits 2-3 of r (2-way bank conflicts at most).
__device__ __forceinline__ int pt_index(int row, int key) {
  return row * kTreeKeys + (((key >> 3) ^ ((row >> 2) & 3)) << 3) + (key & 7);
}

// B operand of O += P V from V rows stored key-major (row stride vrow halves;
// seg = row 0 of a 16-dim tile): lane (l16, lq) needs dim column l16 of keys
// 8 lq .. 8 lq + 7.  ds_read_b64_tr_b16 over a 16-lane group returns to lane i
// column i of the 4 x 16 block whose row r is the 4 x 8 bytes the group's lanes
// 4 r .. 4 r + 3 address, so lane i addresses key (i / 4) of the group's four,
// dims 4 (i % 4) .. + 3; two reads give keys 8 lq .. + 3 and 8 lq + 4 .. + 7.
typedef short tr_v4s __attribute__((vector_size(8)));
__device__ __forceinline__ f16x8 v_operand(const f16* seg, int vrow, int l16, int lq) {
  typedef __attribute__((address_space(3))) tr_v4s lds_v4s;
  const f16* p0 = seg + (8 * lq + (l16 >> 2)) * vrow + 4 * (l16 & 3);
  const tr_v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p0);
  const tr_v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p0 + 4 * vrow));
  f16x8 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    r[e] = __builtin_bit_cast(f16, (short)a[e]);
    r[4 + e] = __builtin_bit_cast(f16, (short)b[e]);
  }
  return r;
}
// Dim of output column c of a 16-dim tile whose V rows were stored in kv_half8's
// order (int4: positions 0..7 of each 8-dim chunk hold dims 0, 2, 4, 6, 1, 3, 5, 7).
template <int KVT>
__device__ __forceinline__ int kv_col_dim(int c) {
  return (c & 8) | kv_dim_of<KVT>(c & 7);
}
constexpr int kTreeRows = 64;    // query rows per workgroup (four waves of 16)

// Online softmax of one 32-key block for the wave's 16-row D tile: lane (l16, lq)
// holds the scaled scores s[v][h] of row 4 lq + v, key 16 h + l16 (kNegBig when
// masked), and the row's running max m[v] (the same in the row's 16 lanes), a
// per-lane partial l[v] of the row's weight sum and the output accumulators o.
// The running max moves only when some score of the wave exceeds it by more
// than kMaxSlack (grows, tested with one ballot); otherwise the weights
// exp2(s - m) stay below 2^kMaxSlack with no row reduction, and only the
// rescaling path takes the row maxima.  The caller sums l over each row's 16
// lanes once after the last block.  The quotient o / l does not depend on m; the
// fp16 weights P keep their relative precision up to 2^kMaxSlack.
constexpr float kMaxSlack = 8.f;
template <int DT>
__device__ __forceinline__ void softmax_block(const float (&s)[4][2], bool grows, float (&m)[4], float (&l)[4],
                                              f32x4 (&o)[DT], f16* pt, int lq, int l16) {
  if (__builtin_amdgcn_ballot_w64(grows)) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float m_new = fmaxf(m[v], row16_max(fmaxf(s[v][0], s[v][1])));
      const float alpha = fast_exp2(m[v] - m_new);
      m[v] = m_new;
      l[v] *= alpha;
#pragma unroll
      for (int d = 0; d < DT; ++d) o[d][v] *= alpha;
    }
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    float pr[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) pr[h] = s[v][h] == kNegBig ? 0.f : fast_exp2(s[v][h] - m[v]);
    l[v] += pr[0] + pr[1];
#pragma unroll
    for (int h = 0; h < 2; ++h) pt[pt_index(4 * lq + v, 16 * h + l16)] = f2h(pr[h]);
  }
}

template <int KVT, int HD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) tree_mfma_kernel(AttnParams p) {
  constexpr int KSTEPS = HD / 32;  // MFMA k-steps over the head dimension
  constexpr int DT = HD / 16;      // 16-wide output dimension tiles
  constexpr int kVec = kTreeKeys * HD / 8;        // 8-element V vectors per key block
  // The block's V rows as stored (key-major, padded rows, read transposed by
  // v_operand) and per wave the P tile of its 16 rows.
  constexpr int VROW = HD + 16;
  __shared__ __align__(16) f16 vr[kTreeKeys * VROW];
  __shared__ __align__(16) f16 pt[4][16 * kTreeKeys];
  auto pt_at = pt_index;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15, lq = lane >> 4;
  const int kvh = blockIdx.x;
  const int R = p.T * p.n_rep;
  const int row0 = blockIdx.y * kTreeRows + wave * 16;
  const int split = blockIdx.z;
  const int prefix = p.prefix_len;
  const int n_keys = prefix + p.T;
  const int per = (n_keys + p.n_splits - 1) / p.n_splits;
  const int k_begin = min(split * per, n_keys);
  const int k_end = min(k_begin + per, n_keys);
  const size_t head_row0 = (size_t)kvh * p.kv.S;  // batch 0
  auto grow = [&](int r) {  // global query row (node * Hq + query head) of row r < R
    return (r / p.n_rep) * p.Hq + kvh * p.n_rep + (r % p.n_rep);
  };
  // Tree key t sits in slot (write_pos + t) % S; the launch guarantees T <= S (and
  // write_pos < S), so one conditional subtraction wraps it.  Selects only: a
  // branch here split the loop body and cost the key buffers their registers.
  auto slot_of = [&](int key) {
    const int w = p.write_pos + (key - prefix);
    const int wrapped = w >= p.kv.S ? w - p.kv.S : w;
    return key < prefix ? key : wrapped;
  };

  // Key / value fetches of one block into register buffer b (two blocks are in
  // flight), each a run of consecutive chunks of one cache row: this lane's K
  // B-operand fragments (keys kb0 + 16 h + l16, dims [HD/4 lq, HD/4 (lq + 1)), of
  // which k-step c takes dims HD/4 lq + 8 c (+ 0..7), the query using the same dim
  // order) and this thread's V run (kVRun chunks, key threadIdx / kRunsPerKey).  Keys
  // at or past k_end read zeros (out-of-range offsets), so every fetch is issued
  // unconditionally and the compiler counts the loads in flight exactly.
  constexpr int kVRun = kVec / 256;          // V chunks per thread
  constexpr int kRunsPerKey = HD / 8 / kVRun;
  static_assert(kVec % 256 == 0, "one V run per thread");
  KvRun<KVT, KSTEPS> krun[2][2];
  KvRun<KVT, kVRun> vrun[2];
  const KvHead kh = kv_head<KVT>(p.kv.k, p.kv.ks, head_row0, p.kv.S, HD);
  const KvHead vh = kv_head<KVT>(p.kv.v, p.kv.vs, head_row0, p.kv.S, HD);
  auto fetch = [&](int kb0, auto bc) {
    constexpr int b = decltype(bc)::value;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int key = kb0 + 16 * h + l16;
      krun[b][h] = kv_fetch_run<KVT, KSTEPS>(kh, slot_of(key), HD, (HD / 4) * lq, key < k_end);
    }
    const int key = kb0 + threadIdx.x / kRunsPerKey;
    vrun[b] = kv_fetch_run<KVT, kVRun>(vh, slot_of(key), HD, 8 * kVRun * (threadIdx.x % kRunsPerKey), key < k_end);
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // A operand: query row row0 + l16, dims HD/4 lq + 8 c .. +7.
  f16x8 qa[KSTEPS];
  {
    const int r = row0 + l16;
#pragma unroll
    for (int c = 0; c < KSTEPS; ++c) {
#pragma unroll
      for (int i = 0; i < 8; ++i) qa[c][i] = f16(0);
      if (r < R)
        qa[c] = kv_order8<KVT>(*reinterpret_cast<const f16x8*>(p.q + (size_t)grow(r) * HD + (HD / 4) * lq + 8 * c));
    }
  }
  // D-tile rows of this lane: row0 + 4 lq + v.
  uint64_t mask[4];
  bool row_ok[4];
  float m[4], l[4];
  f32x4 o[DT];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int r = row0 + 4 * lq + v;
    row_ok[v] = r < R;
    mask[v] = row_ok[v] ? p.masks[r / p.n_rep] : 0ull;
    m[v] = kNegBig;
    l[v] = 0.f;
  }
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The first two blocks' keys and values are requested after the query rows and
  // masks: loads complete in order, so the loop's waits for a key block then also
  // cover them (requested last, they made every iteration wait for all loads).
  fetch(k_begin, B0{});
  fetch(k_begin + kTreeKeys, B1{});

  // One key block from register buffer b, whose registers then take the block
  // two ahead.
  auto block = [&](int kb0, auto bc) {
    constexpr int b = decltype(bc)::value;
    f16x8 kf[2][KSTEPS], vv[kVRun];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) kf[h][c] = kv_half8<KVT>(krun[b][h].chunk(c));
#pragma unroll
    for (int c = 0; c < kVRun; ++c) vv[c] = kv_half8<KVT>(vrun[b].chunk(c));
    // The refill is not scheduled above the conversions: the old and new contents of
    // buffer b then never overlap and keep the same registers across iterations
    // (otherwise the loop head copied the new ones, waiting for every load).
    __builtin_amdgcn_sched_barrier(0);
    fetch(kb0 + 2 * kTreeKeys, bc);
    // Stage V rows as converted: this thread's run covers key kb0 + tid /
    // kRunsPerKey, dims 8 kVRun (tid % kRunsPerKey) onwards (16-byte stores; int4
    // chunks keep kv_half8's order).
    {
      const int kk = threadIdx.x / kRunsPerKey, e0 = 8 * kVRun * (threadIdx.x % kRunsPerKey);
#pragma unroll
      for (int c = 0; c < kVRun; ++c) *reinterpret_cast<f16x8*>(&vr[kk * VROW + e0 + 8 * c]) = vv[c];
    }
    // S = Q K^T for the block's two 16-key halves.
    f32x4 sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], kf[h][c], sc[h], 0, 0, 0);
    }
    // Mask and scale; online softmax per D-tile row; P to the wave's LDS tile.
    float s2[4][2];
    bool grows = false;
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int key = kb0 + 16 * h + l16;
        const bool in_tree = ((mask[v] >> ((key - prefix) & 63)) & 1ull) != 0;
        const bool vis = row_ok[v] && key < k_end && (key < prefix || in_tree);
        s2[v][h] = vis ? sc[h][v] * p.scale_log2 : kNegBig;
        grows |= s2[v][h] > m[v] + kMaxSlack;
      }
    softmax_block(s2, grows, m, l, o, pt[wave], lq, l16);
    __syncthreads();  // V staged by every wave; P tiles written
    // O += P V: A = P[row l16][keys 8 lq ..], B = V^T[dim 16 d + l16][keys 8 lq ..].
    const f16x8 pa = *reinterpret_cast<const f16x8*>(&pt[wave][pt_at(l16, 8 * lq)]);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const f16x8 vb = v_operand(&vr[16 * d], VROW, l16, lq);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[d], 0, 0, 0);
    }
    __syncthreads();  // before the next block overwrites vt / pt
  };
  // Both blocks of an iteration run unconditionally and an odd last block is peeled
  // off: with a conditional second block the two register buffers reach the loop
  // head from two paths, and the compiler copied the freshly requested ones there,
  // waiting for every load in flight on each iteration.
  int kb0 = k_begin;
  for (; kb0 + kTreeKeys < k_end; kb0 += 2 * kTreeKeys) {
    block(kb0, B0{});
    block(kb0 + kTreeKeys, B1{});
  }
  if (kb0 < k_end) block(kb0, B0{});

#pragma unroll
  for (int v = 0; v < 4; ++v) l[v] = row16_sum(l[v]);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (!row_ok[v]) continue;
    const int gr = grow(row0 + 4 * lq + v);
    if (p.n_splits == 1) {
      const float inv = l[v] > 0.f ? 1.f / l[v] : 0.f;
#pragma unroll
      for (int d = 0; d < DT; ++d)
        p.out[(size_t)gr * HD + 16 * d + kv_col_dim<KVT>(l16)] = f2h(l[v] > 0.f ? o[d][v] * inv : 0.f);
    } else {
      float* dst = p.ws + ((size_t)gr * p.n_splits + split) * (2 + HD);
      if (l16 == 0) {
        dst[0] = m[v];
        dst[1] = l[v];
      }
#pragma unroll
      for (int d = 0; d < DT; ++d) dst[2 + 16 * d + kv_col_dim<KVT>(l16)] = o[d][v];
    }
  }
}

template <int HD>
int launch_tree_mfma(const AttnParams& p, dim3 grid, hipStream_t s) {
  switch (p.kv.kv_dtype) {
    case AXM_KV_FP16:
      hipLaunchKernelGGL((tree_mfma_kernel<AXM_KV_FP16, HD>), grid, dim3(256), 0, s, p);
      return 0;
    case AXM_KV_FP8:
      hipLaunchKernelGGL((tree_mfma_kernel<AXM_KV_FP8, HD>), grid, dim3(256), 0, s, p);
      return 0;
    case AXM_KV_INT4:
      hipLaunchKernelGGL((tree_mfma_kernel<AXM_KV_INT4, HD>), grid, dim3(256), 0, s, p);
      return 0;
  }
  axm_set_error("tree attention: bad kv dtype %d", p.kv.kv_dtype);
  return -1;
}

// ---------------------------------------------------------------------------
// Batched GQA decode attention on the matrix cores: the n_rep (2..16) query
// heads of one (batch, KV head) are the rows of one 16-row MFMA tile, so every
// key / value row loaded serves all of them through q K^T and P V tiles instead
// of n_rep vector dot products.  A workgroup is one (batch, KV head, split);
// its four waves take interleaved 32-key blocks of the split independently
// (wave-private transposed V and P tiles, no barrier in the loop) and merge
// their (m, l, o) through LDS at the end.
// ---------------------------------------------------------------------------
template <int KVT, int HD>
__global__ void __launch_bounds__(256) decode_mfma_kernel(AttnParams p) {
  constexpr int KSTEPS = HD / 32;
  constexpr int DT = HD / 16;
  constexpr int kVPL = kTreeKeys * HD / 8 / 64;  // 8-element V vectors per lane and block
  // V rows as stored (key-major, padded rows) for the transposing LDS reads.
  constexpr int VROW = HD + 16;
  __shared__ __align__(16) f16 vr[4][kTreeKeys * VROW];
  __shared__ __align__(16) f16 pt[4][16 * kTreeKeys];
  __shared__ float mrg[4][16][2 + HD];
  auto pt_at = pt_index;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int b = blockIdx.x / p.kv.Hkv, kvh = blockIdx.x % p.kv.Hkv;
  const int R = p.n_rep;
  const int split = blockIdx.y;
  const int n_keys = p.prefix_dev ? p.prefix_dev[0] : p.prefix_len;
  const int per = (n_keys + p.n_splits - 1) / p.n_splits;
  const int k_begin = min(split * per, n_keys);
  const int k_end = min(k_begin + per, n_keys);
  const size_t head_row0 = ((size_t)b * p.kv.Hkv + kvh) * p.kv.S;
  const size_t qrow0 = (size_t)b * p.Hq + (size_t)kvh * p.n_rep;  // global query row of replica 0

  // A wave's key blocks are fetched DEPTH ahead into DEPTH register buffers;
  // keys at or past k_end read zeros, so every fetch is issued unconditionally.
  // Two ahead pays for the fp8 cache (C3 shape, 32k keys: 187 -> 163 us).  The
  // int4 form is slower with a second buffer (with one-load runs: 32k keys 86.9 ->
  // 92.8 us, the ring of 4096 slots 17.9 -> 19.3 us), and for fp16 it takes hd 128
  // past 256 VGPRs, i.e. from two waves per SIMD to one.
  constexpr int DEPTH = KVT == AXM_KV_FP8 ? 2 : 1;
  // A lane fetches runs of KSTEPS chunks (a quarter of a row, HD / 4 elements): the
  // keys of a half-block as dims [HD/4 lq, HD/4 (lq + 1)) of key l16, so k-step c
  // pairs dims HD/4 lq + 8 c (+ 0..7) with the same dims of the query (the MFMA's
  // k order is a permutation of the head dims, the same for both operands); the
  // values as runs j = i 64 + lane, key j / 4, dims HD/4 (j % 4).
  constexpr int kRuns = kVPL / KSTEPS;  // value runs per lane and block
  KvRun<KVT, KSTEPS> krun[DEPTH][2], vrun[DEPTH][kRuns];
  // The key / value descriptors end at the split's last key, so fetches past it
  // read zeros without a per-chunk select.
  const KvHead kh = kv_head<KVT>(p.kv.k, p.kv.ks, head_row0, k_end, HD);
  const KvHead vh = kv_head<KVT>(p.kv.v, p.kv.vs, head_row0, k_end, HD);
  auto fetch = [&](int kb0, auto bc) {
    constexpr int bf = decltype(bc)::value;
#pragma unroll
    for (int h = 0; h < 2; ++h) krun[bf][h] = kv_fetch_run<KVT, KSTEPS>(kh, kb0 + 16 * h + l16, HD, (HD / 4) * lq);
#pragma unroll
    for (int i = 0; i < kRuns; ++i) {
      const int j = i * 64 + lane;
      vrun[bf][i] = kv_fetch_run<KVT, KSTEPS>(vh, kb0 + j / 4, HD, (HD / 4) * (j % 4));
    }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  constexpr int kStride = 4 * kTreeKeys;  // the four waves interleave their blocks
  const int kb_first = k_begin + kTreeKeys * wave;

  f16x8 qa[KSTEPS];
#pragma unroll
  for (int c = 0; c < KSTEPS; ++c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) qa[c][i] = f16(0);
    if (l16 < R)
      qa[c] = kv_order8<KVT>(*reinterpret_cast<const f16x8*>(p.q + (qrow0 + l16) * HD + (HD / 4) * lq + 8 * c));
  }
  bool row_ok[4];
  float m[4], l[4];
  f32x4 o[DT];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    row_ok[v] = 4 * lq + v < R;
    m[v] = kNegBig;
    l[v] = 0.f;
  }
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  // The first key blocks are requested after the query rows: loads complete in
  // order, so the loop's waits for a key block also cover the query loads
  // (requested last, they made every iteration wait for all loads in flight).
  fetch(kb_first, B0{});
  if constexpr (DEPTH == 2) fetch(kb_first + kStride, B1{});

  auto block = [&](int kb0, auto bc) {
    constexpr int bf = decltype(bc)::value;
    f16x8 kf[2][KSTEPS], vv[kRuns][KSTEPS];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) kf[h][c] = kv_half8<KVT>(krun[bf][h].chunk(c));
#pragma unroll
    for (int i = 0; i < kRuns; ++i)
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) vv[i][c] = kv_half8<KVT>(vrun[bf][i].chunk(c));
    fetch(kb0 + DEPTH * kStride, bc);
    // V rows to LDS as converted (16-byte stores; int4 chunks keep kv_half8's order).
#pragma unroll
    for (int i = 0; i < kRuns; ++i) {
      const int j = i * 64 + lane;
      const int kk = j / 4, e0 = (HD / 4) * (j % 4);
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) *reinterpret_cast<f16x8*>(&vr[wave][kk * VROW + e0 + 8 * c]) = vv[i][c];
    }
    f32x4 sc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      sc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) sc[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[c], kf[h][c], sc[h], 0, 0, 0);
    }
    float s2[4][2];
    bool grows = false;
#pragma unroll
    for (int v = 0; v < 4; ++v)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool vis = row_ok[v] && kb0 + 16 * h + l16 < k_end;
        s2[v][h] = vis ? sc[h][v] * p.scale_log2 : kNegBig;
        grows |= s2[v][h] > m[v] + kMaxSlack;
      }
    softmax_block(s2, grows, m, l, o, pt[wave], lq, l16);
    // The wave reads back its own LDS writes: DS operations of one wave complete
    // in order, and the reads below wait for them.
    const f16x8 pa = *reinterpret_cast<const f16x8*>(&pt[wave][pt_at(l16, 8 * lq)]);
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const f16x8 vb = v_operand(&vr[wave][16 * d], VROW, l16, lq);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[d], 0, 0, 0);
    }
  };
  // With two buffers both blocks of an iteration run unconditionally and an odd
  // last block is peeled off, so each buffer keeps its registers across iterations
  // (a conditional second block made the compiler copy the buffers at the loop
  // head, waiting for every load in flight).
  int kb0 = kb_first;
  if constexpr (DEPTH == 2) {
    for (; kb0 + kStride < k_end; kb0 += 2 * kStride) {
      block(kb0, B0{});
      block(kb0 + kStride, B1{});
    }
    if (kb0 < k_end) block(kb0, B0{});
  } else {
    for (; kb0 < k_end; kb0 += kStride) block(kb0, B0{});
  }

  // Merge the four waves' (m, l, o) per query row.
#pragma unroll
  for (int v = 0; v < 4; ++v) l[v] = row16_sum(l[v]);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int row = 4 * lq + v;
    if (l16 == 0) {
      mrg[wave][row][0] = m[v];
      mrg[wave][row][1] = l[v];
    }
    // Output column l16 of tile d is dim 16 d + kv_col_dim<KVT>(l16).
#pragma unroll
    for (int d = 0; d < DT; ++d) mrg[wave][row][2 + 16 * d + kv_col_dim<KVT>(l16)] = o[d][v];
  }
  __syncthreads();
  for (int t = threadIdx.x; t < R * HD; t += 256) {
    const int row = t / HD, e = t % HD;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < 4; ++w) mm = fmaxf(mm, mrg[w][row][0]);
    float ll = 0.f, oo = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float a = fast_exp2(mrg[w][row][0] - mm);
      ll += mrg[w][row][1] * a;
      oo += mrg[w][row][2 + e] * a;
    }
    const size_t gr = qrow0 + row;
    if (p.n_splits == 1) {
      p.out[gr * HD + e] = f2h(ll > 0.f ? oo / ll : 0.f);
    } else {
      float* dst = p.ws + (gr * p.n_splits + split) * (2 + HD);
      if (e == 0) {
        dst[0] = mm;
        dst[1] = ll;
      }
      dst[2 + e] = oo;
    }
  }
}

int launch_decode_mfma(const AttnParams& p, dim3 grid, hipStream_t s) {
  const int hd = p.kv.hd;
  switch (p.kv.kv_dtype) {
    case AXM_KV_FP16:
      if (hd == 128) hipLaunchKernelGGL((decode_mfma_kernel<AXM_KV_FP16, 128>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((decode_mfma_kernel<AXM_KV_FP16, 64>), grid, dim3(256), 0, s, p);
      return 0;
    case AXM_KV_FP8:
      if (hd == 128) hipLaunchKernelGGL((decode_mfma_kernel<AXM_KV_FP8, 128>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((decode_mfma_kernel<AXM_KV_FP8, 64>), grid, dim3(256), 0, s, p);
      return 0;
    case AXM_KV_INT4:
      if (hd == 128) hipLaunchKernelGGL((decode_mfma_kernel<AXM_KV_INT4, 128>), grid, dim3(256), 0, s, p);
      else hipLaunchKernelGGL((decode_mfma_kernel<AXM_KV_INT4, 64>), grid, dim3(256), 0, s, p);
      return 0;
  }
  axm_set_error("decode attention: bad kv dtype %d", p.kv.kv_dtype);
  return -1;
}

int tree_choose_splits(int T, int Hq, int Hkv, int n_keys) {
  // Workgroups of 64 query rows per KV head; splits of >= 64 keys until about
  // one workgroup per CU (with key blocks fetched two ahead, fewer and longer
  // splits cost no latency and halve the partials: 7B verify step 4.03 -> 4.00
  // ms against two workgroups per CU).
  const int rows = T * (Hq / Hkv);
  const int wgs = Hkv * ((rows + kTreeRows - 1) / kTreeRows);
  int splits = 1;
  while (splits < 64 && wgs * splits * 2 <= 256 && n_keys >= 64 * splits * 2) splits *= 2;
  return splits;
}

int launch_tree_attention(const f16* q, const KvView& kv, f16* out, int Hq, int T, int prefix_len, int write_pos,
                          const uint64_t* masks_dev, int n_splits, float* ws, hipStream_t s) {
  AttnParams p{};
  p.q = q;
  p.kv = kv;
  p.out = out;
  p.ws = ws;
  p.Hq = Hq;
  p.n_rep = Hq / kv.Hkv;
  p.n_splits = n_splits;
  p.prefix_len = prefix_len;
  p.T = T;
  p.write_pos = write_pos;
  p.masks = masks_dev;
  p.scale_log2 = kLog2e / sqrtf((float)kv.hd);
  const int rows = T * p.n_rep;
  int rc;
  if (kv.B == 1 && (kv.hd == 64 || kv.hd == 128) && T <= kv.S) {
    const dim3 grid(kv.Hkv, (rows + kTreeRows - 1) / kTreeRows, n_splits);
    rc = kv.hd == 128 ? launch_tree_mfma<128>(p, grid, s) : launch_tree_mfma<64>(p, grid, s);
  } else {
    const int qr = pick_qr(rows);
    dim3 grid(kv.Hkv * ((rows + qr - 1) / qr), n_splits, 1);
    rc = launch_attn_dispatch<true>(p, qr, grid, s);
  }
  if (rc) return rc;
  if (n_splits > 1)
    launch_attn_reduce(ws, out, T * Hq, n_splits, kv.hd, s);
  return 0;
}

// ---------------------------------------------------------------------------
// C ABI.
// ---------------------------------------------------------------------------
static int check_kv(const KvView& kv, const char* who) {
  AXM_CHECK_ARG(kv.k && kv.v, -1, "%s: null cache pointer", who);
  AXM_CHECK_ARG(kv.hd > 0 && kv.hd <= 128 && kv.hd % 64 == 0, -1, "%s: head_dim=%d must be 64 or 128", who, kv.hd);
  AXM_CHECK_ARG(kv.kv_dtype >= 0 && kv.kv_dtype <= 2, -1, "%s: bad kv dtype %d", who, kv.kv_dtype);
  AXM_CHECK_ARG(kv.kv_dtype == AXM_KV_FP16 || (kv.ks && kv.vs), -1, "%s: quantized cache needs scales", who);
  AXM_CHECK_ARG(kv.B > 0 && kv.Hkv > 0 && kv.S > 0, -1, "%s: bad cache shape", who);
  return 0;
}

extern "C" int axm_tree_attention_num_splits(int T, int n_head, int n_kv_head, int n_keys) {
  if (T < 1 || n_kv_head < 1 || n_head < n_kv_head || n_keys < 1) return 1;
  return tree_choose_splits(T, n_head, n_kv_head, n_keys);
}

extern "C" size_t axm_attention_workspace_bytes(int B, int n_query_rows_per_batch, int head_dim, int n_splits) {
  return attn_workspace_bytes(B, n_query_rows_per_batch, head_dim, n_splits);
}

extern "C" int axm_attention_num_splits(int B, int n_head, int n_kv_head, int head_dim, int kv_dtype,
                                        int active_len) {
  if (B < 1 || n_head < 1 || n_kv_head < 1 || head_dim < 1 || active_len < 1) return 1;
  return attn_flash_splits(B, n_head, n_kv_head, head_dim, kv_dtype, active_len);
}

extern "C" int axm_gqa_flash_decode(const void* q, const void* k_cache, const void* v_cache, const void* k_scales,
                                    const void* v_scales, int kv_dtype, void* out, int B, int n_head, int n_kv_head,
                                    int head_dim, int max_seq_len, int active_len, int num_splits, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  KvView kv{(void*)k_cache, (void*)v_cache, (f16*)k_scales, (f16*)v_scales, kv_dtype, B, n_kv_head, max_seq_len,
            head_dim};
  if (int rc = check_kv(kv, "gqa_flash_decode")) return rc;
  AXM_CHECK_ARG(q && out, -1, "gqa_flash_decode: null q/out");
  AXM_CHECK_ARG(n_head % n_kv_head == 0 && n_head / n_kv_head <= 64, -1,
                "gqa_flash_decode: n_head=%d not a multiple of n_kv_head=%d", n_head, n_kv_head);
  AXM_CHECK_ARG(active_len >= 1 && active_len <= max_seq_len, -1, "gqa_flash_decode: active_len=%d out of [1, %d]",
                active_len, max_seq_len);
  if (num_splits <= 0) num_splits = attn_flash_splits(B, n_head, n_kv_head, head_dim, kv_dtype, active_len);
  AXM_CHECK_ARG(num_splits <= 1024, -1, "gqa_flash_decode: num_splits=%d too large", num_splits);
  const size_t need = attn_workspace_bytes(B, n_head, head_dim, num_splits);
  AXM_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace), -1,
                "gqa_flash_decode: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  int rc = launch_flash_decode((const f16*)q, kv, (f16*)out, n_head, active_len, nullptr, num_splits,
                               (float*)workspace, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("gqa_flash_decode");
  return 0;
}

// ---------------------------------------------------------------------------
// No-allocation flash decode: the split partials live in `scratch`, a file-scope
// device array (one copy per GPU).  Its device address is resolved once per
// device with hipGetSymbolAddress (the array's name in host code is only a
// host-side stand-in) and that address is what the kernels receive.  Every
// split writes its partial row before the reduce reads it, so nothing in the
// array has to start at zero.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[AXM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kScratchMaxDevices] = {};

// Device address of the current device's scratch array (resolved on first use).
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchMaxDevices) {
    (void)hipGetLastError();
    axm_set_error("gqa_flash_decode_noalloc: no current device (or device index >= %d)", kScratchMaxDevices);
    return -5;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      axm_set_error("gqa_flash_decode_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                    hipGetErrorString(e));
      return -5;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}
}  // namespace

extern "C" int axm_gqa_flash_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                            const void* k_scales, const void* v_scales, int kv_dtype, void* out,
                                            int B, int n_head, int n_kv_head, int head_dim, int max_seq_len,
                                            int active_len, int num_splits, void* stream) {
  KvView kv{(void*)k_cache, (void*)v_cache, (f16*)k_scales, (f16*)v_scales, kv_dtype, B, n_kv_head, max_seq_len,
            head_dim};
  if (int rc = check_kv(kv, "gqa_flash_decode_noalloc")) return rc;
  AXM_CHECK_ARG(q && out, -1, "gqa_flash_decode_noalloc: null q/out");
  AXM_CHECK_ARG(n_head % n_kv_head == 0 && n_head / n_kv_head <= 64, -1,
                "gqa_flash_decode_noalloc: n_head=%d not a multiple of n_kv_head=%d", n_head, n_kv_head);
  AXM_CHECK_ARG(active_len >= 1 && active_len <= max_seq_len, -1,
                "gqa_flash_decode_noalloc: active_len=%d out of [1, %d]", active_len, max_seq_len);
  if (num_splits <= 0) num_splits = attn_flash_splits(B, n_head, n_kv_head, head_dim, kv_dtype, active_len);
  AXM_CHECK_ARG(num_splits <= 1024, -1, "gqa_flash_decode_noalloc: num_splits=%d too large", num_splits);
  const size_t need = attn_workspace_bytes(B, n_head, head_dim, num_splits);
  AXM_CHECK_ARG(need <= (size_t)AXM_NOALLOC_SCRATCH_BYTES, -1,
                "gqa_flash_decode_noalloc: %zu bytes of split partials (B=%d, %d heads of %d, %d splits) exceed "
                "the fixed %u-byte scratch array",
                need, B, n_head, head_dim, num_splits, (unsigned)AXM_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_address(&ws)) return rc;
  }
  int rc = launch_flash_decode((const f16*)q, kv, (f16*)out, n_head, active_len, nullptr, num_splits, (float*)ws,
                               (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("gqa_flash_decode_noalloc");
  return 0;
}

extern "C" int axm_gqa_tree_verify(const void* q, const void* k_cache, const void* v_cache, const void* k_scales,
                                   const void* v_scales, int kv_dtype, void* out, int T, int n_head, int n_kv_head,
                                   int head_dim, int max_seq_len, int prefix_len, int write_pos,
                                   const void* masks_u64_dev, int num_splits, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  KvView kv{(void*)k_cache, (void*)v_cache, (f16*)k_scales, (f16*)v_scales, kv_dtype, 1, n_kv_head, max_seq_len,
            head_dim};
  if (int rc = check_kv(kv, "gqa_tree_verify")) return rc;
  AXM_CHECK_ARG(q && out && masks_u64_dev, -1, "gqa_tree_verify: null pointer");
  AXM_CHECK_ARG(T >= 1 && T <= 64, -1, "gqa_tree_verify: T=%d must be in [1, 64]", T);
  AXM_CHECK_ARG(n_head % n_kv_head == 0, -1, "gqa_tree_verify: n_head %% n_kv_head != 0");
  AXM_CHECK_ARG(prefix_len >= 0 && prefix_len <= max_seq_len, -1, "gqa_tree_verify: bad prefix_len %d", prefix_len);
  AXM_CHECK_ARG(write_pos >= 0 && write_pos < max_seq_len, -1, "gqa_tree_verify: bad write_pos %d", write_pos);
  if (num_splits <= 0) num_splits = tree_choose_splits(T, n_head, n_kv_head, prefix_len + T);
  const size_t need = tree_workspace_bytes(T, n_head, head_dim, num_splits);
  AXM_CHECK_ARG(workspace_bytes >= need && (need == 0 || workspace), -1,
                "gqa_tree_verify: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  int rc = launch_tree_attention((const f16*)q, kv, (f16*)out, n_head, T, prefix_len, write_pos,
                                 (const uint64_t*)masks_u64_dev, num_splits, (float*)workspace, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("gqa_tree_verify");
  return 0;
}

extern "C" int axm_kv_cache_write(const void* k_rows, const void* v_rows, int ld_rows, int T, void* k_cache,
                                  void* v_cache, void* k_scales, void* v_scales, int kv_dtype, int n_kv_head,
                                  int head_dim, int max_seq_len, int write_pos, void* stream) {
  KvView kv{k_cache, v_cache, (f16*)k_scales, (f16*)v_scales, kv_dtype, 1, n_kv_head, max_seq_len, head_dim};
  if (int rc = check_kv(kv, "kv_cache_write")) return rc;
  AXM_CHECK_ARG(k_rows && v_rows && T >= 1, -1, "kv_cache_write: bad rows");
  AXM_CHECK_ARG(write_pos >= 0 && write_pos < max_seq_len, -1, "kv_cache_write: write_pos %d out of range",
                write_pos);
  launch_kv_write(kv, (const f16*)k_rows, (const f16*)v_rows, ld_rows, T, write_pos, nullptr, (hipStream_t)stream);
  AXM_LAUNCH_CHECK("kv_cache_write");
  return 0;
}

extern "C" int axm_rope_kv_cache_write(void* qkv, int T, const void* freqs, int rope_len, int start_pos,
                                       const int* depths_host, const void* qkv_bias, void* k_cache, void* v_cache,
                                       void* k_scales, void* v_scales, int kv_dtype, int q_dim, int kv_dim,
                                       int head_dim, int max_seq_len, int write_pos, void* stream) {
  KvView kv{k_cache, v_cache, (f16*)k_scales, (f16*)v_scales, kv_dtype, 1, 0, max_seq_len, head_dim};
  AXM_CHECK_ARG(qkv && freqs && k_cache && v_cache, -1, "rope_kv_cache_write: null pointer");
  AXM_CHECK_ARG(T >= 1 && T <= 64, -1, "rope_kv_cache_write: T=%d outside [1, 64]", T);
  AXM_CHECK_ARG(head_dim >= 2 && head_dim % 2 == 0 && q_dim > 0 && kv_dim > 0 && q_dim % head_dim == 0 &&
                    kv_dim % head_dim == 0,
                -1, "rope_kv_cache_write: bad dims q_dim=%d kv_dim=%d head_dim=%d", q_dim, kv_dim, head_dim);
  kv.Hkv = kv_dim / head_dim;
  if (kv_dtype != AXM_KV_FP16) {
    AXM_CHECK_ARG(kv_dtype == AXM_KV_FP8 || kv_dtype == AXM_KV_INT4, -1, "rope_kv_cache_write: bad kv dtype %d",
                  kv_dtype);
    AXM_CHECK_ARG(head_dim % 64 == 0 && k_scales && v_scales, -1,
                  "rope_kv_cache_write: quantized caches need head_dim %% 64 == 0 and scale tensors");
  }
  AXM_CHECK_ARG(rope_len >= 1 && start_pos >= 0 && max_seq_len >= 1 && write_pos >= 0 && write_pos < max_seq_len, -1,
                "rope_kv_cache_write: bad positions start_pos=%d write_pos=%d", start_pos, write_pos);
  RopePositions rp{};
  for (int t = 0; t < T; ++t) {
    const int d = depths_host ? depths_host[t] : t;
    AXM_CHECK_ARG(d >= 0, -1, "rope_kv_cache_write: negative depth at %d", t);
    rp.pos[t] = (int)(((long long)start_pos + d) % rope_len);
  }
  const int qkv_dim = q_dim + 2 * kv_dim;
  const dim3 grid((qkv_dim + 63) / 64, T);
  hipLaunchKernelGGL(rope_kv_write_kernel, grid, dim3(64), 0, (hipStream_t)stream, (f16*)qkv, (const f16*)qkv_bias,
                     (const float*)freqs, rp, q_dim, kv_dim, kv, write_pos);
  AXM_LAUNCH_CHECK("rope_kv_cache_write");
  return 0;
}

// ---------------------------------------------------------------------------
// KV dequantization (dequantize_kv_cache_{fp8,int4}_mps, mps_kernels.mm:930-1004;
// dequantize_kv_fp8 / dequantize_kv_int4, quant.py:727-852): rows of hd codes
// with hd/64 fp16 scales -> fp16, rounded as the reference does (fp8 -> fp16
// exact then one rounding of the product; int4 (q ^ 8) - 8 times the scale).
// One thread per 8 elements.
// ---------------------------------------------------------------------------
namespace {
template <int KVT>
__global__ void dequant_kv_kernel(const void* __restrict__ codes, const f16* __restrict__ scales, long rows, int hd,
                                  f16* __restrict__ out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = hd / 8;
  if (i >= rows * per_row) return;
  const long row = i / per_row;
  const int e0 = (int)(i % per_row) * 8;
  float v[8];
  load_kv8<KVT>(codes, scales, (size_t)row, hd, e0, v);
  f16x8 h;
#pragma unroll
  for (int k = 0; k < 8; ++k) h[k] = f2h(v[k]);
  *reinterpret_cast<f16x8*>(out + row * hd + e0) = h;
}
}  // namespace

extern "C" int axm_dequantize_kv(const void* codes, const void* scales, int kv_dtype, long rows, int head_dim,
                                 void* out, void* stream) {
  AXM_CHECK_ARG(codes && scales && out, -1, "dequantize_kv: null pointer");
  AXM_CHECK_ARG(kv_dtype == AXM_KV_FP8 || kv_dtype == AXM_KV_INT4, -1, "dequantize_kv: kv dtype %d is not quantized",
                kv_dtype);
  AXM_CHECK_ARG(rows >= 0 && head_dim >= 64 && head_dim % 64 == 0, -1, "dequantize_kv: bad shape rows=%ld hd=%d", rows,
                head_dim);
  if (rows == 0) return 0;
  const long n = rows * (head_dim / 8);
  const dim3 grid((unsigned)((n + 255) / 256));
  if (kv_dtype == AXM_KV_FP8)
    hipLaunchKernelGGL(dequant_kv_kernel<AXM_KV_FP8>, grid, dim3(256), 0, (hipStream_t)stream, codes,
                       (const f16*)scales, rows, head_dim, (f16*)out);
  else
    hipLaunchKernelGGL(dequant_kv_kernel<AXM_KV_INT4>, grid, dim3(256), 0, (hipStream_t)stream, codes,
                       (const f16*)scales, rows, head_dim, (f16*)out);
  AXM_LAUNCH_CHECK("dequantize_kv");
  return 0;
}

// ---------------------------------------------------------------------------
// Tree-path KV compaction (compact_tree_kv_{half,fp8,int4}_kernel,
// metal_kernels.metal:3145-3179 / :3875-3978; StaticKVCache.compact_tree_path,
// axiomlm/engine/paged_cache.py:376-462): slot (wp + acc[m]) % S moves to
// (wp + m) % S for every (layer, k|v, batch, head) row block.  One wave owns one
// row block and stages all accepted source rows in LDS before it writes any
// destination, so overlapping source / destination slots cannot race.
// ---------------------------------------------------------------------------
namespace {

constexpr int kMaxAccepted = 64;

struct Accepted {
  int idx[kMaxAccepted];
};

// words: 32-bit words per slot row of the cache; halves: fp16 scales per slot (0 = none).
__global__ void __launch_bounds__(64) compact_tree_kernel(uint32_t* __restrict__ cache, f16* __restrict__ scales,
                                                          int S, int words, int halves, int write_pos, Accepted acc,
                                                          int n) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint32_t* stage_w = reinterpret_cast<uint32_t*>(smem);         // [n][words]
  f16* stage_s = reinterpret_cast<f16*>(stage_w + (size_t)n * words);  // [n][halves]
  const int lane = threadIdx.x;
  const size_t block = blockIdx.x;
  uint32_t* rows = cache + block * (size_t)S * words;
  f16* srows = scales != nullptr ? scales + block * (size_t)S * halves : nullptr;
  for (int m = 0; m < n; ++m) {
    const int src = (write_pos + acc.idx[m]) % S;
    for (int w = lane; w < words; w += 64) stage_w[m * words + w] = rows[(size_t)src * words + w];
    if (srows != nullptr)
      for (int h = lane; h < halves; h += 64) stage_s[m * halves + h] = srows[(size_t)src * halves + h];
  }
  __syncthreads();
  for (int m = 0; m < n; ++m) {
    const int dst = (write_pos + m) % S;
    for (int w = lane; w < words; w += 64) rows[(size_t)dst * words + w] = stage_w[m * words + w];
    if (srows != nullptr)
      for (int h = lane; h < halves; h += 64) srows[(size_t)dst * halves + h] = stage_s[m * halves + h];
  }
}

}  // namespace

extern "C" int axm_compact_tree_kv(void* cache, void* scales, int n_blocks, int max_seq_len, int slot_bytes,
                                   int scale_halves, int write_pos, const int* accepted_host, int n_accepted,
                                   void* stream) {
  AXM_CHECK_ARG(cache && n_blocks > 0 && max_seq_len > 0, -1, "compact_tree_kv: bad cache");
  AXM_CHECK_ARG(slot_bytes > 0 && slot_bytes % 4 == 0, -1, "compact_tree_kv: slot_bytes %d must be a multiple of 4",
                slot_bytes);
  AXM_CHECK_ARG(scales == nullptr || scale_halves > 0, -1, "compact_tree_kv: scales need scale_halves > 0");
  AXM_CHECK_ARG(n_accepted >= 0 && n_accepted <= kMaxAccepted, -1, "compact_tree_kv: %d accepted slots (max %d)",
                n_accepted, kMaxAccepted);
  AXM_CHECK_ARG(write_pos >= 0 && write_pos < max_seq_len, -1, "compact_tree_kv: write_pos %d out of range",
                write_pos);
  if (n_accepted == 0) return 0;
  AXM_CHECK_ARG(accepted_host != nullptr, -1, "compact_tree_kv: null accepted list");
  Accepted acc{};
  for (int m = 0; m < n_accepted; ++m) {
    AXM_CHECK_ARG(accepted_host[m] >= 0 && accepted_host[m] < max_seq_len, -1,
                  "compact_tree_kv: accepted index %d out of range", accepted_host[m]);
    acc.idx[m] = accepted_host[m];
  }
  const int words = slot_bytes / 4;
  const int halves = scales != nullptr ? scale_halves : 0;
  const size_t smem = (size_t)n_accepted * words * 4 + (size_t)n_accepted * halves * 2;
  AXM_CHECK_ARG(smem <= 64 * 1024, -1, "compact_tree_kv: slot rows too large (%zu B of staging)", smem);
  hipLaunchKernelGGL(compact_tree_kernel, dim3((unsigned)n_blocks), dim3(64), smem, (hipStream_t)stream,
                     (uint32_t*)cache, (f16*)scales, max_seq_len, words, halves, write_pos, acc, n_accepted);
  AXM_LAUNCH_CHECK("compact_tree_kv");
  return 0;
}
