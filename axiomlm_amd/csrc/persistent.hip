// Persistent whole-step decode kernel: one cooperative launch runs every layer
// of a batch-1 decode token (the work of QuantizedDecodeGraphState::step,
// axiomlm/kernels/mps_kernels.mm:3195-3263) with grid-wide barriers between
// the dependent phases instead of kernel boundaries.
//
// One 512-thread workgroup per CU.  Wave 0 is the control wave: it stages the
// phase's activation vector into LDS, reduces the per-wave partial tiles, runs
// the epilogue and takes part in the grid barrier.  Waves 1..7 are workers:
// they stream tile16 weight chunks (1 KB per wave, the B operand of four
// v_mfma_f32_16x16x32_f16) through a ring of kDepth in-flight loads.  The ring
// is one continuous stream across phases: while a worker consumes the last
// chunks of one GEMV its refills already fetch the first chunks of the next
// GEMV, so those loads are in flight through the epilogue, the grid barrier and
// the staging of the next phase.  The control wave never has weight loads
// outstanding, so its barrier atomics and activation loads are not queued
// behind them.
//
// Phases per layer (grid barrier after each):
//   A  RMSNorm(x, ln1) -> QKV GEMV -> bias -> RoPE -> q, K/V slot (fp16 cache)
//   B  split-KV attention per (query head, split); the last split of a head to
//      finish merges the head (per-head arrival counter)
//   C  O GEMV + residual  -> x
//   D  RMSNorm(x, ln2) -> gate|up GEMV -> SwiGLU -> h
//   E  down GEMV + residual -> x
// then RMSNorm(x, lnf) -> lm_head GEMV -> logits + per-tile argmax keys, a last
// barrier, and workgroup 0 reduces the keys to the greedy token.
//
// Cross-workgroup data (activations, split partials, the new K/V slot) is
// written and read with device-coherent (sc1) buffer operations, so the grid
// barrier needs no L2 write-back or invalidate: the control wave waits for its
// own stores to complete before it arrives.  Every wait on another workgroup
// is bounded; on expiry the kernel raises an error flag and all workgroups
// leave.
#include "axm.h"
#include "kernels.h"
#include "persistent.h"
#include "t16_device.h"

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = 8;
constexpr int kWorkers = 7;
constexpr int kDepth = 8;         // chunk loads in flight per worker
constexpr int kMaxLocal = 32;     // local 16-row units per workgroup per phase
constexpr int kOOB = 0x7FFFFFF0;  // out-of-range buffer offset: reads zero
constexpr int kAuxStream = 2;     // weight stream: nontemporal
constexpr int kAuxDev = 16;       // sc1: device-coherent access
constexpr float kNegBig = -1e30f;
constexpr long kSpinLimit = 1L << 21;

typedef __amdgpu_buffer_rsrc_t Rsrc;

__device__ __forceinline__ Rsrc rsrc_of(const void* p, long bytes) {
  const long lim = bytes < 0x7FFFFFF0L ? bytes : 0x7FFFFFF0L;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)lim, 0x00020000);
}

// Device-coherent loads / stores of cross-workgroup data.
__device__ __forceinline__ u32x4 ld_dev16(Rsrc r, int off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxDev));
}
__device__ __forceinline__ uint32_t ld_dev4(Rsrc r, int off) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kAuxDev));
}
__device__ __forceinline__ void st_dev2(Rsrc r, int off, f16 v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), r, off, 0, kAuxDev);
}
__device__ __forceinline__ void st_dev4(Rsrc r, int off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kAuxDev);
}
__device__ __forceinline__ void st_dev8(Rsrc r, int off, unsigned long long v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, kAuxDev);
}

__device__ __forceinline__ unsigned long long ld_relaxed(unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until this wave's memory operations (stores included) have completed.
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }

struct Smem {
  f16* x0;     // [D] raw residual input of the current sub-layer
  f16* xs;     // [KBmax*128] staged GEMV activations
  f16* zero;   // 16 zero halves
  f32x2* cx;   // [2*KBmax] magic-offset correction sums per 64-group
  float* red;  // [kMaxLocal][kWaves][16] partial tiles
  float* att;  // [kWaves][2 + 128] attention wave partials
  float* fr;   // [kMaxLocal*16][2] RoPE cos/sin of this workgroup's QKV rows
  f16* bias;   // [kMaxLocal*16]
  float* misc; // [16]
  int* flag;   // [4]
};

// ---------------------------------------------------------------------------
// Grid barrier: two-level arrival counters (8 groups, then a top counter) and
// a generation word.  Counters only grow; barrier k of a launch completes at
// generation bar_base + k + 1.
// ---------------------------------------------------------------------------
__device__ bool grid_sync(const PArgs& a, const Smem& sm, int k) {
  __syncthreads();
  if (threadIdx.x == 0) {
    wait_all_mem();
    const unsigned long long target = a.bar_base + (unsigned long long)k + 1ull;
    const int G = gridDim.x;
    const int g = blockIdx.x & 7;
    const unsigned long long n_g = (unsigned long long)((G - g + 7) / 8);
    unsigned long long* grp = a.bar + 32 * g;
    unsigned long long* top = a.bar + 32 * 8;
    unsigned long long* gen = a.bar + 32 * 9;
    const unsigned long long old = __hip_atomic_fetch_add(grp, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1ull == target * n_g) {
      const unsigned long long o2 = __hip_atomic_fetch_add(top, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (o2 + 1ull == target * 8ull) __hip_atomic_store(gen, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    int ok = 1;
    long spins = 0;
    while (ld_relaxed(gen) < target) {
      if (__hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 || ++spins > kSpinLimit) {
        __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    sm.flag[0] = ok;
  }
  __syncthreads();
  return sm.flag[0] != 0;
}

// ---------------------------------------------------------------------------
// GEMV phase description (wave-uniform).
// ---------------------------------------------------------------------------
struct Phase {
  const u32x4* w;
  const u32x2* sb;
  long w_bytes, sb_bytes;
  int KB;    // 128-wide k blocks per unit
  int n;     // units (pairs for gate|up) owned by this workgroup
  int nl;    // local tiles: n, or 2n for gate|up
  int u0;    // first owned unit
  int pair_off;  // gate|up: tile distance from a gate tile to its up tile (0 otherwise)
  int C;     // local chunks nl * KB
  int nblk;  // this worker's blocks of kDepth chunks (0 for the control wave)
};

__device__ __forceinline__ Phase make_phase(const u32x4* w, const u32x2* sb, int rows_alloc, int K, int units,
                                            bool pair, int pair_off, int worker) {
  Phase p;
  p.w = w;
  p.sb = sb;
  p.KB = (K + 127) / 128;
  p.w_bytes = (long)((rows_alloc + 15) / 16) * p.KB * 1024;
  p.sb_bytes = (long)((rows_alloc + 15) / 16) * p.KB * 128;
  const int G = gridDim.x;
  const int base = units / G, rem = units % G;
  const int g = blockIdx.x;
  p.n = base + (g < rem ? 1 : 0);
  p.u0 = g * base + (g < rem ? g : rem);
  p.nl = pair ? 2 * p.n : p.n;
  p.pair_off = pair ? pair_off : 0;
  p.C = p.nl * p.KB;
  const int NB = (p.C + kDepth - 1) / kDepth;
  p.nblk = (worker >= 0 && worker < NB) ? (NB - worker + kWorkers - 1) / kWorkers : 0;
  return p;
}

__device__ __forceinline__ Phase empty_phase() {
  Phase p{};
  p.KB = 1;
  return p;
}

__device__ __forceinline__ int unit_of(const Phase& p, int ul) {
  if (p.pair_off == 0) return p.u0 + ul;
  return ul < p.n ? p.u0 + ul : p.u0 + (ul - p.n) + p.pair_off;
}

struct Pipe {
  u32x4 w[kDepth];
  u32x2 s[kDepth];
};

// Issue the load of stream position t of phase p into ring slot j (out-of-range
// positions and padding chunks read zero).
__device__ __forceinline__ void issue(Pipe& pp, int j, const Phase& p, int worker, int t, int lane) {
  int wo = kOOB, so = kOOB;
  if (t < p.nblk * kDepth) {
    const int blk = worker + kWorkers * (t / kDepth);
    const int c = blk * kDepth + (t % kDepth);
    if (c < p.C) {
      const int ul = c / p.KB;
      const int kb = c - ul * p.KB;
      const int base = unit_of(p, ul) * p.KB + kb;
      wo = (base * 64 + lane) * 16;
      so = (base * 16 + (lane & 15)) * 8;
    }
  }
  const Rsrc rw = rsrc_of(p.w, p.w_bytes);
  const Rsrc rs = rsrc_of(p.sb, p.sb_bytes);
  pp.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, kAuxStream));
  pp.s[j] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0));
}

// Fill the ring with the first kDepth positions of phase p.
__device__ __forceinline__ void prime(Pipe& pp, const Phase& p, int worker, int lane) {
#pragma unroll
  for (int j = 0; j < kDepth; ++j) issue(pp, j, p, worker, j, lane);
}

// Worker: consume this worker's chunks of `cur`; refills continue into `nxt`.
// Partial tiles are added into red[ul][wave][row] (lanes 0..15 hold rows).
__device__ __forceinline__ void gemv_worker(Pipe& pp, const Phase& cur, const Phase& nxt, int worker, int wave,
                                            int lane, const Smem& sm, const Unpack& U) {
  const int n = cur.nblk * kDepth;
  if (n == 0) {
    prime(pp, nxt, worker, lane);
    return;
  }
  const f16* xa = (lane & 15) == 0 ? sm.xs + 8 * (lane >> 4) : sm.zero;
  const int a_kb = (lane & 15) == 0 ? 128 : 0;
  const int a_c = (lane & 15) == 0 ? 32 : 0;
  float acc = 0.f;
  int cur_ul = -1;
  for (int t0 = 0; t0 < n; t0 += kDepth) {
    const int blk = worker + kWorkers * (t0 / kDepth);
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      const int c = blk * kDepth + j;
      if (c < cur.C) {
        const int ul = c / cur.KB;
        const int kb = c - ul * cur.KB;
        if (ul != cur_ul) {
          if (cur_ul >= 0 && lane < 16) sm.red[(cur_ul * kWaves + wave) * 16 + lane] += acc;
          acc = 0.f;
          cur_ul = ul;
        }
        const f16* xk = xa + kb * a_kb;
        f16x8 A[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) A[q] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(xk + q * a_c));
        const f32x4 cxv = *reinterpret_cast<const f32x4*>(sm.cx + 2 * kb);
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
        f32x4 d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], unpack_word(pp.w[j][0], U), z4, 0, 0, 0);
        f32x4 d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[2], unpack_word(pp.w[j][2], U), z4, 0, 0, 0);
        d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1], unpack_word(pp.w[j][1], U), d0, 0, 0, 0);
        d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[3], unpack_word(pp.w[j][3], U), d1, 0, 0, 0);
        const f16x2 sb0 = as_h2(pp.s[j][0]);
        const f16x2 sb1 = as_h2(pp.s[j][1]);
        acc = __builtin_fmaf(h2f(sb0.x), d0[0] - cxv[0], acc);
        acc = __builtin_fmaf(h2f(sb0.y), cxv[1], acc);
        acc = __builtin_fmaf(h2f(sb1.x), d1[0] - cxv[2], acc);
        acc = __builtin_fmaf(h2f(sb1.y), cxv[3], acc);
      }
      const int tn = t0 + j + kDepth;
      if (tn < n)
        issue(pp, j, cur, worker, tn, lane);
      else
        issue(pp, j, nxt, worker, tn - n, lane);
    }
  }
  if (cur_ul >= 0 && lane < 16) sm.red[(cur_ul * kWaves + wave) * 16 + lane] += acc;
}

// Sum of the partial tiles of local unit ul, row j (control wave).
__device__ __forceinline__ float unit_row(const Smem& sm, int ul, int j) {
  float v = 0.f;
#pragma unroll
  for (int w = 1; w < kWaves; ++w) v += sm.red[(ul * kWaves + w) * 16 + j];
  return v;
}

// ---------------------------------------------------------------------------
// Staging: activations (device-coherent) -> LDS, optional fp16 RMSNorm, the
// per-64-group correction sums, zeroed partial tiles.  keep_raw also copies the
// raw vector into x0.  emb >= 0 stages the embedding row of that token instead.
// ---------------------------------------------------------------------------
__device__ void stage(const PArgs& a, const Smem& sm, const f16* src, int K, const f16* ln_w, bool keep_raw,
                      bool embed, long long emb, int nl_max) {
  const int tid = threadIdx.x;
  const int KB = (K + 127) / 128;
  const int nv = K / 8, nv_pad = KB * 16;
  if (tid < 64) {
    if (embed) {
      // Token ids outside [0, V) give a zero row (as the stand-alone gathers do).
      const bool in_range = emb >= 0 && emb < a.V;
      for (int i = tid; i < nv; i += 64) {
        f16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = f16(0);
        if (in_range) {
          if (a.wte_fmt == 0) {
            v = *reinterpret_cast<const f16x8*>((const f16*)a.wte + (size_t)emb * K + 8 * i);
          } else {
            const u32x2 qv = *reinterpret_cast<const u32x2*>((const uint8_t*)a.wte + (size_t)emb * K + 8 * i);
            const f16* sbr = a.wte_sb + ((size_t)emb * (K / 64) + (8 * i) / 64) * 2;
            const float s = h2f(sbr[0]), b = h2f(sbr[1]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float qq = (float)((qv[e >> 2] >> (8 * (e & 3))) & 0xFFu);
              v[e] = f2h(add_rn(mul_rn(qq, s), b));
            }
          }
        }
        reinterpret_cast<f16x8*>(sm.xs)[i] = v;
        if (keep_raw) reinterpret_cast<f16x8*>(sm.x0)[i] = v;
      }
    } else {
      const Rsrc r = rsrc_of(src, (long)K * 2);
      for (int i = tid; i < nv; i += 64) {
        const u32x4 v = ld_dev16(r, 16 * i);
        reinterpret_cast<u32x4*>(sm.xs)[i] = v;
        if (keep_raw) reinterpret_cast<u32x4*>(sm.x0)[i] = v;
      }
    }
    for (int i = nv + tid; i < nv_pad; i += 64) reinterpret_cast<u32x4*>(sm.xs)[i] = u32x4{0u, 0u, 0u, 0u};
    for (int i = tid; i < nl_max * kWaves * 16; i += 64) sm.red[i] = 0.f;
    if (tid < 8) reinterpret_cast<uint32_t*>(sm.zero)[tid] = 0u;
  }
  __syncthreads();
  float rinv = 1.f;
  if (ln_w != nullptr) {
    // Same summation order as the stand-alone tile16 kernel: per-thread strided
    // partials over 8-element vectors, wave sums, then the 8 waves in order.
    float s = 0.f;
    for (int i = tid; i < nv; i += kThreads) {
      const f16x8 v = reinterpret_cast<const f16x8*>(sm.xs)[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = h2f(v[e]);
        s += h2f(f2h(f * f));
      }
    }
    s = wave_sum(s);
    if ((tid & 63) == 0) sm.misc[tid >> 6] = s;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += sm.misc[w];
    rinv = rms_inv_fp16(tot, K, a.eps);
  }
  for (int i0 = 0; i0 < nv_pad; i0 += kThreads) {
    const int i = i0 + tid;
    f16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = f16(0);
    if (i < nv) {
      v = reinterpret_cast<const f16x8*>(sm.xs)[i];
      if (ln_w != nullptr) {
        const f16x8 w = reinterpret_cast<const f16x8*>(ln_w)[i];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = f2h(h2f(f2h(h2f(v[e]) * rinv)) * h2f(w[e]));
        reinterpret_cast<f16x8*>(sm.xs)[i] = v;
      }
    }
    float corr = 0.f, sum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = h2f(v[e]);
      sum += f;
      corr += f * (((e >> 1) & 1) ? 64.f : 1024.f);
    }
    corr = group_sum<8>(corr);
    sum = group_sum<8>(sum);
    if (i < nv_pad && (tid & 7) == 0) sm.cx[i >> 3] = f32x2{corr, sum};
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------
// Attention (fp16 cache): one workgroup per (query head, split) item.
// ---------------------------------------------------------------------------
__device__ bool attention_phase(const PArgs& a, const Smem& sm, const PLayer& Ly, int layer) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hd = a.hd;
  const int LPT = hd / 8, KPW = 64 / LPT;
  const int sub = lane / LPT, e0 = (lane % LPT) * 8;
  const int ns = a.n_splits;
  const int n_rep = a.Hq / a.Hkv;
  const int n_keys = a.active_len;
  const int per = (n_keys + ns - 1) / ns;
  const Rsrc rq = rsrc_of(a.q, (long)a.Hq * hd * 2);
  const Rsrc rk = rsrc_of(Ly.kc, (long)a.Hkv * a.S * hd * 2);
  const Rsrc rv = rsrc_of(Ly.vc, (long)a.Hkv * a.S * hd * 2);
  const Rsrc rws = rsrc_of(a.ws, (long)a.Hq * ns * (2 + hd) * 4);
  const Rsrc rat = rsrc_of(a.attn, (long)a.Hq * hd * 2);
  for (int item = blockIdx.x; item < a.Hq * ns; item += gridDim.x) {
    const int hq = item / ns, split = item % ns;
    const int kvh = hq / n_rep;
    float q[8];
    {
      const u32x4 qv = ld_dev16(rq, (hq * hd + e0) * 2);
      const f16x8 qh = __builtin_bit_cast(f16x8, qv);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = h2f(qh[i]);
    }
    const int k_begin = min(split * per, n_keys);
    const int k_end = min(k_begin + per, n_keys);
    float m = kNegBig, l = 0.f, o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0.f;
    const long head_row0 = (long)kvh * a.S;
    for (int kb = k_begin + wave * KPW; kb < k_end; kb += kWaves * KPW) {
      const int key = kb + sub;
      const bool valid = key < k_end;
      float kf[8], vf[8];
      if (valid) {
        const int off = (int)(((head_row0 + key) * hd + e0) * 2);
        const f16x8 kh = __builtin_bit_cast(f16x8, ld_dev16(rk, off));
        const f16x8 vh = __builtin_bit_cast(f16x8, ld_dev16(rv, off));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kf[i] = h2f(kh[i]);
          vf[i] = h2f(vh[i]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) kf[i] = vf[i] = 0.f;
      }
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d = __builtin_fmaf(q[i], kf[i], d);
      for (int off = LPT / 2; off > 0; off >>= 1) d += __shfl_xor(d, off, 64);
      const float s = valid ? d * a.scale_log2 : kNegBig;
      const float m_new = fmaxf(m, s);
      const float alpha = exp2f(m - m_new);
      const float pr = valid ? exp2f(s - m_new) : 0.f;
      l = l * alpha + pr;
      m = m_new;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = __builtin_fmaf(o[i], alpha, pr * vf[i]);
    }
    for (int off = LPT; off < 64; off <<= 1) {
      const float m2 = __shfl_xor(m, off, 64);
      const float l2 = __shfl_xor(l, off, 64);
      const float mn = fmaxf(m, m2);
      const float a1 = exp2f(m - mn), a2 = exp2f(m2 - mn);
      l = l * a1 + l2 * a2;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float o2 = __shfl_xor(o[i], off, 64);
        o[i] = o[i] * a1 + o2 * a2;
      }
      m = mn;
    }
    float* att = sm.att + wave * (2 + 128);
    if (lane < LPT) {
      if (lane == 0) {
        att[0] = m;
        att[1] = l;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) att[2 + e0 + i] = o[i];
    }
    __syncthreads();
    if (wave == 0) {
      // Lanes 0..hd/2-1 hold two elements each.
      float mm = kNegBig;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm.att[w * (2 + 128)]);
      float ll = 0.f, oa = 0.f, ob = 0.f;
      const int ea = lane, eb = lane + 64;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float* aw = sm.att + w * (2 + 128);
        const float sc = exp2f(aw[0] - mm);
        ll += aw[1] * sc;
        if (ea < hd) oa += aw[2 + ea] * sc;
        if (eb < hd) ob += aw[2 + eb] * sc;
      }
      if (ns == 1) {
        if (ea < hd) st_dev2(rat, (hq * hd + ea) * 2, f2h(ll > 0.f ? oa / ll : 0.f));
        if (eb < hd) st_dev2(rat, (hq * hd + eb) * 2, f2h(ll > 0.f ? ob / ll : 0.f));
      } else {
        const int pbase = (hq * ns + split) * (2 + hd);
        if (lane == 0) {
          st_dev4(rws, pbase * 4, __builtin_bit_cast(uint32_t, mm));
          st_dev4(rws, (pbase + 1) * 4, __builtin_bit_cast(uint32_t, ll));
        }
        if (ea < hd) st_dev4(rws, (pbase + 2 + ea) * 4, __builtin_bit_cast(uint32_t, oa));
        if (eb < hd) st_dev4(rws, (pbase + 2 + eb) * 4, __builtin_bit_cast(uint32_t, ob));
        wait_all_mem();
        unsigned long long old = 0;
        if (lane == 0)
          old = __hip_atomic_fetch_add(a.head_cnt + hq, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0, 64);
        const unsigned long long target = a.merge_base + (unsigned long long)(layer + 1) * ns;
        if (old + 1ull == target) {
          // Last split of this head: merge all partials.
          float gm = kNegBig;
          for (int s2 = 0; s2 < ns; ++s2)
            gm = fmaxf(gm, __builtin_bit_cast(float, ld_dev4(rws, ((hq * ns + s2) * (2 + hd)) * 4)));
          float gl = 0.f, ga = 0.f, gb = 0.f;
          for (int s2 = 0; s2 < ns; ++s2) {
            const int pb = (hq * ns + s2) * (2 + hd);
            const float ms = __builtin_bit_cast(float, ld_dev4(rws, pb * 4));
            const float ls = __builtin_bit_cast(float, ld_dev4(rws, (pb + 1) * 4));
            const float sc = exp2f(ms - gm);
            gl += ls * sc;
            if (ea < hd) ga += __builtin_bit_cast(float, ld_dev4(rws, (pb + 2 + ea) * 4)) * sc;
            if (eb < hd) gb += __builtin_bit_cast(float, ld_dev4(rws, (pb + 2 + eb) * 4)) * sc;
          }
          if (ea < hd) st_dev2(rat, (hq * hd + ea) * 2, f2h(gl > 0.f ? ga / gl : 0.f));
          if (eb < hd) st_dev2(rat, (hq * hd + eb) * 2, f2h(gl > 0.f ? gb / gl : 0.f));
        }
      }
    }
    __syncthreads();
  }
  return true;
}

// ---------------------------------------------------------------------------
// The kernel.  Phases are enumerated as one sequence (per layer A B C D E, then
// the lm_head) so the weight-stream loop has a single instance and the ring
// registers stay in VGPRs.
// ---------------------------------------------------------------------------
enum { PH_QKV = 0, PH_ATTN = 1, PH_O = 2, PH_GU = 3, PH_DN = 4, PH_LM = 5, PH_NONE = 6 };

__device__ __forceinline__ int phase_kind(int ph, int L) {
  if (ph >= 5 * L) return ph == 5 * L ? PH_LM : PH_NONE;
  return ph % 5;
}

__device__ __forceinline__ Phase phase_desc(const PArgs& a, int kind, int layer, int worker) {
  const int D = a.D, H = a.H, q_dim = a.Hq * a.hd, kv_dim = a.Hkv * a.hd;
  const int qkv_rows = q_dim + 2 * kv_dim;
  if (kind == PH_LM) return make_phase(a.lm_w, a.lm_sb, a.V, D, (a.V + 15) / 16, false, 0, worker);
  if (kind == PH_NONE || kind == PH_ATTN) return empty_phase();
  const PLayer& L = a.layers[layer];
  if (kind == PH_QKV) return make_phase(L.qkv_w, L.qkv_sb, qkv_rows, D, (qkv_rows + 15) / 16, false, 0, worker);
  if (kind == PH_O) return make_phase(L.o_w, L.o_sb, D, q_dim, (D + 15) / 16, false, 0, worker);
  if (kind == PH_GU) return make_phase(L.gu_w, L.gu_sb, 2 * H, D, H / 16, true, H / 16, worker);
  return make_phase(L.dn_w, L.dn_sb, D, H, (D + 15) / 16, false, 0, worker);
}

// The GEMV phase that follows phase ph in the weight stream (attention skipped).
__device__ __forceinline__ Phase next_gemv(const PArgs& a, int ph, int worker) {
  int nx = ph + 1;
  if (phase_kind(nx, a.L) == PH_ATTN) ++nx;
  return phase_desc(a, phase_kind(nx, a.L), nx / 5, worker);
}

// Control-wave epilogues.
__device__ void epilogue_qkv(const PArgs& a, const Smem& sm, const Phase& cur, const PLayer& Ly) {
  const int lane = threadIdx.x & 63;
  const int hd = a.hd, q_dim = a.Hq * hd, kv_dim = a.Hkv * hd;
  const int qkv_rows = q_dim + 2 * kv_dim;
  const Rsrc rq = rsrc_of(a.q, (long)q_dim * 2);
  const Rsrc rk = rsrc_of(Ly.kc, (long)a.Hkv * a.S * hd * 2);
  const Rsrc rv = rsrc_of(Ly.vc, (long)a.Hkv * a.S * hd * 2);
  for (int ul0 = 0; ul0 < cur.nl; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const bool have = ul < cur.nl;
    const int row = (cur.u0 + ul) * 16 + j;
    const float v = have ? unit_row(sm, ul, j) : 0.f;
    f16 h = f2h(v);
    if (have) h = f2h(h2f(h) + h2f(sm.bias[ul * 16 + j]));
    const float partner = __shfl_xor(h2f(h), 1, 64);
    if (have && row < qkv_rows) {
      f16 out = h;
      if (row < q_dim + kv_dim) {
        const bool even = (row & 1) == 0;
        const f16 x0 = even ? h : f2h(partner);
        const f16 x1 = even ? f2h(partner) : h;
        const float c = sm.fr[2 * (ul * 16 + j)], s = sm.fr[2 * (ul * 16 + j) + 1];
        out = rope_out(x0, x1, c, s, even);
      }
      if (row < q_dim) {
        st_dev2(rq, row * 2, out);
      } else {
        const bool is_k = row < q_dim + kv_dim;
        const int within = is_k ? row - q_dim : row - q_dim - kv_dim;
        const int kvh = within / hd, e = within % hd;
        const int off = (int)((((long)kvh * a.S + a.write_pos) * hd + e) * 2);
        st_dev2(is_k ? rk : rv, off, out);
      }
    }
  }
}

// x[row] = x0[row] + y[row] for this workgroup's rows (O and down projections).
__device__ void epilogue_resid(const PArgs& a, const Smem& sm, const Phase& cur) {
  const int lane = threadIdx.x & 63;
  const Rsrc rx = rsrc_of(a.x, (long)a.D * 2);
  for (int ul0 = 0; ul0 < cur.nl; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const int row = (cur.u0 + ul) * 16 + j;
    if (ul < cur.nl && row < a.D) {
      const f16 y = f2h(unit_row(sm, ul, j));
      st_dev2(rx, row * 2, f2h(h2f(sm.x0[row]) + h2f(y)));
    }
  }
}

__device__ void epilogue_swiglu(const PArgs& a, const Smem& sm, const Phase& cur) {
  const int lane = threadIdx.x & 63;
  const Rsrc rh = rsrc_of(a.h, (long)a.H * 2);
  for (int ul0 = 0; ul0 < cur.n; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const int row = (cur.u0 + ul) * 16 + j;
    if (ul < cur.n && row < a.H) {
      const f16 g = f2h(unit_row(sm, ul, j));
      const f16 u = f2h(unit_row(sm, ul + cur.n, j));
      const f16 sg = f2h(t16_silu(h2f(g)));
      st_dev2(rh, row * 2, f2h(h2f(sg) * h2f(u)));
    }
  }
}

__device__ void epilogue_lm(const PArgs& a, const Smem& sm, const Phase& cur) {
  const int lane = threadIdx.x & 63;
  const Rsrc rl = rsrc_of(a.logits, (long)a.V * 2);
  const Rsrc rkey = rsrc_of(a.keys, (long)((a.V + 15) / 16) * 8);
  for (int ul0 = 0; ul0 < cur.nl; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const int unit = cur.u0 + ul;
    const int row = unit * 16 + j;
    const bool have = ul < cur.nl;
    unsigned long long key = 0ull;
    if (have && row < a.V) {
      const f16 hv = f2h(unit_row(sm, ul, j));
      st_dev2(rl, row * 2, hv);
      const uint32_t u = __builtin_bit_cast(uint32_t, h2f(hv));
      const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
      key = ((unsigned long long)ord << 32) | (0xFFFFFFFFu - (uint32_t)row);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const unsigned long long other = __shfl_xor(key, o, 64);
      key = other > key ? other : key;
    }
    if (have && j == 0) st_dev8(rkey, unit * 8, key);
  }
}

// RoPE cos/sin and bias of the QKV rows this workgroup owns (control wave).
__device__ void load_qkv_tables(const PArgs& a, const Smem& sm, const Phase& cur, const PLayer& Ly) {
  const int lane = threadIdx.x & 63;
  const int hd = a.hd, q_dim = a.Hq * hd, kv_dim = a.Hkv * hd;
  const int qkv_rows = q_dim + 2 * kv_dim;
  for (int i = lane; i < cur.nl * 16; i += 64) {
    const int row = cur.u0 * 16 + i;
    float c = 1.f, s = 0.f;
    if (row < q_dim + kv_dim) {
      const int within = row < q_dim ? row : row - q_dim;
      const int fi = (within % hd) >> 1;
      c = a.freqs[((size_t)a.rope_pos * (hd / 2) + fi) * 2 + 0];
      s = a.freqs[((size_t)a.rope_pos * (hd / 2) + fi) * 2 + 1];
    }
    sm.fr[2 * i] = c;
    sm.fr[2 * i + 1] = s;
    sm.bias[i] = (Ly.qkv_bias != nullptr && row < qkv_rows) ? Ly.qkv_bias[row] : f16(0);
  }
}

__global__ void __launch_bounds__(kThreads) persistent_step_kernel(PArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int worker = wave - 1;  // -1 for the control wave
  const int D = a.D, H = a.H;
  const int KBmax = ((D > H ? D : H) + 127) / 128;

  Smem sm;
  {
    unsigned char* p = smem_raw;
    sm.x0 = reinterpret_cast<f16*>(p);
    p += ((size_t)D * 2 + 15) / 16 * 16;
    sm.xs = reinterpret_cast<f16*>(p);
    p += (size_t)KBmax * 256;
    sm.zero = reinterpret_cast<f16*>(p);
    p += 32;
    sm.cx = reinterpret_cast<f32x2*>(p);
    p += (size_t)KBmax * 2 * 8;
    sm.red = reinterpret_cast<float*>(p);
    p += (size_t)kMaxLocal * kWaves * 16 * 4;
    sm.att = reinterpret_cast<float*>(p);
    p += (size_t)kWaves * (2 + 128) * 4;
    sm.fr = reinterpret_cast<float*>(p);
    p += (size_t)kMaxLocal * 16 * 2 * 4;
    sm.bias = reinterpret_cast<f16*>(p);
    p += (size_t)kMaxLocal * 16 * 2;
    sm.misc = reinterpret_cast<float*>(p);
    p += 16 * 4;
    sm.flag = reinterpret_cast<int*>(p);
  }
  const Unpack U{to_vgpr(0x000F000Fu), to_vgpr(0x00F000F0u), 0x64006400u, 0x54005400u};

  // Token of this step.
  long long tok;
  if (a.idx_dev != nullptr)
    tok = a.idx_dev[0];
  else if (a.tok_host >= 0)
    tok = a.tok_host;
  else
    tok = (long long)__hip_atomic_load(a.tok_next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (blockIdx.x == 0 && tid == 0) *a.tok_used = tok;

  Pipe pp;
  if (worker >= 0) prime(pp, phase_desc(a, PH_QKV, 0, worker), worker, lane);

  const int n_phases = 5 * a.L + 1;
  for (int ph = 0; ph < n_phases; ++ph) {
    const int kind = phase_kind(ph, a.L);
    const int layer = ph / 5;
    if (kind == PH_ATTN) {
      attention_phase(a, sm, a.layers[layer], layer);
      if (!grid_sync(a, sm, ph)) return;
      continue;
    }
    const Phase cur = phase_desc(a, kind, layer, worker);
    const Phase nxt = next_gemv(a, ph, worker);
    // Staging.
    if (kind == PH_QKV) {
      if (wave == 0) load_qkv_tables(a, sm, cur, a.layers[layer]);
      stage(a, sm, a.x, D, a.layers[layer].ln1, true, layer == 0, tok, cur.nl);
    } else if (kind == PH_O) {
      stage(a, sm, a.attn, a.Hq * a.hd, nullptr, false, false, 0, cur.nl);
    } else if (kind == PH_GU) {
      stage(a, sm, a.x, D, a.layers[layer].ln2, true, false, 0, cur.nl);
    } else if (kind == PH_DN) {
      stage(a, sm, a.h, H, nullptr, false, false, 0, cur.nl);
    } else {
      stage(a, sm, a.x, D, a.lnf, false, false, 0, cur.nl);
      if (blockIdx.x == 0 && wave == 0) {
        const Rsrc rn = rsrc_of(a.norm_out, (long)D * 2);
        for (int i = lane; i < D / 2; i += 64) st_dev4(rn, 4 * i, reinterpret_cast<const uint32_t*>(sm.xs)[i]);
      }
    }
    // Weight stream.
    if (worker >= 0) gemv_worker(pp, cur, nxt, worker, wave, lane, sm, U);
    __syncthreads();
    // Epilogue.
    if (wave == 0) {
      if (kind == PH_QKV)
        epilogue_qkv(a, sm, cur, a.layers[layer]);
      else if (kind == PH_O || kind == PH_DN)
        epilogue_resid(a, sm, cur);
      else if (kind == PH_GU)
        epilogue_swiglu(a, sm, cur);
      else
        epilogue_lm(a, sm, cur);
    }
    if (!grid_sync(a, sm, ph)) return;
  }
  // Greedy token: workgroup 0 reduces the per-unit keys of every workgroup.
  if (blockIdx.x == 0 && wave == 0) {
    const int n_units = (a.V + 15) / 16;
    const Rsrc rkey = rsrc_of(a.keys, (long)n_units * 8);
    unsigned long long best = 0ull;
    for (int u = lane; u < n_units; u += 64) {
      const uint32_t lo = ld_dev4(rkey, 8 * u), hi = ld_dev4(rkey, 8 * u + 4);
      const unsigned long long k = ((unsigned long long)hi << 32) | lo;
      best = k > best ? k : best;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const unsigned long long other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    if (lane == 0)
      __hip_atomic_store(a.tok_next, (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull)), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

static size_t persist_smem_bytes(int D, int H) {
  const int KBmax = ((D > H ? D : H) + 127) / 128;
  return ((size_t)D * 2 + 15) / 16 * 16 + (size_t)KBmax * 256 + 32 + (size_t)KBmax * 2 * 8 +
         (size_t)kMaxLocal * kWaves * 16 * 4 + (size_t)kWaves * (2 + 128) * 4 + (size_t)kMaxLocal * 16 * 2 * 4 +
         (size_t)kMaxLocal * 16 * 2 + 16 * 4 + 16;
}

int persist_check(int D, int H, int Hq, int hd, int V, int* grid_out, size_t* smem_out) {
  const int cus = axm_num_cus();
  const size_t smem = persist_smem_bytes(D, H);
  if (smem > 160 * 1024) return -1;
  if (hd != 64 && hd != 128) return -1;
  if (H % 16 != 0 || D % 64 != 0 || H % 64 != 0) return -1;
  if (cus < 8) return -1;
  auto max_local = [cus](int units, int mult) { return mult * ((units + cus - 1) / cus); };
  const int qkv_units = (3 * D + 15) / 16;  // upper bound (Hkv <= Hq)
  if (max_local(qkv_units, 1) > kMaxLocal || max_local(H / 16, 2) > kMaxLocal ||
      max_local((V + 15) / 16, 1) > kMaxLocal || max_local((D + 15) / 16, 1) > kMaxLocal)
    return -1;
  if (hipFuncSetAttribute((const void*)persistent_step_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)smem) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, persistent_step_kernel, kThreads, smem) != hipSuccess ||
      occ < 1) {
    (void)hipGetLastError();
    return -1;
  }
  int coop = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) {
    (void)hipGetLastError();
    return -1;
  }
  *grid_out = cus;
  *smem_out = smem;
  return 0;
}

int persist_choose_splits(int grid, int Hq, int hd, int active_len) {
  const int keys_per_step = kWaves * (64 / (hd / 8));
  int ns = grid / Hq;
  const int by_len = (active_len + keys_per_step - 1) / keys_per_step;
  if (ns > by_len) ns = by_len;
  if (ns > 64) ns = 64;
  if (ns < 1) ns = 1;
  return ns;
}

int persist_launch(const PArgs& a, int grid, size_t smem, hipStream_t s) {
  PArgs args = a;
  void* kargs[] = {&args};
  const hipError_t e = hipLaunchCooperativeKernel((const void*)persistent_step_kernel, dim3(grid), dim3(kThreads),
                                                  kargs, (unsigned)smem, s);
  if (e != hipSuccess) {
    axm_set_error("persistent step: cooperative launch failed: %s", hipGetErrorString(e));
    return -5;
  }
  return 0;
}
