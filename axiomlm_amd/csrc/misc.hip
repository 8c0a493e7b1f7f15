// Row-wise kernels of the decode step: RMSNorm (+ residual add), SwiGLU,
// argmax, embedding gathers, the fp16 GEMV of the fp16 runner, and the C-ABI
// entry points of these ops and of the Q8_G64 GEMV (q8_gemv.hip).
//
// Numerics follow the reference CPU path on a half-precision model: every
// elementwise fp16 op rounds its fp32 result to fp16 (torch CPU semantics),
// reductions accumulate in fp32.
#include "kernels.h"

namespace {

constexpr int kNormThreads = 256;

__device__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) s += red[i];
  return s;
}

// y = half(half(x * rinv) * w)   (modules.py:41-43)
__global__ void __launch_bounds__(kNormThreads)
    rmsnorm_kernel(const f16* __restrict__ x, const f16* __restrict__ w, f16* __restrict__ y, int D, float eps) {
  __shared__ float red[kNormThreads / 64];
  const f16* xr = x + (size_t)blockIdx.x * D;
  f16* yr = y + (size_t)blockIdx.x * D;
  float s = 0.f;
  for (int k = threadIdx.x; k < D; k += kNormThreads) {
    float v = h2f(xr[k]);
    s += h2f(f2h(v * v));
  }
  const float rinv = rms_inv_fp16(block_sum_256(s, red), D, eps);
  for (int k = threadIdx.x; k < D; k += kNormThreads) {
    f16 t = f2h(h2f(xr[k]) * rinv);
    yr[k] = f2h(h2f(t) * h2f(w[k]));
  }
}

// Row-vectorized forms of the two norms (same per-element rounding) for rows of
// D % 8 == 0, D <= 8 * kNormThreads * kNormVec with 16-byte aligned rows: every
// thread loads its 8-element vectors once, keeps them in registers across the
// block reduction and writes the normalized vectors.  ADD: x = half(x + r) first.
constexpr int kNormVec = 4;
template <bool ADD>
__global__ void __launch_bounds__(kNormThreads)
    rmsnorm_vec_kernel(f16* __restrict__ x, const f16* __restrict__ r, const f16* __restrict__ w,
                       f16* __restrict__ y, int D, float eps) {
  __shared__ float red[kNormThreads / 64];
  const int nv = D / 8;
  f16x8* xr = reinterpret_cast<f16x8*>(x + (size_t)blockIdx.x * D);
  const f16x8* rr = reinterpret_cast<const f16x8*>(r + (size_t)blockIdx.x * D);
  f16x8* yr = reinterpret_cast<f16x8*>(y + (size_t)blockIdx.x * D);
  const f16x8* wr = reinterpret_cast<const f16x8*>(w);
  f16x8 v[kNormVec];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kNormVec; ++i) {
    const int j = threadIdx.x + i * kNormThreads;
    if (j < nv) {
      v[i] = xr[j];
      if (ADD) {
        const f16x8 rv = rr[j];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] = f2h(h2f(v[i][e]) + h2f(rv[e]));
        xr[j] = v[i];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = h2f(v[i][e]);
        s += h2f(f2h(f * f));
      }
    }
  }
  const float rinv = rms_inv_fp16(block_sum_256(s, red), D, eps);
#pragma unroll
  for (int i = 0; i < kNormVec; ++i) {
    const int j = threadIdx.x + i * kNormThreads;
    if (j < nv) {
      const f16x8 wv = wr[j];
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = f2h(h2f(f2h(h2f(v[i][e]) * rinv)) * h2f(wv[e]));
      yr[j] = o;
    }
  }
}

bool norm_vec_ok(const void* x, const void* r, const void* w, const void* y, int D) {
  const uintptr_t al = (uintptr_t)x | (uintptr_t)r | (uintptr_t)w | (uintptr_t)y;
  return D % 8 == 0 && D <= 8 * kNormThreads * kNormVec && (al & 15) == 0;
}

// x = half(x + r);  y = rmsnorm(x)   (transformer.py:1176-1178)
__global__ void __launch_bounds__(kNormThreads)
    add_rmsnorm_kernel(f16* __restrict__ x, const f16* __restrict__ r, const f16* __restrict__ w,
                       f16* __restrict__ y, int D, float eps) {
  __shared__ float red[kNormThreads / 64];
  f16* xr = x + (size_t)blockIdx.x * D;
  const f16* rr = r + (size_t)blockIdx.x * D;
  f16* yr = y + (size_t)blockIdx.x * D;
  float s = 0.f;
  for (int k = threadIdx.x; k < D; k += kNormThreads) {
    f16 h = f2h(h2f(xr[k]) + h2f(rr[k]));
    xr[k] = h;
    float v = h2f(h);
    s += h2f(f2h(v * v));
  }
  const float rinv = rms_inv_fp16(block_sum_256(s, red), D, eps);
  for (int k = threadIdx.x; k < D; k += kNormThreads) {
    f16 t = f2h(h2f(xr[k]) * rinv);
    yr[k] = f2h(h2f(t) * h2f(w[k]));
  }
}

// y = half(half(silu(g)) * u) with [g || u] rows (transformer.py:1188-1189)
__global__ void swiglu_kernel(const f16* __restrict__ gu, f16* __restrict__ y, int rows, int H) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)rows * H) return;
  const long r = i / H, c = i % H;
  const float g = h2f(gu[r * 2 * H + c]);
  const f16 sg = f2h(g / (1.0f + expf(-g)));
  y[i] = f2h(h2f(sg) * h2f(gu[r * 2 * H + H + c]));
}

// Argmax with lowest-index tie break; NaN compares as smaller than anything.
__global__ void __launch_bounds__(256) argmax_kernel(const f16* __restrict__ logits, int V, int64_t* __restrict__ out) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  const f16* lr = logits + (size_t)blockIdx.x * V;
  float best = -INFINITY;
  int besti = 0x7fffffff;
  auto take = [&](float v, int k) {
    if (v > best || (v == best && k < besti)) {
      best = v;
      besti = k;
    }
  };
  if (V % 8 == 0 && ((uintptr_t)lr & 15) == 0) {
    // 16-byte vectors, kArgVec requested per thread before any is compared (a
    // 32000-entry row in one batch); a thread visits its indices in increasing order,
    // so a strict > keeps the lowest of a tie.
    constexpr int kArgVec = 16;
    const f16x8* l8 = reinterpret_cast<const f16x8*>(lr);
    const int nv = V / 8;
    for (int v0 = threadIdx.x; v0 < nv; v0 += kArgVec * 256) {
      f16x8 h[kArgVec];
#pragma unroll
      for (int u = 0; u < kArgVec; ++u) h[u] = v0 + u * 256 < nv ? l8[v0 + u * 256] : f16x8{};
#pragma unroll
      for (int u = 0; u < kArgVec; ++u) {
        const int v = v0 + u * 256;
        if (v < nv) {
#pragma unroll
          for (int e = 0; e < 8; ++e) take(h2f(h[u][e]), 8 * v + e);
        }
      }
    }
  } else {
    for (int k = threadIdx.x; k < V; k += 256) take(h2f(lr[k]), k);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(besti, o, 64);
    if (ov > best || (ov == best && oi < besti)) {
      best = ov;
      besti = oi;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bv[w] = best;
    bi[w] = besti;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; ++i)
      if (bv[i] > best || (bv[i] == best && bi[i] < besti)) {
        best = bv[i];
        besti = bi[i];
      }
    out[blockIdx.x] = besti == 0x7fffffff ? 0 : besti;
  }
}

__device__ __forceinline__ long token_of(const int64_t* tokens, const int* tok_dev, int t) {
  return tokens != nullptr ? (long)tokens[t] : (long)tok_dev[t];
}

// Out-of-range token ids produce a zero row instead of reading outside the table.
__global__ void embed_f16_kernel(const f16* __restrict__ table, const int64_t* __restrict__ tokens,
                                 const int* __restrict__ tok_dev, f16* __restrict__ out, int D, int V) {
  const int t = blockIdx.x;
  const long tok = token_of(tokens, tok_dev, t);
  const bool ok = tok >= 0 && tok < V;
  for (int k = threadIdx.x; k < D; k += blockDim.x) out[(size_t)t * D + k] = ok ? table[(size_t)tok * D + k] : f16(0);
}

// Q8_G64 row dequantization: half(q * scale + bias) in fp32 (quant.py:132-163).
__global__ void embed_q8_kernel(const uint8_t* __restrict__ wq, const f16* __restrict__ sb,
                                const int64_t* __restrict__ tokens, const int* __restrict__ tok_dev,
                                f16* __restrict__ out, int D, int V) {
  const int t = blockIdx.x;
  const long tok = token_of(tokens, tok_dev, t);
  const int G = D / 64;
  if (tok < 0 || tok >= V) {
    for (int k = threadIdx.x; k < D; k += blockDim.x) out[(size_t)t * D + k] = f16(0);
    return;
  }
  for (int k = threadIdx.x; k < D; k += blockDim.x) {
    const float q = (float)wq[(size_t)tok * D + k];
    const f16* sbr = sb + ((size_t)tok * G + k / 64) * 2;
    out[(size_t)t * D + k] = f2h(add_rn(mul_rn(q, h2f(sbr[0])), h2f(sbr[1])));
  }
}

// ---------------------------------------------------------------------------
constexpr int kQ8Threads = 256;

// fp16 GEMV (the dense layers of the fp16 decode runner):  y[n] = sum_k w[n][k] x[k].
// Activations (optionally RMS-normalized with the fp16 op order of the quantized
// paths) are staged in LDS as fp16 pairs; one wave per output per iteration, each
// lane streaming 16 bytes (8 weights) per step into v_dot2_f32_f16 with fp32
// accumulation.  A wave requests its first weights before the activation staging and
// each next step's (the next output's, after a row's last) before the current row's
// reduction and epilogue.  Epilogues (kF16Store / kF16Resid / kF16Swiglu) as those of the Q8_G64
// GEMV: y = fp16(acc) (+ bias); resid = fp16(resid + fp16(acc)) in place; or, over a
// [W_gate; W_up] matrix of N = 2 H rows, y[c] = fp16(fp16(silu(g)) * u) with g, u the
// fp16 outputs of rows c and H + c, which one wave computes together; kF16Qkv: the QKV
// RoPE / KV-slot epilogue of QkvRope on the row pairs (2 p, 2 p + 1) of one wave.
enum { kF16Store = 0, kF16Resid = 1, kF16Swiglu = 2, kF16Qkv = 3 };
// 512-element steps whose weight loads a lane issues together (fp16 runner: three 329.7,
// four 334.5 tok/s).
constexpr int kF16Unroll = 4;
// Activation vectors (8 values) per thread held in registers across the RMSNorm
// reduction when the launch's M K / 8 vectors fit (one token up to K = 12288).
constexpr int kF16RegVec = 6;
template <int EPI>
__global__ void __launch_bounds__(kQ8Threads)
    f16_gemv_kernel(const f16* __restrict__ x, const f16* __restrict__ w, const f16* __restrict__ bias,
                    f16* __restrict__ y, int M, int K, int N, const f16* __restrict__ ln_w, float eps,
                    QkvRope qr, f16* __restrict__ xn_out) {
  extern __shared__ __align__(16) f16 xh[];  // [M][K]
  __shared__ float red[kQ8Threads / 64][4];
  __shared__ float rinv_m[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_waves_total = gridDim.x * (kQ8Threads / 64);
  constexpr bool kPair = EPI == kF16Swiglu || EPI == kF16Qkv;  // two rows per wave and output
  const int outs = kPair ? N / 2 : N;
  const int nvec = M * K / 8;  // 8-value vectors of x (K % 8 == 0)
  const f16x8* x8 = reinterpret_cast<const f16x8*>(x);
  const bool one_pass = nvec <= kF16RegVec * kQ8Threads;

  // The activation vectors first (loads complete in issue order: the norm waits for
  // them only), then the weights of the wave's first step, which stream in meanwhile.
  f16x8 xv[kF16RegVec];
  if (one_pass) {
#pragma unroll
    for (int i = 0; i < kF16RegVec; ++i) {
      const int v = tid + i * kQ8Threads;
      xv[i] = v < nvec ? x8[v] : f16x8{};
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // kF16Unroll 512-element steps per pass, all of their weight loads issued before
  // any is consumed (one load per lane in flight left the stream latency-bound).
  // Nontemporal loads: each weight is read once (fp16 runner 347.2 -> 369.4 tok/s).
  // Rows of output n: n (store / residual), c = n and H + c (SwiGLU), 2 n and 2 n + 1 (QKV).
  u32x4 wv[kF16Unroll], uv[kF16Unroll];
  auto load = [&](int n, int kb) {
    const f16* wr = w + (size_t)(EPI == kF16Qkv ? 2 * n : n) * K;
    const f16* wu = w + (size_t)(EPI == kF16Qkv ? 2 * n + 1 : n + outs) * K;
#pragma unroll
    for (int u = 0; u < kF16Unroll; ++u) {
      const int k0 = kb + 64 * 8 * u + lane * 8;
      const bool ok = k0 < K;
      wv[u] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + k0)) : u32x4{0u, 0u, 0u, 0u};
      uv[u] = kPair && ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wu + k0)) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  int n = blockIdx.x * (kQ8Threads / 64) + wave;
  if (n < outs) load(n, 0);

  // Stage vector v (normalized when ln_w is set); vectors past the last store nothing.
  auto stage = [&](int v, f16x8 h) {
    if (v >= nvec) return;
    const int m = v / (K / 8), c = v % (K / 8);
    if (ln_w != nullptr) {
      const f16x8 lw = *reinterpret_cast<const f16x8*>(ln_w + 8 * c);
      const float ri = rinv_m[m];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = f2h(h2f(f2h(h2f(h[e]) * ri)) * h2f(lw[e]));
    }
    *reinterpret_cast<f16x8*>(xh + (size_t)m * K + 8 * c) = h;
    if (xn_out != nullptr && blockIdx.x == 0) *reinterpret_cast<f16x8*>(xn_out + (size_t)m * K + 8 * c) = h;
  };
  // RMSNorm scale per token (fp16-rounded squares summed in fp32, the mean rounded to
  // fp16 as in the other normed GEMVs) from the per-thread partial sums.
  auto norm_scales = [&](const float (&ssq)[4]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (m < M) {  // launch-uniform
        const float t = wave_sum(ssq[m]);
        if (lane == 0) red[wave][m] = t;
      }
    }
    __syncthreads();
    if (tid < M) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < kQ8Threads / 64; ++i) t += red[i][tid];
      rinv_m[tid] = rms_inv_fp16(t, K, eps);
    }
    __syncthreads();
  };

  if (one_pass) {
    if (ln_w != nullptr) {
      float ssq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < kF16RegVec; ++i) {
        const int v = tid + i * kQ8Threads;
        if (v < nvec) {
          float part = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f = h2f(xv[i][e]);
            part += h2f(f2h(f * f));
          }
          const int mv = v / (K / 8);
#pragma unroll
          for (int m = 0; m < 4; ++m) ssq[m] += m == mv ? part : 0.f;
        }
      }
      norm_scales(ssq);
    }
#pragma unroll
    for (int i = 0; i < kF16RegVec; ++i) {
      if (i * kQ8Threads < nvec) stage(tid + i * kQ8Threads, xv[i]);  // workgroup-uniform bound
    }
  } else {
    // More activations than the registers hold: the norm scale from a pass over x,
    // then a second pass that stages.
    if (ln_w != nullptr) {
      float ssq[4] = {0.f, 0.f, 0.f, 0.f};
      for (int v = tid; v < nvec; v += kQ8Threads) {
        const f16x8 h = x8[v];
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = h2f(h[e]);
          part += h2f(f2h(f * f));
        }
        const int mv = v / (K / 8);
#pragma unroll
        for (int m = 0; m < 4; ++m) ssq[m] += m == mv ? part : 0.f;
      }
      norm_scales(ssq);
    }
    for (int v = tid; v < nvec; v += kQ8Threads) stage(v, x8[v]);
  }
  __syncthreads();

  // Steps of 512 kF16Unroll elements over the wave's outputs n, n + n_waves_total, ...:
  // the weights of the next step (the next output's first one after a row's last) are
  // requested before this row's reduction and epilogue.
  float acc[4] = {0.f, 0.f, 0.f, 0.f}, accu[4] = {0.f, 0.f, 0.f, 0.f};
  int kb = 0;
  while (n < outs) {
#pragma unroll
    for (int u = 0; u < kF16Unroll; ++u) {
      const int k0 = kb + 64 * 8 * u + lane * 8;
      if (k0 >= K) break;
      for (int mi = 0; mi < M && mi < 4; ++mi) {
        const u32x4 xq = *reinterpret_cast<const u32x4*>(xh + (size_t)mi * K + k0);
        float d = acc[mi];
#pragma unroll
        for (int c = 0; c < 4; ++c) d = __builtin_amdgcn_fdot2(as_h2(xq[c]), as_h2(wv[u][c]), d, false);
        acc[mi] = d;
        if (kPair) {
          float e = accu[mi];
#pragma unroll
          for (int c = 0; c < 4; ++c) e = __builtin_amdgcn_fdot2(as_h2(xq[c]), as_h2(uv[u][c]), e, false);
          accu[mi] = e;
        }
      }
    }
    const int cur = n;
    kb += 64 * 8 * kF16Unroll;
    if (kb < K) {
      load(n, kb);
      continue;
    }
    kb = 0;
    n += n_waves_total;
    if (n < outs) load(n, 0);
    for (int mi = 0; mi < M && mi < 4; ++mi) {
      const float v = wave_sum(acc[mi]);
      const float u = kPair ? wave_sum(accu[mi]) : 0.f;
      acc[mi] = 0.f;
      accu[mi] = 0.f;
      if (lane == 0) {
        if (EPI == kF16Qkv) {
          const int row0 = 2 * cur, hd = qr.head_dim;
          f16 h0 = f2h(v), h1 = f2h(u);
          if (bias != nullptr) {
            h0 = f2h(h2f(h0) + h2f(bias[row0]));
            h1 = f2h(h2f(h1) + h2f(bias[row0 + 1]));
          }
          f16 o[2] = {h0, h1};
          if (row0 < qr.q_dim + qr.kv_dim) {
            const int pos = (qr.rope_pos_dev ? qr.rope_pos_dev[0] : qr.rope_pos) + mi;
            const int within = row0 < qr.q_dim ? row0 : row0 - qr.q_dim;
            const float* f = qr.freqs + ((size_t)(pos % qr.rope_len) * (hd / 2) + ((within % hd) >> 1)) * 2;
            o[0] = rope_out(h0, h1, f[0], f[1], true);
            o[1] = rope_out(h0, h1, f[0], f[1], false);
          }
          for (int j = 0; j < 2; ++j) {
            const int row = row0 + j;
            if (row < qr.q_dim) {
              qr.q_out[(size_t)mi * qr.q_dim + row] = o[j];
            } else {
              const bool is_k = row < qr.q_dim + qr.kv_dim;
              const int within = is_k ? row - qr.q_dim : row - qr.q_dim - qr.kv_dim;
              const int wp = (qr.write_pos_dev ? qr.write_pos_dev[0] : qr.write_pos) + mi;
              (is_k ? qr.k_out : qr.v_out)[(size_t)(within / hd) * qr.kv_stride_h +
                                           (size_t)(wp % qr.max_seq) * hd + within % hd] = o[j];
            }
          }
        } else if (EPI == kF16Swiglu) {
          const float g = h2f(f2h(v));
          const f16 sg = f2h(g / (1.0f + expf(-g)));
          y[(size_t)mi * outs + cur] = f2h(h2f(sg) * h2f(f2h(u)));
        } else {
          f16 h = f2h(v);
          if (bias != nullptr) h = f2h(h2f(h) + h2f(bias[cur]));
          f16* o = y + (size_t)mi * N + cur;
          *o = EPI == kF16Resid ? f2h(add_rn(h2f(*o), h2f(h))) : h;
        }
      }
    }
  }
}

template <int EPI>
int f16_gemv_rows(const f16* x, const f16* w, const f16* bias, f16* y, int M, int K, int N, const f16* ln_w,
                  float eps, hipStream_t s, const QkvRope& qr = QkvRope{}, f16* xn_out = nullptr) {
  constexpr bool kPair = EPI == kF16Swiglu || EPI == kF16Qkv;
  if (K % 8 != 0 || (kPair && N % 2 != 0)) {
    axm_set_error("f16 gemv: K=%d must be a multiple of 8 (N=%d even for SwiGLU)", K, N);
    return -2;
  }
  if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)ln_w | (uintptr_t)xn_out) & 15) {
    axm_set_error("f16 gemv: x, w, ln_w and xn_out must be 16-byte aligned");
    return -2;
  }
  int rows_max = 4;
  while (rows_max > 1 && (size_t)rows_max * K * sizeof(f16) > 150 * 1024) --rows_max;
  if ((size_t)K * sizeof(f16) > 150 * 1024) {
    axm_set_error("f16 gemv: K=%d too large for LDS staging", K);
    return -2;
  }
  const int outs = kPair ? N / 2 : N;
  const int ld_out = EPI == kF16Swiglu ? N / 2 : N;
  if (EPI == kF16Qkv && M > rows_max && (qr.rope_pos_dev || qr.write_pos_dev)) {
    axm_set_error("f16 gemv: a QKV epilogue with device positions takes at most %d tokens", rows_max);
    return -2;
  }
  for (int m0 = 0; m0 < M; m0 += rows_max) {
    QkvRope qk = qr;  // tokens m0 ..: q rows, positions and slots move with them
    qk.q_out = qr.q_out ? qr.q_out + (size_t)m0 * qr.q_dim : nullptr;
    qk.rope_pos += m0;
    qk.write_pos += m0;
    const int mc = (M - m0) < rows_max ? (M - m0) : rows_max;
    const size_t smem = (size_t)mc * K * sizeof(f16);
    static size_t attr_bytes = 0;
    if (smem > 48 * 1024 && smem > attr_bytes) {
      if (hipFuncSetAttribute((const void*)f16_gemv_kernel<EPI>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)smem) != hipSuccess) {
        (void)hipGetLastError();
        axm_set_error("f16 gemv: cannot reserve %zu bytes of LDS", smem);
        return -2;
      }
      attr_bytes = smem;
    }
    const int rows_per_block = kQ8Threads / 64;
    int grid = (outs + rows_per_block - 1) / rows_per_block;
    // One round of resident workgroups (the kernel's registers allow five or six per CU)
    // that loop over the outputs: a grid of eight per CU queued the rest behind the first
    // round (fp16 runner 334.5 -> 347.2 tok/s).
    int per_cu = 8;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f16_gemv_kernel<EPI>, kQ8Threads, smem) != hipSuccess) {
      (void)hipGetLastError();
      per_cu = 8;
    }
    if (per_cu < 1) per_cu = 1;
    const int cap = axm_num_cus() * per_cu;
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL(f16_gemv_kernel<EPI>, dim3(grid), dim3(kQ8Threads), smem, s, x + (size_t)m0 * K, w, bias,
                       y == nullptr ? nullptr : y + (size_t)m0 * ld_out, mc, K, N, ln_w, eps, qk,
                       xn_out == nullptr ? nullptr : xn_out + (size_t)m0 * K);
  }
  return 0;
}

}  // namespace

int launch_f16_gemv(const f16* x, const f16* w, const f16* bias, f16* y, int M, int K, int N, const f16* ln_w,
                    float eps, hipStream_t s, f16* xn_out) {
  return f16_gemv_rows<kF16Store>(x, w, bias, y, M, K, N, ln_w, eps, s, QkvRope{}, xn_out);
}
int launch_f16_gemv_qkv(const f16* x, const f16* w, const f16* bias, int M, int K, int N, const f16* ln_w, float eps,
                        const QkvRope& r, hipStream_t s) {
  return f16_gemv_rows<kF16Qkv>(x, w, bias, nullptr, M, K, N, ln_w, eps, s, r);
}
int launch_f16_gemv_resid(const f16* x, const f16* w, f16* resid, int M, int K, int N, const f16* ln_w, float eps,
                          hipStream_t s) {
  return f16_gemv_rows<kF16Resid>(x, w, nullptr, resid, M, K, N, ln_w, eps, s);
}
int launch_f16_gemv_swiglu(const f16* x, const f16* w, f16* y, int M, int K, int N2, const f16* ln_w, float eps,
                           hipStream_t s) {
  return f16_gemv_rows<kF16Swiglu>(x, w, nullptr, y, M, K, N2, ln_w, eps, s);
}

int launch_rmsnorm(const f16* x, const f16* w, f16* y, int rows, int D, float eps, hipStream_t s) {
  if (norm_vec_ok(x, x, w, y, D))
    hipLaunchKernelGGL(rmsnorm_vec_kernel<false>, dim3(rows), dim3(kNormThreads), 0, s, (f16*)x, (const f16*)nullptr,
                       w, y, D, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, s, x, w, y, D, eps);
  return 0;
}
int launch_add_rmsnorm(f16* x, const f16* r, const f16* w, f16* y, int rows, int D, float eps, hipStream_t s) {
  if (norm_vec_ok(x, r, w, y, D))
    hipLaunchKernelGGL(rmsnorm_vec_kernel<true>, dim3(rows), dim3(kNormThreads), 0, s, x, r, w, y, D, eps);
  else
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, s, x, r, w, y, D, eps);
  return 0;
}
int launch_swiglu(const f16* gu, f16* y, int rows, int H, hipStream_t s) {
  const long n = (long)rows * H;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gu, y, rows, H);
  return 0;
}
int launch_argmax(const f16* logits, int rows, int V, int64_t* out, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(256), 0, s, logits, V, out);
  return 0;
}
int launch_embed_f16(const f16* table, const int64_t* tokens, const int* tok_dev, f16* out, int T, int D, int V,
                     hipStream_t s) {
  hipLaunchKernelGGL(embed_f16_kernel, dim3(T), dim3(256), 0, s, table, tokens, tok_dev, out, D, V);
  return 0;
}
int launch_embed_q8(const uint8_t* wq, const f16* sb, const int64_t* tokens, const int* tok_dev, f16* out, int T,
                    int D, int V, hipStream_t s) {
  hipLaunchKernelGGL(embed_q8_kernel, dim3(T), dim3(256), 0, s, wq, sb, tokens, tok_dev, out, D, V);
  return 0;
}


// ---------------------------------------------------------------------------
// C ABI wrappers.
// ---------------------------------------------------------------------------
extern "C" int axm_rmsnorm(const void* x, const void* w, void* y, int rows, int D, float eps, void* stream) {
  AXM_CHECK_ARG(x && w && y && rows > 0 && D > 0, -1, "rmsnorm: bad arguments");
  launch_rmsnorm((const f16*)x, (const f16*)w, (f16*)y, rows, D, eps, (hipStream_t)stream);
  AXM_LAUNCH_CHECK("rmsnorm");
  return 0;
}
extern "C" int axm_add_rmsnorm(void* x, const void* r, const void* w, void* y, int rows, int D, float eps,
                               void* stream) {
  AXM_CHECK_ARG(x && r && w && y && rows > 0 && D > 0, -1, "add_rmsnorm: bad arguments");
  launch_add_rmsnorm((f16*)x, (const f16*)r, (const f16*)w, (f16*)y, rows, D, eps, (hipStream_t)stream);
  AXM_LAUNCH_CHECK("add_rmsnorm");
  return 0;
}
extern "C" int axm_swiglu_gate_up(const void* gu, void* y, int rows, int H, void* stream) {
  AXM_CHECK_ARG(gu && y && rows > 0 && H > 0, -1, "swiglu_gate_up: bad arguments");
  launch_swiglu((const f16*)gu, (f16*)y, rows, H, (hipStream_t)stream);
  AXM_LAUNCH_CHECK("swiglu_gate_up");
  return 0;
}
extern "C" int axm_argmax(const void* logits, int rows, int V, void* out_i64, void* stream) {
  AXM_CHECK_ARG(logits && out_i64 && rows > 0 && V > 0, -1, "argmax: bad arguments");
  launch_argmax((const f16*)logits, rows, V, (int64_t*)out_i64, (hipStream_t)stream);
  AXM_LAUNCH_CHECK("argmax");
  return 0;
}
extern "C" int axm_embed_q8_g64(const void* w_packed, const void* sb, const void* tokens_i64, void* out, int T,
                                int D, int V, void* stream) {
  AXM_CHECK_ARG(w_packed && sb && tokens_i64 && out && T > 0 && D % 64 == 0 && V > 0, -1,
                "embed_q8_g64: bad arguments");
  launch_embed_q8((const uint8_t*)w_packed, (const f16*)sb, (const int64_t*)tokens_i64, nullptr, (f16*)out, T, D, V,
                  (hipStream_t)stream);
  AXM_LAUNCH_CHECK("embed_q8_g64");
  return 0;
}
extern "C" int axm_qmv_q8_g64(const void* x, const void* w_packed, const void* sb, const void* bias, void* y, int M,
                              int K, int N, void* stream) {
  AXM_CHECK_ARG(x && w_packed && sb && y && M > 0 && N > 0 && K % 64 == 0, -1, "qmv_q8_g64: bad arguments");
  int rc = launch_q8_gemv((const f16*)x, (const uint8_t*)w_packed, (const f16*)sb, (const f16*)bias, (f16*)y, M, K,
                          N, nullptr, 0.f, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmv_q8_g64");
  return 0;
}
