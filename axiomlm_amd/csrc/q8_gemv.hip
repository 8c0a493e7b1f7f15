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
// the current ones are consumed; waves of one or two rows take two 16-code vectors per
// lane and step.
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

// Epilogues: kQ8Store y = fp16(acc) (+ bias, fp16 add); kQ8Resid: resid = fp16(resid +
// fp16(acc)) in place (the residual stream); kQ8Swiglu: y[c] = fp16(fp16(silu(g)) * u)
// with g, u = fp16(acc) of rows c and H + c of the [W_gate; W_up] matrix (N = 2 H).  The
// rounding is that of the GEMV's fp16 output followed by an fp16 add / swiglu_kernel.
// kQ8Qkv: the QKV RoPE / KV-slot epilogue described with QkvRope (R even: a wave's rows
// hold whole rotation pairs).
enum { kQ8Store = 0, kQ8Resid = 1, kQ8Swiglu = 2, kQ8Qkv = 3 };
// Activation vectors (8 values) per thread kept in registers across the RMSNorm
// reduction, so that the normed prologue reads x once.
constexpr int kQ8vRegVec = 8;

template <int M, int R, int EPI, int V>
__global__ void __launch_bounds__(kQ8vThreads)
    q8v_kernel(const f16* __restrict__ x, int K, int N, const uint8_t* __restrict__ w, const f16* __restrict__ sb,
               const f16* __restrict__ bias, f16* __restrict__ y, const f16* __restrict__ ln_w, float eps,
               QkvRope qr, f16* __restrict__ xn_out) {
  extern __shared__ __align__(16) unsigned char smem[];
  f16* xs = reinterpret_cast<f16*>(smem);                       // [M][K]
  float* s16 = reinterpret_cast<float*>(xs + (size_t)M * K);    // [M][K / 16]
  __shared__ float red[kQ8vWaves][M];
  __shared__ float rinv_m[M];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nvec = M * K / 8;  // 8-value vectors of x
  const f16x8* x8 = reinterpret_cast<const f16x8*>(x);
  const bool one_pass = nvec <= kQ8vRegVec * kQ8vThreads;

  // Rows of this wave: R consecutive rows, or for SwiGLU R / 2 output columns c, each
  // with its gate row c and up row H + c.
  const int H = N / 2;
  const int wrow = blockIdx.x * kQ8vWaves + wave;
  auto row_of = [&](int i) {
    if (EPI == kQ8Swiglu) {
      const int c = wrow * (R / 2) + (i % (R / 2));
      return c < H ? (i < R / 2 ? c : H + c) : N;
    }
    return wrow * R + i;
  };

  // The activation vectors first (loads complete in issue order: the norm then waits
  // for them only), then the codes and (scale, bias) of step 0.
  f16x8 xv[kQ8vRegVec];
  if (one_pass) {
#pragma unroll
    for (int i = 0; i < kQ8vRegVec; ++i) {
      const int v = tid + i * kQ8vThreads;
      xv[i] = v < nvec ? x8[v] : f16x8{};
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, N * K, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)sb, (short)0, N * (K / 64) * 4, 0x00020000);
  // Lane l of step s takes the V * 16 codes at 1024 V s + 16 V l of each row (one
  // 64-column group: 16 V divides 64).  Codes and scales are read once: nontemporal
  // loads (q4_k_m 677.5 -> 682.7, q8 483.4 -> 488.0 tok/s).
  const int steps = (K + 1024 * V - 1) / (1024 * V);
  u32x4 cw[R][V];
  uint32_t sv[R];
  auto load = [&](int s) {
    const int k0 = 1024 * V * s + 16 * V * lane;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int row = row_of(i);
      const bool ok = row < N && k0 < K;  // K % 64 == 0: the lane's V vectors are in range together
#pragma unroll
      for (int v = 0; v < V; ++v)
        cw[i][v] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? row * K + k0 + 16 * v : kOOB, 0, 2));
      sv[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (row * (K / 64) + k0 / 64) * 4 : kOOB, 0, 2);
    }
  };
  load(0);

  // Stage vector v (normalized when ln_w is set) and its share of the 16-element sums:
  // vectors c and c ^ 1 of a row are adjacent threads (K / 8 is even).  Every lane of
  // the wave takes part in the sum's lane swap; lanes past the last vector (both of a
  // pair, nvec being even) store nothing.
  auto stage = [&](int v, f16x8 h) {
    const bool valid = v < nvec;
    if (!valid) v = nvec - 1;
    const int m = v / (K / 8), c = v % (K / 8);
    if (ln_w != nullptr) {
      const f16x8 lw = *reinterpret_cast<const f16x8*>(ln_w + 8 * c);
      const float ri = rinv_m[m];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = f2h(h2f(f2h(h2f(h[e]) * ri)) * h2f(lw[e]));
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s = add_rn(s, h2f(h[e]));
    s = add_rn(s, __shfl_xor(s, 1, 64));
    if (valid) {
      *reinterpret_cast<f16x8*>(xs + (size_t)m * K + 8 * c) = h;
      if (xn_out != nullptr && blockIdx.x == 0) *reinterpret_cast<f16x8*>(xn_out + (size_t)m * K + 8 * c) = h;
      if ((c & 1) == 0) s16[(size_t)m * (K / 16) + c / 2] = s;
    }
  };

  if (one_pass) {
    if (ln_w != nullptr) {
      // RMSNorm scale per token from the vectors in registers (fp16-rounded squares
      // summed in fp32, the mean rounded to fp16 as in the other normed GEMVs).
      float ssq[M];
#pragma unroll
      for (int m = 0; m < M; ++m) ssq[m] = 0.f;
#pragma unroll
      for (int i = 0; i < kQ8vRegVec; ++i) {
        const int v = tid + i * kQ8vThreads;
        if (v < nvec) {
          float part = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f = h2f(xv[i][e]);
            part += h2f(f2h(f * f));
          }
          const int mv = v / (K / 8);
#pragma unroll
          for (int m = 0; m < M; ++m) ssq[m] += m == mv ? part : 0.f;
        }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float t = wave_sum(ssq[m]);
        if (lane == 0) red[wave][m] = t;
      }
      __syncthreads();
      if (tid < M) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < kQ8vWaves; ++i) t += red[i][tid];
        rinv_m[tid] = rms_inv_fp16(t, K, eps);
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kQ8vRegVec; ++i) {
      const int v = tid + i * kQ8vThreads;
      if (i * kQ8vThreads < nvec) stage(v, xv[i]);  // workgroup-uniform bound
    }
  } else {
    // More activations than the registers hold: the norm scale from a strided pass over
    // x, then a second pass that stages.
    if (ln_w != nullptr) {
      for (int m = 0; m < M; ++m) {
        float sq = 0.f;
        for (int k = tid; k < K; k += kQ8vThreads) {
          const float v = h2f(x[(size_t)m * K + k]);
          sq += h2f(f2h(v * v));
        }
        sq = wave_sum(sq);
        if (lane == 0) red[wave][m] = sq;
      }
      __syncthreads();
      if (tid < M) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < kQ8vWaves; ++i) t += red[i][tid];
        rinv_m[tid] = rms_inv_fp16(t, K, eps);
      }
      __syncthreads();
    }
    for (int v0 = 0; v0 < nvec; v0 += kQ8vThreads) {
      const int v = v0 + tid;
      stage(v, v < nvec ? x8[v] : f16x8{});
    }
  }
  __syncthreads();

  float r[R][M];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) r[i][m] = 0.f;
  for (int s = 0; s < steps; ++s) {
    u32x4 c0[R][V];
    uint32_t s0[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
#pragma unroll
      for (int v = 0; v < V; ++v) c0[i][v] = cw[i][v];
      s0[i] = sv[i];
    }
    if (s + 1 < steps) load(s + 1);
    const int k0 = 1024 * V * s + 16 * V * lane;
    if (k0 < K) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int kv = k0 + 16 * v;
        u32x4 xa[M], xb[M];
        float sx[M];
#pragma unroll
        for (int m = 0; m < M; ++m) {
          xa[m] = *reinterpret_cast<const u32x4*>(xs + (size_t)m * K + kv);
          xb[m] = *reinterpret_cast<const u32x4*>(xs + (size_t)m * K + kv + 8);
          sx[m] = s16[(size_t)m * (K / 16) + kv / 16];
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
              const uint32_t cwd = c0[i][v][g];
              const u32x4& xq = g < 2 ? xa[m] : xb[m];
              acc = dot2(xq[2 * (g & 1)], q8_pair(cwd, kSelLo), acc);
              acc = dot2(xq[2 * (g & 1) + 1], q8_pair(cwd, kSelHi), acc);
            }
            r[i][m] += sc * (acc - 1024.f * sx[m]) + bi * sx[m];
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int m = 0; m < M; ++m) r[i][m] = wave_sum(r[i][m]);
  if (lane == 0) {
    if (EPI == kQ8Qkv) {
      const int hd = qr.head_dim;
      auto put = [&](int row, int m, f16 v) {
        if (row < qr.q_dim) {
          qr.q_out[(size_t)m * qr.q_dim + row] = v;
        } else {
          const bool is_k = row < qr.q_dim + qr.kv_dim;
          const int within = is_k ? row - qr.q_dim : row - qr.q_dim - qr.kv_dim;
          const int wp = (qr.write_pos_dev ? qr.write_pos_dev[0] : qr.write_pos) + m;
          (is_k ? qr.k_out : qr.v_out)[(size_t)(within / hd) * qr.kv_stride_h + (size_t)(wp % qr.max_seq) * hd +
                                       within % hd] = v;
        }
      };
#pragma unroll
      for (int i = 0; i < R; i += 2) {
        const int row0 = row_of(i);
        if (row0 >= N) continue;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          f16 h0 = f2h(r[i][m]), h1 = f2h(r[i + 1][m]);
          if (bias != nullptr) {
            h0 = f2h(h2f(h0) + h2f(bias[row0]));
            h1 = f2h(h2f(h1) + h2f(bias[row0 + 1]));
          }
          f16 o0 = h0, o1 = h1;
          if (row0 < qr.q_dim + qr.kv_dim) {
            const int pos = (qr.rope_pos_dev ? qr.rope_pos_dev[0] : qr.rope_pos) + m;
            const int within = row0 < qr.q_dim ? row0 : row0 - qr.q_dim;
            const float* f = qr.freqs + ((size_t)(pos % qr.rope_len) * (hd / 2) + ((within % hd) >> 1)) * 2;
            o0 = rope_out(h0, h1, f[0], f[1], true);
            o1 = rope_out(h0, h1, f[0], f[1], false);
          }
          put(row0, m, o0);
          put(row0 + 1, m, o1);
        }
      }
    } else if (EPI == kQ8Swiglu) {
#pragma unroll
      for (int i = 0; i < R / 2; ++i) {
        const int c = wrow * (R / 2) + i;
        if (c >= H) continue;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const float g = h2f(f2h(r[i][m]));
          const f16 sg = f2h(g / (1.0f + expf(-g)));
          y[(size_t)m * H + c] = f2h(h2f(sg) * h2f(f2h(r[R / 2 + i][m])));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int row = row_of(i);
        if (row >= N) continue;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          f16 h = f2h(r[i][m]);
          if (bias != nullptr) h = f2h(h2f(h) + h2f(bias[row]));
          f16* o = y + (size_t)m * N + row;
          if (EPI == kQ8Resid)
            *o = f2h(add_rn(h2f(*o), h2f(h)));
          else
            *o = h;
        }
      }
    }
  }
}

// 16-code vectors per lane and step: two for waves of one or two rows (the 4096-row O
// and down projections, whose waves otherwise keep too few bytes in flight: mode
// q4_k_m 653 -> 676, q8 460 -> 472 tok/s), one for more rows (two there: q8 460 ->
// 448, the registers cost occupancy).
template <int M, int R, int EPI>
int q8v_launch(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int K, int N,
               const f16* ln_w, float eps, const QkvRope& qr, hipStream_t s, f16* xn_out) {
  constexpr int V = R <= 2 ? 2 : 1;
  const size_t smem = (size_t)M * K * sizeof(f16) + (size_t)M * (K / 16) * sizeof(float);
  static bool attr_set = false;
  if (smem > 48 * 1024 && !attr_set) {
    if (hipFuncSetAttribute((const void*)q8v_kernel<M, R, EPI, V>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            150 * 1024) != hipSuccess) {
      (void)hipGetLastError();
      axm_set_error("q8 gemv: cannot reserve %zu bytes of LDS", smem);
      return -2;
    }
    attr_set = true;
  }
  const int rows = kQ8vWaves * R;
  const int units = EPI == kQ8Swiglu ? N / 2 : N;   // output columns
  const int per_wg = EPI == kQ8Swiglu ? rows / 2 : rows;
  hipLaunchKernelGGL((q8v_kernel<M, R, EPI, V>), dim3((units + per_wg - 1) / per_wg), dim3(kQ8vThreads), smem, s, x, K,
                     N, w, sb, bias, y, ln_w, eps, qr, xn_out);
  return 0;
}

// Rows per wave: for one token eight when four would need more than one round of
// workgroups (the one-token four-row kernel holds 81-84 VGPRs, five waves per SIMD:
// 7B gate / up has 1376 workgroups of four-row waves for 1280 slots; the eight-row one
// 124, four waves; mode q8 432.5 -> 440 tok/s), else two while the two-row waves (78
// VGPRs, six per SIMD) fit one round (7B QKV, 12288 rows: 6144 waves of two steps in
// place of 3072 four-row waves of four, q8 473.0 -> 481.2 tok/s), else four.  For
// several tokens four while that leaves two workgroups per CU.  Then two, else one (two
// at least for SwiGLU and QKV, whose waves take row pairs).  Measured and not kept: a
// two-step prefetch ring (three register slots, the step loop unrolled by three):
// q4_k_m 659.6 -> 663 tok/s, q8 439 -> 435; one-row waves with four vectors per lane for
// the 4096-row O and down projections: q8 473.0 -> 468.8.
template <int M, int EPI>
int q8v_launch_m(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int K, int N,
                 const f16* ln_w, float eps, const QkvRope& qr, hipStream_t s, f16* xn_out) {
  constexpr bool kPairs = EPI == kQ8Swiglu || EPI == kQ8Qkv;  // rows come in pairs per wave
  const int cus = axm_num_cus();
  if constexpr (M == 1) {
    if (N > 5 * cus * kQ8vWaves * 4) return q8v_launch<M, 8, EPI>(x, w, sb, bias, y, K, N, ln_w, eps, qr, s, xn_out);
    if (N > 6 * cus * kQ8vWaves * 2) return q8v_launch<M, 4, EPI>(x, w, sb, bias, y, K, N, ln_w, eps, qr, s, xn_out);
  } else {
    if (N >= 2 * cus * kQ8vWaves * 4) return q8v_launch<M, 4, EPI>(x, w, sb, bias, y, K, N, ln_w, eps, qr, s, xn_out);
  }
  if (kPairs || N >= cus * kQ8vWaves * 2)
    return q8v_launch<M, 2, EPI>(x, w, sb, bias, y, K, N, ln_w, eps, qr, s, xn_out);
  return q8v_launch<M, (kPairs ? 2 : 1), EPI>(x, w, sb, bias, y, K, N, ln_w, eps, qr, s, xn_out);
}

template <int EPI>
int q8v_rows(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int M, int K, int N,
             const f16* ln_w, float eps, hipStream_t s, const QkvRope& qr = QkvRope{}, f16* xn_out = nullptr) {
  if (K % 64 != 0 || (long)N * K >= 0x7FFFFFF0L || ((EPI == kQ8Swiglu || EPI == kQ8Qkv) && N % 2 != 0)) {
    axm_set_error("q8 gemv: K=%d must be a multiple of 64, the codes under 2 GiB (N=%d), N even for SwiGLU", K, N);
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
  const int ld_out = EPI == kQ8Swiglu ? N / 2 : N;
  for (int m0 = 0; m0 < M; m0 += rows_max) {
    const int mc = (M - m0) < rows_max ? (M - m0) : rows_max;
    const f16* xm = x + (size_t)m0 * K;
    f16* ym = y + (size_t)m0 * ld_out;
    f16* xnm = xn_out != nullptr ? xn_out + (size_t)m0 * K : nullptr;
    QkvRope qk = qr;  // tokens m0 ..: q rows, positions and slots move with them
    if (EPI == kQ8Qkv) {
      qk.q_out = qr.q_out + (size_t)m0 * qr.q_dim;
      qk.rope_pos += qr.rope_pos_dev ? 0 : m0;
      qk.write_pos += qr.write_pos_dev ? 0 : m0;
      if (m0 > 0 && (qr.rope_pos_dev || qr.write_pos_dev)) {
        axm_set_error("q8 gemv: a QKV epilogue with device positions takes at most %d tokens", rows_max);
        return -2;
      }
    }
    int rc;
    switch (mc) {
      case 1: rc = q8v_launch_m<1, EPI>(xm, w, sb, bias, ym, K, N, ln_w, eps, qk, s, xnm); break;
      case 2: rc = q8v_launch_m<2, EPI>(xm, w, sb, bias, ym, K, N, ln_w, eps, qk, s, xnm); break;
      case 3: rc = q8v_launch_m<3, EPI>(xm, w, sb, bias, ym, K, N, ln_w, eps, qk, s, xnm); break;
      default: rc = q8v_launch_m<4, EPI>(xm, w, sb, bias, ym, K, N, ln_w, eps, qk, s, xnm); break;
    }
    if (rc) return rc;
  }
  return 0;
}

}  // namespace

int launch_q8_gemv(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int M, int K, int N,
                   const f16* ln_w, float eps, hipStream_t s, f16* xn_out) {
  return q8v_rows<kQ8Store>(x, w, sb, bias, y, M, K, N, ln_w, eps, s, QkvRope{}, xn_out);
}

int launch_q8_gemv_qkv(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, int M, int K, int N,
                       const f16* ln_w, float eps, const QkvRope& r, hipStream_t s) {
  return q8v_rows<kQ8Qkv>(x, w, sb, bias, r.q_out, M, K, N, ln_w, eps, s, r);
}

int launch_q8_gemv_resid(const f16* x, const uint8_t* w, const f16* sb, f16* resid, int M, int K, int N,
                         const f16* ln_w, float eps, hipStream_t s) {
  return q8v_rows<kQ8Resid>(x, w, sb, nullptr, resid, M, K, N, ln_w, eps, s);
}

int launch_q8_gemv_swiglu(const f16* x, const uint8_t* w, const f16* sb, f16* y, int M, int K, int N2,
                          const f16* ln_w, float eps, hipStream_t s) {
  return q8v_rows<kQ8Swiglu>(x, w, sb, nullptr, y, M, K, N2, ln_w, eps, s);
}
