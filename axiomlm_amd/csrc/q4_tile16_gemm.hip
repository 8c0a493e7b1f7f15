// Multi-token tile16 GEMM (M <= 64 tokens per launch) for gfx950: the verify /
// prefill steps of the decode runner and the qmm entry points.
//
// The decode GEMV (q4_tile16.hip) fills only 1..4 of the 16 token rows of the
// v_mfma_f32_16x16x32_f16 A operand; here MB tiles of 16 token rows each carry
// tokens, so every weight chunk (16 rows x 128 k, 1 KB) is read from HBM once
// for up to 16 MB tokens and dequantized once (the B operand) for all of them.
//
// A wave owns one unit for the workgroup's K split, so the eight waves of a
// workgroup cover 128 output rows and share one staged copy of the activations
// (16 MB tokens, RC chunks at a time, double-buffered).  K is split across
// workgroups until the grid covers the CUs; with more than one split each
// workgroup writes its fp32 partial tile and t16g_reduce_kernel sums the splits
// in order and applies the epilogue.  Activations come in normalized (the
// runner runs the RMSNorm first, with the same rounding as the GEMV prologue).
#include "kernels.h"
#include "q4_tile16.h"
#include "t16_device.h"

namespace {

constexpr int kGThreads = 512;
constexpr int kGWaves = kGThreads / 64;   // one tile16 unit per wave
constexpr int kGOOB = 0x7FFFFFF0;

// Shapes of one instantiation: MB token tiles (16 MB tokens per weight pass)
// and RC chunks (128 k) per staged activation range.  Staged rows are padded by
// 16 bytes so that the A-operand reads of 16 token rows do not all fall into the
// same LDS banks.
template <int MB, int RC>
struct GemmShape {
  static constexpr int TOK = 16 * MB;
  static constexpr int XROW = RC * 128 + 8;             // halves per staged activation row
  static constexpr size_t XS = (size_t)TOK * XROW;      // halves per buffer
  static constexpr int VPR = 16 * RC;                   // 8-element vectors per token row and range
  static constexpr int RPP = kGThreads / VPR;           // token rows staged per pass of the workgroup
  static constexpr int PER = TOK / RPP;                 // vectors staged per thread
  static constexpr size_t smem = 2 * XS * sizeof(f16);
  static_assert(RPP * VPR == kGThreads && PER * RPP == TOK, "staging map");
  static_assert(smem <= 160 * 1024, "LDS");
};

// The instantiations by tokens per launch: one, two or four 16-token tiles per
// weight pass, each with 4-chunk activation ranges (LDS holds two 64-token ranges,
// 133 KB) and every chunk dequantized once for all of its token tiles.  Up to 16
// tokens once kept the GEMV's arithmetic instead (raw magic-exponent nibbles into
// the MFMA, per-group corrections from staged activation sums, 8-chunk ranges):
// the dequantized form is faster there too (7B layer at 4 tokens 69.2 -> 62.2 us,
// at 16 tokens 72.3 -> 63.7 us).
// upw = units per wave of the store epilogue at 64 tokens: two adjacent units
// share each A fragment read from LDS, as the gate / up pair of the SwiGLU form
// always does.  Measured in the 7B verify step it sped up the QKV and lm_head
// GEMMs (19.4 -> 16.7 us) but slowed the residual O / down GEMMs (13.2 -> 14.4
// us: their K splits double, leaving O on 128 workgroups), which keep one.
struct GemmCfg {
  int mb, rc, upw;
};
GemmCfg gemm_cfg(int M) {
  if (M <= 16) return {1, 4, 1};
  if (M <= 32) return {2, 4, 1};
  return {4, 4, 2};
}
// Units per wave / partial-tile columns per unit of an (epilogue, config).
int gemm_upw(int epi, GemmCfg cfg) { return epi == Q4_EPI_STORE ? cfg.upw : 1; }
int gemm_cols_per_unit(int epi) { return epi == Q4_EPI_SWIGLU ? 2 * 16 : 16; }

// Workgroups per K split: upw units per wave, eight waves per workgroup.  The kernel
// needs 140-200 VGPRs, so one 8-wave workgroup is resident per CU: K is split
// as far as the grid still fits one round of workgroups (a grid even one
// workgroup past the CU count runs a second round, e.g. 7B gate/up at M=16:
// 172 workgroups 21 us, 258 workgroups 32 us), keeping >= RC chunks per split.
int gemm_splits(int KB, int n_units, int rc, int upw) {
  const int wg = (n_units + kGWaves * upw - 1) / (kGWaves * upw);
  int splits = axm_num_cus() / wg;
  const int max_splits = KB / rc > 0 ? KB / rc : 1;
  if (splits > max_splits) splits = max_splits;
  if (splits > kTile16GemmMaxSplits) splits = kTile16GemmMaxSplits;
  return splits < 1 ? 1 : splits;
}

// One output element of the epilogue (identical arithmetic to the GEMV's):
// v0 the gate / plain accumulator, v1 the up accumulator (SwiGLU).
template <int EPI>
__device__ __forceinline__ void t16g_store(const T16Args& a, int tok, int row, float v0, float v1) {
  if (EPI == Q4_EPI_SWIGLU) {
    const f16 g = f2h(v0);
    const f16 u = f2h(v1);
    const f16 sg = f2h(t16_silu(h2f(g)));
    a.y[(size_t)tok * a.ldy + row] = f2h(h2f(sg) * h2f(u));
  } else {
    f16 h = f2h(v0);
    if (a.bias != nullptr) h = f2h(h2f(h) + h2f(a.bias[row]));
    if (EPI == Q4_EPI_STORE) {
      a.y[(size_t)tok * a.ldy + row] = h;
    } else {
      f16* xr = a.resid + (size_t)tok * a.ldr + row;
      *xr = f2h(h2f(*xr) + h2f(h));
    }
  }
}

// Each wave owns NT weight tiles over the workgroup's K split: a gate/up pair
// (SwiGLU) or NT adjacent units (store / residual epilogues).  The split's activations of all 16 MB token rows are staged range by
// range (RC chunks, double-buffered in LDS: range r + 1 is loaded while range r
// is consumed), and the weight chunks of range r + 1 are requested into the
// register slots that range r's chunks free, so the weight stream does not stop
// at range boundaries.
//
// Every weight is dequantized once per chunk to fp16 q * scale + bias (one
// rounding, the "dequantize to half, then MMA" of the reference's multi-token
// kernel) and the MFMAs accumulate the dot products directly, so a token tile
// costs its four A reads and four MFMAs and no per-tile vector math.
template <int NT, int EPI, int MB, int RC, bool G128>
__global__ void __launch_bounds__(kGThreads) t16g_kernel(T16Args a) {
  using G = GemmShape<MB, RC>;
  extern __shared__ __align__(16) unsigned char smem[];
  f16* xs0 = reinterpret_cast<f16*>(smem);                     // [2][TOK][XROW]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = lane >> 4;
  constexpr bool kPair = EPI == Q4_EPI_SWIGLU;
  const int unit = (blockIdx.x * kGWaves + wave) * (kPair ? 1 : NT);  // first unit of the wave
  const int tstride = kPair ? a.pair_offset : 1;                      // unit step between tiles
  const int kbA = blockIdx.y * a.kb_per_split;
  const int kbN = min(a.KB, kbA + a.kb_per_split) - kbA;  // chunks of this split (>= 1)
  const int n_ranges = (kbN + RC - 1) / RC;
  const Unpack U{to_vgpr(a.unpack[0]), to_vgpr(a.unpack[1]), a.unpack[2], a.unpack[3]};
  const __amdgpu_buffer_rsrc_t rw =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w16, (short)0, (int)a.w16_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.sb16, (short)0, (int)a.sb16_bytes, 0x00020000);

  u32x4 wr[RC][NT];
  u32x2 sr[RC][NT];
  // Chunk c of range r into slot c (zeros past the split or the matrix).
  auto load = [&](int r, int c) {
    const int kl = r * RC + c;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool ok = unit + (kPair ? 0 : t) < a.n_units && kl < kbN;
      const int base = (unit + t * tstride) * a.KB + kbA + kl;
      const int wo = ok ? (base * 64 + lane) * 16 : kGOOB;
      const int so = ok ? (base * 16 + (lane & 15)) * (G128 ? 4 : 8) : kGOOB;
      wr[c][t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, 2));
      if (G128) {
        const uint32_t v = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(rs, so, 0, 0));
        sr[c][t] = u32x2{v, v};
      } else {
        sr[c][t] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0));
      }
    }
  };
  // Activations of range r: thread tid stages vector svi = tid % VPR of token
  // rows stok + RPP i (i < PER); eight consecutive lanes hold a 64-group.
  // Buffer loads with out-of-range offsets (tokens >= M, k past the split or K,
  // ranges past the last) read zeros, so every load is issued unconditionally
  // and the compiler can count the loads in flight exactly.
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.M_tokens * a.ldx * (int)sizeof(f16), 0x00020000);
  const int svi = tid & (G::VPR - 1);
  const int stok = tid / G::VPR;
  f16x8 xv[G::PER];
  auto stage_load = [&](int r) {
    const int k = (kbA + r * RC) * 128 + 8 * svi;
    const int kok = (int)(k < a.K) & (int)(8 * svi < (kbN - r * RC) * 128);
#pragma unroll
    for (int i = 0; i < G::PER; ++i) {
      const int tok = stok + G::RPP * i;
      // Branch-free select of the offset (a conditional here became divergent
      // control flow with full memory waits inside it).
      const int m = -(kok & (int)(tok < a.M_tokens));
      const int off = (((tok * a.ldx + k) * (int)sizeof(f16)) & m) | (kGOOB & ~m);
      xv[i] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    }
  };
  auto stage_store = [&](int buf) {
    f16* xs = xs0 + buf * G::XS;
#pragma unroll
    for (int i = 0; i < G::PER; ++i)
      *reinterpret_cast<f16x8*>(xs + (size_t)(stok + G::RPP * i) * G::XROW + 8 * svi) = xv[i];
  };

  // Weights of range 0 first, then its activations (both one latency away).
#pragma unroll
  for (int c = 0; c < RC; ++c) load(0, c);
  stage_load(0);
  stage_store(0);
  __syncthreads();

  f32x4 acc[NT][MB];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[t][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int r = 0; r < n_ranges; ++r) {
    // The next range's weights are requested unconditionally (past the last
    // range they read zeros and are never used); its activations only when it
    // exists.
    const bool more = r + 1 < n_ranges;
    if (more) stage_load(r + 1);
    const f16* xs = xs0 + (r & 1) * G::XS;
    // A operand: token 16 mb + lane % 16 (rows past M are zeros), k sub-block lane / 16.
    const f16* xa = xs + (size_t)(lane & 15) * G::XROW + 8 * kq;
    // Only the last range of a split can be partial (uniform across the
    // workgroup); keeping the guard makes each chunk its own block, which the
    // register allocator needs.
    const int n_here = min(RC, kbN - r * RC);
#pragma unroll
    for (int c = 0; c < RC; ++c) {
      if (c < n_here) {
        // Word q of a lane holds 8 k of group q / 2; its unpacked elements are
        // 1024 + n or 64 + n (pattern of unpack_word), subtracted exactly.
        const f16x8 magic = {(f16)1024.f, (f16)1024.f, (f16)64.f, (f16)64.f,
                             (f16)1024.f, (f16)1024.f, (f16)64.f, (f16)64.f};
        f16x8 B[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f16x2 sb = as_h2(sr[c][t][q >> 1]);
            const f16x8 sc = {sb.x, sb.x, sb.x, sb.x, sb.x, sb.x, sb.x, sb.x};
            const f16x8 bi = {sb.y, sb.y, sb.y, sb.y, sb.y, sb.y, sb.y, sb.y};
            B[t][q] = __builtin_elementwise_fma(unpack_word(wr[c][t][q], U) - magic, sc, bi);
          }
        // Every A fragment of the chunk is read from LDS first, then the MFMAs run
        // k-step by k-step across the token tiles: consecutive MFMAs accumulate
        // into different tiles instead of waiting on each other, and none waits on
        // an LDS read issued just before it.
        f16x8 A[MB][4];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          const f16* xk = xa + (size_t)16 * mb * G::XROW + c * 128;
#pragma unroll
          for (int q = 0; q < 4; ++q) A[mb][q] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(xk + 32 * q));
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              acc[t][mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mb][q], B[t][q], acc[t][mb], 0, 0, 0);
      }
      load(r + 1, c);
    }
    if (more) stage_store((r + 1) & 1);
    __syncthreads();
  }

  const int j = lane & 15;
  if (gridDim.y == 1) {
#pragma unroll
    for (int t = 0; t < (kPair ? 1 : NT); ++t) {
      if (unit + t >= a.n_units) break;
      const int row = (unit + t) * 16 + j;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int vi = 0; vi < 4; ++vi) {
          const int tok = 16 * mb + 4 * kq + vi;
          if (tok < a.M_tokens && row < a.N)
            t16g_store<EPI>(a, tok, row, acc[t][mb][vi], acc[kPair ? NT - 1 : t][mb][vi]);
        }
    }
  } else {
    // Partial tile of this K split: [split][token][column], column = tile * 16 + row in tile.
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (unit + (kPair ? 0 : t) >= a.n_units) break;
      const int col = (unit + t * tstride) * 16 + j;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int vi = 0; vi < 4; ++vi)
          a.part_ws[((size_t)blockIdx.y * G::TOK + 16 * mb + 4 * kq + vi) * a.part_cols + col] = acc[t][mb][vi];
    }
  }
}

// Sums the K-split partials in split order and applies the epilogue: one thread
// per (token, output row); tok_stride = token rows per split in the workspace.
template <int EPI>
__global__ void t16g_reduce_kernel(T16Args a, int n_splits, int up_col, int tok_stride) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int tok = (int)(idx / a.N), row = (int)(idx % a.N);
  if (tok >= a.M_tokens) return;
  float v0 = 0.f, v1 = 0.f;
#pragma unroll 4
  for (int sp = 0; sp < n_splits; ++sp) {
    const float* p = a.part_ws + ((size_t)sp * tok_stride + tok) * a.part_cols;
    v0 += p[row];
    if (EPI == Q4_EPI_SWIGLU) v1 += p[up_col + row];
  }
  t16g_store<EPI>(a, tok, row, v0, v1);
}

// Residual epilogue over the split partials of whole token rows, then RMSNorm of
// each updated row into post_norm_out: one 1024-thread workgroup per token,
// thread tid owns the 4-row vectors tid + 1024 i (N % 4 == 0, N <= 16384,
// 8-byte aligned rows), so each thread issues one 16-byte partial load per split
// and vector.  The arithmetic is t16g_reduce_kernel's followed by the norm
// kernel's.
constexpr int kRnThreads = 1024;
constexpr int kRnVec = 4;
__global__ void __launch_bounds__(kRnThreads) t16g_reduce_resid_norm_kernel(T16Args a, int n_splits, int tok_stride) {
  __shared__ float red[kRnThreads / 64];
  const int tok = blockIdx.x;
  const int nv = a.N / 4;
  f16* xr = a.resid + (size_t)tok * a.ldr;
  f16x4 xv[kRnVec];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kRnVec; ++i) {
    const int j = threadIdx.x + i * kRnThreads;
    if (j < nv) {
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int sp = 0; sp < n_splits; ++sp)
        v += *reinterpret_cast<const f32x4*>(a.part_ws + ((size_t)sp * tok_stride + tok) * a.part_cols + 4 * j);
      f16x4 xo = *reinterpret_cast<const f16x4*>(xr + 4 * j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f16 h = f2h(v[e]);
        if (a.bias != nullptr) h = f2h(h2f(h) + h2f(a.bias[4 * j + e]));
        xo[e] = f2h(h2f(xo[e]) + h2f(h));
        const float f = h2f(xo[e]);
        ss += h2f(f2h(f * f));
      }
      *reinterpret_cast<f16x4*>(xr + 4 * j) = xo;
      xv[i] = xo;
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kRnThreads / 64; ++w) tot += red[w];
  const float rinv = rms_inv_fp16(tot, a.N, a.eps);
  f16* yr = a.post_norm_out + (size_t)tok * a.N;
#pragma unroll
  for (int i = 0; i < kRnVec; ++i) {
    const int j = threadIdx.x + i * kRnThreads;
    if (j < nv) {
      const f16x4 wv = *reinterpret_cast<const f16x4*>(a.post_ln_w + 4 * j);
      f16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = f2h(h2f(f2h(h2f(xv[i][e]) * rinv)) * h2f(wv[e]));
      *reinterpret_cast<f16x4*>(yr + 4 * j) = o;
    }
  }
}

bool post_norm_fusable(const T16Args& a) {
  const uintptr_t al = (uintptr_t)a.resid | (uintptr_t)a.post_ln_w | (uintptr_t)a.post_norm_out;
  return a.N % 4 == 0 && a.N <= 4 * kRnThreads * kRnVec && a.ldr % 4 == 0 && (al & 7) == 0;
}

template <int NT, int EPI, int MB, int RC, bool G128>
void t16g_launch_group(const T16Args& a, dim3 grid, hipStream_t s) {
  using G = GemmShape<MB, RC>;
  static bool set = false;
  if (!set) {
    set = true;
    if (hipFuncSetAttribute((const void*)t16g_kernel<NT, EPI, MB, RC, G128>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)G::smem) != hipSuccess)
      (void)hipGetLastError();
  }
  hipLaunchKernelGGL((t16g_kernel<NT, EPI, MB, RC, G128>), grid, dim3(kGThreads), G::smem, s, a);
}

template <int NT, int EPI, int MB, int RC>
void t16g_launch_shape(const T16Args& a, dim3 grid, hipStream_t s) {
  if (a.g128)
    t16g_launch_group<NT, EPI, MB, RC, true>(a, grid, s);
  else
    t16g_launch_group<NT, EPI, MB, RC, false>(a, grid, s);
}

// The (MB, RC, units per wave) shapes here are the ones gemm_cfg returns.
template <int EPI>
void t16g_launch_epi(const T16Args& a, GemmCfg cfg, dim3 grid, hipStream_t s) {
  constexpr int P = EPI == Q4_EPI_SWIGLU ? 2 : 1;  // tiles per unit
  if (cfg.mb == 1)
    t16g_launch_shape<P, EPI, 1, 4>(a, grid, s);
  else if (cfg.mb == 2)
    t16g_launch_shape<P, EPI, 2, 4>(a, grid, s);
  else if (gemm_upw(EPI, cfg) == 1)
    t16g_launch_shape<P, EPI, 4, 4>(a, grid, s);
  else
    t16g_launch_shape<2, EPI, 4, 4>(a, grid, s);
}

size_t gemm_ws_bytes_cfg(int KB, int n_units, int epi, GemmCfg cfg) {
  const int splits = gemm_splits(KB, n_units, cfg.rc, gemm_upw(epi, cfg));
  return splits <= 1 ? 0 : (size_t)splits * 16 * cfg.mb * n_units * gemm_cols_per_unit(epi) * sizeof(float);
}

}  // namespace

size_t t16_gemm_ws_bytes(int K, int n_units, int NT) {
  const int KB = (K + 127) / 128;
  const int epi = NT == 2 ? Q4_EPI_SWIGLU : Q4_EPI_STORE;
  size_t need = 0;
  for (int m = 16; m <= kTile16GemmMaxTokens; m *= 2) {
    const size_t b = gemm_ws_bytes_cfg(KB, n_units, epi, gemm_cfg(m));
    if (b > need) need = b;
  }
  return need;
}

int t16_gemm_launch(T16Args a, int M, int epi, float* ws, size_t ws_bytes, hipStream_t s) {
  if (M < 1 || M > kTile16GemmMaxTokens || a.ln_w != nullptr || a.argmax_keys != nullptr || a.x_parts != nullptr ||
      (epi != Q4_EPI_STORE && epi != Q4_EPI_RESID && epi != Q4_EPI_SWIGLU) || a.K <= 0 || a.K % 64 != 0 ||
      (a.post_ln_w != nullptr && (epi != Q4_EPI_RESID || a.post_norm_out == nullptr || a.ldr != a.N))) {
    axm_set_error("tile16 gemm: M=%d (1..%d), epi=%d, K=%d unsupported (normalized activations, store / "
                  "residual / SwiGLU epilogues, post-norm only with the residual one over contiguous rows)", M,
                  kTile16GemmMaxTokens, epi, a.K);
    return -2;
  }
  const GemmCfg cfg = gemm_cfg(M);
  const int upw = gemm_upw(epi, cfg);
  a.KB = (a.K + 127) / 128;
  const int splits = gemm_splits(a.KB, a.n_units, cfg.rc, upw);
  const int kbps = (a.KB + splits - 1) / splits;
  const size_t need = gemm_ws_bytes_cfg(a.KB, a.n_units, epi, cfg);
  if (need > 0 && (ws == nullptr || ws_bytes < need)) {
    axm_set_error("tile16 gemm: workspace of %zu bytes needed, %zu given", need, ws_bytes);
    return -1;
  }
  a.split = 1;
  a.M_tokens = M;
  a.kb_per_split = kbps;
  a.part_ws = ws;
  a.part_cols = a.n_units * gemm_cols_per_unit(epi);
  a.w16_bytes = t16_weight_bytes(a.N_rows_alloc, a.K);
  a.sb16_bytes = t16_sb_bytes(a.N_rows_alloc, a.K, a.g128);
  a.unpack[0] = 0x000F000Fu;
  a.unpack[1] = 0x00F000F0u;
  a.unpack[2] = 0x64006400u;
  a.unpack[3] = 0x54005400u;
  const dim3 grid((a.n_units + kGWaves * upw - 1) / (kGWaves * upw), splits);
  switch (epi) {
    case Q4_EPI_STORE:
      t16g_launch_epi<Q4_EPI_STORE>(a, cfg, grid, s);
      break;
    case Q4_EPI_RESID:
      t16g_launch_epi<Q4_EPI_RESID>(a, cfg, grid, s);
      break;
    default:
      t16g_launch_epi<Q4_EPI_SWIGLU>(a, cfg, grid, s);
      break;
  }
  const int ts = 16 * cfg.mb;
  if (a.split_info != nullptr) {
    a.split_info[0] = a.split_info[1] = a.split_info[2] = 0;
    if (splits > 1 && epi == Q4_EPI_STORE && a.post_ln_w == nullptr) {
      a.split_info[0] = splits;
      a.split_info[1] = ts;
      a.split_info[2] = a.part_cols;
      return 0;
    }
  }
  if (a.post_ln_w != nullptr) {
    // Residual rows then their RMSNorm: one fused launch over the partials, or
    // the norm kernel after an unsplit GEMM (and as the general fallback).
    if (splits > 1 && post_norm_fusable(a)) {
      hipLaunchKernelGGL(t16g_reduce_resid_norm_kernel, dim3(M), dim3(kRnThreads), 0, s, a, splits, ts);
      return 0;
    }
    if (splits > 1) {
      const long n = (long)M * a.N;
      hipLaunchKernelGGL(t16g_reduce_kernel<Q4_EPI_RESID>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a,
                         splits, 0, ts);
    }
    return launch_rmsnorm(a.resid, a.post_ln_w, a.post_norm_out, M, a.N, a.eps, s);
  }
  if (splits > 1) {
    const long n = (long)M * a.N;
    const dim3 rg((unsigned)((n + 255) / 256));
    const int up_col = a.pair_offset * 16;
    if (epi == Q4_EPI_STORE)
      hipLaunchKernelGGL(t16g_reduce_kernel<Q4_EPI_STORE>, rg, dim3(256), 0, s, a, splits, up_col, ts);
    else if (epi == Q4_EPI_RESID)
      hipLaunchKernelGGL(t16g_reduce_kernel<Q4_EPI_RESID>, rg, dim3(256), 0, s, a, splits, up_col, ts);
    else
      hipLaunchKernelGGL(t16g_reduce_kernel<Q4_EPI_SWIGLU>, rg, dim3(256), 0, s, a, splits, up_col, ts);
  }
  return 0;
}

// ---------------------------------------------------------------------------
// C ABI: multi-token GEMM on tile16 copies (up to 64 tokens per weight pass).
// ---------------------------------------------------------------------------
extern "C" size_t axm_qmm_q4_tile16_workspace_bytes(int K, int N, int swiglu) {
  if (K <= 0 || N <= 0) return 0;
  return t16_gemm_ws_bytes(K, (N + 15) / 16, swiglu ? 2 : 1);
}

static int qmm_tile16_rows(const void* x, const void* w16, const void* sb16, const void* bias, void* y, int M, int K,
                           int N, int group_size, int epi, void* ws, size_t ws_bytes, hipStream_t s) {
  for (int m0 = 0; m0 < M; m0 += kTile16GemmMaxTokens) {
    const int mc = (M - m0) < kTile16GemmMaxTokens ? (M - m0) : kTile16GemmMaxTokens;
    T16Args a{};
    a.x = (const f16*)x + (size_t)m0 * K;
    a.ldx = K;
    a.w16 = (const u32x4*)w16;
    a.sb16 = (const u32x2*)sb16;
    a.g128 = group_size == 128;
    a.K = K;
    a.N = N;
    a.n_units = (N + 15) / 16;
    if (epi == Q4_EPI_SWIGLU) {
      a.N_rows_alloc = 2 * N;
      a.pair_offset = N / 16;
    } else {
      a.N_rows_alloc = N;
    }
    a.y = (f16*)y + (size_t)m0 * N;
    a.ldy = N;
    a.bias = (const f16*)bias;
    const int rc = t16_gemm_launch(a, mc, epi, (float*)ws, ws_bytes, s);
    if (rc) return rc;
  }
  return 0;
}

extern "C" int axm_qmm_q4_tile16(const void* x, const void* w16, const void* sb16, const void* bias, void* y, int M,
                                 int K, int N, int group_size, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  AXM_CHECK_ARG(x && w16 && sb16 && y, -1, "qmm_q4_tile16: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && N > 0 && M >= 1, -1, "qmm_q4_tile16: bad shape M=%d K=%d N=%d", M, K, N);
  AXM_CHECK_ARG(group_size == 64 || (group_size == 128 && K % 128 == 0), -1,
                "qmm_q4_tile16: group_size %d (64, or 128 with K %% 128 == 0)", group_size);
  const int rc = qmm_tile16_rows(x, w16, sb16, bias, y, M, K, N, group_size, Q4_EPI_STORE, workspace,
                                 workspace_bytes, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmm_q4_tile16");
  return 0;
}

extern "C" int axm_qmm_q4_tile16_swiglu(const void* x_normed, const void* gu16, const void* gusb16, void* y, int M,
                                        int K, int H, int group_size, void* workspace, size_t workspace_bytes,
                                        void* stream) {
  AXM_CHECK_ARG(x_normed && gu16 && gusb16 && y, -1, "qmm_q4_tile16_swiglu: null pointer");
  AXM_CHECK_ARG(K > 0 && K % 64 == 0 && H > 0 && H % 16 == 0 && M >= 1, -1,
                "qmm_q4_tile16_swiglu: bad shape M=%d K=%d H=%d (H %% 16 == 0)", M, K, H);
  AXM_CHECK_ARG(group_size == 64 || (group_size == 128 && K % 128 == 0), -1,
                "qmm_q4_tile16_swiglu: group_size %d (64, or 128 with K %% 128 == 0)", group_size);
  const int rc = qmm_tile16_rows(x_normed, gu16, gusb16, nullptr, y, M, K, H, group_size, Q4_EPI_SWIGLU, workspace,
                                 workspace_bytes, (hipStream_t)stream);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("qmm_q4_tile16_swiglu");
  return 0;
}
