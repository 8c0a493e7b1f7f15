// Whole-model quantized decode runner (the MI355X counterpart of the
// reference QuantizedDecodeGraphState, axiomlm/kernels/mps_kernels.mm:2982-3738).
//
// Per token and layer the step is five launches:
//   1. QKV GEMV   : RMSNorm(x, ln1) prologue, RoPE + KV-slot write epilogue
//   2. attention  : split-KV decode over the (fp16 | FP8 | INT4) cache (+ merge)
//   3. O GEMV     : residual add epilogue (x += o)
//   4. gate/up    : RMSNorm(x, ln2) prologue, SwiGLU epilogue over tile pairs
//   5. down GEMV  : residual add epilogue (x += d)
// followed by the lm_head GEMV with the final RMSNorm fused in.  Quantized KV
// caches add one quantize-and-store launch after the QKV GEMV.
//
// Positions (rope position, write slot, active length) and the token id live
// in a small device parameter block written by one tiny kernel before the
// graph is replayed, so a single captured hipGraph serves every step; graphs
// are cached per attention split count.
#include <algorithm>
#include <chrono>
#include <cstring>
#include <map>
#include <vector>

#include "axm.h"
#include "kernels.h"
#include "step_kernel.h"
#include "q4_tile16.h"

namespace {

enum { P_TOKEN = 0, P_ROPE = 1, P_WRITE = 2, P_ACTIVE = 3, P_COUNT = 4 };
// Token rows from which a multi-token step (verify / prompt chunk) runs the
// multi-token GEMM instead of the decode GEMV per group of up to four rows.
// Measured as verify_tree_step(N) / step on the 7B FP8 prefix-2048 model: the
// GEMV is faster at three rows (1.49 -> 1.42 steps), the GEMM from four (GEMV
// 1.69, GEMM 1.50).
constexpr int kGemmMinTokens = 4;
// Byte offset inside the parameter block of the int64 token id used by the
// current step.
constexpr int kTokenOffset = 72;

// Token source: idx_dev[0] if non-null, else tok_host if >= 0, else the greedy
// argmax of the previous step's logits, reduced here from the per-tile keys the
// lm_head launch wrote (largest fp16 logit, lowest index on ties).
//
// With `emb` set the same workgroup also gathers the token's embedding row into
// emb->x (the first kernel of the decode graph otherwise), with the arithmetic
// of embed_f16_kernel / embed_q8_kernel: 16 elements per thread and pass.
struct EmbedArgs {
  const void* wte;    // fp16 [V][D] (format 0) or Q8 codes u8 [V][D] (format 1)
  const f16* wte_sb;  // Q8: (scale, bias) fp16 [V][D / 64][2]
  int format;
  int D, V;           // D % 64 == 0
  f16* x;
};
__global__ void __launch_bounds__(256) set_params_kernel(int* params, const int64_t* idx_dev, int64_t tok_host,
                                                         int rope_pos, int write_pos, int active_len,
                                                         const unsigned long long* keys, int n_keys,
                                                         EmbedArgs emb) {
  __shared__ unsigned long long red[4];
  int64_t tok = 0;
  if (idx_dev == nullptr && tok_host < 0) {
    // Sixteen keys per thread and pass, all requested before any is compared
    // (keys past n_keys read 0, below every real key).
    constexpr int kPerThread = 16;
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)keys, (short)0, n_keys * 8, 0x00020000);
    unsigned long long best = 0ull;
    for (int base = 0; base < n_keys; base += 256 * kPerThread) {
      unsigned long long k[kPerThread];
#pragma unroll
      for (int u = 0; u < kPerThread; ++u)
        k[u] = __builtin_bit_cast(unsigned long long,
                                  __builtin_amdgcn_raw_buffer_load_b64(rk, (base + u * 256 + threadIdx.x) * 8, 0, 0));
#pragma unroll
      for (int u = 0; u < kPerThread; ++u) best = k[u] > best ? k[u] : best;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const unsigned long long other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    best = red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) best = red[w] > best ? red[w] : best;
    tok = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
  } else {
    tok = idx_dev != nullptr ? idx_dev[0] : tok_host;
  }
  if (threadIdx.x == 0) {
    *reinterpret_cast<int64_t*>(reinterpret_cast<unsigned char*>(params) + kTokenOffset) = tok;
    params[P_TOKEN] = (int)tok;
    params[P_ROPE] = rope_pos;
    params[P_WRITE] = write_pos;
    params[P_ACTIVE] = active_len;
  }
  if (emb.x == nullptr) return;
  // Out-of-range token ids produce a zero row (params[P_TOKEN] is the int cast,
  // as the embed kernels read it).
  const long t = (long)(int)tok;
  const bool ok = t >= 0 && t < emb.V;
  for (int k0 = 16 * threadIdx.x; k0 < emb.D; k0 += 16 * 256) {
    f16x8 o[2];
    if (!ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[0][e] = o[1][e] = f16(0);
    } else if (emb.format == 0) {
      const f16x8* src = reinterpret_cast<const f16x8*>((const f16*)emb.wte + (size_t)t * emb.D + k0);
      o[0] = src[0];
      o[1] = src[1];
    } else {
      const u32x4 c = *reinterpret_cast<const u32x4*>((const uint8_t*)emb.wte + (size_t)t * emb.D + k0);
      const f16* sbr = emb.wte_sb + ((size_t)t * (emb.D / 64) + k0 / 64) * 2;
      const float sc = h2f(sbr[0]), bi = h2f(sbr[1]);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float q = (float)((c[e >> 2] >> (8 * (e & 3))) & 0xFFu);
        o[e >> 3][e & 7] = f2h(add_rn(mul_rn(q, sc), bi));
      }
    }
    f16x8* dst = reinterpret_cast<f16x8*>(emb.x + k0);
    dst[0] = o[0];
    dst[1] = o[1];
  }
}

constexpr int kMaxVerify = 64;

struct TreeParams {
  int pos[kMaxVerify];               // rope position of each token
  unsigned long long mask[kMaxVerify];
};

// Copies the per-call tree description into device memory (kernel arguments,
// so no host-to-device copy is needed).
__global__ void set_tree_kernel(TreeParams p, int T, int* pos_dev, unsigned long long* mask_dev) {
  const int t = threadIdx.x;
  if (t < T) {
    pos_dev[t] = p.pos[t];
    mask_dev[t] = p.mask[t];
  }
}

// Multi-token RoPE (rope_tree_kv_cache_write_half_kernel, metal_kernels.metal:2862-2918):
// token t of qkv [T][qkv_dim] (bias already added) is rotated at pos_dev[t]; q rows go to
// q [T][q_dim], rotated k and raw v rows to kv [T][2 kv_dim] for the cache writer.
__global__ void rope_tokens_kernel(const f16* __restrict__ qkv, int q_dim, int kv_dim, int hd,
                                   const float* __restrict__ freqs, const int* __restrict__ pos_dev,
                                   f16* __restrict__ q, f16* __restrict__ kv) {
  // Thread (token blockIdx.y, vector i): elements 8 i .. 8 i + 7 (four rotation
  // pairs of one head; q_dim, kv_dim and hd are multiples of 8).
  const int t = blockIdx.y;
  const int qkv_dim = q_dim + 2 * kv_dim;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (8 * i >= qkv_dim) return;
  const int e = 8 * i;
  const f16x8 v = *reinterpret_cast<const f16x8*>(qkv + (size_t)t * qkv_dim + e);
  f16x8 out = v;
  if (e < q_dim + kv_dim) {
    const int within = e < q_dim ? e : e - q_dim;
    const int fi = (within % hd) >> 1;
    const float* f = freqs + ((size_t)pos_dev[t] * (hd / 2) + fi) * 2;
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
      const float c = f[2 * pr], sn = f[2 * pr + 1];
      out[2 * pr] = rope_out(v[2 * pr], v[2 * pr + 1], c, sn, true);
      out[2 * pr + 1] = rope_out(v[2 * pr], v[2 * pr + 1], c, sn, false);
    }
  }
  if (e < q_dim)
    *reinterpret_cast<f16x8*>(q + (size_t)t * q_dim + e) = out;
  else
    *reinterpret_cast<f16x8*>(kv + (size_t)t * 2 * kv_dim + (e - q_dim)) = out;
}

}  // namespace

// One packed matrix: the caller's reference MARLIN tensors and, when the
// runner re-tiled them for the matrix cores, its own tile16 copy.
struct Mat {
  const void* w = nullptr;
  const void* sb = nullptr;
  void* w16 = nullptr;
  void* sb16 = nullptr;
  int N = 0, K = 0;
  int g128 = 0;  // one (scale, bias) per 128 columns (tile16 copy only)
  int fmt = 0;   // 0: MARLIN Q4 (w int32 [N/8][K/64][32][2]); 1: Q8_G64 (w uint8 [N][K], sb fp16 [N][K/64][2]);
                 // 2: fp16 (w fp16 [N][K], no sb)
};

// Prologue / epilogue settings shared by both GEMV paths.
struct GemvCall {
  const f16* x = nullptr;
  int ldx = 0;
  f16* y = nullptr;
  int ldy = 0;
  const f16* bias = nullptr;
  const f16* ln_w = nullptr;
  float eps = 0.f;
  f16* x_norm_out = nullptr;
  f16* resid = nullptr;
  int ldr = 0;
  int pair_rows = 0;  // SWIGLU: rows of the gate half (H)
  int q_dim = 0, kv_dim = 0, head_dim = 0;
  const float* freqs = nullptr;
  int rope_len = 0;
  const int* rope_pos_dev = nullptr;
  int write_pos = 0;
  const int* write_pos_dev = nullptr;
  f16* k_out = nullptr;
  f16* v_out = nullptr;
  long kv_stride_h = 0;
  int max_seq = 1;
  unsigned long long* argmax_keys = nullptr;
  // tile16 O projection: activations merged from attention split partials.
  const f16* x_parts = nullptr;
  const f32x2* x_ml = nullptr;
  int n_parts = 0, parts_hd = 0;
  // RESID: RMSNorm (weight post_ln_w, eps) of the updated residual rows into
  // post_norm_out, the input of the next normed GEMM.
  const f16* post_ln_w = nullptr;
  f16* post_norm_out = nullptr;
  // Multi-token GEMM with the store epilogue: see T16Args::split_info.
  int* split_info = nullptr;
};

template <class A>
static void fill_common(A& a, const GemvCall& c, int K, int N) {
  a.x = c.x;
  a.ldx = c.ldx;
  a.K = K;
  a.N = N;
  a.y = c.y;
  a.ldy = c.ldy;
  a.bias = c.bias;
  a.ln_w = c.ln_w;
  a.eps = c.eps;
  a.x_norm_out = c.x_norm_out;
  a.resid = c.resid;
  a.ldr = c.ldr;
  a.q_dim = c.q_dim;
  a.kv_dim = c.kv_dim;
  a.head_dim = c.head_dim;
  a.freqs = c.freqs;
  a.rope_len = c.rope_len;
  a.rope_pos_dev = c.rope_pos_dev;
  a.write_pos = c.write_pos;
  a.write_pos_dev = c.write_pos_dev;
  a.k_out = c.k_out;
  a.v_out = c.v_out;
  a.kv_stride_h = c.kv_stride_h;
  a.max_seq = c.max_seq;
  a.argmax_keys = c.argmax_keys;
}

// out_rows: valid output rows (H for the SwiGLU pair, N otherwise).
static int run_gemv(const Mat& m, int epi, int out_rows, const GemvCall& c, int M, hipStream_t s) {
  if (m.w16 != nullptr) {
    T16Args a{};
    fill_common(a, c, m.K, out_rows);
    a.w16 = (const u32x4*)m.w16;
    a.sb16 = (const u32x2*)m.sb16;
    a.g128 = m.g128;
    a.KB = (m.K + 127) / 128;
    a.N_rows_alloc = m.N;
    a.n_units = (out_rows + 15) / 16;
    a.pair_offset = c.pair_rows / 16;
    a.x_parts = c.x_parts;
    a.x_ml = c.x_ml;
    a.n_parts = c.n_parts;
    a.parts_hd = c.parts_hd;
    return t16_gemv_launch(a, M, epi, s);
  }
  Q4GemvArgs a{};
  fill_common(a, c, m.K, out_rows);
  a.w = (const u32x4*)m.w;
  a.sb = (const u32x4*)m.sb;
  a.KG = m.K / 64;
  a.n_units = (out_rows + 7) / 8;
  a.pair_offset = c.pair_rows / 8;
  return q4m_gemv_launch(a, M, epi, s);
}

struct axm_runner {
  axm_runner_desc d{};
  std::vector<const void*> ln1, ln2, qkv_w, qkv_sb, qkv_b, o_w, o_sb, gu_w, gu_sb, dn_w, dn_sb;
  std::vector<Mat> m_qkv, m_o, m_gu, m_dn;
  Mat m_lmh;
  std::vector<void*> owned;  // runner-owned tile16 copies
  std::vector<void*> kc, vc, ks, vs;
  int q_dim = 0, kv_dim = 0, qkv_dim = 0;
  // device buffers
  int* params = nullptr;
  f16* x = nullptr;
  f16* q = nullptr;
  f16* kvst = nullptr;
  f16* attn_y = nullptr;
  f16* hbuf = nullptr;
  f16* logits = nullptr;
  f16* norm = nullptr;
  f16* qkvbuf = nullptr;                 // [T][qkv_dim] (multi-token paths)
  int* tree_pos = nullptr;               // [kMaxVerify]
  unsigned long long* tree_mask = nullptr;  // [kMaxVerify]
  float* ws = nullptr;
  size_t ws_bytes = 0;
  // Decode: attention split partials merged by the tile16 O projection (no
  // reduce launch) when parts_ok.
  bool parts_ok = false;
  f16* parts_o = nullptr;
  f32x2* parts_ml = nullptr;
  unsigned long long* argmax_keys = nullptr;  // per lm_head tile: ordered (logit, index) key
  int max_splits = 64;
  int mode = AXM_RUNNER_MODE_GRAPH;
  hipStream_t cap_stream = nullptr;
  std::map<int, hipGraphExec_t> graphs;
  // Persistent whole-step kernel state (step_kernel.hip).
  bool persist_ok = false;
  sp::Shape p_shape{};
  size_t p_smem = 0;
  StepLayer* p_layers = nullptr;           // device copy of the per-layer table
  unsigned long long* p_words = nullptr;   // cross-workgroup words (sp::words_layout)
  size_t p_words_bytes = 0;
  int64_t* p_tok_next = nullptr;
  int* p_err = nullptr;
  int* p_err_host = nullptr;               // pinned mirror, refreshed after each step
  unsigned p_tag = 1;                      // tag of the next launch's first phase (0 never matches)
  bool tok_next_valid = false;

  ~axm_runner() {
    for (auto& kv : graphs) (void)hipGraphExecDestroy(kv.second);
    if (cap_stream) (void)hipStreamDestroy(cap_stream);
    void* bufs[] = {params, x, q, kvst, attn_y, hbuf, logits, norm, ws, argmax_keys, parts_o,
                    qkvbuf, tree_pos, tree_mask, p_layers, p_words, p_tok_next, p_err};
    for (void* b : bufs)
      if (b) (void)hipFree(b);
    if (p_err_host) (void)hipHostFree(p_err_host);
    for (void* b : owned) (void)hipFree(b);
  }

  // Set up the persistent kernel when the configuration allows it: tile16 copies
  // of every MARLIN Q4 matrix (group 64 or 128) and of a MARLIN lm_head, an fp16
  // KV cache, head size 64 or 128, and co-residency of one 512-thread workgroup
  // on every CU (step_check).
  void setup_persistent() {
    if (m_qkv.empty() || d.kv_dtype != AXM_KV_FP16 || d.lm_head_format != 0 || m_lmh.w16 == nullptr ||
        d.qkv_format != 0 || d.o_format != 0 || d.gu_format != 0 || d.down_format != 0)
      return;
    for (int i = 0; i < d.n_layer; ++i)
      if (!m_qkv[i].w16 || !m_o[i].w16 || !m_gu[i].w16 || !m_dn[i].w16) return;
    sp::Shape sh{};
    sh.L = d.n_layer;
    sh.D = d.d_model;
    sh.H = d.hidden_dim;
    sh.Hq = d.n_head;
    sh.Hkv = d.n_kv_head;
    sh.hd = d.head_dim;
    sh.V = d.vocab_size;
    sh.S = d.max_seq_len;
    sh.g128 = d.group_size == 128 ? 1 : 0;
    if (step_check(sh, &p_smem) != 0) return;
    const int L = d.n_layer;
    std::vector<StepLayer> host(L);
    for (int i = 0; i < L; ++i) {
      StepLayer& p = host[i];
      p.qkv_w = m_qkv[i].w16;
      p.qkv_sb = m_qkv[i].sb16;
      p.o_w = m_o[i].w16;
      p.o_sb = m_o[i].sb16;
      p.gu_w = m_gu[i].w16;
      p.gu_sb = m_gu[i].sb16;
      p.dn_w = m_dn[i].w16;
      p.dn_sb = m_dn[i].sb16;
      p.ln1 = (const f16*)ln1[i];
      p.ln2 = (const f16*)ln2[i];
      p.qkv_bias = (const f16*)qkv_b[i];
      p.kc = (f16*)kc[i];
      p.vc = (f16*)vc[i];
    }
    p_words_bytes = (size_t)sp::words_layout(sh).total * sizeof(unsigned long long);
#ifdef AXM_STEP_STAMPS
    // Diagnostic build: phase timestamps follow the words (4 per workgroup and phase).
    p_words_bytes += (size_t)sh.G * sp::n_phases(sh) * 6 * sizeof(unsigned long long);
#endif
    if (hipMalloc(&p_layers, sizeof(StepLayer) * L) != hipSuccess ||
        hipMemcpy(p_layers, host.data(), sizeof(StepLayer) * L, hipMemcpyHostToDevice) != hipSuccess ||
        hipMalloc(&p_words, p_words_bytes) != hipSuccess || hipMemset(p_words, 0, p_words_bytes) != hipSuccess ||
        hipMalloc(&p_tok_next, sizeof(int64_t)) != hipSuccess || hipMemset(p_tok_next, 0, sizeof(int64_t)) != hipSuccess ||
        hipMalloc(&p_err, sizeof(int)) != hipSuccess || hipMemset(p_err, 0, sizeof(int)) != hipSuccess ||
        hipHostMalloc(&p_err_host, sizeof(int), hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      return;
    }
    *p_err_host = 0;
    p_shape = sh;
    persist_ok = true;
  }

  int step_persistent(const int64_t* idx_dev, int64_t tok_host, int rope_pos, int write_pos, int active_len,
                      hipStream_t s) {
    if (*p_err_host != 0) {
      axm_set_error("runner_step: an earlier persistent step gave up waiting for another workgroup");
      return -6;
    }
    const int nph = sp::n_phases(p_shape);
    if (p_tag > 0xFFFFFFFFu - (unsigned)nph) {
      // Tags would wrap: clear every word so that no stale tag can match, restart at 1.
      if (hipMemsetAsync(p_words, 0, p_words_bytes, s) != hipSuccess) {
        axm_set_error("runner_step: clearing the persistent step's words failed");
        return -5;
      }
      p_tag = 1;
    }
    StepArgs a{};
    a.sh = p_shape;
    a.layers = p_layers;
    a.lm_w = m_lmh.w16;
    a.lm_sb = m_lmh.sb16;
    a.lnf = (const f16*)d.lnf_w;
    a.freqs = d.freqs;
    a.rope_len = d.rope_len;
    a.wte_fmt = d.wte_format;
    a.wte = d.wte;
    a.wte_sb = (const f16*)d.wte_sb;
    a.eps = d.eps;
    a.scale_log2 = 1.4426950408889634f / sqrtf((float)d.head_dim);
    a.idx_dev = idx_dev;
    a.tok_host = tok_host;
    a.tok_prev = p_tok_next;
    a.tok_used = reinterpret_cast<int64_t*>(reinterpret_cast<unsigned char*>(params) + kTokenOffset);
    if (idx_dev == nullptr && tok_host < 0 && !tok_next_valid) {
      // Greedy feedback after a step of another mode: reduce its argmax keys first.
      hipLaunchKernelGGL(set_params_kernel, dim3(1), dim3(256), 0, s, params, (const int64_t*)nullptr, (int64_t)-1,
                         rope_pos, write_pos, active_len, argmax_keys, (d.vocab_size + 7) / 8, EmbedArgs{});
      a.idx_dev = a.tok_used;
    }
    a.rope_pos = rope_pos;
    a.write_pos = write_pos;
    a.active_len = active_len;
    a.n_splits = sp::choose_splits(p_shape, active_len);
    a.tag0 = p_tag;
    a.spin_limit = 1 << 20;
    a.words = p_words;
    a.logits = logits;
    a.norm_out = norm;
    a.argmax_keys = argmax_keys;
    a.tok_next = p_tok_next;
    a.err = p_err;
    const int rc = step_launch(a, p_smem, s);
    if (rc) return rc;
    p_tag += (unsigned)nph;
    if (hipMemcpyAsync(p_err_host, p_err, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess) {
      axm_set_error("runner_step: error-flag copy failed");
      return -5;
    }
    tok_next_valid = true;
    return 0;
  }

  KvView kv_view(int layer) const {
    KvView v{kc[layer], vc[layer], d.kv_dtype ? (f16*)ks[layer] : nullptr, d.kv_dtype ? (f16*)vs[layer] : nullptr,
             d.kv_dtype, 1, d.n_kv_head, d.max_seq_len, d.head_dim};
    return v;
  }

  // Enqueue the whole single-token step on stream s (no host synchronization).
  // The decode step after set_params_kernel, which has written the token's
  // embedding row into x.  Each launch group of a layer is its own member
  // (axm_runner_time_kernels times them one at a time).
  int enqueue_step(int n_splits, bool short_splits, hipStream_t s) {
    for (int i = 0; i < d.n_layer; ++i) {
      int rc = enqueue_qkv(i, s);
      if (rc) return rc;
      rc = enqueue_attention(i, n_splits, short_splits, s);
      if (rc) return rc;
      rc = enqueue_o(i, n_splits, s);
      if (rc) return rc;
      rc = enqueue_gate_up(i, s);
      if (rc) return rc;
      rc = enqueue_down(i, s);
      if (rc) return rc;
    }
    return enqueue_lm_head(s);
  }

  // The attention split count of a one-token step over active_len keys, bucketed
  // so that one graph covers a range of lengths; splits of at most 64 keys use a
  // smaller attention launch shape (the graph key carries both).
  void split_shape(int active_len, int* bucket_out, bool* short_out) const {
    const int splits = parts_ok ? attn_parts_splits(1, d.n_kv_head, active_len)
                                : attn_choose_splits(1, d.n_kv_head, active_len);
    int bucket = 1;
    while (bucket < splits) bucket <<= 1;
    if (bucket > max_splits) bucket = max_splits;
    *bucket_out = bucket;
    *short_out = active_len <= 64 * bucket;
  }

  // With parts_ok and more than one split, the attention leaves its split
  // partials for the O projection to merge while staging its activations.
  bool merge_in_o(int n_splits) const { return parts_ok && n_splits > 1; }

  // 1. QKV with RMSNorm prologue and RoPE / KV-write epilogue.
  int enqueue_qkv(int i, hipStream_t s) {
    const int D = d.d_model;
    KvView kv = kv_view(i);
    GemvCall a{};
    a.x = x;
    a.ldx = D;
    a.y = q;
    a.ldy = q_dim;
    a.bias = (const f16*)qkv_b[i];
    a.ln_w = (const f16*)ln1[i];
    a.eps = d.eps;
    a.q_dim = q_dim;
    a.kv_dim = kv_dim;
    a.head_dim = d.head_dim;
    a.freqs = d.freqs;
    a.rope_len = d.rope_len;
    a.rope_pos_dev = params + P_ROPE;
    if (d.kv_dtype == AXM_KV_FP16) {
      a.write_pos_dev = params + P_WRITE;
      a.k_out = (f16*)kc[i];
      a.v_out = (f16*)vc[i];
      a.kv_stride_h = (long)d.max_seq_len * d.head_dim;
      a.max_seq = d.max_seq_len;
    } else {
      // Stage fp16 k / v rows; the quantizer writes the cache slot.
      a.k_out = kvst;
      a.v_out = kvst + kv_dim;
      a.kv_stride_h = d.head_dim;
      a.max_seq = 1;
    }
    int rc = 0;
    if (m_qkv[i].fmt != 0) {
      // Q8_G64 / fp16 QKV: the GEMV's own RoPE / KV-slot epilogue, as the tile16 one.
      QkvRope r;
      r.q_dim = q_dim;
      r.kv_dim = kv_dim;
      r.head_dim = d.head_dim;
      r.rope_len = d.rope_len;
      r.freqs = d.freqs;
      r.rope_pos_dev = a.rope_pos_dev;
      r.write_pos_dev = a.write_pos_dev;
      r.q_out = q;
      r.k_out = a.k_out;
      r.v_out = a.v_out;
      r.kv_stride_h = a.kv_stride_h;
      r.max_seq = a.max_seq;
      const Mat& m = m_qkv[i];
      rc = m.fmt == 1 ? launch_q8_gemv_qkv(x, (const uint8_t*)m.w, (const f16*)m.sb, a.bias, 1, D, qkv_dim, a.ln_w,
                                           d.eps, r, s)
                      : launch_f16_gemv_qkv(x, (const f16*)m.w, a.bias, 1, D, qkv_dim, a.ln_w, d.eps, r, s);
      if (rc) return rc;
      if (d.kv_dtype != AXM_KV_FP16) launch_kv_write(kv, kvst, kvst + kv_dim, 2 * kv_dim, 1, 0, params + P_WRITE, s);
    } else {
      rc = run_gemv(m_qkv[i], Q4_EPI_QKV_ROPE, qkv_dim, a, 1, s);
      if (rc) return rc;
      if (d.kv_dtype != AXM_KV_FP16) launch_kv_write(kv, kvst, kvst + kv_dim, 2 * kv_dim, 1, 0, params + P_WRITE, s);
    }
    return 0;
  }

  // 2. attention over slots [0, active_len).
  int enqueue_attention(int i, int n_splits, bool short_splits, hipStream_t s) {
    KvView kv = kv_view(i);
    if (merge_in_o(n_splits))
      return launch_flash_decode_parts(q, kv, d.n_head, 0, params + P_ACTIVE, n_splits, parts_o, parts_ml,
                                       short_splits, s);
    return launch_flash_decode(q, kv, attn_y, d.n_head, 0, params + P_ACTIVE, n_splits, ws, s);
  }

  // 3. O projection, residual add into x.
  int enqueue_o(int i, int n_splits, hipStream_t s) {
    GemvCall o{};
    o.x = attn_y;
    o.ldx = q_dim;
    o.resid = x;
    o.ldr = d.d_model;
    if (merge_in_o(n_splits)) {
      o.x_parts = parts_o;
      o.x_ml = parts_ml;
      o.n_parts = n_splits;
      o.parts_hd = d.head_dim;
    }
    return gemv(m_o[i], Q4_EPI_RESID, d.d_model, o, 1, s);
  }

  // 4. gate/up with RMSNorm prologue and SwiGLU epilogue.
  int enqueue_gate_up(int i, hipStream_t s) {
    GemvCall g{};
    g.x = x;
    g.ldx = d.d_model;
    g.y = hbuf;
    g.ldy = d.hidden_dim;
    g.ln_w = (const f16*)ln2[i];
    g.eps = d.eps;
    g.pair_rows = d.hidden_dim;
    return gemv(m_gu[i], Q4_EPI_SWIGLU, d.hidden_dim, g, 1, s);
  }

  // 5. down projection, residual add.
  int enqueue_down(int i, hipStream_t s) {
    GemvCall dn{};
    dn.x = hbuf;
    dn.ldx = d.hidden_dim;
    dn.resid = x;
    dn.ldr = d.d_model;
    return gemv(m_dn[i], Q4_EPI_RESID, d.d_model, dn, 1, s);
  }

  // Final RMSNorm + lm_head (+ per-tile greedy argmax keys).
  int enqueue_lm_head(hipStream_t s) {
    const int D = d.d_model;
    if (d.lm_head_format == 0) {
      GemvCall l{};
      l.x = x;
      l.ldx = D;
      l.y = logits;
      l.ldy = d.vocab_size;
      l.ln_w = (const f16*)d.lnf_w;
      l.eps = d.eps;
      l.x_norm_out = norm;
      l.argmax_keys = argmax_keys;
      return run_gemv(m_lmh, Q4_EPI_STORE, d.vocab_size, l, 1, s);
    }
    return lm_head_dense(x, 1, (const f16*)d.lnf_w, norm, s);
  }

  // Q8_G64 (format 1) or fp16 (format 2) lm_head over T rows into logits: with ln_w the
  // GEMV applies the final RMSNorm itself and writes the normalized rows to xn_out (one
  // launch where a separate norm took two); without, the rows are normalized already.
  int lm_head_dense(const f16* x, int T, const f16* ln_w, f16* xn_out, hipStream_t s) {
    if (d.lm_head_format == 2)
      return launch_f16_gemv(x, (const f16*)d.lm_head_w, nullptr, logits, T, d.d_model, d.vocab_size, ln_w, d.eps,
                             s, xn_out);
    return launch_q8_gemv(x, (const uint8_t*)d.lm_head_w, (const f16*)d.lm_head_sb, nullptr, logits, T, d.d_model,
                          d.vocab_size, ln_w, d.eps, s, xn_out);
  }

  // The GEMV of a Q8_G64 (fmt 1) or fp16 (fmt 2) matrix, [M][K] -> [M][N] rows.
  static int dense_gemv(const Mat& m, const f16* x, const f16* bias, f16* y, int M, int N, const f16* ln,
                        float eps, hipStream_t s) {
    if (m.fmt == 2) return launch_f16_gemv(x, (const f16*)m.w, bias, y, M, m.K, N, ln, eps, s);
    return launch_q8_gemv(x, (const uint8_t*)m.w, (const f16*)m.sb, bias, y, M, m.K, N, ln, eps, s);
  }

  // A Q8_G64 or fp16 matrix: its GEMV (RMSNorm prologue, bias) with the residual /
  // SwiGLU epilogue fused, with the rounding of the tile16 epilogues (residual add in
  // fp16, silu(fp16 g) * fp16 u).  Activation and output rows are contiguous ([M][K]
  // in, [M][N] out), as every caller lays them out.
  int run_dense(const Mat& m, int epi, int out_rows, const GemvCall& c, int M, hipStream_t s) {
    if (c.x_parts != nullptr || c.argmax_keys != nullptr || epi == Q4_EPI_QKV_ROPE || c.ldx != m.K) {
      axm_set_error("runner: unsupported call on a Q8_G64 / fp16 matrix (epilogue %d)", epi);
      return -2;
    }
    const f16* xin = c.x;
    const f16* ln = c.ln_w;
    if (c.x_norm_out != nullptr && ln != nullptr) {
      launch_rmsnorm(c.x, ln, c.x_norm_out, M, m.K, c.eps, s);
      xin = c.x_norm_out;
      ln = nullptr;
    }
    int rc = 0;
    if (epi == Q4_EPI_STORE) {
      if (c.ldy != out_rows) {
        axm_set_error("runner: a Q8 store needs contiguous output rows");
        return -2;
      }
      return dense_gemv(m, xin, c.bias, c.y, M, out_rows, ln, c.eps, s);
    }
    if (epi == Q4_EPI_SWIGLU) {
      if (c.ldy != out_rows) {
        axm_set_error("runner: a Q8 SwiGLU needs contiguous output rows");
        return -2;
      }
      if (m.fmt == 1)
        return launch_q8_gemv_swiglu(xin, (const uint8_t*)m.w, (const f16*)m.sb, c.y, M, m.K, 2 * out_rows, ln,
                                     c.eps, s);
      return launch_f16_gemv_swiglu(xin, (const f16*)m.w, c.y, M, m.K, 2 * out_rows, ln, c.eps, s);
    }
    // Q4_EPI_RESID
    if (c.ldr != out_rows) {
      axm_set_error("runner: a Q8 residual needs contiguous rows");
      return -2;
    }
    rc = m.fmt == 1 ? launch_q8_gemv_resid(xin, (const uint8_t*)m.w, (const f16*)m.sb, c.resid, M, m.K, out_rows, ln,
                                           c.eps, s)
                    : launch_f16_gemv_resid(xin, (const f16*)m.w, c.resid, M, m.K, out_rows, ln, c.eps, s);
    if (rc) return rc;
    if (c.post_ln_w != nullptr) launch_rmsnorm(c.resid, c.post_ln_w, c.post_norm_out, M, out_rows, c.eps, s);
    return 0;
  }

  int gemv(const Mat& m, int epi, int out_rows, const GemvCall& c, int M, hipStream_t s) {
    return m.fmt != 0 ? run_dense(m, epi, out_rows, c, M, s) : run_gemv(m, epi, out_rows, c, M, s);
  }

  // GEMV over T token rows in launches of at most 4 rows, or the multi-token GEMM
  // from kGemmMinTokens rows on.
  int gemv_rows(const Mat& m, int epi, int out_rows, GemvCall c, int T, hipStream_t s) {
    if (m.w16 != nullptr && T >= kGemmMinTokens && c.argmax_keys == nullptr && c.q_dim == 0 &&
        (epi == Q4_EPI_STORE || epi == Q4_EPI_RESID || epi == Q4_EPI_SWIGLU)) {
      // Multi-token GEMM: up to 64 tokens per weight pass, activations normalized first
      // (into x_norm_out when the caller wants them, else into the norm scratch).
      const f16* xall = c.x;
      if (c.ln_w != nullptr) {
        f16* nrm = c.x_norm_out ? c.x_norm_out : norm;
        launch_rmsnorm(c.x, c.ln_w, nrm, T, m.K, c.eps, s);
        xall = nrm;
      }
      for (int t0 = 0; t0 < T; t0 += kTile16GemmMaxTokens) {
        const int mc = (T - t0) < kTile16GemmMaxTokens ? (T - t0) : kTile16GemmMaxTokens;
        const f16* xin = xall + (size_t)t0 * c.ldx;
        T16Args a{};
        a.x = xin;
        a.ldx = c.ldx;
        a.w16 = (const u32x4*)m.w16;
        a.sb16 = (const u32x2*)m.sb16;
        a.g128 = m.g128;
        a.K = m.K;
        a.KB = (m.K + 127) / 128;
        a.N = out_rows;
        a.N_rows_alloc = m.N;
        a.n_units = (out_rows + 15) / 16;
        a.pair_offset = c.pair_rows / 16;
        a.y = c.y ? c.y + (size_t)t0 * c.ldy : nullptr;
        a.ldy = c.ldy;
        a.bias = c.bias;
        a.resid = c.resid ? c.resid + (size_t)t0 * c.ldr : nullptr;
        a.ldr = c.ldr;
        a.post_ln_w = c.post_ln_w;
        a.post_norm_out = c.post_ln_w ? c.post_norm_out + (size_t)t0 * out_rows : nullptr;
        a.eps = c.eps;
        a.split_info = T <= kTile16GemmMaxTokens ? c.split_info : nullptr;
        const int rc = t16_gemm_launch(a, mc, epi, ws, ws_bytes, s);
        if (rc) return rc;
      }
      return 0;
    }
    for (int t0 = 0; t0 < T; t0 += 4) {
      const int mc = (T - t0) < 4 ? (T - t0) : 4;
      GemvCall cc = c;
      cc.x = c.x + (size_t)t0 * c.ldx;
      if (c.y) cc.y = c.y + (size_t)t0 * c.ldy;
      if (c.resid) cc.resid = c.resid + (size_t)t0 * c.ldr;
      if (c.x_norm_out) cc.x_norm_out = c.x_norm_out + (size_t)t0 * c.ldx;
      GemvCall cq = cc;
      if (m.fmt != 0) cq.post_ln_w = nullptr;  // normalized once below
      const int rc = gemv(m, epi, out_rows, cq, mc, s);
      if (rc) return rc;
    }
    if (c.post_ln_w != nullptr) return launch_rmsnorm(c.resid, c.post_ln_w, c.post_norm_out, T, out_rows, c.eps, s);
    return 0;
  }

  // Multi-token step (verify_step / verify_tree_step, mps_kernels.mm:3265-3464).
  // tree: token t is rotated at start_pos + depth[t], written to slot
  // (write_pos + t) % S and attends to [0, prefix) plus the tree slots its mask
  // selects.  !tree (ring wrap-around): all T rows are written, then every token
  // attends over all S slots, as the reference does in that case.
  int enqueue_verify(const int64_t* idx_dev, int T, int write_pos, int prefix, bool tree, hipStream_t s) {
    const int D = d.d_model, H = d.hidden_dim;
    // Multi-token GEMMs take normalized activations: there the residual GEMMs
    // (O, down) also write the RMSNorm of the rows they update into `norm` for
    // the next GEMM (fused into their split reduce), instead of a norm launch
    // per normed GEMM.  Fewer tokens keep the GEMVs' fused norm prologue.
    const bool post = T >= kGemmMinTokens;
    if (d.wte_format == 0)
      launch_embed_f16((const f16*)d.wte, idx_dev, nullptr, x, T, D, d.vocab_size, s);
    else
      launch_embed_q8((const uint8_t*)d.wte, (const f16*)d.wte_sb, idx_dev, nullptr, x, T, D, d.vocab_size, s);
    for (int i = 0; i < d.n_layer; ++i) {
      KvView kv = kv_view(i);
      GemvCall a{};
      a.x = post && i > 0 ? norm : x;
      a.ldx = D;
      a.y = qkvbuf;
      a.ldy = qkv_dim;
      a.bias = (const f16*)qkv_b[i];
      a.ln_w = post && i > 0 ? nullptr : (const f16*)ln1[i];
      a.eps = d.eps;
      // With head size 128 a K-split QKV GEMM leaves its partials to the RoPE /
      // cache-write launch, which sums them (no separate split reduce).
      int split_info[3] = {0, 0, 0};
      if (d.head_dim == 128) a.split_info = split_info;
      int rc = gemv_rows(m_qkv[i], Q4_EPI_STORE, qkv_dim, a, T, s);
      if (rc) return rc;
      if (d.head_dim == 128) {
        // RoPE and the cache write in one launch.
        if (split_info[0] > 1)
          rc = launch_reduce_rope_kv_write(kv, ws, split_info[0], split_info[1], split_info[2], a.bias, d.n_head, T,
                                           d.freqs, tree_pos, q, write_pos, s);
        else
          rc = launch_rope_kv_write(kv, qkvbuf, d.n_head, T, d.freqs, tree_pos, q, write_pos, s);
        if (rc) return rc;
      } else {
        hipLaunchKernelGGL(rope_tokens_kernel, dim3((qkv_dim / 8 + 255) / 256, T), dim3(256), 0, s, qkvbuf, q_dim,
                           kv_dim, d.head_dim, d.freqs, tree_pos, q, kvst);
        launch_kv_write(kv, kvst, kvst + kv_dim, 2 * kv_dim, T, write_pos, nullptr, s);
      }
      if (tree) {
        const int splits = tree_choose_splits(T, d.n_head, d.n_kv_head, prefix + T);
        rc = launch_tree_attention(q, kv, attn_y, d.n_head, T, prefix, write_pos, (const uint64_t*)tree_mask, splits, ws,
                                   s);
      } else {
        const int splits = attn_flash_splits(1, d.n_head, d.n_kv_head, d.head_dim, d.kv_dtype, d.max_seq_len);
        for (int t = 0; t < T && rc == 0; ++t)
          rc = launch_flash_decode(q + (size_t)t * q_dim, kv, attn_y + (size_t)t * q_dim, d.n_head, d.max_seq_len,
                                   nullptr, splits, ws, s);
      }
      if (rc) return rc;
      GemvCall o{};
      o.x = attn_y;
      o.ldx = q_dim;
      o.resid = x;
      o.ldr = D;
      if (post) {
        o.post_ln_w = (const f16*)ln2[i];
        o.post_norm_out = norm;
        o.eps = d.eps;
      }
      rc = gemv_rows(m_o[i], Q4_EPI_RESID, D, o, T, s);
      if (rc) return rc;
      GemvCall g{};
      g.x = post ? norm : x;
      g.ldx = D;
      g.y = hbuf;
      g.ldy = H;
      g.ln_w = post ? nullptr : (const f16*)ln2[i];
      g.eps = d.eps;
      g.pair_rows = H;
      rc = gemv_rows(m_gu[i], Q4_EPI_SWIGLU, H, g, T, s);
      if (rc) return rc;
      GemvCall dn{};
      dn.x = hbuf;
      dn.ldx = H;
      dn.resid = x;
      dn.ldr = D;
      if (post) {
        dn.post_ln_w = (const f16*)(i + 1 < d.n_layer ? ln1[i + 1] : d.lnf_w);
        dn.post_norm_out = norm;
        dn.eps = d.eps;
      }
      rc = gemv_rows(m_dn[i], Q4_EPI_RESID, D, dn, T, s);
      if (rc) return rc;
    }
    if (d.lm_head_format == 0) {
      GemvCall l{};
      l.x = post ? norm : x;
      l.ldx = D;
      l.y = logits;
      l.ldy = d.vocab_size;
      l.ln_w = post ? nullptr : (const f16*)d.lnf_w;
      l.eps = d.eps;
      l.x_norm_out = post ? nullptr : norm;
      return gemv_rows(m_lmh, Q4_EPI_STORE, d.vocab_size, l, T, s);
    }
    if (!post) return lm_head_dense(x, T, (const f16*)d.lnf_w, norm, s);
    return lm_head_dense(norm, T, nullptr, nullptr, s);
  }

  // Re-tile one matrix for the matrix-core GEMV (runner-owned copy).
  int make_tile16(Mat& m) {
    m.g128 = d.group_size == 128;
    const size_t wb = t16_weight_bytes(m.N, m.K), sbb = t16_sb_bytes(m.N, m.K, d.group_size == 128);
    if (hipMalloc(&m.w16, wb) != hipSuccess) return -4;
    owned.push_back(m.w16);
    if (hipMalloc(&m.sb16, sbb) != hipSuccess) return -4;
    owned.push_back(m.sb16);
    return t16_repack(m.w, m.sb, m.N, m.K, m.w16, m.sb16, nullptr, d.group_size == 128);
  }
};

static bool q4_shape_ok(int N, int K) { return N > 0 && K > 0 && K % 64 == 0; }

extern "C" int axm_runner_create(const axm_runner_desc* desc, axm_runner_t* out) {
  AXM_CHECK_ARG(desc && out, -1, "runner_create: null argument");
  const axm_runner_desc& d = *desc;
  AXM_CHECK_ARG(d.n_layer >= 1 && d.n_head >= 1 && d.n_kv_head >= 1 && d.n_head % d.n_kv_head == 0, -1,
                "runner_create: bad head configuration");
  AXM_CHECK_ARG(d.head_dim == 64 || d.head_dim == 128, -1, "runner_create: head_dim %d must be 64 or 128",
                d.head_dim);
  AXM_CHECK_ARG(d.d_model == d.n_head * d.head_dim, -1, "runner_create: d_model != n_head * head_dim");
  AXM_CHECK_ARG(q4_shape_ok(d.hidden_dim, d.d_model) && d.hidden_dim % 64 == 0 && d.hidden_dim % 8 == 0, -1,
                "runner_create: hidden_dim %d must be a multiple of 64", d.hidden_dim);
  AXM_CHECK_ARG(d.vocab_size > 0 && d.max_seq_len > 0 && d.rope_len > 0, -1, "runner_create: bad sizes");
  AXM_CHECK_ARG(d.kv_dtype >= 0 && d.kv_dtype <= 2, -1, "runner_create: bad kv dtype");
  AXM_CHECK_ARG(d.wte && d.lm_head_w && d.freqs && d.lnf_w, -1, "runner_create: null global weight");
  AXM_CHECK_ARG(d.ln1_w && d.ln2_w && d.qkv_w && d.qkv_sb && d.o_w && d.o_sb && d.gu_w && d.gu_sb && d.down_w &&
                    d.down_sb && d.k_cache && d.v_cache,
                -1, "runner_create: null per-layer array");
  AXM_CHECK_ARG(d.kv_dtype == AXM_KV_FP16 || (d.k_scales && d.v_scales), -1,
                "runner_create: quantized KV cache needs scale arrays");
  AXM_CHECK_ARG(d.lm_head_format >= 0 && d.lm_head_format <= 2, -1, "runner_create: bad lm_head format");
  AXM_CHECK_ARG(d.lm_head_format == 2 || d.lm_head_sb, -1, "runner_create: lm_head scales missing");
  AXM_CHECK_ARG(d.group_size == 0 || d.group_size == 64 || d.group_size == 128, -1,
                "runner_create: group_size %d must be 64 or 128", d.group_size);
  for (int f : {d.qkv_format, d.o_format, d.gu_format, d.down_format})
    AXM_CHECK_ARG(f >= 0 && f <= 2, -1,
                  "runner_create: layer matrix format %d must be 0 (MARLIN Q4), 1 (Q8_G64) or 2 (fp16)", f);
  AXM_CHECK_ARG(d.qkv_format == 0 || (d.n_head + 2 * d.n_kv_head) * d.head_dim % 8 == 0, -1,
                "runner_create: a Q8_G64 QKV needs q, k and v rows in multiples of 8");
  AXM_CHECK_ARG(d.group_size != 128 ||
                    (d.layout != 1 && d.d_model % 128 == 0 && d.hidden_dim % 128 == 0 &&
                     (d.n_head * d.head_dim) % 128 == 0 && d.hidden_dim % 16 == 0 && d.hidden_dim <= kTile16MaxK &&
                     d.d_model <= kTile16MaxK && d.n_head * d.head_dim <= kTile16MaxK),
                -1, "runner_create: group-128 weights need the tile16 layout and K %% 128 == 0 for every matrix");

  axm_runner* r = new axm_runner();
  r->d = d;
  const int L = d.n_layer;
  auto copy = [L](const void* const* src, std::vector<const void*>& dst, bool allow_null) {
    dst.assign(L, nullptr);
    if (!src) return allow_null;
    for (int i = 0; i < L; ++i) {
      dst[i] = src[i];
      if (!dst[i] && !allow_null) return false;
    }
    return true;
  };
  // fp16 matrices (format 2) have no scale arrays
  bool ok = copy(d.ln1_w, r->ln1, false) && copy(d.ln2_w, r->ln2, false) && copy(d.qkv_w, r->qkv_w, false) &&
            copy(d.qkv_sb, r->qkv_sb, d.qkv_format == 2) && copy(d.qkv_bias, r->qkv_b, true) &&
            copy(d.o_w, r->o_w, false) && copy(d.o_sb, r->o_sb, d.o_format == 2) && copy(d.gu_w, r->gu_w, false) &&
            copy(d.gu_sb, r->gu_sb, d.gu_format == 2) && copy(d.down_w, r->dn_w, false) &&
            copy(d.down_sb, r->dn_sb, d.down_format == 2);
  if (!ok) {
    delete r;
    axm_set_error("runner_create: a per-layer weight pointer is null");
    return -1;
  }
  r->kc.assign(d.k_cache, d.k_cache + L);
  r->vc.assign(d.v_cache, d.v_cache + L);
  if (d.kv_dtype != AXM_KV_FP16) {
    r->ks.assign(d.k_scales, d.k_scales + L);
    r->vs.assign(d.v_scales, d.v_scales + L);
  } else {
    r->ks.assign(L, nullptr);
    r->vs.assign(L, nullptr);
  }
  r->d.max_tokens = d.max_tokens > 0 ? d.max_tokens : 1;
  {
    const int qkv_rows = (d.n_head + 2 * d.n_kv_head) * d.head_dim;
    for (int i = 0; i < L; ++i) {
      r->m_qkv.push_back(Mat{r->qkv_w[i], r->qkv_sb[i], nullptr, nullptr, qkv_rows, d.d_model, 0, d.qkv_format});
      r->m_o.push_back(Mat{r->o_w[i], r->o_sb[i], nullptr, nullptr, d.d_model, d.n_head * d.head_dim, 0, d.o_format});
      r->m_gu.push_back(Mat{r->gu_w[i], r->gu_sb[i], nullptr, nullptr, 2 * d.hidden_dim, d.d_model, 0, d.gu_format});
      r->m_dn.push_back(Mat{r->dn_w[i], r->dn_sb[i], nullptr, nullptr, d.d_model, d.hidden_dim, 0, d.down_format});
    }
    r->m_lmh = Mat{d.lm_head_w, d.lm_head_sb, nullptr, nullptr, d.vocab_size, d.d_model};
    // The gate/up pair shares a tile16 boundary when H % 16 == 0, and the tile16
    // GEMV stages at most kTile16MaxK activations; otherwise keep the reference
    // layout everywhere.
    const bool t16 = d.hidden_dim % 16 == 0 && d.layout != 1 && d.hidden_dim <= kTile16MaxK &&
                     d.d_model <= kTile16MaxK && d.n_head * d.head_dim <= kTile16MaxK;
    if (t16) {
      int rc = 0;
      for (int i = 0; i < L && rc == 0; ++i) {
        // Q8_G64 matrices keep the reference layout (the Q8 GEMV streams it).
        for (Mat* m : {&r->m_qkv[i], &r->m_o[i], &r->m_gu[i], &r->m_dn[i]})
          if (m->fmt == 0) rc = rc ? rc : r->make_tile16(*m);
      }
      if (rc == 0 && d.lm_head_format == 0) rc = r->make_tile16(r->m_lmh);
      if (rc != 0 || hipDeviceSynchronize() != hipSuccess) {
        delete r;
        axm_set_error("runner_create: tile16 repack failed");
        return -4;
      }
    }
  }
  r->q_dim = d.n_head * d.head_dim;
  r->kv_dim = d.n_kv_head * d.head_dim;
  r->qkv_dim = r->q_dim + 2 * r->kv_dim;
  const int T = r->d.max_tokens;
  r->ws_bytes = attn_workspace_bytes(T, d.n_head, d.head_dim, r->max_splits);
  if (r->m_o.size() == (size_t)L && r->m_o[0].w16 != nullptr) {
    // Partial tiles of the multi-token GEMM share the attention workspace.
    const size_t g[] = {t16_gemm_ws_bytes(d.d_model, r->qkv_dim / 16 + ((r->qkv_dim % 16) != 0), 1),
                        t16_gemm_ws_bytes(r->q_dim, (d.d_model + 15) / 16, 1),
                        t16_gemm_ws_bytes(d.d_model, d.hidden_dim / 16, 2),
                        t16_gemm_ws_bytes(d.hidden_dim, (d.d_model + 15) / 16, 1),
                        t16_gemm_ws_bytes(d.d_model, (d.vocab_size + 15) / 16, 1)};
    for (size_t b : g) r->ws_bytes = b > r->ws_bytes ? b : r->ws_bytes;
  }
  struct {
    void** p;
    size_t bytes;
  } allocs[] = {
      {(void**)&r->params, 64 * sizeof(int)},
      {(void**)&r->x, (size_t)T * d.d_model * sizeof(f16)},
      {(void**)&r->q, (size_t)T * r->q_dim * sizeof(f16)},
      {(void**)&r->kvst, (size_t)T * 2 * r->kv_dim * sizeof(f16)},
      {(void**)&r->attn_y, (size_t)T * r->q_dim * sizeof(f16)},
      {(void**)&r->hbuf, (size_t)T * d.hidden_dim * sizeof(f16)},
      {(void**)&r->logits, (size_t)T * d.vocab_size * sizeof(f16)},
      {(void**)&r->norm, (size_t)T * d.d_model * sizeof(f16)},
      {(void**)&r->ws, r->ws_bytes > 0 ? r->ws_bytes : 256},
      {(void**)&r->parts_o, attn_parts_bytes(1, d.n_head, d.head_dim)},
      {(void**)&r->argmax_keys, (size_t)((d.vocab_size + 7) / 8) * sizeof(unsigned long long)},
      {(void**)&r->qkvbuf, (size_t)T * r->qkv_dim * sizeof(f16)},
      {(void**)&r->tree_pos, kMaxVerify * sizeof(int)},
      {(void**)&r->tree_mask, kMaxVerify * sizeof(unsigned long long)},
  };
  for (auto& al : allocs) {
    if (hipMalloc(al.p, al.bytes) != hipSuccess) {
      delete r;
      axm_set_error("runner_create: hipMalloc of %zu bytes failed", al.bytes);
      return -4;
    }
  }
  if (hipMemset(r->params, 0, 64 * sizeof(int)) != hipSuccess ||
      hipMemset(r->argmax_keys, 0, (size_t)((d.vocab_size + 7) / 8) * sizeof(unsigned long long)) != hipSuccess ||
      hipStreamCreateWithFlags(&r->cap_stream, hipStreamNonBlocking) != hipSuccess) {
    delete r;
    axm_set_error("runner_create: stream/memset setup failed");
    return -4;
  }
  r->parts_ml = reinterpret_cast<f32x2*>(r->parts_o + (size_t)kAttnMaxParts * r->q_dim);
  r->parts_ok = true;
  for (const Mat& m : r->m_o) r->parts_ok = r->parts_ok && m.w16 != nullptr;
  r->parts_ok = r->parts_ok && r->q_dim <= kTile16PartsMaxK && d.head_dim % 8 == 0 &&
                kAttnMaxParts <= kTile16MaxParts;
  q4m_prepare_attributes();
  r->setup_persistent();
  *out = r;
  return 0;
}

extern "C" void axm_runner_destroy(axm_runner_t r) { delete r; }

extern "C" int axm_runner_set_graph(axm_runner_t r, int enable) {
  AXM_CHECK_ARG(r, -1, "runner_set_graph: null runner");
  r->mode = enable != 0 ? AXM_RUNNER_MODE_GRAPH : AXM_RUNNER_MODE_EAGER;
  return 0;
}

extern "C" int axm_runner_set_mode(axm_runner_t r, int mode) {
  AXM_CHECK_ARG(r, -1, "runner_set_mode: null runner");
  AXM_CHECK_ARG(mode == AXM_RUNNER_MODE_GRAPH || mode == AXM_RUNNER_MODE_EAGER || mode == AXM_RUNNER_MODE_PERSISTENT,
                -1, "runner_set_mode: unknown mode %d", mode);
  AXM_CHECK_ARG(mode != AXM_RUNNER_MODE_PERSISTENT || r->persist_ok, -1,
                "runner_set_mode: the persistent step needs tile16 copies of MARLIN Q4 layer and lm_head weights, an "
                "fp16 KV cache, head size 64 or 128 and one co-resident 512-thread workgroup per CU");
  r->mode = mode;
  return 0;
}

extern "C" int axm_runner_get_mode(axm_runner_t r) { return r ? r->mode : -1; }

extern "C" int axm_runner_check(axm_runner_t r) {
  AXM_CHECK_ARG(r, -1, "runner_check: null runner");
  if (!r->persist_ok) return 0;
  int e = 0;
  if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(&e, r->p_err, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) {
    axm_set_error("runner_check: device error");
    return -5;
  }
  if (e != 0) {
    axm_set_error("runner_check: a persistent step gave up waiting for another workgroup");
    return -6;
  }
  return 0;
}

extern "C" int axm_runner_step(axm_runner_t r, const void* idx_dev, int64_t tok_host, int start_pos, int write_pos,
                               int active_len, void* stream, void** logits_out) {
  AXM_CHECK_ARG(r, -1, "runner_step: null runner");
  const axm_runner_desc& d = r->d;
  AXM_CHECK_ARG(write_pos >= 0 && write_pos < d.max_seq_len, -1, "runner_step: write_pos %d out of [0, %d)",
                write_pos, d.max_seq_len);
  AXM_CHECK_ARG(active_len >= 1 && active_len <= d.max_seq_len, -1, "runner_step: active_len %d out of [1, %d]",
                active_len, d.max_seq_len);
  AXM_CHECK_ARG(start_pos >= 0, -1, "runner_step: negative start_pos");
  AXM_CHECK_ARG(idx_dev != nullptr || tok_host < d.vocab_size, -1, "runner_step: token id %lld out of range",
                (long long)tok_host);
  AXM_CHECK_ARG(idx_dev != nullptr || tok_host >= 0 || d.lm_head_format == 0, -1,
                "runner_step: greedy feedback needs the MARLIN lm_head");
  hipStream_t s = (hipStream_t)stream;
  const int rope_pos = start_pos % d.rope_len;
  if (r->mode == AXM_RUNNER_MODE_PERSISTENT) {
    const int rc = r->step_persistent((const int64_t*)idx_dev, tok_host, rope_pos, write_pos, active_len, s);
    if (rc) return rc;
    AXM_LAUNCH_CHECK("runner_step");
    if (logits_out) *logits_out = r->logits;
    return 0;
  }
  r->tok_next_valid = false;
  // The step's token and its embedding row (the graph starts at layer 0).
  const EmbedArgs emb{d.wte, (const f16*)d.wte_sb, d.wte_format, d.d_model, d.vocab_size, r->x};
  hipLaunchKernelGGL(set_params_kernel, dim3(1), dim3(256), 0, s, r->params, (const int64_t*)idx_dev, tok_host,
                     rope_pos, write_pos, active_len, r->argmax_keys, (d.vocab_size + 7) / 8, emb);
  int bucket = 1;
  bool short_splits = false;
  r->split_shape(active_len, &bucket, &short_splits);
  const int key = 2 * bucket + (short_splits ? 1 : 0);
  if (r->mode == AXM_RUNNER_MODE_EAGER) {
    int rc = r->enqueue_step(bucket, short_splits, s);
    if (rc) return rc;
  } else {
    auto it = r->graphs.find(key);
    if (it == r->graphs.end()) {
      hipGraph_t g = nullptr;
      if (hipStreamBeginCapture(r->cap_stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        axm_set_error("runner_step: stream capture failed to start");
        return -5;
      }
      int rc = r->enqueue_step(bucket, short_splits, r->cap_stream);
      hipError_t e = hipStreamEndCapture(r->cap_stream, &g);
      if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
      }
      if (e != hipSuccess) {
        axm_set_error("runner_step: capture failed: %s", hipGetErrorString(e));
        return -5;
      }
      hipGraphExec_t ge = nullptr;
      e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (e != hipSuccess) {
        axm_set_error("runner_step: graph instantiate failed: %s", hipGetErrorString(e));
        return -5;
      }
      it = r->graphs.emplace(key, ge).first;
    }
    if (hipGraphLaunch(it->second, s) != hipSuccess) {
      axm_set_error("runner_step: graph launch failed");
      return -5;
    }
  }
  AXM_LAUNCH_CHECK("runner_step");
  if (logits_out) *logits_out = r->logits;
  return 0;
}

extern "C" int axm_runner_time_kernels(axm_runner_t r, int position, int active_len, int reps, void* stream,
                                       float* us_out) {
  AXM_CHECK_ARG(r && us_out, -1, "runner_time_kernels: null argument");
  const axm_runner_desc& d = r->d;
  AXM_CHECK_ARG(reps >= 1 && reps <= 100000, -1, "runner_time_kernels: reps %d out of [1, 100000]", reps);
  AXM_CHECK_ARG(position >= 0 && position < d.max_seq_len, -1, "runner_time_kernels: position %d out of [0, %d)",
                position, d.max_seq_len);
  AXM_CHECK_ARG(active_len >= 1 && active_len <= d.max_seq_len, -1,
                "runner_time_kernels: active_len %d out of [1, %d]", active_len, d.max_seq_len);
  hipStream_t s = (hipStream_t)stream;
  const EmbedArgs emb{d.wte, (const f16*)d.wte_sb, d.wte_format, d.d_model, d.vocab_size, r->x};
  hipLaunchKernelGGL(set_params_kernel, dim3(1), dim3(256), 0, s, r->params, (const int64_t*)nullptr, (int64_t)0,
                     position % d.rope_len, position, active_len, r->argmax_keys, (d.vocab_size + 7) / 8, emb);
  int bucket = 1;
  bool short_splits = false;
  r->split_shape(active_len, &bucket, &short_splits);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0) (void)hipEventDestroy(e0);
    axm_set_error("runner_time_kernels: event creation failed");
    return -5;
  }
  int rc = 0;
  for (int k = 0; k < 6 && rc == 0; ++k) {
    auto one = [&](int j, hipStream_t cs) -> int {
      const int i = j % d.n_layer;
      switch (k) {
        case 0: return r->enqueue_qkv(i, cs);
        case 1: return r->enqueue_attention(i, bucket, short_splits, cs);
        case 2: return r->enqueue_o(i, bucket, cs);
        case 3: return r->enqueue_gate_up(i, cs);
        case 4: return r->enqueue_down(i, cs);
        default: return r->enqueue_lm_head(cs);
      }
    };
    // The reps launches are captured into a graph (as the step's launches are), so
    // the host's launch rate does not bound short kernels; one untimed replay first.
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    if (hipStreamBeginCapture(r->cap_stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
      axm_set_error("runner_time_kernels: stream capture failed to start");
      rc = -5;
      break;
    }
    for (int j = 0; j < reps && rc == 0; ++j) rc = one(j, r->cap_stream);
    const hipError_t ce = hipStreamEndCapture(r->cap_stream, &g);
    if (rc == 0 && ce != hipSuccess) {
      axm_set_error("runner_time_kernels: capture failed: %s", hipGetErrorString(ce));
      rc = -5;
    }
    if (rc == 0 && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) {
      axm_set_error("runner_time_kernels: graph instantiate failed");
      rc = -5;
    }
    if (g) (void)hipGraphDestroy(g);
    if (rc) break;
    if (hipGraphLaunch(ge, s) != hipSuccess || hipEventRecord(e0, s) != hipSuccess || hipGraphLaunch(ge, s) != hipSuccess ||
        hipEventRecord(e1, s) != hipSuccess) {
      axm_set_error("runner_time_kernels: graph launch failed");
      (void)hipGraphExecDestroy(ge);
      rc = -5;
      break;
    }
    float ms = 0.f;
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) {
      axm_set_error("runner_time_kernels: event timing failed");
      (void)hipGraphExecDestroy(ge);
      rc = -5;
      break;
    }
    us_out[k] = ms * 1000.f / (float)reps;
    (void)hipGraphExecDestroy(ge);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("runner_time_kernels");
  return 0;
}

extern "C" int axm_runner_token_slot(axm_runner_t r, void** tok_out) {
  AXM_CHECK_ARG(r && tok_out, -1, "runner_token_slot: null argument");
  *tok_out = reinterpret_cast<unsigned char*>(r->params) + kTokenOffset;
  return 0;
}

extern "C" int axm_runner_persistent_words(axm_runner_t r, void** words_out, int64_t* n_words) {
  AXM_CHECK_ARG(r && words_out && n_words, -1, "runner_persistent_words: null argument");
  *words_out = r->persist_ok ? (void*)r->p_words : nullptr;
  *n_words = r->persist_ok ? (int64_t)(r->p_words_bytes / sizeof(unsigned long long)) : 0;
  return 0;
}

extern "C" int axm_runner_last_norm(axm_runner_t r, void** norm_out) {
  AXM_CHECK_ARG(r && norm_out, -1, "runner_last_norm: null argument");
  *norm_out = r->norm;
  return 0;
}

static int verify_common(axm_runner_t r, const void* idx_dev, int T, int start_pos, int write_pos, int prefix,
                         const int* depths, const unsigned long long* masks, bool tree, void* stream,
                         void** logits_out) {
  const axm_runner_desc& d = r->d;
  TreeParams tp{};
  for (int t = 0; t < T; ++t) {
    AXM_CHECK_ARG(depths[t] >= 0, -1, "verify: negative tree depth at %d", t);
    tp.pos[t] = (int)(((long long)start_pos + depths[t]) % d.rope_len);
    tp.mask[t] = masks ? masks[t] : 0ull;
  }
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(set_tree_kernel, dim3(1), dim3(kMaxVerify), 0, s, tp, T, r->tree_pos, r->tree_mask);
  r->tok_next_valid = false;
  const int rc = r->enqueue_verify((const int64_t*)idx_dev, T, write_pos, prefix, tree, s);
  if (rc) return rc;
  AXM_LAUNCH_CHECK("runner_verify");
  if (logits_out) *logits_out = r->logits;
  return 0;
}

extern "C" int axm_runner_verify_step(axm_runner_t r, const void* idx_dev, int T, int start_pos, int write_pos,
                                      int active_len, void* stream, void** logits_out) {
  AXM_CHECK_ARG(r && idx_dev, -1, "runner_verify_step: null argument");
  const axm_runner_desc& d = r->d;
  AXM_CHECK_ARG(T >= 1 && T <= d.max_tokens && T <= kMaxVerify, -1,
                "runner_verify_step: T=%d outside [1, %d] (runner max_tokens)", T, d.max_tokens);
  AXM_CHECK_ARG(write_pos >= 0 && write_pos < d.max_seq_len && start_pos >= 0, -1, "runner_verify_step: bad positions");
  AXM_CHECK_ARG(active_len >= 1 && active_len <= d.max_seq_len, -1, "runner_verify_step: bad active_len %d",
                active_len);
  int depths[kMaxVerify];
  unsigned long long masks[kMaxVerify];
  for (int t = 0; t < T; ++t) {
    depths[t] = t;
    masks[t] = (t == 63) ? ~0ull : ((1ull << (t + 1)) - 1ull);
  }
  // A contiguous chain is a tree with causal masks over the prefix [0, write_pos)
  // (mps_kernels.mm:3371-3378); otherwise the ring case attends over all slots.
  const bool chain = write_pos + T <= d.max_seq_len && active_len == write_pos + T;
  return verify_common(r, idx_dev, T, start_pos, write_pos, write_pos, depths, masks, chain, stream, logits_out);
}

extern "C" int axm_runner_verify_tree_step(axm_runner_t r, const void* idx_dev, int T, int start_pos, int write_pos,
                                           int prefix_len, const int* depths_host, const uint64_t* masks_host,
                                           void* stream, void** logits_out) {
  AXM_CHECK_ARG(r && idx_dev && depths_host && masks_host, -1, "runner_verify_tree_step: null argument");
  const axm_runner_desc& d = r->d;
  AXM_CHECK_ARG(T >= 1 && T <= d.max_tokens && T <= kMaxVerify, -1,
                "runner_verify_tree_step: T=%d outside [1, %d] (runner max_tokens)", T, d.max_tokens);
  AXM_CHECK_ARG(write_pos >= 0 && write_pos < d.max_seq_len && start_pos >= 0, -1,
                "runner_verify_tree_step: bad positions");
  AXM_CHECK_ARG(prefix_len >= 0 && prefix_len + T <= d.max_seq_len, -1, "runner_verify_tree_step: bad prefix_len %d",
                prefix_len);
  return verify_common(r, idx_dev, T, start_pos, write_pos, prefix_len, depths_host,
                       (const unsigned long long*)masks_host, true, stream, logits_out);
}

// ---------------------------------------------------------------------------
// Prompt-lookup speculative decoding with greedy acceptance, run natively
// (speculative_decode, mps_kernels.mm:3639-3730; find_candidate_ngram_cpp,
// :368-396).  Each iteration either decodes one token (no n-gram match) or
// verifies [last token, candidates...] in one multi-token pass and accepts the
// matching prefix plus the first corrected / bonus token.
// ---------------------------------------------------------------------------
static std::vector<int64_t> find_candidate_ngram(const std::vector<int64_t>& ids, int64_t n, int64_t max_spec) {
  const int64_t len = (int64_t)ids.size();
  if (len < n + 1) return {};
  const int64_t search_end = len - n;
  for (int64_t i = search_end - 1; i >= 0; --i) {
    bool match = true;
    for (int64_t k = 0; k < n; ++k)
      if (ids[i + k] != ids[search_end + k]) {
        match = false;
        break;
      }
    if (match) {
      const int64_t start = i + n;
      const int64_t end = std::min(start + max_spec, search_end);
      if (start < end) return std::vector<int64_t>(ids.begin() + start, ids.begin() + end);
    }
  }
  return {};
}

extern "C" int axm_runner_speculative_decode(axm_runner_t r, const int64_t* initial_tokens, int n_initial,
                                             int max_new_tokens, int ngram_size, int max_spec_tokens, int start_pos,
                                             int64_t* out_tokens, int out_capacity, int64_t* stats, void* stream) {
  AXM_CHECK_ARG(r && initial_tokens && out_tokens && stats, -1, "speculative_decode: null argument");
  AXM_CHECK_ARG(n_initial >= 1 && max_new_tokens >= 0 && ngram_size >= 1 && max_spec_tokens >= 0 && start_pos >= 0,
                -1, "speculative_decode: bad arguments");
  AXM_CHECK_ARG(out_capacity >= n_initial + max_new_tokens, -1, "speculative_decode: output capacity too small");
  const axm_runner_desc& d = r->d;
  AXM_CHECK_ARG(1 + max_spec_tokens <= d.max_tokens, -1, "speculative_decode: max_spec_tokens + 1 exceeds max_tokens %d",
                d.max_tokens);
  AXM_CHECK_ARG(d.lm_head_format >= 0 && d.lm_head_format <= 2, -1, "speculative_decode: bad lm_head");
  hipStream_t s = (hipStream_t)stream;
  std::vector<int64_t> gen(initial_tokens, initial_tokens + n_initial);
  const int64_t target = (int64_t)n_initial + max_new_tokens;
  int64_t seen = start_pos, calls = 0, drafted = 0, accepted_total = 0;
  int64_t* host = nullptr;  // pinned staging: [0, 64) tokens in, [64, 128) predictions out
  int64_t* dev = nullptr;
  if (hipHostMalloc((void**)&host, 128 * sizeof(int64_t), hipHostMallocDefault) != hipSuccess ||
      hipMalloc((void**)&dev, 128 * sizeof(int64_t)) != hipSuccess) {
    if (host) (void)hipHostFree(host);
    axm_set_error("speculative_decode: staging allocation failed");
    return -4;
  }
  int rc = 0;
  if (hipStreamSynchronize(s) != hipSuccess) rc = -5;
  const auto t0 = std::chrono::high_resolution_clock::now();
  while (rc == 0 && (int64_t)gen.size() < target) {
    const std::vector<int64_t> cand = find_candidate_ngram(gen, ngram_size, max_spec_tokens);
    const int64_t k = (int64_t)cand.size();
    const int T = (int)(1 + k);
    host[0] = gen.back();
    for (int64_t c = 0; c < k; ++c) host[1 + c] = cand[c];
    if (hipMemcpyAsync(dev, host, T * sizeof(int64_t), hipMemcpyHostToDevice, s) != hipSuccess) {
      rc = -5;
      break;
    }
    const int write_pos = (int)(seen % d.max_seq_len);
    const int rope_pos = (int)(seen % d.rope_len);
    if (k == 0) {
      const int active = (int)std::min<int64_t>(seen + 1, d.max_seq_len);
      rc = axm_runner_step(r, dev, 0, rope_pos, write_pos, active, stream, nullptr);
    } else {
      // Chain verification when the T slots do not wrap (prefix = write_pos), else the
      // all-slots branch (mps_kernels.mm:3555-3620).
      int depths[kMaxVerify];
      unsigned long long masks[kMaxVerify];
      for (int t = 0; t < T; ++t) {
        depths[t] = t;
        masks[t] = (t == 63) ? ~0ull : ((1ull << (t + 1)) - 1ull);
      }
      const bool chain = write_pos + T <= d.max_seq_len;
      rc = verify_common(r, dev, T, rope_pos, write_pos, write_pos, depths, masks, chain, stream, nullptr);
    }
    if (rc) break;
    launch_argmax(r->logits, T, d.vocab_size, dev + 64, s);
    if (hipMemcpyAsync(host + 64, dev + 64, T * sizeof(int64_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
      rc = -5;
      break;
    }
    ++calls;
    if (k == 0) {
      gen.push_back(host[64]);
      seen += 1;
      continue;
    }
    drafted += k;
    int64_t acc = 0;
    bool all_matched = true;
    for (int64_t j = 0; j < k; ++j) {
      const int64_t pred = host[64 + j];
      gen.push_back(pred);
      acc += 1;
      if (pred != cand[j] || (int64_t)gen.size() >= target) {
        all_matched = false;
        break;
      }
    }
    if (all_matched && (int64_t)gen.size() < target) {
      gen.push_back(host[64 + k]);
      acc += 1;
    }
    accepted_total += std::max<int64_t>(0, acc - 1);
    seen += acc;
  }
  const double secs = std::chrono::duration<double>(std::chrono::high_resolution_clock::now() - t0).count();
  (void)hipHostFree(host);
  (void)hipFree(dev);
  if (rc) {
    if (rc == -5) axm_set_error("speculative_decode: device error");
    return rc;
  }
  const int n = (int)std::min<int64_t>((int64_t)gen.size(), out_capacity);
  for (int i = 0; i < n; ++i) out_tokens[i] = gen[i];
  stats[0] = n;
  stats[1] = seen;
  stats[2] = calls;
  stats[3] = drafted;
  stats[4] = accepted_total;
  std::memcpy(&stats[5], &secs, sizeof(double));
  return 0;
}
