// Internal host-side launchers shared between the C-ABI wrappers and the
// decode runner.  All pointers are device pointers; every launcher enqueues on
// the given stream and never synchronizes.
#pragma once
#include "axm_common.h"
#include "q4_marlin.h"

// ---- norms / activations (torch-CPU fp16 op semantics) ---------------------
int launch_rmsnorm(const f16* x, const f16* w, f16* y, int rows, int D, float eps, hipStream_t s);
int launch_add_rmsnorm(f16* x, const f16* r, const f16* w, f16* y, int rows, int D, float eps, hipStream_t s);
int launch_swiglu(const f16* gu, f16* y, int rows, int H, hipStream_t s);
// Row-wise argmax of fp16 logits; the lowest index wins ties.
int launch_argmax(const f16* logits, int rows, int V, int64_t* out, hipStream_t s);

// ---- embeddings -------------------------------------------------------------
// tokens: int64 device array of length T (or nullptr with tok_dev pointing to
// one int32 slot written by the runner's parameter kernel).
// Token ids outside [0, V) produce zero rows.
int launch_embed_f16(const f16* table, const int64_t* tokens, const int* tok_dev, f16* out, int T, int D, int V,
                     hipStream_t s);
int launch_embed_q8(const uint8_t* wq, const f16* sb, const int64_t* tokens, const int* tok_dev, f16* out, int T,
                    int D, int V, hipStream_t s);

// ---- Q8_G64 GEMV (affine 8-bit, group 64), optional fused fp16 RMSNorm -------
// xn_out (optional, with ln_w): the RMS-normalized rows [M][K] the GEMV staged, written
// by its first workgroup.
int launch_f16_gemv(const f16* x, const f16* w, const f16* bias, f16* y, int M, int K, int N, const f16* ln_w,
                    float eps, hipStream_t s, f16* xn_out = nullptr);
int launch_f16_gemv_resid(const f16* x, const f16* w, f16* resid, int M, int K, int N, const f16* ln_w, float eps,
                          hipStream_t s);
int launch_f16_gemv_swiglu(const f16* x, const f16* w, f16* y, int M, int K, int N2, const f16* ln_w, float eps,
                           hipStream_t s);
int launch_q8_gemv(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, f16* y, int M, int K, int N,
                   const f16* ln_w, float eps, hipStream_t s, f16* xn_out = nullptr);
// The Q8_G64 / fp16 GEMVs with the residual add fused (resid[m][n] = fp16(resid +
// fp16(acc)), in place) or with SwiGLU over a [W_gate; W_up] matrix of N2 rows (y
// [M][N2 / 2]), each with the rounding of the GEMV's fp16 output followed by an fp16
// residual add / launch_swiglu.
// QKV epilogue of the dense GEMVs (the tile16 Q4_EPI_QKV_ROPE step for one token): the
// fp16 outputs (+ bias) of adjacent rows (2 j, 2 j + 1) of q and k rotated at position
// rope_pos_dev[0] (or rope_pos) + token with freqs [rope_len][hd / 2][(cos, sin)]; q rows
// to q_out [M][q_dim], k / v rows to k_out / v_out + kvh kv_stride_h + (wp % max_seq) hd
// + e with wp = write_pos_dev[0] (or write_pos) + token (the fp16 cache slot, or staging
// rows with kv_stride_h = hd and max_seq = 1).
struct QkvRope {
  int q_dim = 0, kv_dim = 0, head_dim = 0, rope_len = 1;
  const float* freqs = nullptr;
  const int* rope_pos_dev = nullptr;
  int rope_pos = 0;
  const int* write_pos_dev = nullptr;
  int write_pos = 0;
  f16* q_out = nullptr;
  f16* k_out = nullptr;
  f16* v_out = nullptr;
  long kv_stride_h = 0;
  int max_seq = 1;
};
int launch_q8_gemv_qkv(const f16* x, const uint8_t* w, const f16* sb, const f16* bias, int M, int K, int N,
                       const f16* ln_w, float eps, const QkvRope& r, hipStream_t s);
int launch_f16_gemv_qkv(const f16* x, const f16* w, const f16* bias, int M, int K, int N, const f16* ln_w, float eps,
                        const QkvRope& r, hipStream_t s);
int launch_q8_gemv_resid(const f16* x, const uint8_t* w, const f16* sb, f16* resid, int M, int K, int N,
                         const f16* ln_w, float eps, hipStream_t s);
int launch_q8_gemv_swiglu(const f16* x, const uint8_t* w, const f16* sb, f16* y, int M, int K, int N2,
                          const f16* ln_w, float eps, hipStream_t s);

// ---- KV cache ---------------------------------------------------------------
#include "axm.h"  // AXM_KV_* codes

struct KvView {
  void* k;        // fp16 [B][Hkv][S][hd] | u8 [B][Hkv][S][hd] | u8 [B][Hkv][S][hd/2]
  void* v;
  f16* ks;        // scales [B][Hkv][S][hd/64] (quantized caches)
  f16* vs;
  int kv_dtype;
  int B, Hkv, S, hd;
};

// Quantize fp16 k/v rows [T][Hkv*hd] and write them at slots (write_pos+t) % S
// (batch 0).  write_pos_dev overrides write_pos when non-null.
int launch_kv_write(const KvView& kv, const f16* k_rows, const f16* v_rows, int ld_rows, int T, int write_pos,
                    const int* write_pos_dev, hipStream_t s);
// RoPE of the query and key rows of qkv [T][Hq hd + 2 Hkv hd] (token t at
// pos_dev[t], freqs as the runner holds them) with the queries into q
// [T][Hq hd] and the keys / values written at slots (write_pos + t) % S, in one
// launch; head size 128 only (-2 otherwise).
int launch_rope_kv_write(const KvView& kv, const f16* qkv, int Hq, int T, const float* freqs, const int* pos_dev,
                         f16* q, int write_pos, hipStream_t s);
// The same, with the qkv rows summed from the K-split partials of the multi-token
// QKV GEMM (part [split][token, stride tok_stride][part_cols] fp32) and rounded as
// the GEMM's store epilogue with the bias would (replaces that split reduce).
int launch_reduce_rope_kv_write(const KvView& kv, const float* part, int n_splits, int tok_stride, int part_cols,
                                const f16* bias, int Hq, int T, const float* freqs, const int* pos_dev, f16* q,
                                int write_pos, hipStream_t s);

// Split-KV decode attention over slots [0, active_len) of every batch entry.
// q: [B][Hq][hd] fp16, out: [B][Hq][hd] fp16.  ws: workspace of
// attn_workspace_bytes(); active_len_dev overrides active_len when non-null.
size_t attn_workspace_bytes(int B, int Hq, int hd, int n_splits);
int attn_choose_splits(int B, int Hkv, int active_len);
// Split count of launch_flash_decode for the attention kernel it picks (matrix-core
// form for 2-16 query heads per KV head and head size 64 / 128).
int attn_flash_splits(int B, int Hq, int Hkv, int hd, int kv_dtype, int active_len);
int launch_flash_decode(const f16* q, const KvView& kv, f16* out, int Hq, int active_len, const int* active_len_dev,
                        int n_splits, float* ws, hipStream_t s);

// The same decode attention with 2..kAttnMaxParts splits whose partials are
// left for the consumer to merge (no reduce launch): parts_o [n_splits][B*Hq][hd]
// holds each split's o / l in fp16, parts_ml [n_splits][B*Hq] its (max, sum);
// the row is sum_s w_s o_s / sum_s w_s with w_s = l_s 2^(m_s - max_s m_s).
constexpr int kAttnMaxParts = 8;
int attn_parts_splits(int B, int Hkv, int active_len);
size_t attn_parts_bytes(int B, int Hq, int hd);  // parts_o + parts_ml for kAttnMaxParts splits
// short_splits: at most 64 keys per split (the launch shape for such splits).
int launch_flash_decode_parts(const f16* q, const KvView& kv, int Hq, int active_len, const int* active_len_dev,
                              int n_splits, f16* parts_o, f32x2* parts_ml, bool short_splits, hipStream_t s);

// Tree / multi-token verification attention (batch 0): T query tokens; prefix
// slots [0, prefix_len) always visible; tree node j lives at slot
// (write_pos + j) % S and is visible to node u iff bit j of mask[u] is set.
int launch_tree_attention(const f16* q, const KvView& kv, f16* out, int Hq, int T, int prefix_len, int write_pos,
                          const uint64_t* masks_dev, int n_splits, float* ws, hipStream_t s);
size_t tree_workspace_bytes(int T, int Hq, int hd, int n_splits);
// Key splits for tree attention (about two 64-row workgroups per CU, >= 64 keys each).
int tree_choose_splits(int T, int Hq, int Hkv, int n_keys);
