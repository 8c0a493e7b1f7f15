// Internal interface of the tile16 (MFMA) MARLIN Q4 GEMV used by the decode runner.
#pragma once
#include "axm_common.h"
#include "q4_marlin.h"  // Q4_EPI_* epilogue codes

struct T16Args {
  const f16* x;        // [M][ldx] activations
  int ldx;
  const u32x4* w16;    // [N16][KB][64] x 16 B
  const u32x2* sb16;   // [N16][KB][16] x 8 B (two groups of (scale, bias)); g128: x 4 B (one)
  int g128;            // one (scale, bias) per 128 columns (group-128 packs)
  int K, KB, N;        // N = valid output rows
  int N_rows_alloc;    // rows the w16 / sb16 arrays were packed for (2 H for gate/up)
  size_t w16_bytes, sb16_bytes;  // set by t16_gemv_launch (buffer bounds)
  int n_units;         // tile16 units (gate tiles for SWIGLU)
  f16* y;
  int ldy;
  const f16* bias;
  const f16* ln_w;     // optional fused RMSNorm (torch-CPU fp16 semantics)
  float eps;
  f16* x_norm_out;     // optional export of the normalized activations [M][K]
  f16* resid;          // Q4_EPI_RESID
  int ldr;
  int pair_offset;     // Q4_EPI_SWIGLU: tile16 distance from a gate tile to its up tile
  int q_dim, kv_dim, head_dim;  // Q4_EPI_QKV_ROPE
  const float* freqs;
  int rope_len;
  int rope_pos;
  const int* rope_pos_dev;
  int write_pos;
  const int* write_pos_dev;
  f16* k_out;
  f16* v_out;
  long kv_stride_h;
  int max_seq;
  unsigned long long* argmax_keys;  // Q4_EPI_STORE, M == 1: per-unit ordered (logit, index) key
  // Q4_EPI_RESID, M == 1, K <= kTile16PartsMaxK: when x_parts is set the
  // activations are merged from decode-attention split partials instead of read
  // from x: x[h hd + e] = sum_s w_s o_s[h hd + e] / sum_s w_s with
  // w_s = l_s 2^(m_s - max_s m_s), (m_s, l_s) = x_ml[s][h], rounded once to fp16.
  const f16* x_parts;  // [n_parts][K] fp16
  const f32x2* x_ml;   // [n_parts][K / parts_hd]
  int n_parts;         // 2..kTile16MaxParts
  int parts_hd;        // elements per head (a multiple of 8)
  int split;           // waves per unit (set by t16_gemv_launch)
  uint32_t unpack[4];  // nibble masks and fp16 magic exponents (set by t16_gemv_launch)
  // Multi-token GEMM (t16_gemm_launch): tokens, chunks of K per grid.y split,
  // fp32 partial tiles [splits][16][part_cols] when K is split across workgroups.
  int M_tokens;
  int kb_per_split;
  float* part_ws;
  int part_cols;
  // Q4_EPI_RESID: when post_ln_w is set, the updated residual rows are also
  // RMS-normalized (weight post_ln_w, eps) into post_norm_out [M][N] (the input
  // of the next normed GEMM), fused into the split reduce when K is split.
  const f16* post_ln_w;
  f16* post_norm_out;
  // Multi-token GEMM, store epilogue: when set (a host array of 3), a K-split launch
  // leaves its partials in part_ws unreduced and reports {splits, token stride,
  // part_cols} here for a consumer that reduces them itself; {0, 0, 0} when the
  // GEMM was not split and stored its rows.
  int* split_info;
};

// Largest K (activation length) the tile16 GEMV stages.
constexpr int kTile16MaxK = 16384;
// Limits of the split-partial activation source (one 8-element vector per thread).
constexpr int kTile16PartsMaxK = 4096;
constexpr int kTile16MaxParts = 8;

// LDS bytes of a GEMV workgroup of `waves` waves (before per-wave scale staging).
size_t t16_smem_bytes(int M, int NT, int K, int waves);
void t16_prepare_attributes();
// Picks split / grid (a.split is overwritten); M in [1, 4].
int t16_gemv_launch(T16Args a, int M, int epi, hipStream_t s);
// g128: sb_marlin holds one (scale, bias) per 128 columns ([N/8][K/128][8]).
int t16_repack(const void* w_marlin, const void* sb_marlin, int N, int K, void* w16, void* sb16, hipStream_t s,
               int g128);
// Multi-token GEMM over the same tile16 weights for M in [1, 64] tokens (one to
// four 16-row MFMA A tiles): every weight chunk is streamed once for all M
// tokens.  Activations must be normalized already (a.ln_w == nullptr); epi is
// Q4_EPI_STORE (+ bias), Q4_EPI_RESID or Q4_EPI_SWIGLU.  K is split across at
// most kTile16GemmMaxSplits workgroups; with more than one split the partial
// tiles go to ws (t16_gemm_ws_bytes, enough for any M) and a reduce launch
// applies the epilogue.
constexpr int kTile16GemmMaxTokens = 64;
constexpr int kTile16GemmMaxSplits = 16;
size_t t16_gemm_ws_bytes(int K, int n_units, int NT);
int t16_gemm_launch(T16Args a, int M, int epi, float* ws, size_t ws_bytes, hipStream_t s);
size_t t16_weight_bytes(int N, int K);
size_t t16_sb_bytes(int N, int K, int g128);
