// Internal interface of the MARLIN Q4 GEMV family (shared by the standalone
// C-ABI entry points and the decode runner).
#pragma once
#include "axm_common.h"

enum {
  Q4_EPI_STORE = 0,     // y = fp16(acc) (+ bias, fp16 add)
  Q4_EPI_RESID = 1,     // resid += fp16(acc)          (fp16 add, in place)
  Q4_EPI_SWIGLU = 2,    // y = silu(fp16(g)) * fp16(u)  over the gate/up tile pair
  Q4_EPI_QKV_ROPE = 3,  // bias + RoPE on q/k rows, q -> y, k/v -> cache slots
};

struct Q4GemvArgs {
  const f16* x;        // [M][ldx] activations
  int ldx;
  const u32x4* w;      // reference MARLIN codes, [n_tiles][KG][16] x 16 B
  const u32x4* sb;     // [n_tiles][KG][2] x 16 B (8 rows of (scale, bias))
  int K, KG, N;        // N = valid output rows (tiles beyond are padding)
  int n_units;         // work units: tiles, or gate tiles for SWIGLU
  f16* y;              // [M][ldy]
  int ldy;
  const f16* bias;     // optional per-row bias (fp16)
  // Optional fused RMSNorm prologue (torch-CPU fp16 semantics).
  const f16* ln_w;
  float eps;
  f16* x_norm_out;     // optional export of the normalized activations [M][K]
  // Q4_EPI_RESID
  f16* resid;
  int ldr;
  // Q4_EPI_SWIGLU: index distance between a gate tile and its up tile.
  int pair_offset;
  // Q4_EPI_QKV_ROPE
  int q_dim, kv_dim, head_dim;
  const float* freqs;  // [rope_len][head_dim/2][2] (cos, sin)
  int rope_len;
  int rope_pos;        // token 0 position (used when rope_pos_dev == nullptr)
  const int* rope_pos_dev;
  int write_pos;
  const int* write_pos_dev;
  f16* k_out;          // destination of k rows: [kv_head][max_seq][head_dim]
  f16* v_out;
  long kv_stride_h;    // elements between kv heads (max_seq * head_dim)
  int max_seq;
  int split;           // waves per unit (set by q4m_gemv_launch)
  // Q4_EPI_STORE, M == 1: optional per-unit argmax of the fp16 outputs as an
  // ordered 64-bit key (value order, then lowest index); keys[unit] is written
  // by every launch, so the array needs no reset.
  unsigned long long* argmax_keys;
};

size_t q4m_gemv_smem_bytes(int M, int NT, int K);
// Picks the split-K factor and grid (a.split is overwritten).
int q4m_gemv_launch(Q4GemvArgs a, int M, int epi, hipStream_t s);
void q4m_prepare_attributes();
