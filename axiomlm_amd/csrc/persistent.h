// Internal interface of the persistent decode-step kernel (one cooperative
// launch per token; see persistent.hip).
#pragma once
#include "axm_common.h"

// Per-layer device pointers (tile16 weights, norms, bias, KV cache views).
struct PLayer {
  const u32x4* qkv_w;
  const u32x2* qkv_sb;
  const u32x4* o_w;
  const u32x2* o_sb;
  const u32x4* gu_w;
  const u32x2* gu_sb;
  const u32x4* dn_w;
  const u32x2* dn_sb;
  const f16* ln1;
  const f16* ln2;
  const f16* qkv_bias;  // may be null
  f16* kc;              // fp16 [Hkv][S][hd] (batch-0 view)
  f16* vc;
};

struct PArgs {
  const PLayer* layers;  // device array [L]
  int L, D, H, Hq, Hkv, hd, V, S, rope_len;
  float eps, scale_log2;
  const float* freqs;  // [rope_len][hd/2][2]
  const f16* lnf;
  const u32x4* lm_w;  // tile16 lm_head
  const u32x2* lm_sb;
  int wte_fmt;  // 0 fp16 table, 1 Q8_G64
  const void* wte;
  const f16* wte_sb;
  // per step
  const int64_t* idx_dev;  // token from device memory when non-null
  long long tok_host;      // else host token when >= 0, else *tok_next (greedy feedback)
  int rope_pos, write_pos, active_len, n_splits;
  unsigned long long bar_base;    // grid barriers completed by earlier launches
  unsigned long long merge_base;  // split arrivals per head recorded by earlier launches
  // activations and state (runner-owned)
  f16* x;
  f16* q;
  f16* attn;
  f16* h;
  f16* logits;
  f16* norm_out;
  float* ws;                      // split partials [Hq][n_splits][2 + hd]
  unsigned long long* keys;       // per lm_head unit argmax key
  int64_t* tok_used;              // token consumed by this step
  int64_t* tok_next;              // greedy argmax of this step's logits
  unsigned long long* bar;        // barrier words (see persistent.hip)
  unsigned long long* head_cnt;   // [Hq] split arrivals
  int* err;                       // set when a bounded wait expires
};

// Grid barriers one launch performs (the host advances bar_base by this).
inline int persist_barriers_per_step(int n_layer) { return 5 * n_layer + 1; }
// Bytes of the barrier word area the runner allocates (zeroed once).
constexpr size_t kPersistBarBytes = 16 * 256;
// Returns 0 when the kernel can run co-resident on every CU with these sizes.
int persist_check(int D, int H, int Hq, int hd, int V, int* grid_out, size_t* smem_out);
int persist_launch(const PArgs& a, int grid, size_t smem, hipStream_t s);
int persist_choose_splits(int grid, int Hq, int hd, int active_len);
