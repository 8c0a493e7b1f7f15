// Host interface of the persistent decode-step kernel (step_kernel.hip): one
// cooperative launch per token runs every layer of the batch-1 decode step.
#pragma once
#include "axm_common.h"
#include "step_plan.h"

// Per-layer device pointers (tile16 weights, norms, bias, fp16 KV cache views).
struct StepLayer {
  const void* qkv_w;
  const void* qkv_sb;
  const void* o_w;
  const void* o_sb;
  const void* gu_w;
  const void* gu_sb;
  const void* dn_w;
  const void* dn_sb;
  const f16* ln1;
  const f16* ln2;
  const f16* qkv_bias;  // may be null
  f16* kc;              // fp16 [Hkv][S][hd] (batch-0 view)
  f16* vc;
};

struct StepArgs {
  sp::Shape sh;
  const StepLayer* layers;  // device array [L]
  const void* lm_w;         // tile16 lm_head
  const void* lm_sb;
  const f16* lnf;
  const float* freqs;  // [rope_len][hd/2][2]
  int rope_len;
  int wte_fmt;  // 0 fp16 table [V][D], 1 Q8_G64 codes [V][D] + (scale, bias) [V][D/64]
  const void* wte;
  const f16* wte_sb;
  float eps, scale_log2;
  // per step
  const int64_t* idx_dev;   // token from device memory when non-null
  long long tok_host;       // else this token when >= 0
  const int64_t* tok_prev;  // else the greedy token the previous launch left here
  int rope_pos, write_pos, active_len, n_splits;
  unsigned tag0;  // tag of this launch's first phase
  int spin_limit;
  unsigned long long* words;  // cross-workgroup words (sp::words_layout)
  f16* logits;                // [V]
  f16* norm_out;              // [D] final normed hidden state
  unsigned long long* argmax_keys;  // [ceil(V/16)] per lm_head tile
  int64_t* tok_used;          // token consumed by this step
  int64_t* tok_next;          // greedy argmax of this step's logits
  int* err;                   // set when a wait on another workgroup gave up
};

// 0 when the kernel runs co-resident with one workgroup on each of the device's
// CUs for this shape (sh.G is set to the CU count); sets the LDS size.
int step_check(sp::Shape& sh, size_t* smem_out);
int step_launch(const StepArgs& a, size_t smem, hipStream_t s);
