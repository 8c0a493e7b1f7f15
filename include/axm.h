/*
 * axm.h -- C ABI of libaxm.so, the MI355X (gfx950) implementation of the
 * AxiomLM quantized decode step.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream); all
 *     calls are asynchronous with respect to the host and never synchronize.
 *   - Return value 0 = success, negative = error; axm_last_error() returns the
 *     message of the last failure on the calling thread.
 *   - Activations and KV values are fp16 (IEEE binary16), accumulation fp32.
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the AxiomLM source tree).
 */
#ifndef AXM_H_
#define AXM_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- library ------------------------------------------------------------ */
const char* axm_last_error(void);
int axm_version(void);

/* ---- MARLIN Q4 (group 64, fp16 scale + bias) ------------------------------
 * w_marlin: int32 [ceil(N/8)][K/64][32][2], sb_marlin: fp16 [ceil(N/8)][K/64][8][2]
 * x: fp16 [M][K], y: fp16 [M][N], bias: fp16 [N] or NULL.
 * Replaces qmv_q4_marlin_mps / qmm_q4_marlin_mps
 *   (axiomlm/kernels/mps_kernels.mm:1272-1396, bound in the pybind module at
 *    :4302-4641; Python entry axiomlm/kernels/quant.py:637-684). */
int axm_qmv_q4_marlin(const void* x, const void* w_marlin, const void* sb_marlin, const void* bias, void* y, int M,
                      int K, int N, void* stream);
/* Fused RMSNorm (ln_w fp16 [K], or NULL for none) -> gate/up GEMV over the packed
 * [W_gate; W_up] rows -> SwiGLU: y fp16 [M][H] = silu(g) * u, M <= 4.  The MLP
 * input half of a decoder layer (transformer.py:1178-1189; runner dispatches
 * mps_kernels.mm:3249-3253 fused into one launch). */
int axm_qmv_q4_marlin_swiglu(const void* x, const void* ln_w, float eps, const void* gu_w, const void* gu_sb,
                             void* y, int M, int K, int H, void* stream);
/* Matrix-core ("tile16") copy of a MARLIN matrix, the layout the decode runner
 * streams: w16 u32 [ceil(N/16)][ceil(K/128)][64][4], sb16 [ceil(N/16)][ceil(K/128)][16][2]
 * (scale, bias).  The re-tiling is bit-exact (same codes, scales and biases).
 * axm_tile16_bytes(N, K, 0) / (N, K, 1) give the two buffer sizes; (N, K, 2) the
 * scale buffer of a group-128 copy (one (scale, bias) per row and kb: [N16][KB][16]). */
size_t axm_tile16_bytes(int N, int K, int which);
int axm_repack_q4_marlin_tile16(const void* w_marlin, const void* sb_marlin, int N, int K, void* w16, void* sb16,
                                void* stream);
/* Group-128 variant (no counterpart in the reference, whose MARLIN groups are 64
 * columns): the same 64-column code layout with one (scale, bias) per 128 columns,
 * sb128 fp16 [N/8][K/128][8][2] (0.53125 bytes per weight).  RTN packer (the rule of
 * quant.py:483-494 over 128 columns), fp16 dequantization, and the re-tiling. */
int axm_pack_q4_marlin_rtn_g128(const void* w, int src_is_fp16, int N, int K, void* w_marlin, void* sb128,
                                void* stream);
int axm_dequantize_q4_marlin_g128(const void* w_marlin, const void* sb128, void* out, int K, int N, void* stream);
int axm_repack_q4_marlin_g128_tile16(const void* w_marlin, const void* sb128, int N, int K, void* w16, void* sb16,
                                     void* stream);
/* y = x W^T (+ bias) on the tile16 copy, MFMA 16x16x32 f16 with fp32 accumulation.
 * group_size: 64, or 128 for a group-128 copy (K % 128 == 0), on every tile16 entry. */
int axm_qmv_q4_tile16(const void* x, const void* w16, const void* sb16, const void* bias, void* y, int M, int K,
                      int N, int group_size, void* stream);
/* axm_qmv_q4_marlin_swiglu on the tile16 copy of the packed [W_gate; W_up] (2 H rows,
 * H % 16 == 0): the runner's MLP-input launch (transformer.py:1178-1189). */
int axm_qmv_q4_tile16_swiglu(const void* x, const void* ln_w, float eps, const void* gu16, const void* gusb16,
                             void* y, int M, int K, int H, int group_size, void* stream);
/* Multi-token GEMM on the tile16 copy: y[M][N] = x @ W^T (+ bias) with every weight
 * chunk streamed once per 64 tokens (the M > 8 path of qmm_q4_marlin_mps: kernels
 * qmm_q4_marlin_m8_apple_kernel / qmm_q4_marlin_apple_kernel, metal_kernels.metal:
 * 2268-2684; dispatch mps_kernels.mm:1272-1312; CPU form quant.py:664-684).  Up to
 * 16 tokens per launch keep the GEMV's arithmetic; 17-64 tokens dequantize each
 * weight to fp16 q * scale + bias before the MFMAs (as the reference's kernel does).
 * K is split across workgroups; `workspace` holds the fp32 partial tiles
 * (axm_qmm_q4_tile16_workspace_bytes: enough for any M, 0 when no split is used). */
size_t axm_qmm_q4_tile16_workspace_bytes(int K, int N, int swiglu);
int axm_qmm_q4_tile16(const void* x, const void* w16, const void* sb16, const void* bias, void* y, int M, int K,
                      int N, int group_size, void* workspace, size_t workspace_bytes, void* stream);
/* silu(g) * u over the tile16 [W_gate; W_up] copy for M tokens whose activations are
 * already RMS-normalized (the multi-token MLP input, transformer.py:1178-1189). */
int axm_qmm_q4_tile16_swiglu(const void* x_normed, const void* gu16, const void* gusb16, void* y, int M, int K,
                             int H, int group_size, void* workspace, size_t workspace_bytes, void* stream);
/* Row-major fp16 [N][K] dequantization (axiomlm/kernels/quant.py:597-634). */
int axm_dequantize_q4_marlin(const void* w_marlin, const void* sb_marlin, void* out, int K, int N, void* stream);
/* Round-to-nearest packer, clip_search=False (axiomlm/kernels/quant.py:447-494, 573-593).
 * w: fp16 (src_is_fp16=1) or fp32 [N][K]. */
int axm_pack_q4_marlin_rtn(const void* w, int src_is_fp16, int N, int K, void* w_marlin, void* sb_marlin,
                           void* stream);
/* Importance-weighted MSE clip-search packer, clip_search=True (quant.py:495-571).
 * col_importance: fp32 [K] or NULL; alphas: fp32 [n_alpha] (device) shrink grid. */
int axm_pack_q4_marlin_mse(const void* w, int src_is_fp16, int N, int K, const float* col_importance,
                           const float* alphas, int n_alpha, void* w_marlin, void* sb_marlin, void* stream);

/* ---- Q8_G64 ------------------------------------------------------------- *
 * w: uint8 [N][K] (the int32 [N][K/4] little-endian view), sb: fp16 [N][K/64][2].
 * Replaces qmv_q8_g64_mps / qmm_q8_g64_mps (mps_kernels.mm:2122-2170; quant.py:201-233). */
int axm_qmv_q8_g64(const void* x, const void* w_packed, const void* sb, const void* bias, void* y, int M, int K,
                   int N, void* stream);
/* Q8_G64 packer (quant.py:72-111): w fp16/fp32 [N][K] -> uint8 [N][K] + sb fp16 [N][K/64][2]. */
int axm_pack_q8_g64(const void* w, int src_is_fp16, int N, int K, void* packed_u8, void* sb, void* stream);
/* Token-row gather + dequantization, dequant_q8_rows (quant.py:132-163) /
 * embed_q8_g64_gather_half_kernel (metal_kernels.metal:357-391). tokens: int64 [T]; ids outside
 * [0, V) give zero rows. */
int axm_embed_q8_g64(const void* w_packed, const void* sb, const void* tokens_i64, void* out, int T, int D, int V,
                     void* stream);

/* ---- BitNet 1.58 ternary and reference "Q2_K" (affine 2-bit), group 64 ----
 * codes: uint8 [N][K/4], element 4b+j at bits 2j.  Ternary code 1 -> +1, 2 -> -1,
 * 0 -> 0 with fp16 scales [N][K/64]; Q2 codes q in [0,3] with sb fp16 [N][K/64][2].
 * Packers: pack_linear_ternary (quant.py:236-276), pack_linear_q2_k (quant.py:339-378). */
int axm_pack_ternary(const void* w, int src_is_fp16, int N, int K, void* packed_u8, void* scales, void* stream);
int axm_pack_q2_k(const void* w, int src_is_fp16, int N, int K, void* packed_u8, void* sb, void* stream);
/* y = x W^T (+ bias) on the packed 2-bit rows, x fp16 [M][K], y fp16 [M][N], fp32
 * accumulation.  Replaces qmv/qmm_ternary_mps (qmv/qmm_ternary_half_kernel,
 * metal_kernels.metal:3990-4160; Python quant.py:298-336) and qmv/qmm_q2_k_mps
 * (metal_kernels.metal:4167-4334; quant.py:406-444).  Exact code products: one or two
 * tokens on v_dot2_f32_f16, three to sixteen per launch on MFMA. */
int axm_qmv_ternary(const void* x, const void* w_packed, const void* scales, const void* bias, void* y, int M, int K,
                    int N, void* stream);
int axm_qmv_q2_k(const void* x, const void* w_packed, const void* scales_biases, const void* bias, void* y, int M,
                 int K, int N, void* stream);

/* ---- GGUF Q2_K super-blocks (ggml block_q2_K, QK_K = 256) ----------------
 * No counterpart in the reference's kernels (its "Q2_K" is the affine group-64
 * format above); this is the GGUF layout the C4 configuration names, read as
 * stored: blocks uint8 [N][K/256][84] = scales[16] (4-bit scale | 4-bit min << 4
 * per 16 elements), qs[64] (element 128h + 32j + l at bits 2j of qs[32h + l]),
 * d, dmin fp16; w = d * (sc & 15) * q - dmin * (sc >> 4).  K % 256 == 0.
 * Packer: round to nearest (per-sub-block min/max, 4-bit scale and min codes
 * against fp16 super-block maxima), not ggml's iterative scale search. */
int axm_pack_q2_k_gguf(const void* w, int src_is_fp16, int N, int K, void* blocks, void* stream);
/* blocks -> fp16 [N][K], fp32 arithmetic, one rounding. */
int axm_dequantize_q2_k_gguf(const void* blocks, int N, int K, void* out, void* stream);
/* y = x W^T (+ bias), x fp16 [M][K], y fp16 [M][N], fp32 accumulation; K <= 16384.  Exact code
 * products: one token on v_dot2_f32_f16, two to sixteen per launch on MFMA. */
int axm_qmv_q2_k_gguf(const void* x, const void* blocks, const void* bias, void* y, int M, int K, int N,
                      void* stream);

/* ---- norms / activations / argmax ---------------------------------------- */
/* rmsnorm_infer_mps (mps_kernels.mm:247-266; math of axiomlm/models/modules.py:41-43). */
int axm_rmsnorm(const void* x, const void* w, void* y, int rows, int D, float eps, void* stream);
/* add_rmsnorm_infer_mps: x += r; y = rmsnorm(x) (mps_kernels.mm:405-425). */
int axm_add_rmsnorm(void* x, const void* r, const void* w, void* y, int rows, int D, float eps, void* stream);
/* swiglu_gate_up_mps: y = silu(g) * u over [g || u] rows (mps_kernels.mm:434-450). */
int axm_swiglu_gate_up(const void* gu, void* y, int rows, int H, void* stream);
/* argmax_last_token_mps / argmax_multi (mps_kernels.mm:292-366): lowest index wins ties. */
int axm_argmax(const void* logits, int rows, int V, void* out_i64, void* stream);

/* ---- KV cache and attention ---------------------------------------------- *
 * kv_dtype: 0 = fp16, 1 = FP8 E4M3FN, 2 = INT4 (symmetric, group 64).
 * Cache layouts: fp16/fp8 [B][Hkv][S][hd], int4 [B][Hkv][S][hd/2], scales fp16 [B][Hkv][S][hd/64]
 * (axiomlm/engine/paged_cache.py:158-198). */
#define AXM_KV_FP16 0
#define AXM_KV_FP8 1
#define AXM_KV_INT4 2

/* Quantize (per 64-element group) and store T rows of k and v at slots
 * (write_pos + t) % S of batch 0.  Replaces the cache write of
 * rope_kv_cache_write{,_fp8,_int4}_mps (mps_kernels.mm:589-681, 817-929) with the
 * CPU quantizer semantics of quantize_kv_fp8 / quantize_kv_int4 (quant.py:692-807). */
/* Tree-path compaction after tree verification: in every row block of the cache
 * (n_blocks = L * 2 * B * Hkv blocks of max_seq_len slots of slot_bytes bytes, plus
 * optional fp16 scales of scale_halves per slot), slot (write_pos + a[m]) % S moves
 * to (write_pos + m) % S for m < n_accepted (<= 64; accepted_host is a host array).
 * Replaces compact_tree_kv{,_quant}_mps (compact_tree_kv_*_kernel,
 * metal_kernels.metal:3145-3179, :3875-3978) behind StaticKVCache.compact_tree_path
 * (axiomlm/engine/paged_cache.py:376-462). */
int axm_compact_tree_kv(void* cache, void* scales, int n_blocks, int max_seq_len, int slot_bytes, int scale_halves,
                        int write_pos, const int* accepted_host, int n_accepted, void* stream);
int axm_kv_cache_write(const void* k_rows, const void* v_rows, int ld_rows, int T, void* k_cache, void* v_cache,
                       void* k_scales, void* v_scales, int kv_dtype, int n_kv_head, int head_dim, int max_seq_len,
                       int write_pos, void* stream);

/* KV dequantization: rows x head_dim codes (fp8: u8 [rows][hd], int4: u8
 * [rows][hd/2]) with fp16 scales [rows][hd/64] -> fp16 out [rows][hd].
 * Replaces dequantize_kv_cache_{fp8,int4}_mps (mps_kernels.mm:930-1004) and the
 * Python dequantize_kv_fp8 / dequantize_kv_int4 (quant.py:727-852). */
int axm_dequantize_kv(const void* codes, const void* scales, int kv_dtype, long rows, int head_dim, void* out,
                      void* stream);

/* Fused QKV bias + RoPE + KV-cache write for T <= 64 tokens, in place on
 * qkv fp16 [T][q_dim + 2 kv_dim]: the (bias-added) query part is rotated in
 * place; token t's rotated key and its value are stored (quantized for fp8 /
 * int4 caches, 64-element groups) at slot (write_pos + t) % max_seq_len of batch
 * 0; token t is rotated at (start_pos + depth[t]) % rope_len with depth[t] =
 * depths_host[t] (tree variant) or t when depths_host is NULL.  freqs fp32
 * [rope_len][head_dim/2][2]; qkv_bias fp16 [q_dim + 2 kv_dim] or NULL.  The key
 * and value parts of qkv are left as they were.
 * Replaces rope_kv_cache_write{,_fp8,_int4}_mps (mps_kernels.mm:788-929),
 * rope_tree_kv_cache_write_mps (:3961-3998), rope_tree_kv_write_{fp8,int4}_mps
 * (:1005-1140); Python entry rope_kv_cache_write_quantized (quant.py:896-1008). */
int axm_rope_kv_cache_write(void* qkv, int T, const void* freqs, int rope_len, int start_pos, const int* depths_host,
                            const void* qkv_bias, void* k_cache, void* v_cache, void* k_scales, void* v_scales,
                            int kv_dtype, int q_dim, int kv_dim, int head_dim, int max_seq_len, int write_pos,
                            void* stream);

/* Split-KV GQA decode attention: q fp16 [B][Hq][hd] -> out fp16 [B][Hq][hd] over
 * slots [0, active_len).  num_splits <= 0 picks a split count
 * (axm_attention_num_splits).  workspace >= axm_attention_workspace_bytes().
 * Replaces gqa_flash_decode{,_fp8,_int4}_mps (mps_kernels.mm:1399-1506, 1672-1906,
 * 2040-2120; Python entry axiomlm/kernels/ops.py:552-654). */
int axm_attention_num_splits(int B, int n_head, int n_kv_head, int head_dim, int kv_dtype, int active_len);
size_t axm_attention_workspace_bytes(int B, int n_query_rows_per_batch, int head_dim, int n_splits);
int axm_gqa_flash_decode(const void* q, const void* k_cache, const void* v_cache, const void* k_scales,
                         const void* v_scales, int kv_dtype, void* out, int B, int n_head, int n_kv_head,
                         int head_dim, int max_seq_len, int active_len, int num_splits, void* workspace,
                         size_t workspace_bytes, void* stream);

/* No-allocation variant of axm_gqa_flash_decode.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split-KV partials go to a fixed device array inside the library (one per GPU,
 * AXM_NOALLOC_SCRATCH_BYTES, held until the process ends) instead of a caller
 * workspace; a call whose partials would exceed it returns -1 with an error
 * message, and the function itself calls no hipMalloc / hipFree.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (other streams,
 * other threads) race.  Same arguments, splits and results as axm_gqa_flash_decode. */
#define AXM_NOALLOC_SCRATCH_BYTES (16u << 20)
int axm_gqa_flash_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, const void* k_scales,
                                 const void* v_scales, int kv_dtype, void* out, int B, int n_head, int n_kv_head,
                                 int head_dim, int max_seq_len, int active_len, int num_splits, void* stream);

/* Key splits the tree-verification attention picks for num_splits <= 0 (T nodes,
 * n_keys = prefix_len + T); the split heuristic of gqa_tree_verify_*_mps
 * (mps_kernels.mm:1508-1631) re-derived for 64-row matrix-core workgroups. */
int axm_tree_attention_num_splits(int T, int n_head, int n_kv_head, int n_keys);
/* Bitmask tree-verification attention (batch 0): q fp16 [T][Hq][hd], T <= 64,
 * masks uint64 [T] (device) ancestor bitmasks.  Prefix slots [0, prefix_len)
 * are visible to every node; node j lives at slot (write_pos + j) % S.  Q K^T and
 * P V run as v_mfma_f32_16x16x32_f16 tiles (hd 64 / 128).
 * workspace >= axm_attention_workspace_bytes(T, Hq, hd, num_splits).
 * Replaces gqa_tree_verify{,_fp8,_int4}_mps (mps_kernels.mm:1508-1631, 1908-2038,
 * 4111-4249; Python entry axiomlm/kernels/ops.py:657-797); masks are widened
 * from uint32 (T <= 32) to uint64 (T <= 64). */
int axm_gqa_tree_verify(const void* q, const void* k_cache, const void* v_cache, const void* k_scales,
                        const void* v_scales, int kv_dtype, void* out, int T, int n_head, int n_kv_head,
                        int head_dim, int max_seq_len, int prefix_len, int write_pos, const void* masks_u64_dev,
                        int num_splits, void* workspace, size_t workspace_bytes, void* stream);

/* ---- whole-model decode runner ------------------------------------------- *
 * Replaces MPSQuantizedDecodeRunner (QuantizedDecodeGraphState,
 * mps_kernels.mm:2982-3738, bound at :4373-4461).  The runner keeps pointers to
 * the caller's packed weights and KV cache (it never frees them), owns its
 * activation buffers, and replays the whole step as one hipGraph. */
typedef struct axm_runner_desc {
  int n_layer, n_head, n_kv_head, head_dim, d_model, hidden_dim, vocab_size;
  int max_seq_len; /* KV slots S */
  int rope_len;    /* rows of freqs */
  float eps;
  int kv_dtype;       /* AXM_KV_* */
  int wte_format;     /* 0: fp16 table [V][d]; 1: Q8_G64 (uint8 [V][d] + sb [V][d/64][2]) */
  const void* wte;
  const void* wte_sb;
  int lm_head_format; /* 0: MARLIN Q4; 1: Q8_G64; 2: fp16 [V][d] (no scales) */
  const void* lm_head_w;
  const void* lm_head_sb;
  const float* freqs; /* [rope_len][head_dim/2][2] (cos, sin) */
  const void* lnf_w;  /* fp16 [d] */
  /* per-layer arrays (host arrays of device pointers), length n_layer */
  const void* const* ln1_w;
  const void* const* ln2_w;
  const void* const* qkv_w;
  const void* const* qkv_sb;
  const void* const* qkv_bias; /* entries may be NULL; the array itself may be NULL */
  const void* const* o_w;
  const void* const* o_sb;
  const void* const* gu_w; /* rows [gate; up] */
  const void* const* gu_sb;
  const void* const* down_w;
  const void* const* down_sb;
  void* const* k_cache; /* per layer, batch-1 views [Hkv][S][hd or hd/2] */
  void* const* v_cache;
  void* const* k_scales; /* quantized caches only */
  void* const* v_scales;
  int max_tokens; /* capacity of the multi-token (verify) paths, <= 64 */
  int layout;     /* 0: re-tile weights for the matrix cores (default); 1: stream the reference layout */
  int group_size; /* MARLIN Q4 packs (layers and a Q4 lm_head): 64 (reference), or 128 (tile16 layout only);
                     0 means 64 */
  /* Format of each kind of layer matrix, as the reference runner dispatches it from the
   * packed shape (mps_kernels.mm:3055-3068): 0 = MARLIN Q4 (4-D pack), 1 = Q8_G64 (uint8
   * [N][K], sb fp16 [N][K/64][2]), 2 = fp16 [N][K] without scales (the weights of the
   * reference's fp16 runner MPSDecodeRunner, mps_kernels.mm:2304-2980).  Mode "q4_k_m" packs
   * down as Q8, mode "q8" every matrix (transformer.py:840-847, 897-903). */
  int qkv_format, o_format, gu_format, down_format;
} axm_runner_desc;

typedef struct axm_runner* axm_runner_t;

int axm_runner_create(const axm_runner_desc* desc, axm_runner_t* out);
void axm_runner_destroy(axm_runner_t r);
/* One decode token.  The token id comes from idx_dev (int64, device) when
 * non-NULL, else from tok_host when >= 0, else (tok_host < 0) from the greedy
 * argmax of the previous step's logits (lowest index on ties), computed inside
 * the lm_head launch -- the device-side loop of speculative_decode / greedy
 * generation (mps_kernels.mm:3466-3527).  Positions follow transformer.py:1453-1462.
 * *logits_out receives the runner's persistent fp16 [V] buffer (valid until the
 * next call).  Replaces QuantizedDecodeGraphState::step (mps_kernels.mm:3195-3263). */
int axm_runner_step(axm_runner_t r, const void* idx_dev, int64_t tok_host, int start_pos, int write_pos,
                    int active_len, void* stream, void** logits_out);
/* T tokens (idx_dev: device int64 [T], T <= desc.max_tokens <= 64) in one pass;
 * *logits_out receives the runner's fp16 [T][V] buffer.  verify_step rotates token t
 * at start_pos + t and writes slot (write_pos + t) % S; when the T slots are contiguous
 * and active_len == write_pos + T it attends causally over [0, write_pos) + the chain,
 * otherwise (ring wrap-around) every token attends over all S slots, as the
 * reference does.  Replaces verify_step (mps_kernels.mm:3359-3464). */
int axm_runner_verify_step(axm_runner_t r, const void* idx_dev, int T, int start_pos, int write_pos, int active_len,
                           void* stream, void** logits_out);
/* Tree verification: token t is rotated at start_pos + depths[t], written to slot
 * (write_pos + t) % S and attends to slots [0, prefix_len) plus the tree slots whose
 * bit is set in masks[t] (64-bit masks; host arrays).  Replaces verify_tree_step
 * (mps_kernels.mm:3265-3357), whose masks are 32-bit. */
int axm_runner_verify_tree_step(axm_runner_t r, const void* idx_dev, int T, int start_pos, int write_pos,
                                int prefix_len, const int* depths_host, const uint64_t* masks_host, void* stream,
                                void** logits_out);
/* Native prompt-lookup speculative decoding with greedy acceptance: n-gram
 * candidates from the token history are verified in one multi-token pass, the
 * matching prefix plus one corrected / bonus token is kept.  Host arrays;
 * out_tokens receives the whole sequence (initial + generated, capacity >=
 * n_initial + max_new_tokens); stats = {n_tokens, seen, model_calls, drafted,
 * accepted, seconds (double bits)}.  Replaces speculative_decode
 * (mps_kernels.mm:3639-3730). */
int axm_runner_speculative_decode(axm_runner_t r, const int64_t* initial_tokens, int n_initial, int max_new_tokens,
                                  int ngram_size, int max_spec_tokens, int start_pos, int64_t* out_tokens,
                                  int out_capacity, int64_t* stats, void* stream);
/* Device int64 slot holding the token id consumed by the latest step. */
int axm_runner_token_slot(axm_runner_t r, void** tok_out);
/* Measurement entry (no counterpart in the reference): times the launch groups of
 * the one-token step one at a time, each run reps times back to back over the
 * layers in turn (layer j % n_layer) as one captured hipGraph, replayed once untimed
 * and once between HIP events on `stream`.  us_out[6] receives the average microseconds per launch group:
 * QKV (with its RoPE / KV-write epilogue), attention over active_len keys, O
 * projection, gate/up + SwiGLU, down projection, final norm + lm_head.  The token
 * parameters are set to id 0 at `position`; the runner's activations and the cache
 * slot at `position` are left overwritten (the next step recomputes them). */
int axm_runner_time_kernels(axm_runner_t r, int position, int active_len, int reps, void* stream, float* us_out);
/* Normalized final hidden state of the last call (fp16 [T][d]),
 * get_last_norm (mps_kernels.mm:3732-3737). */
int axm_runner_last_norm(axm_runner_t r, void** norm_out);
/* Diagnostic view of the persistent step's cross-workgroup words (uint64: 32-bit
 * payload | 32-bit phase tag << 32) as the last persistent step left them: the
 * residual stream, queries, new key / value rows, attention output and SwiGLU output
 * of the last layer (layout in csrc/step_plan.h, sp::words_layout).  *n_words = 0
 * when the persistent step is unavailable.  No counterpart in the reference. */
int axm_runner_persistent_words(axm_runner_t r, void** words_out, int64_t* n_words);
/* 1 = replay the per-op step as a captured hipGraph, 0 = eager launches
 * (equivalent to axm_runner_set_mode GRAPH / EAGER). */
int axm_runner_set_graph(axm_runner_t r, int enable);
/* Execution of a decode step:
 *   GRAPH      the per-op kernels (five per layer) replayed as a hipGraph;
 *   EAGER      the same kernels launched one by one;
 *   PERSISTENT one cooperative launch per token that runs every layer; each
 *              phase polls the tagged words its inputs arrive in instead of
 *              waiting at a grid barrier, and the next phase's weights stream
 *              while it waits (available with tile16 copies of MARLIN Q4 layer
 *              and lm_head weights, an fp16 KV cache, head size 64 or 128).
 * No counterpart in the reference, whose step is a single Metal command
 * buffer (mps_kernels.mm:3195-3263). */
#define AXM_RUNNER_MODE_GRAPH 0
#define AXM_RUNNER_MODE_EAGER 1
#define AXM_RUNNER_MODE_PERSISTENT 2
int axm_runner_set_mode(axm_runner_t r, int mode);
int axm_runner_get_mode(axm_runner_t r);
/* Synchronizes and returns -6 if a persistent step gave up waiting for another
 * workgroup's output (the runner must then be recreated), 0 otherwise. */
int axm_runner_check(axm_runner_t r);

#ifdef __cplusplus
}
#endif
#endif /* AXM_H_ */
