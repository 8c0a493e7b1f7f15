// Persistent decode-step kernel: one cooperative launch runs a whole batch-1
// decode token (the work of QuantizedDecodeGraphState::step,
// axiomlm/kernels/mps_kernels.mm:3195-3263) on one 1024-thread workgroup per CU.
//
// Phases (step_plan.h): per layer QKV, ATTN, O, GU, DN, then LM.  There is no
// grid barrier.  Every value a phase hands to the next travels through 64-bit
// words of (32-bit payload, 32-bit phase tag) written with device-scope
// relaxed atomic stores; a consumer polls the words it needs until each carries
// the tag of the phase that produces it.  Each phase consumes all of the
// previous phase's outputs (the attention of a head needs only its own rows),
// so no workgroup can run two phases ahead of another, and a buffer is never
// rewritten while a reader still expects an older tag.
//
// Waves 0..kCtl-1 of each workgroup stage the input vector (poll, RMSNorm, LDS),
// prepare the epilogue operands, reduce the per-wave partial tiles and run the
// epilogues; waves kCtl..15 are workers that stream tile16 weight chunks (1 KB
// each, the B operand of four v_mfma_f32_16x16x32_f16) through a ring of kDepth
// in-flight loads and never poll.  The ring runs across phases: while a worker
// consumes its last chunks of one GEMV, its refills already request the first
// chunks of the next GEMV, so those loads are in flight through the epilogue,
// the wait for the next phase's input and its staging.
//
// Every offset the kernel forms comes from step_plan.h, which a CPU check
// (tests/cpu/step_plan_check.cpp) enumerates over whole launches.
#include "axm.h"
#include "kernels.h"
#include "step_kernel.h"
#include "t16_device.h"

namespace {

using sp::Gemv;
using sp::Lds;
using sp::Shape;
using sp::Words;
using u64 = unsigned long long;
typedef __amdgpu_buffer_rsrc_t Rsrc;

constexpr int kThreads = sp::kThreads;
constexpr int kWaves = sp::kWaves;
constexpr int kCtl = sp::kCtl;
constexpr int kWorkers = sp::kWorkers;
constexpr int kDepth = sp::kDepth;
// Blocks of kDepth chunks a worker runs as straight-line code (more run in a loop,
// where the compiler waits for every load in flight at the loop head).
constexpr int kStraightBlocks = 4;
constexpr int kSlots = sp::kStageSlots;
constexpr float kNegBig = -1e30f;
constexpr int kAuxStream = 2;  // nontemporal weight stream

__device__ __forceinline__ Rsrc rsrc_of(const void* p, long bytes) {
  const long lim = bytes < 0x7FFFFFF0L ? bytes : 0x7FFFFFF0L;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)lim, 0x00020000);
}

// A pointer read from the per-layer table, made wave-uniform (scalar registers),
// so that the buffer descriptors built from it are scalar.
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const unsigned long long v = (unsigned long long)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (T*)(((unsigned long long)hi << 32) | lo);
}

// Cross-workgroup words.
__device__ __forceinline__ u64 w_load(const u64* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void w_store(u64* p, uint32_t payload, unsigned tag) {
  __hip_atomic_store(p, ((u64)tag << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned w_tag(u64 w) { return (unsigned)(w >> 32); }
__device__ __forceinline__ uint32_t w_val(u64 w) { return (uint32_t)w; }
__device__ __forceinline__ bool err_set(const StepArgs& a) {
  return __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void raise_err(const StepArgs& a) {
  __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll words src[idx[k]] (k < N; idx[k] < 0 skips slot k) until each carries
// `tag`; w[k] receives the words.  Returns false when the wait gave up.
template <int N>
__device__ __forceinline__ bool poll_words(const StepArgs& a, const u64* src, unsigned tag, const int (&idx)[N],
                                           u64 (&w)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) w[k] = idx[k] >= 0 ? w_load(src + idx[k]) : ((u64)tag << 32);
  for (int spins = 0;; ++spins) {
    bool pend = false;
#pragma unroll
    for (int k = 0; k < N; ++k) pend = pend || w_tag(w[k]) != tag;
    if (!pend) return true;
    if (spins >= a.spin_limit || err_set(a)) {
      raise_err(a);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
#pragma unroll
    for (int k = 0; k < N; ++k)
      if (w_tag(w[k]) != tag) w[k] = w_load(src + idx[k]);
  }
}

// Poll the staging words src[i], i = stage_word(r0, tid, k) < nw (k < N), until each
// carries `tag`.  Waiting on the whole vector would re-read it every round from
// every workgroup (megabytes per round trip across the chip, in the memory
// queues the weight stream uses), so each lane first polls one sentinel word of
// a sample that spans every producer (stage_sentinel),
// then reads its words once and re-polls only those not yet written.
template <int N>
__device__ __forceinline__ bool poll_stage(const StepArgs& a, const u64* src, unsigned tag, int r0, int tid, int nw,
                                           u64 (&w)[N]) {
  if (r0 == 0) {
    // Probes go out every ~0.1 us with up to four in flight, so a written
    // sentinel is seen about one probe interval after it lands rather than up to
    // a full round trip later.
    const int sent = sp::stage_sentinel(tid, nw);
    u64 p0 = w_load(src + sent);
    __builtin_amdgcn_s_sleep(4);
    u64 p1 = w_load(src + sent);
    __builtin_amdgcn_s_sleep(4);
    u64 p2 = w_load(src + sent);
    __builtin_amdgcn_s_sleep(4);
    u64 p3 = w_load(src + sent);
    for (int spins = 0;; ++spins) {
      if (w_tag(p0) == tag) break;
      if (spins >= a.spin_limit || err_set(a)) {
        raise_err(a);
        return false;
      }
      p0 = p1;
      p1 = p2;
      p2 = p3;
      __builtin_amdgcn_s_sleep(4);
      p3 = w_load(src + sent);
    }
  }
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int i = sp::stage_word(r0, tid, k);
    w[k] = i < nw ? w_load(src + i) : ((u64)tag << 32);
  }
  for (int spins = 0;; ++spins) {
    bool pend = false;
#pragma unroll
    for (int k = 0; k < N; ++k) pend = pend || w_tag(w[k]) != tag;
    if (!pend) return true;
    if (spins >= a.spin_limit || err_set(a)) {
      raise_err(a);
      return false;
    }
    __builtin_amdgcn_s_sleep(2);
#pragma unroll
    for (int k = 0; k < N; ++k)
      if (w_tag(w[k]) != tag) w[k] = w_load(src + sp::stage_word(r0, tid, k));
  }
}

__device__ __forceinline__ uint32_t pack_h2(f16 a, f16 b) { return as_u32(f16x2{a, b}); }

// Embedding word i (elements 2i, 2i+1) of token tok: the gather of
// embed_q8_g64_gather_half_kernel (metal_kernels.metal:357-391) or an fp16 row;
// ids outside [0, V) give zeros (as the stand-alone gathers do).
__device__ __forceinline__ uint32_t embed_word(const StepArgs& a, long tok, int i) {
  if (tok < 0 || tok >= a.sh.V) return 0u;
  const int D = a.sh.D;
  if (a.wte_fmt == 0) return reinterpret_cast<const uint32_t*>((const f16*)a.wte + (size_t)tok * D)[i];
  const uint16_t q2 = reinterpret_cast<const uint16_t*>((const uint8_t*)a.wte + (size_t)tok * D)[i];
  const f16* sbr = a.wte_sb + ((size_t)tok * (D / 64) + (2 * i) / 64) * 2;
  const float sc = h2f(sbr[0]), bi = h2f(sbr[1]);
  const f16 e0 = f2h(add_rn(mul_rn((float)(q2 & 0xFFu), sc), bi));
  const f16 e1 = f2h(add_rn(mul_rn((float)(q2 >> 8), sc), bi));
  return pack_h2(e0, e1);
}

struct Smem {
  unsigned char* base;
  Lds L;
  __device__ f16* xs() const { return reinterpret_cast<f16*>(base + L.xs); }
  __device__ f16* lnw() const { return reinterpret_cast<f16*>(base + L.lnw); }
  __device__ f16* zero() const { return reinterpret_cast<f16*>(base + L.zero); }
  __device__ f32x2* cx() const { return reinterpret_cast<f32x2*>(base + L.cx); }
  __device__ float* red() const { return reinterpret_cast<float*>(base + L.red); }
  __device__ f32x2* cs() const { return reinterpret_cast<f32x2*>(base + L.cs); }
  __device__ f16* bias() const { return reinterpret_cast<f16*>(base + L.bias); }
  __device__ f16* xold() const { return reinterpret_cast<f16*>(base + L.xold); }
  __device__ float* att() const { return reinterpret_cast<float*>(base + L.att); }
  __device__ float* qv() const { return reinterpret_cast<float*>(base + L.qv); }
  __device__ float* misc() const { return reinterpret_cast<float*>(base + L.misc); }
  __device__ int* flag() const { return reinterpret_cast<int*>(base + L.flag); }
};

// ---------------------------------------------------------------------------
// Weight stream.
// ---------------------------------------------------------------------------
struct Stream {
  sp::Run r;
  Rsrc rw, rs;
};

// Weight stream of phase ph for this workgroup's worker `worker`.
__device__ __forceinline__ Stream stream_of(const StepArgs& a, int ph, int worker) {
  const Shape& s = a.sh;
  Stream st;
  const int kind = sp::kind_of(s, ph);
  const Gemv p = sp::gemv_plan(s, kind, blockIdx.x);
  st.r = sp::worker_run(p, worker);
  const void* w = nullptr;
  const void* sb = nullptr;
  if (kind == sp::K_LM) {
    w = a.lm_w;
    sb = a.lm_sb;
  } else if (kind == sp::K_QKV || kind == sp::K_O || kind == sp::K_GU || kind == sp::K_DN) {
    const StepLayer* Ly = a.layers + sp::layer_of(ph);
    if (kind == sp::K_QKV) {
      w = Ly->qkv_w;
      sb = Ly->qkv_sb;
    } else if (kind == sp::K_O) {
      w = Ly->o_w;
      sb = Ly->o_sb;
    } else if (kind == sp::K_GU) {
      w = Ly->gu_w;
      sb = Ly->gu_sb;
    } else {
      w = Ly->dn_w;
      sb = Ly->dn_sb;
    }
    w = uniform_ptr(w);
    sb = uniform_ptr(sb);
  }
  const bool has = w != nullptr;
  st.rw = rsrc_of(w, has ? sp::w_bytes(p) : 0);
  st.rs = rsrc_of(sb, has ? sp::sb_bytes(p, s.g128) : 0);
  return st;
}

// Ring slots: the 16 code bytes of a lane and its row's scale words (two (scale,
// bias) pairs for group 64, one for group 128, used for both 64-column halves).
template <bool G128>
struct Ring {
  u32x4 w[kDepth];
  u32x2 s[G128 ? 1 : kDepth];
  uint32_t s1[G128 ? kDepth : 1];
};

template <bool G128>
__device__ __forceinline__ void issue(Ring<G128>& r, int j, const Stream& st, int t, int lane) {
  const int c = sp::run_chunk(st.r, t);
  const int wo = sp::w_off(st.r, c, lane);
  const int so = sp::sb_off(st.r, c, lane, G128 ? 1 : 0);
  r.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(st.rw, wo, 0, kAuxStream));
  if constexpr (G128)
    r.s1[j] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(st.rs, so, 0, 0));
  else
    r.s[j] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(st.rs, so, 0, 0));
}

template <bool G128>
__device__ __forceinline__ void prime(Ring<G128>& r, const Stream& st, int lane) {
#pragma unroll
  for (int j = 0; j < kDepth; ++j) issue<G128>(r, j, st, j, lane);
}

// Adds a wave's running partial of local tile ul (rows in lanes 0..15) into the
// tile's LDS slot.  Every lane takes part (lanes 16..63 add zero to the same 16
// slots) so the chunk loop has no divergent branch: one would make the compiler
// wait for every load in flight before the next chunk.
__device__ __forceinline__ void flush_tile(const Smem& sm, int ul, int worker, int lane, float acc) {
  if (ul >= 0) atomicAdd(sm.red() + sp::red_index(ul, worker, lane & 15), lane < 16 ? acc : 0.f);
}

// Chunk in ring slot j (local chunk c >= 0) into the running partial of its tile.
template <bool G128>
__device__ __forceinline__ void consume(const Ring<G128>& r, int j, int c, int KB, int worker, int lane, const f16* xa,
                                        int a_kb, int a_c, const Smem& sm, const Unpack& U, float& acc,
                                        int& cur_ul) {
  const int ul = c / KB;
  const int kb = c - ul * KB;
  if (ul != cur_ul) {
    flush_tile(sm, cur_ul, worker, lane, acc);
    acc = 0.f;
    cur_ul = ul;
  }
  const f16* xk = xa + kb * a_kb;
  f16x8 A[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) A[q] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(xk + q * a_c));
  const f32x4 cxv = *reinterpret_cast<const f32x4*>(sm.cx() + 2 * kb);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[0], unpack_word(r.w[j][0], U), z4, 0, 0, 0);
  f32x4 d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[2], unpack_word(r.w[j][2], U), z4, 0, 0, 0);
  d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[1], unpack_word(r.w[j][1], U), d0, 0, 0, 0);
  d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[3], unpack_word(r.w[j][3], U), d1, 0, 0, 0);
  if constexpr (G128) {
    const f16x2 sb = as_h2(r.s1[j]);
    acc = __builtin_fmaf(h2f(sb.x), (d0[0] - cxv[0]) + (d1[0] - cxv[2]), acc);
    acc = __builtin_fmaf(h2f(sb.y), cxv[1] + cxv[3], acc);
  } else {
    const uint32_t s0 = r.s[j][0];
    const uint32_t s1 = r.s[j][1];
    const f16x2 sb0 = as_h2(s0);
    const f16x2 sb1 = as_h2(s1);
    acc = __builtin_fmaf(h2f(sb0.x), d0[0] - cxv[0], acc);
    acc = __builtin_fmaf(h2f(sb0.y), cxv[1], acc);
    acc = __builtin_fmaf(h2f(sb1.x), d1[0] - cxv[2], acc);
    acc = __builtin_fmaf(h2f(sb1.y), cxv[3], acc);
  }
}

// Worker state of one GEMV phase.
template <bool G128>
struct WorkerPhase {
  Stream cur, nxt;
  int nblk;
  const f16* xa;
  int a_kb, a_c;
  float acc;
  int cur_ul;
};

// Block b: consume the chunks at positions b * kDepth + j; refill slot j with
// position (b + 1) * kDepth + j of this phase, or, in the last block, position j
// of the next GEMV phase.  The scheduling barrier after each slot keeps "consume
// slot j, refill slot j" in program order, so consuming a slot waits only for
// that slot's loads (left to itself the scheduler gathers the MFMAs of all slots
// ahead of the refills, which waits for every load in flight).
template <bool G128>
__device__ __forceinline__ void worker_block(Ring<G128>& r, WorkerPhase<G128>& w, int b, int worker, int lane,
                                             const Smem& sm, const Unpack& U) {
  const bool last = b + 1 >= w.nblk;
#pragma unroll
  for (int j = 0; j < kDepth; ++j) {
    const int c = sp::run_chunk(w.cur.r, b * kDepth + j);
    if (c >= 0) consume<G128>(r, j, c, w.cur.r.KB, worker, lane, w.xa, w.a_kb, w.a_c, sm, U, w.acc, w.cur_ul);
    issue<G128>(r, j, last ? w.nxt : w.cur, last ? j : (b + 1) * kDepth + j, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Blocks B.. as nested straight-line code (every path a chain, so the compiler
// counts the loads in flight exactly), then a loop for any beyond kStraightBlocks.
template <bool G128, int B>
__device__ __forceinline__ void worker_blocks(Ring<G128>& r, WorkerPhase<G128>& w, int worker, int lane,
                                              const Smem& sm, const Unpack& U) {
  if constexpr (B < kStraightBlocks) {
    if (B < w.nblk) {
      worker_block<G128>(r, w, B, worker, lane, sm, U);
      worker_blocks<G128, B + 1>(r, w, worker, lane, sm, U);
    }
  } else {
    for (int b = B; b < w.nblk; ++b) worker_block<G128>(r, w, b, worker, lane, sm, U);
  }
}

// Consume this worker's chunks of phase `ph` (partial tiles added into
// red[ul][worker]); the refills of the last block request the first chunks of
// the next GEMV phase `nph`.
template <bool G128>
__device__ __forceinline__ void worker_phase(Ring<G128>& r, const StepArgs& a, int ph, int nph, int worker, int lane,
                                             const Smem& sm, const Unpack& U) {
  WorkerPhase<G128> w;
  w.cur = stream_of(a, ph, worker);
  w.nxt = stream_of(a, nph, worker);
  w.nblk = w.cur.r.nt / kDepth;
  if (w.nblk > 0) {
    // A operand: lanes 0, 16, 32, 48 hold the token's activations, the others a zero block.
    w.xa = (lane & 15) == 0 ? sm.xs() + 8 * (lane >> 4) : sm.zero();
    w.a_kb = (lane & 15) == 0 ? 128 : 0;
    w.a_c = (lane & 15) == 0 ? 32 : 0;
    w.acc = 0.f;
    w.cur_ul = -1;
    worker_blocks<G128, 0>(r, w, worker, lane, sm, U);
    flush_tile(sm, w.cur_ul, worker, lane, w.acc);
  } else {
    // The ring holds this phase's (all padding) positions: request the next phase's.
    prime<G128>(r, w.nxt, lane);
  }
}

// Sum of the worker partials of local tile ul, row j.
__device__ __forceinline__ float tile_row(const Smem& sm, int ul, int j) {
  const float* red = sm.red();
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < kWorkers; ++w) v += red[sp::red_index(ul, w, j)];
  return v;
}

// ---------------------------------------------------------------------------
// Staging (control waves): the phase's input vector (K elements, K/2 words)
// polled from `src` (or the embedding row of tok when src is null) into LDS xs,
// then the optional fp16 RMSNorm (weights already in LDS lnw) and the
// per-64-group sums that remove the magic offsets of the nibble expansion.  The
// workers take part only in the barriers (stage_sync): their loads complete in
// issue order, so a poll behind their prefetched weight chunks would wait for
// those chunks.  Returns false (on every thread) when a wait gave up.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool stage_ctl(const StepArgs& a, const Smem& sm, const u64* src, int K, unsigned tag,
                                          bool norm, long tok, f16* norm_out) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int nw = K / 2;
  const int nwp = sp::cdiv(K, 128) * 64;
  uint32_t* xs = reinterpret_cast<uint32_t*>(sm.xs());
  bool ok = true;
  for (int r0 = 0; r0 < nwp && ok; r0 += sp::kStagePass) {
    u64 w[kSlots];
    if (src != nullptr) ok = poll_stage(a, src, tag, r0, tid, nw, w);
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const int i = sp::stage_word(r0, tid, j);
      if (i < nwp) xs[i] = i >= nw ? 0u : (src != nullptr ? w_val(w[j]) : embed_word(a, tok, i));
    }
  }
  if (!ok) sm.flag()[0] = 1;
  __syncthreads();
  float rinv = 1.f;
  if (norm) {
    float ss = 0.f;
    for (int i = tid; i < nw; i += kCtl * 64) {
      const f16x2 h = as_h2(xs[i]);
      const float f0 = h2f(h.x), f1 = h2f(h.y);
      ss += h2f(f2h(f0 * f0));
      ss += h2f(f2h(f1 * f1));
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) sm.misc()[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kCtl; ++w) tot += sm.misc()[w];
    rinv = rms_inv_fp16(tot, K, a.eps);
  }
  const uint32_t* lw = reinterpret_cast<const uint32_t*>(sm.lnw());
  // nwp is a multiple of 64, so each wave's words are all inside or all past it.
  for (int i = tid; i < nwp; i += kCtl * 64) {
    f16x2 h = as_h2(xs[i]);
    if (norm && i < nw) {
      const f16x2 g = as_h2(lw[i]);
      h.x = f2h(h2f(f2h(h2f(h.x) * rinv)) * h2f(g.x));
      h.y = f2h(h2f(f2h(h2f(h.y) * rinv)) * h2f(g.y));
      xs[i] = as_u32(h);
      if (norm_out != nullptr) reinterpret_cast<uint32_t*>(norm_out)[i] = as_u32(h);
    }
    // Elements 2i, 2i+1 sit at positions 2i mod 8, 2i+1 mod 8 of an 8-element chunk,
    // whose nibbles expand as 1024 + q (positions 0, 1, 4, 5) or 64 + q (2, 3, 6, 7).
    const float m = (i & 1) ? 64.f : 1024.f;
    const float f0 = h2f(h.x), f1 = h2f(h.y);
    float corr = f0 * m + f1 * m;
    float sum = f0 + f1;
    corr = group_sum<32>(corr);
    sum = group_sum<32>(sum);
    if ((tid & 31) == 0) sm.cx()[i >> 5] = f32x2{corr, sum};
  }
  __syncthreads();
  return sm.flag()[0] == 0;
}

// The workers' side of stage_ctl: the same barriers.
__device__ __forceinline__ bool stage_sync(const Smem& sm, bool norm) {
  __syncthreads();
  if (norm) __syncthreads();
  __syncthreads();
  return sm.flag()[0] == 0;
}

// ---------------------------------------------------------------------------
// Epilogues (control wave; lanes 16 u + j hold row j of local tile ul0 + u).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void epi_qkv(const StepArgs& a, const Smem& sm, const Gemv& p, const StepLayer* Ly, unsigned tag,
                        const Words& W) {
  const Shape& s = a.sh;
  const int lane = threadIdx.x & 63;
  const int qd = sp::q_dim(s), kvd = sp::kv_dim(s), rows = sp::qkv_rows(s);
  f16* kc = uniform_ptr(Ly->kc);
  f16* vc = uniform_ptr(Ly->vc);
  for (int ul0 = 0; ul0 < p.nl; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const int lr = ul * 16 + j;
    const int row = sp::epi_row(p, ul, j);
    const bool have = ul < p.nl && row < rows;
    f16 h = f2h(have ? tile_row(sm, ul, j) : 0.f);
    if (have) h = f2h(h2f(h) + h2f(sm.bias()[lr]));
    const f16 partner = f2h(__shfl_xor(h2f(h), 1, 64));
    f16 out = h;
    if (have && row < qd + kvd) {
      const bool even = (row & 1) == 0;
      const f32x2 cs = sm.cs()[lr];
      out = rope_out(even ? h : partner, even ? partner : h, cs[0], cs[1], even);
    }
    const f16 other = f2h(__shfl_xor(h2f(out), 1, 64));
    if (have && (row & 1) == 0) {
      const uint32_t pair = pack_h2(out, other);
      w_store(a.words + sp::qkv_word(s, W, row), pair, tag);
      if (row >= qd) {
        const bool is_k = row < qd + kvd;
        const int within = is_k ? row - qd : row - qd - kvd;
        const int kvh = within / s.hd, e = within % s.hd;
        f16* dst = (is_k ? kc : vc) + sp::cache_elem(s, kvh, a.write_pos, e);
        *reinterpret_cast<uint32_t*>(dst) = pair;
      }
    }
  }
}

// x[row] = x_old[row] + y[row] (O and down projections).
__device__ __forceinline__ void epi_resid(const StepArgs& a, const Smem& sm, const Gemv& p, unsigned tag, const Words& W) {
  const int lane = threadIdx.x & 63;
  for (int ul0 = 0; ul0 < p.nl; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const int lr = ul * 16 + j;
    const int row = sp::epi_row(p, ul, j);
    const bool have = ul < p.nl && row < p.N;
    const f16 y = f2h(have ? tile_row(sm, ul, j) : 0.f);
    const f16 x = f2h(h2f(sm.xold()[have ? lr : 0]) + h2f(y));
    const f16 other = f2h(__shfl_xor(h2f(x), 1, 64));
    if (have && (row & 1) == 0) w_store(a.words + sp::x_word(W, row), pack_h2(x, other), tag);
  }
}

__device__ __forceinline__ void epi_swiglu(const StepArgs& a, const Smem& sm, const Gemv& p, unsigned tag, const Words& W) {
  const int lane = threadIdx.x & 63;
  for (int ul0 = 0; ul0 < p.n; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const int row = sp::epi_row(p, ul, j);
    const bool have = ul < p.n && row < p.N;
    const f16 g = f2h(have ? tile_row(sm, ul, j) : 0.f);
    const f16 u = f2h(have ? tile_row(sm, ul + p.n, j) : 0.f);
    const f16 sg = f2h(t16_silu(h2f(g)));
    const f16 hv = f2h(h2f(sg) * h2f(u));
    const f16 other = f2h(__shfl_xor(h2f(hv), 1, 64));
    if (have && (row & 1) == 0) w_store(a.words + sp::h_word(W, row), pack_h2(hv, other), tag);
  }
}

// Ordered key of (logit, row): larger logit first, then the lower row.
__device__ __forceinline__ u64 logit_key(f16 v, int row) {
  const uint32_t u = __builtin_bit_cast(uint32_t, h2f(v));
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((u64)ord << 32) | (0xFFFFFFFFu - (uint32_t)row);
}

// Logits, per-tile argmax keys (the graph path's format, for greedy feedback in
// either mode) and the workgroup's best key.
__device__ __forceinline__ u64 epi_lm(const StepArgs& a, const Smem& sm, const Gemv& p) {
  const int lane = threadIdx.x & 63;
  u64 best = 0ull;
  for (int ul0 = 0; ul0 < p.nl; ul0 += 4) {
    const int ul = ul0 + (lane >> 4), j = lane & 15;
    const int unit = p.u0 + ul;
    const int row = sp::epi_row(p, ul, j);
    const bool have = ul < p.nl && row < p.N;
    u64 key = 0ull;
    if (have) {
      const f16 hv = f2h(tile_row(sm, ul, j));
      a.logits[row] = hv;
      key = logit_key(hv, row);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const u64 other = __shfl_xor(key, o, 64);
      key = other > key ? other : key;
    }
    if (ul < p.nl && j == 0) a.argmax_keys[unit] = key;
    best = key > best ? key : best;
  }
#pragma unroll
  for (int o = 16; o < 64; o <<= 1) {
    const u64 other = __shfl_xor(best, o, 64);
    best = other > best ? other : best;
  }
  return best;
}

// Epilogue operands of this workgroup's rows, requested by the control wave
// before the staging: RoPE (cos, sin) and bias of the QKV rows; the residual
// input of the O / DN rows (x words of phase `xtag`, or the embedding row).
__device__ __forceinline__ bool epi_operands(const StepArgs& a, const Smem& sm, const Gemv& p, int kind, const StepLayer* Ly,
                             unsigned xtag, bool x_from_embedding, long tok, const Words& W) {
  const Shape& s = a.sh;
  const int lane = threadIdx.x & 63;
  const int nrows = p.nl * 16;
  if (kind == sp::K_QKV) {
    const int qd = sp::q_dim(s), kvd = sp::kv_dim(s), rows = sp::qkv_rows(s);
    const f16* bias = uniform_ptr(Ly->qkv_bias);
    for (int lr = lane; lr < nrows; lr += 64) {
      const int row = sp::epi_row(p, lr >> 4, lr & 15);
      float c = 1.f, sn = 0.f;
      if (row < qd + kvd) {
        const int within = row < qd ? row : row - qd;
        const int fi = (within % s.hd) >> 1;
        const float* f = a.freqs + ((size_t)a.rope_pos * (s.hd / 2) + fi) * 2;
        c = f[0];
        sn = f[1];
      }
      sm.cs()[lr] = f32x2{c, sn};
      sm.bias()[lr] = (bias != nullptr && row < rows) ? bias[row] : f16(0);
    }
    return true;
  }
  if (kind != sp::K_O && kind != sp::K_DN) return true;
  // nrows / 2 words from word p.u0 * 8; at most kMaxLocal * 8 = 256 words: 4 per lane.
  constexpr int kPer = sp::kMaxLocal * 8 / 64;
  const int nwords = min(nrows, p.N - sp::epi_row(p, 0, 0)) / 2;
  uint32_t v[kPer];
  bool ok = true;
  if (x_from_embedding) {
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = lane + 64 * k;
      v[k] = i < nwords ? embed_word(a, tok, (int)(sp::x_word(W, sp::epi_row(p, 0, 2 * i)) - W.x)) : 0u;
    }
  } else {
    int idx[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      idx[k] = lane + 64 * k < nwords ? (int)sp::x_word(W, sp::epi_row(p, 0, 2 * (lane + 64 * k))) : -1;
    u64 w[kPer];
    ok = poll_words(a, a.words, xtag, idx, w);
#pragma unroll
    for (int k = 0; k < kPer; ++k) v[k] = w_val(w[k]);
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = lane + 64 * k;
    if (i < nwords) reinterpret_cast<uint32_t*>(sm.xold())[i] = v[k];
  }
  return ok;
}

// ---------------------------------------------------------------------------
// Attention (fp16 cache).  Item = (query head, split); every wave takes key
// steps of KPW keys; the slot write_pos holds this step's key / value, taken
// from the kv words by the control wave.  Split partials merge in the
// workgroup of split 0, which writes the head's output words.  The control
// waves poll and merge (attn_ctl), the workers run only the key loop
// (attn_work); both follow the same barriers.
// ---------------------------------------------------------------------------
struct AttnItem {
  int hq, spl, kvh, k0, k1;
  bool has_new;
};
__device__ __forceinline__ AttnItem attn_item(const StepArgs& a, int item) {
  const Shape& s = a.sh;
  AttnItem it;
  const int ns = a.n_splits;
  it.hq = item / ns;
  it.spl = item - it.hq * ns;
  it.kvh = it.hq / (s.Hq / s.Hkv);
  it.k0 = sp::attn_k0(a.active_len, ns, it.spl);
  it.k1 = sp::attn_k1(a.active_len, ns, it.spl);
  it.has_new = a.write_pos >= it.k0 && a.write_pos < it.k1;
  return it;
}

// Key loop of wave `wave` over the item's cache keys (the new key excluded), its
// (m, l, o) state into att[wave].
__device__ __forceinline__ void attn_keys(const StepArgs& a, const Smem& sm, int layer, const AttnItem& it, int wave,
                                          int lane) {
  const Shape& s = a.sh;
  const int hd = s.hd;
  const int LPT = hd / 8, KPW = 64 / LPT;
  const int sub = lane / LPT, e0 = (lane % LPT) * 8;
  const StepLayer* Ly = a.layers + layer;
  const long cache_bytes = (long)s.Hkv * s.S * hd * 2;
  const Rsrc rk = rsrc_of(uniform_ptr(Ly->kc), cache_bytes);
  const Rsrc rv = rsrc_of(uniform_ptr(Ly->vc), cache_bytes);
  const float* qv = sm.qv();
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = qv[e0 + i];
  float m = kNegBig, l = 0.f, o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;
  for (int kb = it.k0 + wave * KPW; kb < it.k1; kb += kWaves * KPW) {
    const int key = kb + sub;
    // Keys past the split and the slot of this step's key read zeros (out-of-range
    // offset), so a stale slot cannot put a NaN into the sums.
    const bool valid = key < it.k1 && key != a.write_pos;
    const int off = valid ? (int)(sp::cache_elem(s, it.kvh, key, e0) * 2) : sp::kOOB;
    const f16x8 kh = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
    const f16x8 vh = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) d = __builtin_fmaf(q[i], h2f(kh[i]), d);
    for (int x = LPT / 2; x > 0; x >>= 1) d += __shfl_xor(d, x, 64);
    const float sc = valid ? d * a.scale_log2 : kNegBig;
    const float m_new = fmaxf(m, sc);
    const float alpha = exp2f(m - m_new);
    const float pr = valid ? exp2f(sc - m_new) : 0.f;
    l = l * alpha + pr;
    m = m_new;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = __builtin_fmaf(o[i], alpha, pr * h2f(vh[i]));
  }
  // Merge the KPW key slots of the wave.
  for (int x = LPT; x < 64; x <<= 1) {
    const float m2 = __shfl_xor(m, x, 64);
    const float l2 = __shfl_xor(l, x, 64);
    const float mn = fmaxf(m, m2);
    const float a1 = exp2f(m - mn), a2 = exp2f(m2 - mn);
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = o[i] * a1 + __shfl_xor(o[i], x, 64) * a2;
    m = mn;
  }
  float* att = sm.att() + wave * (2 + 128);
  if (lane < LPT) {
    if (lane == 0) {
      att[0] = m;
      att[1] = l;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) att[2 + e0 + i] = o[i];
  }
}

// Control waves: per item, wave 0 polls the query (and the new key / value rows)
// into LDS, every control wave runs its key steps, wave 0 merges the waves' and
// the splits' states and writes the head's output.
__device__ __forceinline__ bool attn_ctl(const StepArgs& a, const Smem& sm, int layer, unsigned tag_in,
                                         unsigned tag_out, const Words& W) {
  const Shape& s = a.sh;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hd = s.hd, nq = hd / 2;
  const int ns = a.n_splits;
  float* qv = sm.qv();
  for (int item = blockIdx.x; item < s.Hq * ns; item += gridDim.x) {
    const AttnItem it = attn_item(a, item);
    if (wave == 0) {
      int idx[3];
      idx[0] = lane < nq ? (int)sp::q_word(s, W, it.hq, lane) : -1;
      idx[1] = (lane < nq && it.has_new) ? (int)sp::kvnew_word(s, W, it.kvh, lane, 0) : -1;
      idx[2] = (lane < nq && it.has_new) ? (int)sp::kvnew_word(s, W, it.kvh, lane, 1) : -1;
      u64 w[3];
      const bool ok = poll_words(a, a.words, tag_in, idx, w);
      if (!ok) sm.flag()[0] = 1;
      if (lane < nq) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          const f16x2 h = as_h2(w_val(w[k]));
          qv[k * 128 + 2 * lane] = h2f(h.x);
          qv[k * 128 + 2 * lane + 1] = h2f(h.y);
        }
      }
    }
    __syncthreads();
    if (sm.flag()[0] != 0) return false;
    attn_keys(a, sm, layer, it, wave, lane);
    __syncthreads();
    if (wave == 0) {
      // Lane i holds dims 2i, 2i+1 (i < hd/2).
      const bool act = lane < nq;
      const int ea = act ? 2 * lane : 0;
      float mm = kNegBig;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm.att()[w * (2 + 128)]);
      float ll = 0.f, oa = 0.f, ob = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float* aw = sm.att() + w * (2 + 128);
        const float sc = exp2f(aw[0] - mm);
        ll += aw[1] * sc;
        oa += aw[2 + ea] * sc;
        ob += aw[3 + ea] * sc;
      }
      if (it.has_new) {
        float d = act ? qv[ea] * qv[128 + ea] + qv[ea + 1] * qv[128 + ea + 1] : 0.f;
        d = wave_sum(d);
        const float sn = d * a.scale_log2;
        const float mn = fmaxf(mm, sn);
        const float c1 = exp2f(mm - mn), pn = exp2f(sn - mn);
        ll = ll * c1 + pn;
        oa = oa * c1 + pn * qv[256 + ea];
        ob = ob * c1 + pn * qv[256 + ea + 1];
        mm = mn;
      }
      bool ok = true;
      if (ns > 1 && it.spl > 0) {
        if (lane == 0) {
          w_store(a.words + sp::part_word(s, W, it.hq, it.spl, 0), __builtin_bit_cast(uint32_t, mm), tag_out);
          w_store(a.words + sp::part_word(s, W, it.hq, it.spl, 1), __builtin_bit_cast(uint32_t, ll), tag_out);
        }
        if (act) {
          w_store(a.words + sp::part_word(s, W, it.hq, it.spl, 2 + ea), __builtin_bit_cast(uint32_t, oa), tag_out);
          w_store(a.words + sp::part_word(s, W, it.hq, it.spl, 3 + ea), __builtin_bit_cast(uint32_t, ob), tag_out);
        }
      } else {
        for (int s2 = 1; s2 < ns && ok; ++s2) {
          int idx[4];
          idx[0] = (int)sp::part_word(s, W, it.hq, s2, 0);
          idx[1] = (int)sp::part_word(s, W, it.hq, s2, 1);
          idx[2] = act ? (int)sp::part_word(s, W, it.hq, s2, 2 + ea) : -1;
          idx[3] = act ? (int)sp::part_word(s, W, it.hq, s2, 3 + ea) : -1;
          u64 w[4];
          ok = poll_words(a, a.words, tag_out, idx, w);
          const float m2 = __builtin_bit_cast(float, w_val(w[0]));
          const float l2 = __builtin_bit_cast(float, w_val(w[1]));
          const float mn = fmaxf(mm, m2);
          const float c1 = exp2f(mm - mn), c2 = exp2f(m2 - mn);
          ll = ll * c1 + l2 * c2;
          oa = oa * c1 + __builtin_bit_cast(float, w_val(w[2])) * c2;
          ob = ob * c1 + __builtin_bit_cast(float, w_val(w[3])) * c2;
          mm = mn;
        }
        if (act) {
          const float inv = ll > 0.f ? 1.f / ll : 0.f;
          w_store(a.words + sp::o_word(s, W, it.hq, lane), pack_h2(f2h(oa * inv), f2h(ob * inv)), tag_out);
        }
      }
      if (!ok) sm.flag()[0] = 1;
    }
    __syncthreads();
    if (sm.flag()[0] != 0) return false;
  }
  return true;
}

// Workers: the key loop of every item, between the control waves' barriers.
__device__ __forceinline__ bool attn_work(const StepArgs& a, const Smem& sm, int layer) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int item = blockIdx.x; item < a.sh.Hq * a.n_splits; item += gridDim.x) {
    const AttnItem it = attn_item(a, item);
    __syncthreads();
    if (sm.flag()[0] != 0) return false;
    attn_keys(a, sm, layer, it, wave, lane);
    __syncthreads();
    __syncthreads();
    if (sm.flag()[0] != 0) return false;
  }
  return true;
}

#ifdef AXM_STEP_STAMPS
// Diagnostic build only: per (workgroup, phase) the 100 MHz clock at the phase's
// start, after its staging, after its weight stream and after its epilogue.
#define STAMP(ph, k)                                                                                       \
  if (threadIdx.x == 0)                                                                                    \
    a.words[sp::words_layout(a.sh).total + ((size_t)blockIdx.x * sp::n_phases(a.sh) + (ph)) * 6 + (k)] = \
        __builtin_amdgcn_s_memrealtime();
// Worker wave 0 (the first worker) stamps slots 4 and 5.
#define STAMPW(ph, k)                                                                                      \
  if (threadIdx.x == kCtl * 64)                                                                            \
    a.words[sp::words_layout(a.sh).total + ((size_t)blockIdx.x * sp::n_phases(a.sh) + (ph)) * 6 + (k)] = \
        __builtin_amdgcn_s_memrealtime();
#else
#define STAMP(ph, k)
#define STAMPW(ph, k)
#endif

// The RMSNorm weight of a GEMV phase's input (null: no norm).
__device__ __forceinline__ const f16* norm_weight(const StepArgs& a, int kind, const StepLayer* Ly) {
  return kind == sp::K_QKV  ? uniform_ptr(Ly->ln1)
         : kind == sp::K_GU ? uniform_ptr(Ly->ln2)
         : kind == sp::K_LM ? a.lnf
                            : nullptr;
}

// Control waves: staging, epilogue operands and epilogues of every phase, the
// attention polls and merges, and (workgroup 0) the greedy token at the end.
__device__ __forceinline__ void control_loop(const StepArgs& a, const Smem& sm, long tok_row) {
  const Shape& s = a.sh;
  const Words W = sp::words_layout(s);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nph = sp::n_phases(s);
  for (int ph = 0; ph < nph; ++ph) {
    const int kind = sp::kind_of(s, ph);
    const int layer = sp::layer_of(ph);
    const unsigned tag = sp::tag_of(a.tag0, ph);
    STAMP(ph, 0)
    if (kind == sp::K_ATTN) {
      if (!attn_ctl(a, sm, layer, sp::tag_of(a.tag0, ph - 1), tag, W)) return;
      STAMP(ph, 3)
      continue;
    }
    const Gemv p = sp::gemv_plan(s, kind, blockIdx.x);
    const StepLayer* Ly = a.layers + (kind == sp::K_LM ? 0 : layer);
    if (p.n > 0) {
      // Input words (all of the previous phase's output): QKV and GU read x (the
      // residual after the previous DN / this layer's O; layer 0's QKV the
      // embedding row), O the attention output, DN the SwiGLU output, LM the last x.
      const u64* src = kind == sp::K_O    ? a.words + W.o
                       : kind == sp::K_DN ? a.words + W.h
                       : (kind == sp::K_QKV && layer == 0) ? nullptr
                                                            : a.words + W.x;
      const f16* ln = norm_weight(a, kind, Ly);
      // Set-up split over two control waves so that no wave chains several round
      // trips ahead of its share of the poll.  Wave 0: the epilogue operands, then
      // zeroed partial tiles (wave 0 itself read the previous phase's tiles in its
      // epilogue; the workers cannot clear them).  Wave 1: RMSNorm weights into LDS.
      // The residual input of O is x as the previous DN (or the embedding) left it,
      // that of DN x as this layer's O left it.
      if (wave == 0) {
        const unsigned xtag = sp::tag_of(a.tag0, kind == sp::K_O ? ph - 3 : ph - 2);
        if (!epi_operands(a, sm, p, kind, Ly, xtag, kind == sp::K_O && layer == 0, tok_row, W)) sm.flag()[0] = 1;
        for (int i = lane; i < p.nl * kWorkers * 16; i += 64) sm.red()[i] = 0.f;
      } else if (wave == 1 && ln != nullptr) {
        const u32x4* lsrc = reinterpret_cast<const u32x4*>(ln);
        u32x4* ldst = reinterpret_cast<u32x4*>(sm.lnw());
        for (int i = lane; i < p.K / 8; i += 64) ldst[i] = lsrc[i];
      }
      f16* norm_out = (kind == sp::K_LM && blockIdx.x == 0) ? a.norm_out : nullptr;
      if (!stage_ctl(a, sm, src, p.K, sp::tag_of(a.tag0, ph - 1), ln != nullptr, tok_row, norm_out)) return;
    }
    STAMP(ph, 1)
    __syncthreads();  // the workers' partial tiles are complete
    STAMP(ph, 2)
    if (wave == 0) {
      if (p.n > 0) {
        if (kind == sp::K_QKV)
          epi_qkv(a, sm, p, Ly, tag, W);
        else if (kind == sp::K_O || kind == sp::K_DN)
          epi_resid(a, sm, p, tag, W);
        else if (kind == sp::K_GU)
          epi_swiglu(a, sm, p, tag, W);
      }
      if (kind == sp::K_LM) {
        const u64 best = p.n > 0 ? epi_lm(a, sm, p) : 0ull;
        if (lane == 0) {
          w_store(a.words + sp::key_word(W, blockIdx.x, 0), (uint32_t)(best >> 32), tag);
          w_store(a.words + sp::key_word(W, blockIdx.x, 1), (uint32_t)best, tag);
        }
      }
    }
    STAMP(ph, 3)
  }
  // Greedy token of this step: workgroup 0 reduces every workgroup's best key.
  if (blockIdx.x == 0 && wave == 0) {
    const unsigned tag = sp::tag_of(a.tag0, nph - 1);
    constexpr int kPer = 4;  // G <= 256 workgroups
    int idx[2 * kPer];
#pragma unroll
    for (int k = 0; k < 2 * kPer; ++k) {
      const int g = lane + 64 * (k >> 1);
      idx[k] = g < (int)gridDim.x ? (int)sp::key_word(W, g, k & 1) : -1;
    }
    u64 w[2 * kPer];
    const bool ok = poll_words(a, a.words, tag, idx, w);
    u64 best = 0ull;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int g = lane + 64 * k;
      const u64 key = ((u64)w_val(w[2 * k]) << 32) | w_val(w[2 * k + 1]);
      if (g < (int)gridDim.x) best = key > best ? key : best;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const u64 other = __shfl_xor(best, o, 64);
      best = other > best ? other : best;
    }
    if (ok && lane == 0) *a.tok_next = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
  }
}

// Workers: the weight stream of every GEMV phase and their share of the attention
// keys, between the control waves' barriers.
template <bool G128>
__device__ __forceinline__ void worker_loop(const StepArgs& a, const Smem& sm, int worker) {
  const Shape& s = a.sh;
  const int lane = threadIdx.x & 63;
  const Unpack U{to_vgpr(0x000F000Fu), to_vgpr(0x00F000F0u), 0x64006400u, 0x54005400u};
  Ring<G128> ring;
  prime<G128>(ring, stream_of(a, 0, worker), lane);
  __syncthreads();  // LDS set-up
  const int nph = sp::n_phases(s);
  for (int ph = 0; ph < nph; ++ph) {
    const int kind = sp::kind_of(s, ph);
    if (kind == sp::K_ATTN) {
      if (!attn_work(a, sm, sp::layer_of(ph))) return;
      continue;
    }
    if (sp::gemv_plan(s, kind, blockIdx.x).n > 0 && !stage_sync(sm, kind == sp::K_QKV || kind == sp::K_GU ||
                                                                      kind == sp::K_LM))
      return;
    STAMPW(ph, 4)
    worker_phase<G128>(ring, a, ph, sp::next_gemv_phase(s, ph), worker, lane, sm, U);
    STAMPW(ph, 5)
    __syncthreads();  // partial tiles complete
  }
}

template <bool G128>
__global__ void __launch_bounds__(kThreads) step_kernel(StepArgs a) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const Smem sm{smem_raw, sp::lds_layout()};
  long long tok;
  if (a.idx_dev != nullptr)
    tok = a.idx_dev[0];
  else if (a.tok_host >= 0)
    tok = a.tok_host;
  else
    tok = a.tok_prev[0];
  if (wave >= kCtl) {
    worker_loop<G128>(a, sm, wave - kCtl);
    return;
  }
  if (tid == 0) sm.flag()[0] = 0;
  if (tid < 8) reinterpret_cast<uint32_t*>(sm.zero())[tid] = 0u;
  if (blockIdx.x == 0 && tid == 0) *a.tok_used = tok;
  __syncthreads();  // LDS set-up
  control_loop(a, sm, (long)(int)tok);  // the embedding gathers read the int32 id
}
#undef STAMP
#undef STAMPW

}  // namespace

int step_check(sp::Shape& sh, size_t* smem_out) {
  const int cus = axm_num_cus();
  sh.G = cus;
  const Lds L = sp::lds_layout();
  const size_t smem = (size_t)L.total;
  if (cus < 1 || cus > 256) return -1;  // the greedy reduction reads four keys per lane
  if (sh.hd != 64 && sh.hd != 128) return -1;
  if (sh.Hkv < 1 || sh.Hq % sh.Hkv != 0) return -1;
  if (sh.H % 16 != 0 || sh.D % 2 != 0 || sp::q_dim(sh) % 2 != 0) return -1;
  const int kmax = std::max(std::max(sh.D, sh.H), sp::q_dim(sh));
  if (sp::cdiv(kmax, 128) > sp::kMaxKB) return -1;
  for (int kind : {sp::K_QKV, sp::K_O, sp::K_GU, sp::K_DN, sp::K_LM})
    if (sp::gemv_plan(sh, kind, 0).nl > sp::kMaxLocal) return -1;
  if (sh.S < 1 || (long)sh.Hkv * sh.S * sh.hd * 2 > 0x7FFFFFF0L) return -1;
  const void* fn = sh.g128 ? (const void*)step_kernel<true> : (const void*)step_kernel<false>;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  int occ = 0;
  const hipError_t e = sh.g128
                           ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, step_kernel<true>, kThreads, smem)
                           : hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, step_kernel<false>, kThreads, smem);
  if (e != hipSuccess || occ < 1) {
    (void)hipGetLastError();
    return -1;
  }
  int coop = 0, dev = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess || !coop) {
    (void)hipGetLastError();
    return -1;
  }
  *smem_out = smem;
  return 0;
}

int step_launch(const StepArgs& a, size_t smem, hipStream_t s) {
  StepArgs args = a;
  void* kargs[] = {&args};
  const void* fn = a.sh.g128 ? (const void*)step_kernel<true> : (const void*)step_kernel<false>;
  const hipError_t e = hipLaunchCooperativeKernel(fn, dim3(a.sh.G), dim3(kThreads), kargs, (unsigned)smem, s);
  if (e != hipSuccess) {
    axm_set_error("persistent step: cooperative launch failed: %s", hipGetErrorString(e));
    return -5;
  }
  return 0;
}
