// Index math of the persistent decode-step kernel (step_kernel.hip), shared
// verbatim between the kernel and a CPU enumeration check that walks every
// workgroup, wave, lane and phase of a launch and asserts that each offset the
// kernel forms lies inside the buffer it addresses.  Plain C++ (no HIP types):
// under hipcc the functions are __host__ __device__, under g++ plain inline.
//
// Work of one decode token (the work of QuantizedDecodeGraphState::step,
// axiomlm/kernels/mps_kernels.mm:3195-3263), as phases of one launch:
//   per layer l:  5l+0 QKV   RMSNorm(x, ln1) -> QKV GEMV -> bias -> RoPE -> q, K/V slot
//                 5l+1 ATTN  split-KV attention per (query head, split)
//                 5l+2 O     O GEMV + residual -> x
//                 5l+3 GU    RMSNorm(x, ln2) -> gate|up GEMV -> SwiGLU -> h
//                 5l+4 DN    down GEMV + residual -> x
//   5L           LM    RMSNorm(x, lnf) -> lm_head GEMV -> logits, argmax keys
#pragma once

#ifdef __HIPCC__
#define SP_HD __host__ __device__ __forceinline__
#else
#define SP_HD inline
#endif

namespace sp {

// Launch shape.
constexpr int kThreads = 1024; // one workgroup per CU
constexpr int kWaves = 16;
constexpr int kCtl = 4;        // waves 0..3: staging (polls), epilogues; wave 0 also the epilogue operands
constexpr int kWorkers = 12;   // waves 4..15 stream weights and never poll
constexpr int kDepth = 8;      // weight chunks in flight per worker (register ring slots)
constexpr int kMaxLocal = 32;  // 16-row tiles a workgroup owns in one GEMV phase
constexpr int kMaxKB = 96;     // 128-column blocks of a GEMV input (K <= 12288)
constexpr int kMaxSplits = 16; // key splits per head
constexpr int kStageSlots = 12;  // input words per control-wave lane and staging pass
constexpr int kStagePass = kCtl * 64 * kStageSlots;  // words per staging pass
constexpr int kOOB = 0x7FFFFFF0;  // buffer offset past every descriptor: loads read zero

enum Kind { K_QKV = 0, K_ATTN = 1, K_O = 2, K_GU = 3, K_DN = 4, K_LM = 5, K_NONE = 6 };

struct Shape {
  int L, D, H, Hq, Hkv, hd, V, S;  // layers, model width, MLP width, heads, KV heads, head dim, vocab, cache slots
  int G;                           // workgroups (one per CU)
  int g128;                        // 1: one (scale, bias) per 128 columns; 0: per 64
};

SP_HD int cdiv(int a, int b) { return (a + b - 1) / b; }
SP_HD int q_dim(const Shape& s) { return s.Hq * s.hd; }
SP_HD int kv_dim(const Shape& s) { return s.Hkv * s.hd; }
SP_HD int qkv_rows(const Shape& s) { return q_dim(s) + 2 * kv_dim(s); }
SP_HD int n_phases(const Shape& s) { return 5 * s.L + 1; }
SP_HD int kind_of(const Shape& s, int ph) {
  if (ph >= 5 * s.L) return ph == 5 * s.L ? K_LM : K_NONE;
  return ph % 5;
}
SP_HD int layer_of(int ph) { return ph / 5; }
// The GEMV phase whose weights follow phase ph's in the weight stream (ATTN skipped).
SP_HD int next_gemv_phase(const Shape& s, int ph) {
  int nx = ph + 1;
  if (kind_of(s, nx) == K_ATTN) ++nx;
  return nx;
}

// ---------------------------------------------------------------------------
// GEMV phases.  Unit = one 16-row tile of the tile16 copy (a gate / up tile pair
// for GU).  Units are dealt to workgroups in contiguous runs; the local tiles of
// a workgroup are numbered ul = 0..nl-1 (GU: gates 0..n-1, then ups n..2n-1) and
// its chunks c = ul * KB + kb (one 1 KB weight chunk = 16 rows x 128 columns).
// Worker w takes chunks w, w + kWorkers, ... in blocks of kDepth.
// ---------------------------------------------------------------------------
struct Gemv {
  int kind;
  int units, KB, pair_off;  // pair_off: tile distance gate -> up (GU), 0 otherwise
  int tiles_alloc;          // tiles of the tile16 buffer (its size)
  int K, N;                 // input length, output rows (H for GU)
  int n, u0, nl, C;         // this workgroup: units, first unit, local tiles, chunks
};

SP_HD Gemv gemv_plan(const Shape& s, int kind, int g) {
  Gemv p{};
  p.kind = kind;
  if (kind == K_QKV) {
    p.K = s.D;
    p.N = qkv_rows(s);
    p.units = cdiv(p.N, 16);
    p.tiles_alloc = p.units;
  } else if (kind == K_O) {
    p.K = q_dim(s);
    p.N = s.D;
    p.units = cdiv(p.N, 16);
    p.tiles_alloc = p.units;
  } else if (kind == K_GU) {
    p.K = s.D;
    p.N = s.H;
    p.units = s.H / 16;
    p.pair_off = s.H / 16;
    p.tiles_alloc = 2 * s.H / 16;
  } else if (kind == K_DN) {
    p.K = s.H;
    p.N = s.D;
    p.units = cdiv(p.N, 16);
    p.tiles_alloc = p.units;
  } else if (kind == K_LM) {
    p.K = s.D;
    p.N = s.V;
    p.units = cdiv(p.N, 16);
    p.tiles_alloc = p.units;
  } else {
    p.KB = 1;
    return p;  // no weights
  }
  p.KB = cdiv(p.K, 128);
  const int base = p.units / s.G, rem = p.units % s.G;
  p.n = base + (g < rem ? 1 : 0);
  p.u0 = g * base + (g < rem ? g : rem);
  p.nl = kind == K_GU ? 2 * p.n : p.n;
  p.C = p.nl * p.KB;
  return p;
}

SP_HD int tile_of(const Gemv& p, int ul) {
  if (p.pair_off == 0) return p.u0 + ul;
  return ul < p.n ? p.u0 + ul : p.u0 + (ul - p.n) + p.pair_off;
}
// Buffer sizes of the tile16 copy (bytes).
SP_HD long w_bytes(const Gemv& p) { return (long)p.tiles_alloc * p.KB * 1024; }
SP_HD long sb_bytes(const Gemv& p, int g128) { return (long)p.tiles_alloc * p.KB * (g128 ? 64 : 128); }

// What one worker needs in its chunk loop: stream position t in [0, nt) maps to
// local chunk c0 + t * kWorkers (padding past C reads zero), so at each step the
// workgroup's workers read consecutive 1 KB chunks (a 12 KB contiguous window),
// spreading the concurrent requests over the HBM channels.
struct Run {
  int c0, nt, C, KB, u0, n, pair_off;
};
SP_HD Run worker_run(const Gemv& p, int w) {
  Run r;
  r.c0 = w < 0 ? 0 : w;
  const int mine = (w < 0 || w >= p.C) ? 0 : cdiv(p.C - w, kWorkers);
  r.nt = cdiv(mine, kDepth) * kDepth;
  r.C = p.C;
  r.KB = p.KB;
  r.u0 = p.u0;
  r.n = p.n;
  r.pair_off = p.pair_off;
  return r;
}
// Local chunk at stream position t, or -1 (padding / past the run).
SP_HD int run_chunk(const Run& r, int t) {
  const int c = r.c0 + t * kWorkers;
  return (t >= 0 && t < r.nt && c < r.C) ? c : -1;
}
SP_HD int run_tile(const Run& r, int ul) {
  if (r.pair_off == 0) return r.u0 + ul;
  return ul < r.n ? r.u0 + ul : r.u0 + (ul - r.n) + r.pair_off;
}
// Byte offsets of lane `lane`'s 16 code bytes and of its row's scale word(s) for
// local chunk c (kOOB for c < 0).
SP_HD int w_off(const Run& r, int c, int lane) {
  if (c < 0) return kOOB;
  const int ul = c / r.KB;
  const int base = run_tile(r, ul) * r.KB + (c - ul * r.KB);
  return (base * 64 + lane) * 16;
}
SP_HD int sb_off(const Run& r, int c, int lane, int g128) {
  if (c < 0) return kOOB;
  const int ul = c / r.KB;
  const int base = run_tile(r, ul) * r.KB + (c - ul * r.KB);
  return (base * 16 + (lane & 15)) * (g128 ? 4 : 8);
}

// ---------------------------------------------------------------------------
// Cross-workgroup words.  Every value one workgroup hands to another travels
// in a 64-bit word: 32 bits of payload (two fp16 values, or one fp32) and the
// 32-bit tag of the phase that wrote it.  A reader polls its words until each
// carries the tag it expects, so no grid barrier is needed; tags grow by one
// per phase over the runner's lifetime.
//   x     D/2 words         residual stream (fp16 pairs)
//   q     q_dim/2           rotated queries
//   kv    kv_dim            new key row (kv_dim/2 words), then the new value row
//   o     q_dim/2           attention output
//   h     H/2               SwiGLU output
//   part  Hq*kMaxSplits*(hd+2)  split partials (m, l, o[hd]) as fp32
//   keys  2*G               per-workgroup best lm_head key (hi, lo)
// ---------------------------------------------------------------------------
struct Words {
  long x, q, kv, o, h, part, keys, total;
};
SP_HD Words words_layout(const Shape& s) {
  Words w{};
  long off = 0;
  w.x = off;
  off += s.D / 2;
  w.q = off;
  off += q_dim(s) / 2;
  w.kv = off;
  off += kv_dim(s);
  w.o = off;
  off += q_dim(s) / 2;
  w.h = off;
  off += s.H / 2;
  w.part = off;
  off += (long)s.Hq * kMaxSplits * (s.hd + 2);
  w.keys = off;
  off += 2L * s.G;
  w.total = off;
  return w;
}
// Word indices (from the start of the words buffer).  Output row r of a GEMV
// lands in word r / 2 of its vector (rows 2i, 2i+1 share word i).
SP_HD long x_word(const Words& w, int row) { return w.x + row / 2; }
SP_HD long h_word(const Words& w, int row) { return w.h + row / 2; }
// QKV rows: q rows [0, q_dim), then key rows, then value rows.
SP_HD long qkv_word(const Shape& s, const Words& w, int row) {
  const int qd = q_dim(s), kvd = kv_dim(s);
  if (row < qd) return w.q + row / 2;
  if (row < qd + kvd) return w.kv + (row - qd) / 2;
  return w.kv + kvd / 2 + (row - qd - kvd) / 2;
}
// Word i (dims 2i, 2i+1) of query head hq, of KV head kvh's new key / value row,
// of head hq's attention output.
SP_HD long q_word(const Shape& s, const Words& w, int hq, int i) { return w.q + (long)hq * (s.hd / 2) + i; }
SP_HD long kvnew_word(const Shape& s, const Words& w, int kvh, int i, int is_v) {
  return w.kv + (is_v ? kv_dim(s) / 2 : 0) + (long)kvh * (s.hd / 2) + i;
}
SP_HD long o_word(const Shape& s, const Words& w, int hq, int i) { return w.o + (long)hq * (s.hd / 2) + i; }
SP_HD long key_word(const Words& w, int g, int k) { return w.keys + 2L * g + k; }

// Tag of phase ph of a launch whose first phase has tag tag0.
SP_HD unsigned tag_of(unsigned tag0, int ph) { return tag0 + (unsigned)ph; }

// Staging: in the pass starting at word r0 (a multiple of kStagePass),
// control-wave thread tid (< kCtl * 64) owns input words i = r0 + tid + kCtl * 64 * j,
// j < kStageSlots.
SP_HD int stage_word(int r0, int tid, int j) { return r0 + tid + kCtl * 64 * j; }
// Sentinel word of control-wave thread tid: an evenly spread sample of the nw words.
SP_HD int stage_sentinel(int tid, int nw) { return (int)(((long)tid * nw) / (kCtl * 64)); }

// ---------------------------------------------------------------------------
// LDS carve-up (bytes).
// ---------------------------------------------------------------------------
struct Lds {
  int xs;     // f16 [kMaxKB * 128] staged GEMV input
  int lnw;    // f16 [kMaxKB * 128] RMSNorm weight of the staged input
  int zero;   // 16 zero halves
  int cx;     // f32x2 [2 * kMaxKB] magic-offset sum and plain sum per 64-group
  int red;    // float [kMaxLocal][kWorkers][16] partial tiles
  int cs;     // float2 [kMaxLocal * 16] RoPE (cos, sin) of the QKV rows
  int bias;   // f16 [kMaxLocal * 16]
  int xold;   // f16 [kMaxLocal * 16] residual input of the O / DN rows
  int att;    // float [kWaves][2 + 128] per-wave attention state
  int qv;     // float [3][128] query, new key, new value of an attention item
  int misc;   // float [16]
  int flag;   // int [4]
  int total;
};
SP_HD Lds lds_layout() {
  Lds l{};
  int off = 0;
  l.xs = off;
  off += kMaxKB * 128 * 2;
  l.lnw = off;
  off += kMaxKB * 128 * 2;
  l.zero = off;
  off += 32;
  l.cx = off;
  off += 2 * kMaxKB * 8;
  l.red = off;
  off += kMaxLocal * kWorkers * 16 * 4;
  l.cs = off;
  off += kMaxLocal * 16 * 8;
  l.bias = off;
  off += kMaxLocal * 16 * 2;
  l.xold = off;
  off += kMaxLocal * 16 * 2;
  l.att = off;
  off += kWaves * (2 + 128) * 4;
  l.qv = off;
  off += 3 * 128 * 4;
  l.misc = off;
  off += 16 * 4;
  l.flag = off;
  off += 16;
  l.total = off;
  return l;
}
// Output row of lane row j of local tile ul (GU: ul < n, the gate tile's row,
// which is also the SwiGLU output row).
SP_HD int epi_row(const Gemv& p, int ul, int j) { return (p.u0 + ul) * 16 + j; }
// Partial tile slot of (local tile ul, worker w, row j) in floats from Lds::red.
SP_HD int red_index(int ul, int w, int j) { return (ul * kWorkers + w) * 16 + j; }

// ---------------------------------------------------------------------------
// Attention.  Item = (query head hq, split sp); the keys of the head, slots
// [0, active), are split into ns contiguous ranges.  The slot write_pos holds
// this step's key and value, which come from the kv words instead of the cache.
// ---------------------------------------------------------------------------
SP_HD int attn_keys_per_split(int active, int ns) { return cdiv(active, ns); }
SP_HD int attn_k0(int active, int ns, int sp) {
  const int k = sp * attn_keys_per_split(active, ns);
  return k < active ? k : active;
}
SP_HD int attn_k1(int active, int ns, int sp) {
  const int k = attn_k0(active, ns, sp) + attn_keys_per_split(active, ns);
  return k < active ? k : active;
}
// Element offset (f16 units) of dims [e0, e0 + 8) of cache slot `slot`, KV head kvh.
SP_HD long cache_elem(const Shape& s, int kvh, int slot, int e0) { return ((long)kvh * s.S + slot) * s.hd + e0; }
// Word of partial (hq, sp): m at +0, l at +1, o[e] at +2+e.
SP_HD long part_word(const Shape& s, const Words& w, int hq, int sp, int e) {
  return w.part + ((long)hq * kMaxSplits + sp) * (s.hd + 2) + e;
}
// Splits per head: at least 32 keys per split, at most one item per workgroup.
SP_HD int choose_splits(const Shape& s, int active) {
  int ns = s.G / s.Hq;
  const int by_len = cdiv(active, 32);
  if (ns > by_len) ns = by_len;
  if (ns > kMaxSplits) ns = kMaxSplits;
  if (ns < 1) ns = 1;
  return ns;
}

}  // namespace sp
