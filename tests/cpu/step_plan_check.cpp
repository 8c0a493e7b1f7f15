// CPU enumeration check of the persistent decode-step kernel's index math
// (axiomlm_amd/csrc/step_plan.h, the same functions the kernel calls).
//
// For each shape it walks a whole launch -- every phase, workgroup, wave, lane,
// ring slot and stream position, every staging word, epilogue row, attention
// item / key step (for many context lengths and write slots) and cross-
// workgroup word -- in the order and with the loop bounds the kernel uses, and
//   * asserts each offset lies inside the buffer it addresses (weights and
//     scales of the tile16 copies, KV cache views, RoPE table, embedding rows,
//     norm weights, logits, argmax keys, the words buffer, the LDS carve-up);
//   * reads or writes a host buffer of exactly that buffer's size at the offset,
//     so that AddressSanitizer (the build uses -fsanitize=address) reports any
//     access the assertions miss;
//   * checks coverage: every weight chunk of every tile is consumed exactly once
//     per phase, every output row is written once, the key splits of every head
//     partition [0, active) and exactly one of them holds the new key.
// Exit status 0 and one "ok" line per shape on success.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "step_plan.h"

using namespace sp;

static int g_fail = 0;
#define CHECK(cond, ...)                                  \
  do {                                                    \
    if (!(cond)) {                                        \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                  \
      std::fprintf(stderr, "\n");                         \
      if (++g_fail > 20) std::exit(1);                    \
    }                                                     \
  } while (0)

// A host stand-in of one device buffer: every access goes through touch().
struct Buf {
  const char* name;
  std::vector<unsigned char> mem;
  Buf(const char* n, long bytes) : name(n), mem((size_t)bytes) {}
  // In-range check, then a real read of the bytes (ASan-instrumented).
  void touch(long off, long len) {
    CHECK(off >= 0 && off + len <= (long)mem.size(), "%s: bytes [%ld, %ld) outside %zu", name, off, off + len,
          mem.size());
    if (off < 0 || off + len > (long)mem.size()) return;
    volatile unsigned char sink = 0;
    unsigned char* p = mem.data() + off;
    for (long i = 0; i < len; ++i) sink ^= p[i];
    (void)sink;
  }
  // Buffer loads with an out-of-range offset read zero and touch nothing.
  void buffer_load(long off, long len) {
    if (off == kOOB) return;
    touch(off, len);
  }
};

struct Bufs {
  Shape s;
  Words W;
  Lds L;
  Buf words, lds, kc, vc, freqs, bias, wte, wte_sb, lnw, logits, keys, norm_out;
  std::vector<Buf> w, sb;  // per GEMV kind: tile16 codes, scales
  Bufs(const Shape& sh, int rope_len)
      : s(sh),
        W(words_layout(sh)),
        L(lds_layout()),
        words("words", W.total * 8),
        lds("lds", L.total),
        kc("k_cache", (long)sh.Hkv * sh.S * sh.hd * 2),
        vc("v_cache", (long)sh.Hkv * sh.S * sh.hd * 2),
        freqs("freqs", (long)rope_len * (sh.hd / 2) * 2 * 4),
        bias("qkv_bias", (long)qkv_rows(sh) * 2),
        wte("wte_q8", (long)sh.V * sh.D),
        wte_sb("wte_sb", (long)sh.V * (sh.D / 64) * 4),
        lnw("ln_w", (long)sh.D * 2),
        logits("logits", (long)sh.V * 2),
        keys("argmax_keys", (long)((sh.V + 7) / 8) * 8),
        norm_out("norm_out", (long)sh.D * 2) {
    for (int k = 0; k < 6; ++k) {
      const Gemv p = gemv_plan(sh, k, 0);
      const bool has = k == K_QKV || k == K_O || k == K_GU || k == K_DN || k == K_LM;
      w.emplace_back("tile16 codes", has ? w_bytes(p) : 0);
      sb.emplace_back("tile16 scales", has ? sb_bytes(p, sh.g128) : 0);
    }
  }
  void word(long i) { words.touch(i * 8, 8); }
  void lds_at(int region, long off, long len, long region_bytes) {
    CHECK(off >= 0 && off + len <= region_bytes, "lds region at %d: [%ld, %ld) outside %ld", region, off, off + len,
          region_bytes);
    lds.touch(region + off, len);
  }
};

static long words_len_of_input(const Shape& s, const Words& W, int kind, long* base) {
  if (kind == K_O) {
    *base = W.o;
    return q_dim(s) / 2;
  }
  if (kind == K_DN) {
    *base = W.h;
    return s.H / 2;
  }
  *base = W.x;
  return s.D / 2;
}

// One GEMV phase of one workgroup: staging, ring, epilogue.
static void check_gemv_phase(Bufs& B, int ph, int g, std::vector<int>& row_writes, int write_pos, int rope_pos,
                             int rope_len) {
  const Shape& s = B.s;
  const Words& W = B.W;
  const Lds& L = B.L;
  const int kind = kind_of(s, ph);
  const Gemv p = gemv_plan(s, kind, g);
  CHECK(p.nl <= kMaxLocal, "phase %d g %d: %d local tiles > %d", ph, g, p.nl, kMaxLocal);
  CHECK(p.KB <= kMaxKB, "phase %d: KB %d > %d", ph, p.KB, kMaxKB);
  const int nxt_ph = next_gemv_phase(s, ph);
  const int nxt_kind = kind_of(s, nxt_ph);
  Buf& wb = B.w[kind];
  Buf& sbb = B.sb[kind];
  const int sbl = s.g128 ? 4 : 8;
  const long xs_bytes = (long)kMaxKB * 128 * 2;
  const long cx_bytes = 2L * kMaxKB * 8;
  const long red_bytes = (long)kMaxLocal * kWorkers * 16 * 4;
  const long rows_bytes = (long)kMaxLocal * 16;

  if (p.n > 0) {
    // control wave: norm weights into LDS, epilogue operands, zeroed tiles
    const bool norm = kind == K_QKV || kind == K_GU || kind == K_LM;
    if (norm)
      for (int lane = 0; lane < 64; ++lane)
        for (int i = lane; i < p.K / 8; i += 64) {
          B.lnw.touch((long)i * 16, 16);
          B.lds_at(L.lnw, (long)i * 16, 16, xs_bytes);
        }
    const int nrows = p.nl * 16;
    if (kind == K_QKV) {
      for (int lane = 0; lane < 64; ++lane)
        for (int lr = lane; lr < nrows; lr += 64) {
          const int row = epi_row(p, lr >> 4, lr & 15);
          if (row < q_dim(s) + kv_dim(s)) {
            const int within = row < q_dim(s) ? row : row - q_dim(s);
            const int fi = (within % s.hd) >> 1;
            B.freqs.touch((((long)rope_pos * (s.hd / 2) + fi) * 2) * 4, 8);
          }
          B.lds_at(L.cs, (long)lr * 8, 8, rows_bytes * 8);
          B.lds_at(L.bias, (long)lr * 2, 2, rows_bytes * 2);
          if (row < qkv_rows(s)) B.bias.touch((long)row * 2, 2);
        }
    } else if (kind == K_O || kind == K_DN) {
      const int nwords = std::min(nrows, p.N - epi_row(p, 0, 0)) / 2;
      for (int lane = 0; lane < 64; ++lane)
        for (int k = 0; k < kMaxLocal * 8 / 64; ++k) {
          const int i = lane + 64 * k;
          if (i >= nwords) continue;
          const long wi = x_word(W, epi_row(p, 0, 2 * i));
          CHECK(wi >= W.x && wi < W.x + s.D / 2, "x_old word %ld", wi);
          B.word(wi);
          if (kind == K_O && ph == 2) {  // layer 0: the embedding row instead
            const long ei = wi - W.x;
            B.wte.touch(2 * ei, 2);
            B.wte_sb.touch(((2 * ei) / 64) * 4, 4);
          }
          B.lds_at(L.xold, (long)i * 4, 4, rows_bytes * 2);
        }
    }
    for (int i = 0; i < p.nl * kWorkers * 16; ++i) B.lds_at(L.red, (long)i * 4, 4, red_bytes);
    // staging, all threads
    long base = 0;
    const long src_len = words_len_of_input(s, W, kind, &base);
    const int nw = p.K / 2, nwp = cdiv(p.K, 128) * 64;
    CHECK(nw <= src_len, "phase %d: %d input words > %ld", ph, nw, src_len);
    const bool embed = kind == K_QKV && ph == 0;
    if (!embed)
      for (int tid = 0; tid < kCtl * 64; ++tid) {
        const int sent = stage_sentinel(tid, nw);
        CHECK(sent >= 0 && sent < nw, "sentinel %d of %d", sent, nw);
        B.word(base + sent);
      }
    std::vector<int> staged(nwp, 0);
    for (int r0 = 0; r0 < nwp; r0 += kStagePass)
      for (int tid = 0; tid < kCtl * 64; ++tid)
        for (int j = 0; j < kStageSlots; ++j) {
        const int i = stage_word(r0, tid, j);
        if (i < nwp) staged[i]++;
        if (i < nw) {
          if (embed) {
            B.wte.touch(2L * i, 2);
            B.wte_sb.touch(((2L * i) / 64) * 4, 4);
          } else {
            B.word(base + i);
          }
        }
        if (i < nwp) B.lds_at(L.xs, (long)i * 4, 4, xs_bytes);
      }
    for (int i = 0; i < nwp; ++i) CHECK(staged[i] == 1, "phase %d: staging word %d written %d times", ph, i, staged[i]);
    for (int tid = 0; tid < kCtl * 64; ++tid)
      for (int i = tid; i < nwp; i += kCtl * 64) {
        B.lds_at(L.xs, (long)i * 4, 4, xs_bytes);
        if (norm && i < nw) B.lds_at(L.lnw, (long)i * 4, 4, xs_bytes);
        if (kind == K_LM && g == 0 && i < nw) B.norm_out.touch((long)i * 4, 4);
        if ((tid & 31) == 0) B.lds_at(L.cx, (long)(i >> 5) * 8, 8, cx_bytes);
      }
  }

  // workers: the chunk loop, refills into the next phase
  std::vector<int> seen(p.C, 0);
  for (int w = 0; w < kWorkers; ++w) {
    const Run cur = worker_run(p, w);
    const Gemv pn = gemv_plan(s, nxt_kind, g);
    const Run nxt = worker_run(pn, w);
    Buf& nwb = B.w[nxt_kind];
    Buf& nsbb = B.sb[nxt_kind];
    auto issue = [&](const Run& r, const Gemv& pp, Buf& bw, Buf& bs, int t) {
      const int c = run_chunk(r, t);
      CHECK(c < pp.C, "chunk %d >= C %d", c, pp.C);
      for (int lane = 0; lane < 64; ++lane) {
        bw.buffer_load(w_off(r, c, lane), 16);
        bs.buffer_load(sb_off(r, c, lane, s.g128), sbl);
      }
    };
    auto consume = [&](int c) {
      CHECK(c >= 0 && c < p.C, "consumed chunk %d outside [0, %d)", c, p.C);
      seen[c]++;
      const int ul = c / cur.KB, kb = c - ul * cur.KB;
      CHECK(ul < p.nl, "local tile %d >= %d", ul, p.nl);
      for (int lane = 0; lane < 64; ++lane) {
        if ((lane & 15) == 0)
          for (int q = 0; q < 4; ++q) B.lds_at(L.xs, ((long)kb * 128 + 8 * (lane >> 4) + 32 * q) * 2, 16, xs_bytes);
        B.lds_at(L.cx, (long)(2 * kb) * 8, 16, cx_bytes);
        B.lds_at(L.red, (long)red_index(ul, w, lane & 15) * 4, 4, red_bytes);
      }
    };
    const int n = cur.nt;
    CHECK(n % kDepth == 0, "run of %d positions", n);
    if (n > 0) {
      for (int t0 = 0; t0 < n - kDepth; t0 += kDepth)
        for (int j = 0; j < kDepth; ++j) {
          const int c = run_chunk(cur, t0 + j);
          if (c >= 0) consume(c);
          issue(cur, p, wb, sbb, t0 + j + kDepth);
        }
      for (int j = 0; j < kDepth; ++j) {
        const int c = run_chunk(cur, n - kDepth + j);
        if (c >= 0) consume(c);
        issue(nxt, pn, nwb, nsbb, j);
      }
    } else {
      for (int j = 0; j < kDepth; ++j) issue(nxt, pn, nwb, nsbb, j);
    }
  }
  for (int c = 0; c < p.C; ++c) CHECK(seen[c] == 1, "phase %d g %d: chunk %d consumed %d times", ph, g, c, seen[c]);

  // control wave epilogue
  if (p.n > 0) {
    for (int ul0 = 0; ul0 < p.nl; ul0 += 4)
      for (int lane = 0; lane < 64; ++lane) {
        const int ul = ul0 + (lane >> 4), j = lane & 15;
        const int lr = ul * 16 + j;
        const int row = epi_row(p, ul, j);
        if (kind == K_GU) {
          if (ul >= p.n || ul0 >= p.n || row >= p.N) continue;
          for (int w = 0; w < kWorkers; ++w) {
            B.lds_at(L.red, (long)red_index(ul, w, j) * 4, 4, red_bytes);
            B.lds_at(L.red, (long)red_index(ul + p.n, w, j) * 4, 4, red_bytes);
          }
          row_writes[row]++;
          if ((row & 1) == 0) {
            const long wi = h_word(W, row);
            CHECK(wi >= W.h && wi < W.h + s.H / 2, "h word");
            B.word(wi);
          }
          continue;
        }
        if (ul >= p.nl || row >= p.N) continue;
        for (int w = 0; w < kWorkers; ++w) B.lds_at(L.red, (long)red_index(ul, w, j) * 4, 4, red_bytes);
        row_writes[row]++;
        if (kind == K_QKV) {
          B.lds_at(L.bias, (long)lr * 2, 2, rows_bytes * 2);
          B.lds_at(L.cs, (long)lr * 8, 8, rows_bytes * 8);
          if ((row & 1) == 0) {
            const long wi = qkv_word(s, W, row);
            CHECK(wi >= W.q && wi < W.kv + kv_dim(s), "qkv word");
            B.word(wi);
            if (row >= q_dim(s)) {
              const bool is_k = row < q_dim(s) + kv_dim(s);
              const int within = is_k ? row - q_dim(s) : row - q_dim(s) - kv_dim(s);
              (is_k ? B.kc : B.vc).touch(cache_elem(s, within / s.hd, write_pos, within % s.hd) * 2, 4);
            }
          }
        } else if (kind == K_O || kind == K_DN) {
          B.lds_at(L.xold, (long)lr * 2, 2, rows_bytes * 2);
          if ((row & 1) == 0) {
            const long wi = x_word(W, row);
            CHECK(wi >= W.x && wi < W.x + s.D / 2, "x word");
            B.word(wi);
          }
        } else if (kind == K_LM) {
          B.logits.touch((long)row * 2, 2);
          if (j == 0) B.keys.touch((long)(p.u0 + ul) * 8, 8);
        }
      }
  }
  if (kind == K_LM) {
    B.word(key_word(W, g, 0));
    B.word(key_word(W, g, 1));
  }
}

static void check_attention(Bufs& B, int active, int write_pos) {
  const Shape& s = B.s;
  const Words& W = B.W;
  const Lds& L = B.L;
  const int hd = s.hd, LPT = hd / 8, KPW = 64 / LPT, nq = hd / 2;
  const int ns = choose_splits(s, active);
  CHECK(ns >= 1 && ns <= kMaxSplits, "splits %d", ns);
  const int n_rep = s.Hq / s.Hkv;
  for (int hq = 0; hq < s.Hq; ++hq) {
    int covered = 0, holders = 0;
    for (int spl = 0; spl < ns; ++spl) {
      const int kvh = hq / n_rep;
      const int k0 = attn_k0(active, ns, spl), k1 = attn_k1(active, ns, spl);
      CHECK(k0 >= 0 && k0 <= k1 && k1 <= active, "split [%d, %d) of %d", k0, k1, active);
      CHECK(k0 == covered, "splits of head %d not contiguous", hq);
      covered = k1;
      const bool has_new = write_pos >= k0 && write_pos < k1;
      holders += has_new ? 1 : 0;
      for (int lane = 0; lane < 64; ++lane) {
        if (lane < nq) {
          B.word(q_word(s, W, hq, lane));
          CHECK(q_word(s, W, hq, lane) < W.q + q_dim(s) / 2, "q word");
          if (has_new) {
            B.word(kvnew_word(s, W, kvh, lane, 0));
            B.word(kvnew_word(s, W, kvh, lane, 1));
            CHECK(kvnew_word(s, W, kvh, lane, 1) < W.kv + kv_dim(s), "kv word");
          }
          for (int k = 0; k < 3; ++k) B.lds_at(L.qv, (long)(k * 128 + 2 * lane + 1) * 4, 4, 3 * 128 * 4);
        }
      }
      for (int wave = 0; wave < kWaves; ++wave)
        for (int lane = 0; lane < 64; ++lane) {
          const int sub = lane / LPT, e0 = (lane % LPT) * 8;
          B.lds_at(L.qv, (long)(e0 + 7) * 4, 4, 3 * 128 * 4);
          for (int kb = k0 + wave * KPW; kb < k1; kb += kWaves * KPW) {
            const int key = kb + sub;
            const bool valid = key < k1 && key != write_pos;
            if (!valid) continue;
            B.kc.touch(cache_elem(s, kvh, key, e0) * 2, 16);
            B.vc.touch(cache_elem(s, kvh, key, e0) * 2, 16);
          }
          if (lane < LPT) B.lds_at(L.att, (long)(wave * (2 + 128) + 2 + e0 + 7) * 4, 4, kWaves * (2 + 128) * 4);
        }
      for (int lane = 0; lane < 64; ++lane) {
        const int ea = lane < nq ? 2 * lane : 0;
        if (ns > 1 && spl > 0) {
          B.word(part_word(s, W, hq, spl, 0));
          B.word(part_word(s, W, hq, spl, 3 + ea));
          CHECK(part_word(s, W, hq, spl, 3 + ea) < W.keys, "part word");
        } else {
          for (int s2 = 1; s2 < ns; ++s2) {
            B.word(part_word(s, W, hq, s2, 1));
            if (lane < nq) B.word(part_word(s, W, hq, s2, 3 + ea));
          }
          if (lane < nq) {
            B.word(o_word(s, W, hq, lane));
            CHECK(o_word(s, W, hq, lane) < W.o + q_dim(s) / 2, "o word");
          }
        }
      }
    }
    CHECK(covered == active, "head %d: splits cover %d of %d keys", hq, covered, active);
    CHECK(holders == 1, "head %d: %d splits hold the new key (write_pos %d, active %d)", hq, holders, write_pos,
          active);
  }
}

static void check_shape(const char* name, Shape s, int rope_len) {
  const int before = g_fail;
  CHECK(words_layout(s).total < 0x7FFFFFFFL, "words do not fit int indices");
  CHECK(lds_layout().total <= 160 * 1024, "LDS %d bytes", lds_layout().total);
  Bufs B(s, rope_len);
  // unit coverage of every GEMV kind
  for (int kind : {K_QKV, K_O, K_GU, K_DN, K_LM}) {
    std::vector<int> cov(gemv_plan(s, kind, 0).units, 0);
    for (int g = 0; g < s.G; ++g) {
      const Gemv p = gemv_plan(s, kind, g);
      for (int u = p.u0; u < p.u0 + p.n; ++u) {
        CHECK(u >= 0 && u < (int)cov.size(), "unit %d", u);
        if (u >= 0 && u < (int)cov.size()) cov[u]++;
      }
      for (int ul = 0; ul < p.nl; ++ul) CHECK(tile_of(p, ul) < p.tiles_alloc, "tile %d", tile_of(p, ul));
    }
    for (size_t u = 0; u < cov.size(); ++u) CHECK(cov[u] == 1, "kind %d unit %zu owned %d times", kind, u, cov[u]);
  }
  // prime of phase 0
  for (int w = 0; w < kWorkers; ++w)
    for (int g = 0; g < s.G; ++g) {
      const Gemv p = gemv_plan(s, K_QKV, g);
      const Run r = worker_run(p, w);
      for (int j = 0; j < kDepth; ++j)
        for (int lane = 0; lane < 64; ++lane) {
          B.w[K_QKV].buffer_load(w_off(r, run_chunk(r, j), lane), 16);
          B.sb[K_QKV].buffer_load(sb_off(r, run_chunk(r, j), lane, s.g128), s.g128 ? 4 : 8);
        }
    }
  // every phase of a launch (GEMV phases of layer 0 and 1 and the lm_head; every
  // layer indexes the same way), with write slots at both ends of the cache
  const int wps[] = {0, s.S / 2, s.S - 1};
  for (int wp : wps) {
    for (int ph = 0; ph < n_phases(s); ++ph) {
      const int kind = kind_of(s, ph);
      if (layer_of(ph) >= 2 && kind != K_LM) continue;
      if (kind == K_ATTN) continue;
      std::vector<int> rows(gemv_plan(s, kind, 0).N, 0);
      for (int g = 0; g < s.G; ++g) check_gemv_phase(B, ph, g, rows, wp, rope_len - 1, rope_len);
      for (size_t r = 0; r < rows.size(); ++r)
        CHECK(rows[r] == 1, "phase %d row %zu written %d times", ph, r, rows[r]);
    }
  }
  // attention over many context lengths, write slot = newest key (and ring wraps)
  for (int active = 1; active <= s.S; active += (active < 300 ? 1 : 97)) {
    check_attention(B, active, active - 1);
    if (active == s.S) check_attention(B, active, s.S / 3);
  }
  check_attention(B, s.S, 0);
  check_attention(B, s.S, s.S - 1);
  // greedy reduction
  for (int g = 0; g < s.G; ++g) {
    B.word(key_word(B.W, g, 0));
    B.word(key_word(B.W, g, 1));
  }
  if (g_fail == before) std::printf("ok %s\n", name);
}

int main() {
  // L, D, H, Hq, Hkv, hd, V, S, G, g128
  check_shape("c1 (4 layers, d 256, 4 x 64 heads, MLP 704, vocab 1024)", Shape{4, 256, 704, 4, 4, 64, 1024, 128, 256, 0},
              256);
  check_shape("smoke (GQA 2, vocab 512, 32 slots)", Shape{2, 256, 704, 4, 2, 64, 512, 32, 256, 0}, 64);
  check_shape("wide GQA-2 (d 1024, 8 x 128 heads, MLP 2816, group 128)", Shape{2, 1024, 2816, 8, 4, 128, 2048, 256, 256, 1},
              256);
  check_shape("7B layer shape, group 128, 4096 slots", Shape{3, 4096, 11008, 32, 32, 128, 32000, 4096, 256, 1}, 16384);
  check_shape("7B layer shape, group 64, 4096 slots", Shape{2, 4096, 11008, 32, 32, 128, 32000, 4096, 256, 0}, 16384);
  check_shape("7B layer shape on 80 CUs", Shape{2, 4096, 11008, 32, 32, 128, 32000, 512, 80, 1}, 1024);
  check_shape("GQA 8:1, d 2048, vocab 49152", Shape{2, 2048, 5632, 16, 2, 128, 49152, 300, 256, 1}, 600);
  if (g_fail) {
    std::fprintf(stderr, "%d check(s) failed\n", g_fail);
    return 1;
  }
  return 0;
}
