// TEST INFRASTRUCTURE ONLY: a C-ABI driver over the reference's own CPU core,
// compiled together with the reference sources csrc/src/mask_cpu.cpp and
// csrc/src/pda_cpu.cpp (read in place from the reference checkout) into
// oracle/_ref/libbpd_ref.so.  It only marshals flat arrays into the
// reference's structs (mask.hpp:18-35, pda.hpp:46-91) and calls its
// functions; no reference code is restated here.
#include <cstring>
#include <thread>
#include <vector>

#include "bpdecode/mask.hpp"
#include "bpdecode/pda.hpp"

using namespace bpdecode;

namespace {

PdaTable table(int32_t n, int32_t rs, int32_t ra, const uint8_t* acc, const uint8_t* live,
               const int32_t* off, const int32_t* kind, const int32_t* lo, const int32_t* hi,
               const int32_t* dst, const int32_t* callee) {
  PdaTable g;
  g.num_states = n;
  g.root_start = rs;
  g.root_accept = ra;
  g.accept.assign(acc, acc + n);
  g.live.assign(live, live + n);
  g.edge_offsets.assign(off, off + n + 1);
  const int32_t nnz = off[n];
  g.edge_kind.assign(kind, kind + nnz);
  g.edge_lo.assign(lo, lo + nnz);
  g.edge_hi.assign(hi, hi + nnz);
  g.edge_dst.assign(dst, dst + nnz);
  g.edge_callee.assign(callee, callee + nnz);
  return g;
}

PdaTokens tokens(int32_t vocab, int32_t eos, const int32_t* off, const uint8_t* bytes) {
  PdaTokens t;
  t.vocab_size = vocab;
  t.eos_id = eos;
  t.offsets.assign(off, off + vocab + 1);
  t.bytes.assign(bytes, bytes + off[vocab]);
  return t;
}

FsaTable fsa(int32_t n, int32_t m, int32_t dead, const int32_t* trans, const uint8_t* acc,
             const uint8_t* live) {
  FsaTable f;
  f.num_states = n;
  f.num_symbols = m;
  f.dead = dead;
  f.trans.assign(trans, trans + int64_t(n) * m);
  f.accept.assign(acc, acc + n);
  if (live) f.live.assign(live, live + n);
  return f;
}

TokenSymbols symbols(int32_t vocab, int32_t eos, const int32_t* off, const int32_t* sym) {
  TokenSymbols t;
  t.vocab_size = vocab;
  t.eos_id = eos;
  t.offsets.assign(off, off + vocab + 1);
  t.symbols.assign(sym, sym + off[vocab]);
  return t;
}

}  // namespace

#define TBL int32_t n, int32_t rs, int32_t ra, const uint8_t *acc, const uint8_t *live, \
            const int32_t *off, const int32_t *kind, const int32_t *lo, const int32_t *hi, \
            const int32_t *dst, const int32_t *callee
#define TPASS n, rs, ra, acc, live, off, kind, lo, hi, dst, callee

extern "C" {

void ref_pda_init(TBL, int32_t* out) {
  PdaTable g = table(TPASS);
  PdaConfigSet c;
  pda_init(g, c);
  std::memcpy(out, &c, sizeof c);
}

int ref_pda_advance_byte(TBL, int32_t* cfg, int32_t byte) {
  PdaTable g = table(TPASS);
  PdaConfigSet c;
  std::memcpy(&c, cfg, sizeof c);
  const bool ok = pda_advance_byte(g, c, byte);
  std::memcpy(cfg, &c, sizeof c);
  return ok ? 1 : 0;
}

void ref_pda_compute_mask(TBL, int32_t vocab, int32_t eos, const int32_t* toff,
                          const uint8_t* tb, const int32_t* configs, int32_t batch,
                          uint32_t* bits) {
  compute_mask_pda_batch(table(TPASS), tokens(vocab, eos, toff, tb),
                         reinterpret_cast<const PdaConfigSet*>(configs), batch, bits);
}

void ref_pda_apply_mask(TBL, int32_t vocab, int32_t eos, const int32_t* toff, const uint8_t* tb,
                        const int32_t* configs, int32_t batch, float* logits, float neg_inf) {
  apply_mask_pda_batch(table(TPASS), tokens(vocab, eos, toff, tb),
                       reinterpret_cast<const PdaConfigSet*>(configs), batch, logits, neg_inf);
}

// The same call split over `threads` host threads by rows (each row's mask
// is independent; the reference's tables are shared read-only): the
// parallel CPU baseline.
void ref_pda_apply_mask_threads(TBL, int32_t vocab, int32_t eos, const int32_t* toff,
                                const uint8_t* tb, const int32_t* configs, int32_t batch,
                                float* logits, float neg_inf, int32_t threads) {
  const PdaTable g = table(TPASS);
  const PdaTokens t = tokens(vocab, eos, toff, tb);
  const PdaConfigSet* cs = reinterpret_cast<const PdaConfigSet*>(configs);
  if (threads < 1) threads = 1;
  std::vector<std::thread> pool;
  const int32_t per = (batch + threads - 1) / threads;
  for (int32_t r0 = 0; r0 < batch; r0 += per) {
    const int32_t n = batch - r0 < per ? batch - r0 : per;
    pool.emplace_back([&, r0, n] { apply_mask_pda_batch(g, t, cs + r0, n, logits + int64_t(r0) * vocab, neg_inf); });
  }
  for (auto& th : pool) th.join();
}

void ref_pda_advance(TBL, int32_t vocab, int32_t eos, const int32_t* toff, const uint8_t* tb,
                     int32_t* configs, const int32_t* token_ids, int32_t batch, uint8_t* ok) {
  advance_state_pda_batch(table(TPASS), tokens(vocab, eos, toff, tb),
                          reinterpret_cast<PdaConfigSet*>(configs), token_ids, batch, ok);
}

void ref_fsa_build_reachability(int32_t n, int32_t m, const int32_t* trans, const uint8_t* acc,
                                uint8_t* live_out) {
  FsaTable f = fsa(n, m, n - 1, trans, acc, nullptr);
  build_reachability(f);
  std::memcpy(live_out, f.live.data(), size_t(n));
}

int32_t ref_fsa_step(int32_t n, int32_t m, int32_t dead, const int32_t* trans, const uint8_t* acc,
                     const uint8_t* live, int32_t vocab, int32_t eos, const int32_t* off,
                     const int32_t* sym, int32_t state, int32_t token) {
  return step(fsa(n, m, dead, trans, acc, live), symbols(vocab, eos, off, sym), state, token);
}

void ref_fsa_step_table(int32_t n, int32_t m, int32_t dead, const int32_t* trans,
                        const uint8_t* acc, const uint8_t* live, int32_t vocab, int32_t eos,
                        const int32_t* off, const int32_t* sym, const int32_t* states,
                        int32_t nstates, int32_t* out) {
  FsaTable f = fsa(n, m, dead, trans, acc, live);
  TokenSymbols t = symbols(vocab, eos, off, sym);
  for (int32_t i = 0; i < nstates; ++i)
    for (int32_t tok = 0; tok < vocab; ++tok)
      out[int64_t(i) * vocab + tok] = step(f, t, states[i], tok);
}

void ref_fsa_compute_mask_batch(int32_t n, int32_t m, int32_t dead, const int32_t* trans,
                                const uint8_t* acc, const uint8_t* live, int32_t vocab,
                                int32_t eos, const int32_t* off, const int32_t* sym,
                                const int32_t* states, int32_t batch, uint32_t* bits) {
  compute_mask_batch(fsa(n, m, dead, trans, acc, live), symbols(vocab, eos, off, sym), states,
                     batch, bits);
}

void ref_fsa_apply_mask_batch(int32_t n, int32_t m, int32_t dead, const int32_t* trans,
                              const uint8_t* acc, const uint8_t* live, int32_t vocab, int32_t eos,
                              const int32_t* off, const int32_t* sym, const int32_t* states,
                              int32_t batch, float* logits, float neg_inf) {
  apply_mask_batch(fsa(n, m, dead, trans, acc, live), symbols(vocab, eos, off, sym), states,
                   batch, logits, neg_inf);
}

}  // extern "C"
