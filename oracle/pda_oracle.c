/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the PDA path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker or as the timed CPU baseline.
 *
 * A plain-C restatement of the reference's bounded config-set PDA:
 *   pda_stack_eq / pda_contains / pda_push_config  pda.hpp:95-121
 *   pda_prune_dead                                 pda.hpp:124-139
 *   pda_close                                      pda.hpp:150-198
 *   pda_init                                       pda.hpp:200-207
 *   pda_advance_byte                               pda.hpp:211-236
 *   pda_is_complete                                pda.hpp:238-244
 *   pda_try_token                                  pda.hpp:248-258
 *   compute_mask / apply_mask / advance batches    pda_cpu.cpp:7-54
 * Candidate stacks are materialised in a temporary array exactly as the
 * reference does, so every write to a config-set happens in the same order
 * and the raw 266-word buffers (stale words included) can be compared.
 */
#include <stdint.h>
#include <string.h>

#define MAXC 8
#define MAXD 32
#define WORDS (2 + MAXC + MAXC * MAXD)

typedef struct {
  int32_t n, sat, depth[MAXC], stack[MAXC][MAXD];
} Cfg;

typedef struct {
  int32_t num_states, root_start, root_accept;
  const uint8_t *accept, *live;
  const int32_t *off, *kind, *lo, *hi, *dst, *callee;
} Table;

static int stack_eq(const int32_t *a, const int32_t *b, int32_t n) {
  for (int32_t i = 0; i < n; ++i)
    if (a[i] != b[i]) return 0;
  return 1;
}

static int contains(const Cfg *c, const int32_t *st, int32_t d) {
  for (int32_t i = 0; i < c->n; ++i)
    if (c->depth[i] == d && stack_eq(c->stack[i], st, d)) return 1;
  return 0;
}

static int push(Cfg *c, const int32_t *st, int32_t d) {
  if (c->n >= MAXC) {
    c->sat = 1;
    return 0;
  }
  int32_t i = c->n++;
  c->depth[i] = d;
  for (int32_t k = 0; k < d; ++k) c->stack[i][k] = st[k];
  return 1;
}

static void prune(const Table *g, Cfg *c) {
  int32_t out = 0;
  for (int32_t i = 0; i < c->n; ++i) {
    int32_t d = c->depth[i];
    if (d <= 0) continue;
    if (!g->live[c->stack[i][d - 1]]) continue;
    if (out != i) {
      c->depth[out] = d;
      for (int32_t k = 0; k < d; ++k) c->stack[out][k] = c->stack[i][k];
    }
    ++out;
  }
  c->n = out;
}

static int close_set(const Table *g, Cfg *c) {
  int changed = 1, guard = 0;
  const int rounds = MAXC * MAXD + 8;
  int32_t tmp[MAXD];
  while (changed && guard++ < rounds) {
    changed = 0;
    int32_t n = c->n;
    for (int32_t i = 0; i < n; ++i) {
      int32_t d = c->depth[i];
      if (d <= 0) continue;
      int32_t top = c->stack[i][d - 1];
      if (g->accept[top] && d > 1 && !contains(c, c->stack[i], d - 1) && push(c, c->stack[i], d - 1))
        changed = 1;
      for (int32_t e = g->off[top]; e < g->off[top + 1]; ++e) {
        if (g->kind[e] == 0) {
          memcpy(tmp, c->stack[i], sizeof(int32_t) * (size_t)(d - 1));
          tmp[d - 1] = g->dst[e];
          if (!contains(c, tmp, d) && push(c, tmp, d)) changed = 1;
        } else if (g->kind[e] == 2) {
          if (d + 1 <= MAXD) {
            memcpy(tmp, c->stack[i], sizeof(int32_t) * (size_t)(d - 1));
            tmp[d - 1] = g->dst[e];
            tmp[d] = g->callee[e];
            if (!contains(c, tmp, d + 1) && push(c, tmp, d + 1)) changed = 1;
          } else {
            c->sat = 1;
          }
        }
      }
    }
  }
  prune(g, c);
  return c->n > 0;
}

static int advance_byte(const Table *g, Cfg *c, int32_t byte) {
  Cfg next;
  memset(&next, 0, sizeof next);
  int32_t tmp[MAXD];
  for (int32_t i = 0; i < c->n; ++i) {
    int32_t d = c->depth[i];
    if (d <= 0) continue;
    int32_t top = c->stack[i][d - 1];
    for (int32_t e = g->off[top]; e < g->off[top + 1]; ++e) {
      if (g->kind[e] != 1 || byte < g->lo[e] || byte > g->hi[e]) continue;
      memcpy(tmp, c->stack[i], sizeof(int32_t) * (size_t)(d - 1));
      tmp[d - 1] = g->dst[e];
      if (!contains(&next, tmp, d)) push(&next, tmp, d);
    }
  }
  next.sat = next.sat || c->sat;
  int ok = close_set(g, &next);
  *c = next;
  return ok;
}

static int is_complete(const Table *g, const Cfg *c) {
  for (int32_t i = 0; i < c->n; ++i)
    if (c->depth[i] == 1 && c->stack[i][0] == g->root_accept) return 1;
  return 0;
}

static int try_token(const Table *g, const int32_t *toff, const uint8_t *tb, int32_t eos,
                     Cfg c, int32_t t) {
  if (t == eos) return is_complete(g, &c);
  for (int32_t i = toff[t]; i < toff[t + 1]; ++i)
    if (!advance_byte(g, &c, tb[i])) return 0;
  return c.n > 0;
}

static Table make_table(int32_t num_states, int32_t root_start, int32_t root_accept,
                        const uint8_t *accept, const uint8_t *live, const int32_t *off,
                        const int32_t *kind, const int32_t *lo, const int32_t *hi,
                        const int32_t *dst, const int32_t *callee) {
  Table g = {num_states, root_start, root_accept, accept, live, off, kind, lo, hi, dst, callee};
  return g;
}

#define TABLE_ARGS                                                                         \
  int32_t num_states, int32_t root_start, int32_t root_accept, const uint8_t *accept,     \
      const uint8_t *live, const int32_t *off, const int32_t *kind, const int32_t *lo,    \
      const int32_t *hi, const int32_t *dst, const int32_t *callee
#define TABLE_PASS num_states, root_start, root_accept, accept, live, off, kind, lo, hi, dst, callee

void oracle_pda_init(TABLE_ARGS, int32_t *out) {
  Table g = make_table(TABLE_PASS);
  Cfg c;
  memset(&c, 0, sizeof c);
  int32_t st[1] = {g.root_start};
  push(&c, st, 1);
  close_set(&g, &c);
  memcpy(out, &c, sizeof c);
}

/* Raw byte step of one config-set in place; returns the non-empty flag. */
int oracle_pda_advance_byte(TABLE_ARGS, int32_t *cfg, int32_t byte) {
  Table g = make_table(TABLE_PASS);
  Cfg c;
  memcpy(&c, cfg, sizeof c);
  int ok = advance_byte(&g, &c, byte);
  memcpy(cfg, &c, sizeof c);
  return ok;
}

void oracle_pda_compute_mask(TABLE_ARGS, int32_t vocab, int32_t eos, const int32_t *toff,
                             const uint8_t *tb, const int32_t *configs, int32_t batch,
                             uint32_t *bits) {
  Table g = make_table(TABLE_PASS);
  int32_t words = (vocab + 31) / 32;
  memset(bits, 0, sizeof(uint32_t) * (size_t)batch * (size_t)words);
  for (int32_t b = 0; b < batch; ++b) {
    Cfg c;
    memcpy(&c, configs + (int64_t)b * WORDS, sizeof c);
    uint32_t *row = bits + (int64_t)b * words;
    for (int32_t t = 0; t < vocab; ++t)
      if (try_token(&g, toff, tb, eos, c, t)) row[t >> 5] |= 1u << (t & 31);
    if (eos >= 0 && is_complete(&g, &c)) row[eos >> 5] |= 1u << (eos & 31);
  }
}

void oracle_pda_apply_mask(TABLE_ARGS, int32_t vocab, int32_t eos, const int32_t *toff,
                           const uint8_t *tb, const int32_t *configs, int32_t batch,
                           float *logits, float neg_inf) {
  Table g = make_table(TABLE_PASS);
  for (int32_t b = 0; b < batch; ++b) {
    Cfg c;
    memcpy(&c, configs + (int64_t)b * WORDS, sizeof c);
    float *row = logits + (int64_t)b * vocab;
    for (int32_t t = 0; t < vocab; ++t)
      if (!try_token(&g, toff, tb, eos, c, t)) row[t] = neg_inf;
  }
}

void oracle_pda_advance(TABLE_ARGS, int32_t eos, const int32_t *toff, const uint8_t *tb,
                        int32_t *configs, const int32_t *tokens, int32_t batch, uint8_t *ok) {
  Table g = make_table(TABLE_PASS);
  for (int32_t b = 0; b < batch; ++b) {
    Cfg *c = (Cfg *)(configs + (int64_t)b * WORDS);
    int32_t t = tokens[b];
    if (t == eos) {
      ok[b] = (uint8_t)is_complete(&g, c);
      continue;
    }
    Cfg trial = *c;
    int acc = 1;
    for (int32_t i = toff[t]; i < toff[t + 1] && acc; ++i) acc = advance_byte(&g, &trial, tb[i]);
    ok[b] = (uint8_t)(acc ? 1 : 0);
    if (acc) *c = trial;
  }
}
