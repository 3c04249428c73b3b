// Config-set pushdown automaton semantics, written once for host and device
// over an abstract storage view.
//
// The semantics are those of the reference's bounded PDA (pda.hpp:95-258):
// a config-set holds at most 8 stacks of at most 32 frames; `push` appends a
// stack unless the set is full (then it only sets `saturated`); the closure
// runs rounds over the configs present at the start of each round, trying
// for each config in order the pop (when its top state accepts and depth > 1)
// and then its top state's edges in CSR order (epsilon: replace the top;
// call: replace the top by the return state and push the callee's start),
// skipping candidates already present; after the rounds, configs whose top
// state is not live are removed by an order-preserving compaction that does
// not clear the vacated words.  Consuming a byte builds a fresh config-set
// from the byte edges of every config's top, in config and edge order, then
// closes it.  Any append order difference changes which stacks are dropped
// under saturation, so the order is kept exactly.
//
// Candidates are never materialised: a candidate is "the first `keep` frames
// of source config `i`, then up to two extra frames", compared and copied in
// place.  Two views implement the storage:
//   FlatView  - the padding-free int32 PdaConfigSet layout (266 words), used
//               for the row configs in global memory, the commit kernel's
//               buffers and all host code; raw words come out bit-identical
//               to the reference, stale words included.
//   LaneView  - the mask kernel's per-lane LDS layout: 16-bit frames, one
//               dword per lane per word index, lanes interleaved so that a
//               wave touching the same word index hits 64 distinct banks.
#pragma once

#include <cstdint>

#include "bpdecode_hip.h"

#if defined(__HIPCC__)
#define BPD_HD __host__ __device__ __forceinline__
#else
#define BPD_HD inline
#endif

namespace bpd {

constexpr int kMaxConfigs = BPD_PDA_MAX_CONFIGS;
constexpr int kMaxDepth = BPD_PDA_MAX_DEPTH;
constexpr int kConfigWords = BPD_PDA_CONFIG_WORDS;

struct PdaTableView {
  int32_t num_states, root_start, root_accept, num_edges;
  const uint8_t* accept;
  const uint8_t* live;
  const int32_t* edge_offsets;
  const int32_t* edge_kind;
  const int32_t* edge_lo;
  const int32_t* edge_hi;
  const int32_t* edge_dst;
  const int32_t* edge_callee;
};

inline PdaTableView table_view(const BpdPdaTable& t) {
  return PdaTableView{t.num_states, t.root_start, t.root_accept, t.num_edges,
                      t.accept, t.live, t.edge_offsets, t.edge_kind,
                      t.edge_lo, t.edge_hi, t.edge_dst, t.edge_callee};
}

// int32 PdaConfigSet layout: {n, saturated, depth[8], stack[8][32]}.
struct FlatView {
  int32_t* w;
  BPD_HD int n() const { return w[0]; }
  BPD_HD void set_n(int v) { w[0] = v; }
  BPD_HD int sat() const { return w[1]; }
  BPD_HD void set_sat(int v) { w[1] = v; }
  BPD_HD int depth(int i) const { return w[2 + i]; }
  BPD_HD void set_depth(int i, int d) { w[2 + i] = d; }
  BPD_HD int frame(int i, int k) const { return w[2 + kMaxConfigs + i * kMaxDepth + k]; }
  BPD_HD void set_frame(int i, int k, int v) { w[2 + kMaxConfigs + i * kMaxDepth + k] = v; }
  // fresh set: the reference value-initialises every word
  BPD_HD void reset_all() {
    for (int k = 0; k < kConfigWords; ++k) w[k] = 0;
  }
  BPD_HD void reset() { reset_all(); }
};

struct ConstFlatView {
  const int32_t* w;
  BPD_HD int n() const { return w[0]; }
  BPD_HD int sat() const { return w[1]; }
  BPD_HD int depth(int i) const { return w[2 + i]; }
  BPD_HD int frame(int i, int k) const { return w[2 + kMaxConfigs + i * kMaxDepth + k]; }
};

// Per-lane LDS config-set: dword 0 = n | sat << 8; dwords 1-2 = depth bytes;
// dwords 3.. = 16-bit frames, two per dword.  Dword j of lane l sits at
// base[j * 64 + l].  Only n, sat, depths and frames below each depth are
// meaningful; reset() does not clear frames.
constexpr int kLaneWords = 3 + kMaxConfigs * kMaxDepth / 2;
struct LaneView {
  uint32_t* base;  // already offset by the lane
  BPD_HD uint32_t& word(int j) const { return base[j * 64]; }
  BPD_HD int n() const { return int(word(0) & 0xFFu); }
  BPD_HD void set_n(int v) { word(0) = (word(0) & ~0xFFu) | uint32_t(v); }
  BPD_HD int sat() const { return int((word(0) >> 8) & 1u); }
  BPD_HD void set_sat(int v) { word(0) = (word(0) & 0xFFu) | (uint32_t(v != 0) << 8); }
  BPD_HD int depth(int i) const { return int((word(1 + (i >> 2)) >> ((i & 3) * 8)) & 0xFFu); }
  BPD_HD void set_depth(int i, int d) {
    uint32_t& x = word(1 + (i >> 2));
    const int sh = (i & 3) * 8;
    x = (x & ~(0xFFu << sh)) | (uint32_t(d) << sh);
  }
  BPD_HD int frame(int i, int k) const {
    const int f = i * kMaxDepth + k;
    return int((word(3 + (f >> 1)) >> ((f & 1) * 16)) & 0xFFFFu);
  }
  BPD_HD void set_frame(int i, int k, int v) {
    const int f = i * kMaxDepth + k;
    uint32_t& x = word(3 + (f >> 1));
    const int sh = (f & 1) * 16;
    x = (x & ~(0xFFFFu << sh)) | (uint32_t(v) << sh);
  }
  BPD_HD void reset() {
    word(0) = 0;
    word(1) = 0;
    word(2) = 0;
  }
};

// Does `dst` hold the stack src[i][0..keep) ++ extra[0..nx)?
template <class Dst, class Src>
BPD_HD bool holds(const Dst& dst, const Src& src, int i, int keep, const int* extra, int nx) {
  const int d = keep + nx;
  const int n = dst.n();
  for (int j = 0; j < n; ++j) {
    if (dst.depth(j) != d) continue;
    bool same = true;
    for (int k = 0; k < keep && same; ++k) same = dst.frame(j, k) == src.frame(i, k);
    for (int k = 0; k < nx && same; ++k) same = dst.frame(j, keep + k) == extra[k];
    if (same) return true;
  }
  return false;
}

// Append src[i][0..keep) ++ extra; false (and saturated) when full.
template <class Dst, class Src>
BPD_HD bool append(Dst& dst, const Src& src, int i, int keep, const int* extra, int nx) {
  const int n = dst.n();
  if (n >= kMaxConfigs) {
    dst.set_sat(1);
    return false;
  }
  dst.set_n(n + 1);
  dst.set_depth(n, keep + nx);
  for (int k = 0; k < keep; ++k) dst.set_frame(n, k, src.frame(i, k));
  for (int k = 0; k < nx; ++k) dst.set_frame(n, keep + k, extra[k]);
  return true;
}

template <class S>
BPD_HD void prune_dead(const PdaTableView& g, S& c) {
  int out = 0;
  const int n = c.n();
  for (int i = 0; i < n; ++i) {
    const int d = c.depth(i);
    if (d <= 0) continue;
    if (!g.live[c.frame(i, d - 1)]) continue;
    if (out != i) {
      c.set_depth(out, d);
      for (int k = 0; k < d; ++k) c.set_frame(out, k, c.frame(i, k));
    }
    ++out;
  }
  c.set_n(out);
}

// The closure visits every config once, in index order, including the
// configs it appends.  This is the reference's round structure (pda.hpp:
// 150-196: rounds over the configs present at each round's start until a
// round appends nothing) without its repeated visits: configs are never
// modified or removed while closing and the set only grows, so a config
// visited again yields only candidates that are already present or that were
// dropped because the set is full -- no append and no new saturation.  The
// appends, their order and the saturated flag are therefore identical.  At
// most kMaxConfigs configs exist, so at most kMaxConfigs + 1 reference rounds
// run and its round guard (pda.hpp:154) is never reached.
template <class S>
BPD_HD bool close(const PdaTableView& g, S& c) {
  for (int i = 0; i < c.n(); ++i) {
    const int d = c.depth(i);
    if (d <= 0) continue;
    const int top = c.frame(i, d - 1);
    if (g.accept[top] && d > 1) {
      if (!holds(c, c, i, d - 1, nullptr, 0)) append(c, c, i, d - 1, nullptr, 0);
    }
    const int eb = g.edge_offsets[top], ee = g.edge_offsets[top + 1];
    for (int e = eb; e < ee; ++e) {
      const int kind = g.edge_kind[e];
      if (kind == BPD_PDA_EDGE_EPS) {
        const int x[1] = {g.edge_dst[e]};
        if (!holds(c, c, i, d - 1, x, 1)) append(c, c, i, d - 1, x, 1);
      } else if (kind == BPD_PDA_EDGE_CALL) {
        if (d + 1 <= kMaxDepth) {
          const int x[2] = {g.edge_dst[e], g.edge_callee[e]};
          if (!holds(c, c, i, d - 1, x, 2)) append(c, c, i, d - 1, x, 2);
        } else {
          c.set_sat(1);
        }
      }
    }
  }
  prune_dead(g, c);
  return c.n() > 0;
}

// next = close(byte step of src); `next` must be a fresh set (reset()).
template <class Dst, class Src>
BPD_HD bool advance_byte(const PdaTableView& g, const Src& src, Dst& next, int byte) {
  const int n = src.n();
  for (int i = 0; i < n; ++i) {
    const int d = src.depth(i);
    if (d <= 0) continue;
    const int top = src.frame(i, d - 1);
    const int eb = g.edge_offsets[top], ee = g.edge_offsets[top + 1];
    for (int e = eb; e < ee; ++e) {
      if (g.edge_kind[e] != BPD_PDA_EDGE_BYTE) continue;
      if (byte < g.edge_lo[e] || byte > g.edge_hi[e]) continue;
      const int x[1] = {g.edge_dst[e]};
      if (!holds(next, src, i, d - 1, x, 1)) append(next, src, i, d - 1, x, 1);
    }
  }
  next.set_sat(next.sat() || src.sat());
  return close(g, next);
}

template <class S>
BPD_HD bool is_complete(const PdaTableView& g, const S& c) {
  const int n = c.n();
  for (int i = 0; i < n; ++i)
    if (c.depth(i) == 1 && c.frame(i, 0) == g.root_accept) return true;
  return false;
}

// Initial closed config-set (pda.hpp:200-207) into a flat buffer.
BPD_HD void init_config(const PdaTableView& g, FlatView c) {
  c.reset_all();
  const int x[1] = {g.root_start};
  append(c, c, 0, 0, x, 1);
  close(g, c);
}

}  // namespace bpd
