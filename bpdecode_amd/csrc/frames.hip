// Frame lists of the PDA mask's fast path (no counterpart in the reference:
// an acceleration of pda_try_token, pda.hpp:248-258): the host enumeration
// of the stack-relative config lists and the device classification of every
// (list, token) walk.
//
// A config-set whose configs all sit on one common stack P is the ordered
// list of the configs' suffixes above P.  While no config pops into P (a
// one-frame suffix whose top accepts) and no suffix grows past
// BPD_PDA_FRAME_SUFFIX frames, the bounded step (pda.hpp:211-236: byte edges
// of each top in config and edge order), the closure (pda.hpp:150-196:
// epsilon edges, pushes of callees, pops of accepting tops inside the
// suffix, each config visited once in index order, no duplicates, at most
// BPD_PDA_MAX_CONFIGS configs) and the compaction of configs whose top is not
// live (pda.hpp:198-209) act on the suffixes alone.
#include <algorithm>
#include <map>
#include <thread>
#include <vector>

#include "bpd_common.hpp"

namespace bpd {
namespace {

constexpr int kSuffix = BPD_PDA_FRAME_SUFFIX;
constexpr int kCap = BPD_PDA_MAX_CONFIGS;
constexpr int32_t kDead = -1, kBoundary = -2;

struct Suffix {
  int8_t len = 0;
  int32_t f[kSuffix] = {};
  bool operator==(const Suffix& o) const {
    if (len != o.len) return false;
    for (int k = 0; k < len; ++k)
      if (f[k] != o.f[k]) return false;
    return true;
  }
};

// An ordered list of suffixes; its key words (BpdPdaFrames.keys) order it.
struct List {
  int n = 0;
  Suffix s[kCap];
  std::vector<int32_t> key() const {
    std::vector<int32_t> k(BPD_PDA_FRAME_KEY_WORDS, 0);
    k[0] = n;
    for (int i = 0; i < n; ++i) {
      k[1 + i] = s[i].len;
      for (int j = 0; j < s[i].len; ++j) k[1 + kCap + i * kSuffix + j] = s[i].f[j];
    }
    return k;
  }
};

struct Tables {
  const BpdPdaTable& g;
  explicit Tables(const BpdPdaTable& t) : g(t) {}
  bool accept(int32_t s) const { return g.accept[s] != 0; }
  bool live(int32_t s) const { return g.live[s] != 0; }
};

// Append x unless present; false when the list is full (x dropped).
bool add(List& l, const Suffix& x) {
  for (int i = 0; i < l.n; ++i)
    if (l.s[i] == x) return true;
  if (l.n >= kCap) return false;
  l.s[l.n++] = x;
  return true;
}

// Closure and compaction of a suffix list: kBoundary when a config pops into
// the common stack or pushes past kSuffix frames, kDead when none is left,
// else 0 with the list in `l`; `sat` gets whether a config was dropped at
// the cap, `pruned` whether the compaction dropped one (a set stepped so
// keeps that config's words in slots past its last).
int32_t close_list(const Tables& t, List& l, bool& sat, bool& pruned) {
  const BpdPdaTable& g = t.g;
  for (int i = 0; i < l.n; ++i) {
    const Suffix sfx = l.s[i];
    const int32_t top = sfx.f[sfx.len - 1];
    if (t.accept(top)) {
      if (sfx.len == 1) return kBoundary;
      Suffix p = sfx;
      p.len = int8_t(sfx.len - 1);
      sat = !add(l, p) || sat;
    }
    for (int32_t e = g.edge_offsets[top]; e < g.edge_offsets[top + 1]; ++e) {
      const int32_t kind = g.edge_kind[e];
      if (kind == BPD_PDA_EDGE_EPS) {
        Suffix x = sfx;
        x.f[sfx.len - 1] = g.edge_dst[e];
        sat = !add(l, x) || sat;
      } else if (kind == BPD_PDA_EDGE_CALL) {
        if (sfx.len + 1 > kSuffix) return kBoundary;
        Suffix x = sfx;
        x.f[sfx.len - 1] = g.edge_dst[e];
        x.f[sfx.len] = g.edge_callee[e];
        x.len = int8_t(sfx.len + 1);
        sat = !add(l, x) || sat;
      }
    }
  }
  int out = 0;
  for (int i = 0; i < l.n; ++i)
    if (t.live(l.s[i].f[l.s[i].len - 1])) l.s[out++] = l.s[i];
  pruned = out < l.n;
  l.n = out;
  return out > 0 ? 0 : kDead;
}

int32_t step_list(const Tables& t, const List& src, int byte, List& out, bool& sat, bool& pruned) {
  const BpdPdaTable& g = t.g;
  out.n = 0;
  sat = false;
  for (int i = 0; i < src.n; ++i) {
    const Suffix& sfx = src.s[i];
    const int32_t top = sfx.f[sfx.len - 1];
    for (int32_t e = g.edge_offsets[top]; e < g.edge_offsets[top + 1]; ++e) {
      if (g.edge_kind[e] != BPD_PDA_EDGE_BYTE || byte < g.edge_lo[e] || byte > g.edge_hi[e]) continue;
      Suffix x = sfx;
      x.f[sfx.len - 1] = g.edge_dst[e];
      sat = !add(out, x) || sat;
    }
  }
  return close_list(t, out, sat, pruned);
}

uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7FEB352Du;
  x ^= x >> 15;
  x *= 0x846CA68Bu;
  x ^= x >> 16;
  return x;
}

// Hash of a key (the device's frame_list_of computes the same sum of
// per-word mixes lane-parallel).
uint32_t key_hash(const std::vector<int32_t>& k) {
  const int n = k[0];
  uint32_t h = mix32(0xC2B2AE35u ^ uint32_t(n));
  for (int i = 0; i < n; ++i) {
    const int len = k[1 + i];
    h += mix32((uint32_t((i << 8) | 0xFF) * 0x85EBCA6Bu) ^ uint32_t(len));
    for (int j = 0; j < len; ++j)
      h += mix32((uint32_t((i << 8) | j) * 0x9E3779B1u) ^ uint32_t(k[1 + kCap + i * kSuffix + j]));
  }
  return mix32(h);
}

// Every (list, token) walk from token position `k` of `order`, list
// blockIdx.y: 0 dead, 1 inside (every byte leads to a list), 2 seed (a
// boundary, EOS or an empty token).  Count pass (offsets null): the bits
// of the inside tokens are or-ed into `allowed` and each block writes its
// number of seeds; fill pass: the seeds go, in walk order, to
// seeds[offsets[list * blocks + block] ..].
constexpr int kClassifyThreads = 256;

__global__ __launch_bounds__(kClassifyThreads) void frame_classify_kernel(
    const int32_t* __restrict__ trans, const int32_t* __restrict__ tok_off, const uint8_t* __restrict__ tok_bytes,
    int32_t V, int32_t eos, const int32_t* __restrict__ order, int32_t words, uint32_t* __restrict__ allowed,
    int32_t* __restrict__ counts, const int64_t* __restrict__ offsets, int32_t* __restrict__ seeds) {
  __shared__ int32_t wave_n[kClassifyThreads / 64];
  const int32_t l = blockIdx.y;
  const int32_t k = int32_t(blockIdx.x) * kClassifyThreads + int32_t(threadIdx.x);
  const int lane = threadIdx.x & 63, w = threadIdx.x / 64;
  int cls = 0;
  int32_t t = -1;
  if (k < V) {
    t = order[k];
    const int32_t s = tok_off[t], e = tok_off[t + 1];
    int32_t cur = l;
    for (int32_t i = s; i < e && cur >= 0; ++i) {
      const int32_t c = trans[int64_t(cur) * 256 + tok_bytes[i]];
      cur = c >= 0 ? (c & (BPD_PDA_FRAME_SAT - 1)) : c;
    }
    const bool special = e == s || t == eos;
    cls = special || cur == kBoundary ? 2 : (cur >= 0 ? 1 : 0);
  }
  const uint64_t seed = __ballot(cls == 2);
  if (!offsets) {
    if (cls == 1) atomicOr(&allowed[int64_t(l) * words + (t >> 5)], 1u << (t & 31));
    if (lane == 0) wave_n[w] = __popcll(seed);
    __syncthreads();
    if (threadIdx.x == 0) {
      int32_t n = 0;
      for (int i = 0; i < kClassifyThreads / 64; ++i) n += wave_n[i];
      counts[int64_t(l) * gridDim.x + blockIdx.x] = n;
    }
    return;
  }
  if (lane == 0) wave_n[w] = __popcll(seed);
  __syncthreads();
  int64_t at = offsets[int64_t(l) * gridDim.x + blockIdx.x];
  for (int i = 0; i < w; ++i) at += wave_n[i];
  if (cls == 2) seeds[at + __popcll(seed & ((uint64_t(1) << lane) - 1u))] = k;
}

}  // namespace
}  // namespace bpd

using namespace bpd;

namespace {

// The enumeration behind bpd_host_frame_lists: 0 or an error code, the
// number of lists in *count.
int frame_lists_impl(const BpdPdaTable* g, int32_t max_lists, int32_t* keys, int32_t* trans, uint32_t* slots,
                     int32_t* count) {
  BPD_REQUIRE(g && keys && trans && slots, "null pointer argument");
  BPD_REQUIRE(max_lists >= 0 && max_lists <= BPD_PDA_MAX_FRAME_LISTS, "max_lists %d outside [0, %d]", max_lists,
              BPD_PDA_MAX_FRAME_LISTS);
  const int32_t N = g->num_states;
  BPD_REQUIRE(N >= 0 && g->num_edges >= 0, "bad table shape");
  for (int32_t s = 0; s < N; ++s)
    BPD_REQUIRE(g->edge_offsets[s] <= g->edge_offsets[s + 1], "edge offsets decrease at state %d", s);
  BPD_REQUIRE(N == 0 || (g->edge_offsets[0] >= 0 && g->edge_offsets[N] <= g->num_edges), "edge offsets out of range");
  for (int32_t e = 0; e < g->num_edges; ++e) {
    BPD_REQUIRE(g->edge_dst[e] >= 0 && g->edge_dst[e] < N, "edge %d: destination out of range", e);
    BPD_REQUIRE(g->edge_kind[e] != BPD_PDA_EDGE_CALL || (g->edge_callee[e] >= 0 && g->edge_callee[e] < N),
                "edge %d: callee out of range", e);
  }
  const Tables t(*g);
  std::vector<List> lists;
  std::map<std::vector<int32_t>, int32_t> index;
  auto intern = [&](const List& l) -> int32_t {
    const std::vector<int32_t> k = l.key();
    const auto it = index.find(k);
    if (it != index.end()) return it->second;
    if (int32_t(lists.size()) >= max_lists) return -1;
    const int32_t id = int32_t(lists.size());
    index.emplace(k, id);
    lists.push_back(l);
    return id;
  };
  // the closure of every single state, then breadth first by byte
  for (int32_t s = 0; s < N; ++s) {
    List l;
    l.n = 1;
    l.s[0].len = 1;
    l.s[0].f[0] = s;
    bool sat = false, pruned = false;
    if (close_list(t, l, sat, pruned) == 0) intern(l);
  }
  std::vector<int32_t> rows;
  for (size_t head = 0; head < lists.size(); ++head) {
    const List src = lists[head];
    // bytes over the same byte edges of the tops step alike
    std::map<std::vector<bool>, int32_t> memo;
    for (int byte = 0; byte < 256; ++byte) {
      std::vector<bool> sig;
      for (int i = 0; i < src.n; ++i) {
        const int32_t top = src.s[i].f[src.s[i].len - 1];
        for (int32_t e = g->edge_offsets[top]; e < g->edge_offsets[top + 1]; ++e)
          if (g->edge_kind[e] == BPD_PDA_EDGE_BYTE) sig.push_back(g->edge_lo[e] <= byte && byte <= g->edge_hi[e]);
      }
      const auto m = memo.find(sig);
      if (m != memo.end()) {
        rows.push_back(m->second);
        continue;
      }
      List nx;
      bool sat = false, pruned = false;
      int32_t code = step_list(t, src, byte, nx, sat, pruned);
      if (code == 0) {
        const int32_t id = intern(nx);
        code = id < 0 ? kBoundary : (id | (sat ? BPD_PDA_FRAME_SAT : 0) | (pruned ? 0 : BPD_PDA_FRAME_RAW));
      }
      memo.emplace(sig, code);
      rows.push_back(code);
    }
  }
  const int32_t L = int32_t(lists.size());
  std::fill(slots, slots + BPD_PDA_FRAME_SLOTS, BPD_PDA_FRAME_EMPTY);
  for (int32_t i = 0; i < L; ++i) {
    const std::vector<int32_t> k = lists[size_t(i)].key();
    std::copy(k.begin(), k.end(), keys + int64_t(i) * BPD_PDA_FRAME_KEY_WORDS);
    const uint32_t h = key_hash(k);
    uint32_t s = h & (BPD_PDA_FRAME_SLOTS - 1);
    while (slots[s] != BPD_PDA_FRAME_EMPTY) s = (s + 1) & (BPD_PDA_FRAME_SLOTS - 1);
    slots[s] = uint32_t(i) | (((h >> 10) & 0xFFFFFu) << 12);
  }
  std::copy(rows.begin(), rows.end(), trans);
  *count = L;
  return BPD_OK;
}

}  // namespace

extern "C" int bpd_host_frame_lists(const BpdPdaTable* g, int32_t max_lists, int32_t* keys, int32_t* trans,
                                    uint32_t* slots) {
  int32_t count = 0;
  const int rc = frame_lists_impl(g, max_lists, keys, trans, slots, &count);
  return rc != BPD_OK ? -rc : count;
}

extern "C" int bpd_frame_classify(const int32_t* trans, int32_t num_lists, const int32_t* tok_offsets,
                                  const uint8_t* tok_bytes, int32_t vocab_size, int32_t eos_id, const int32_t* order,
                                  uint32_t* allowed, int32_t* block_counts, const int64_t* block_offsets,
                                  int32_t* seeds, void* stream) {
  BPD_REQUIRE(num_lists >= 0 && num_lists <= BPD_PDA_MAX_FRAME_LISTS && vocab_size >= 0, "bad shape");
  if (num_lists == 0 || vocab_size == 0) return BPD_OK;
  BPD_REQUIRE(trans && tok_offsets && tok_bytes && order && block_counts, "null pointer argument");
  BPD_REQUIRE(block_offsets ? seeds != nullptr : allowed != nullptr, "count pass needs allowed, fill pass seeds");
  const unsigned blocks = unsigned((vocab_size + kClassifyThreads - 1) / kClassifyThreads);
  frame_classify_kernel<<<dim3(blocks, unsigned(num_lists)), kClassifyThreads, 0, static_cast<hipStream_t>(stream)>>>(
      trans, tok_offsets, tok_bytes, vocab_size, eos_id, order, (vocab_size + 31) / 32, allowed, block_counts,
      block_offsets, seeds);
  BPD_LAUNCHED();
  return BPD_OK;
}

extern "C" int32_t bpd_frame_classify_blocks(int32_t vocab_size) {
  return vocab_size > 0 ? (vocab_size + kClassifyThreads - 1) / kClassifyThreads : 0;
}
