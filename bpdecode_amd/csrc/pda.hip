// Config-set PDA step on gfx950: token mask (fused into the logits or packed
// bits) and the per-row commit, plus the host forms of both and pda_init.
//
// Mask kernel: one wave64 per (row, vocab chunk).  The row's config-set is
// staged in LDS (int32 layout) and shared by the wave; each lane walks one
// token at a time through its own two LDS config-sets (LaneView, 16-bit
// frames, lane-interleaved).  Before walking, the wave evaluates all 256
// first bytes from the row's set (4 per lane) and packs the survivors into a
// 256-bit table with ballots, so a token whose first byte empties the set is
// rejected with one bit test.  Verdicts of the 64 lanes are written as one
// coalesced store (logits) or packed into two words with a ballot (bits).
//
// Commit kernel without a workspace: one thread per row with two int32
// config-sets in LDS; the walk starts from the row's set in global memory and
// every byte step writes a freshly cleared set, so the 266 words written back
// on acceptance are exactly those the reference produces.  With the mask's
// workspace the commit walks the mask's tables first (pda_memo_advance_kernel).
//
// Memoised mask kernel (pda_memo_mask_kernel, the default with a workspace):
// see the section below.
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "bpd_common.hpp"
#include "pda_core.hpp"

namespace bpd {
namespace {

constexpr int kWave = 64;
constexpr int kCommitRows = 16;

struct MaskArgs {
  PdaTableView g;
  const int32_t* tok_off;
  const uint8_t* tok_bytes;
  int32_t vocab;
  int32_t eos;
  const int32_t* configs;
  const int64_t* slots;
  const uint8_t* broken;
  int64_t rows;
  uint8_t* logits;  // null when writing bits
  int64_t ld_bytes;
  int32_t elem;
  uint32_t fill;
  uint32_t* bits;  // null when writing logits
  int64_t words;
  int32_t chunk_tokens;  // multiple of 64
  int32_t* err;
  const int32_t* only_rows;  // non-null: process only rows b with only_rows[b] != 0
  const int32_t* order;      // memo walk order (null: id order)
  const int32_t* runs;       // first-byte runs of order (null: none)
  BpdPdaFrames frames;       // num_lists 0: no frame lists
  // the launch after a memoised mask (only_rows set): the workspace header
  // (the pack key is stamped there, the deferred slots read), the deferred
  // rows' verdict bits (null: none), the mask launch's generation and pack key
  uint32_t* header;
  const uint32_t* defer_bits;
  uint32_t gen;
  uint64_t pkey;
};

// Structural check of a row's config-set before any table lookup with its
// frames: counts in range and every frame a valid state id.
__device__ bool config_ok(const int32_t* c, int32_t num_states, int lane) {
  const int n = c[0];
  bool ok = n >= 0 && n <= kMaxConfigs;
  if (lane < kMaxConfigs) {
    const int d = c[2 + lane];
    ok = ok && (lane >= n || (d >= 0 && d <= kMaxDepth));
  }
  for (int f = lane; f < kMaxConfigs * kMaxDepth; f += kWave) {
    const int i = f / kMaxDepth, k = f % kMaxDepth;
    if (i < n && i < kMaxConfigs) {
      const int d = c[2 + i];
      if (d >= 0 && d <= kMaxDepth && k < d) {
        const int v = c[2 + kMaxConfigs + f];
        ok = ok && v >= 0 && v < num_states;
      }
    }
  }
  return __ballot(!ok) == 0;
}

// Chunk `blockIdx.x` of row b's verdicts by one wave.
__device__ void mask_row_chunk(const MaskArgs& a, int64_t b) {
  __shared__ int32_t row_cfg[kConfigWords];
  __shared__ uint32_t lane_sets[2 * kLaneWords * kWave];
  __shared__ uint32_t first_ok[8];

  const int lane = threadIdx.x;
  const int64_t row = a.slots ? a.slots[b] : b;
  for (int k = lane; k < kConfigWords; k += kWave) row_cfg[k] = a.configs[row * kConfigWords + k];
  __syncthreads();

  bool dead_row = a.broken != nullptr && a.broken[row] != 0;
  if (!config_ok(row_cfg, a.g.num_states, lane)) {
    if (lane == 0 && blockIdx.x == 0 && a.err) atomicOr(a.err, BPD_FLAG_STATE_RANGE);
    dead_row = true;
  }
  const ConstFlatView C{row_cfg};
  LaneView A{lane_sets + lane};
  LaneView Bv{lane_sets + kLaneWords * kWave + lane};

  if (!dead_row) {
    for (int q = 0; q < 4; ++q) {
      A.reset();
      const bool ok = advance_byte(a.g, C, A, q * kWave + lane);
      const uint64_t m = __ballot(ok);
      if (lane == 0) {
        first_ok[2 * q] = uint32_t(m);
        first_ok[2 * q + 1] = uint32_t(m >> 32);
      }
    }
  }
  __syncthreads();
  const bool complete = !dead_row && is_complete(a.g, C);
  const bool nonempty = !dead_row && C.n() > 0;

  const int64_t t_begin = int64_t(blockIdx.x) * a.chunk_tokens;
  const int64_t t_end = t_begin + a.chunk_tokens < a.vocab ? t_begin + a.chunk_tokens : a.vocab;
  for (int64_t t0 = t_begin; t0 < t_end; t0 += kWave) {
    const int64_t t = t0 + lane;
    bool allow = false;
    if (!dead_row && t < t_end) {
      if (t == a.eos) {
        allow = complete;
      } else {
        const int32_t s = a.tok_off[t], e = a.tok_off[t + 1];
        if (s == e) {
          allow = nonempty;
        } else {
          const int b0 = a.tok_bytes[s];
          if ((first_ok[b0 >> 5] >> (b0 & 31)) & 1u) {
            LaneView cur = A, nxt = Bv;
            cur.reset();
            allow = advance_byte(a.g, C, cur, b0);
            for (int32_t i = s + 1; i < e && allow; ++i) {
              nxt.reset();
              allow = advance_byte(a.g, cur, nxt, a.tok_bytes[i]);
              const LaneView tmp = cur;
              cur = nxt;
              nxt = tmp;
            }
          }
        }
      }
    }
    if (a.logits) {
      if (t < t_end && !allow) {
        uint8_t* p = a.logits + b * a.ld_bytes + t * a.elem;
        if (a.elem == 2)
          *reinterpret_cast<uint16_t*>(p) = uint16_t(a.fill);
        else
          *reinterpret_cast<uint32_t*>(p) = a.fill;
      }
    } else {
      const uint64_t m = __ballot(allow);
      if (lane == 0) {
        const int64_t w0 = t0 >> 5;
        if (w0 < a.words) a.bits[b * a.words + w0] = uint32_t(m);
        if (w0 + 1 < a.words) a.bits[b * a.words + w0 + 1] = uint32_t(m >> 32);
      }
    }
  }
  __syncthreads();  // the LDS arrays are reused by the next row of the block
}

// ------------------------------------------------------- memoised mask --
// One workgroup per row.  A token's verdict depends only on the config-sets
// its bytes walk through, and advance_byte is a pure function of a set's
// meaningful words (n, saturated, depths, frames below each depth).  The
// workgroup therefore interns the sets it meets (pool, global workspace) and
// fills a transition table T[set][byte] in LDS on demand: threads walk their
// tokens through T; a missing entry pauses the token and is requested; the
// requests of a round are computed in parallel (one wave each, the set
// being built in LDS), de-duplicated against the pool and among themselves,
// and entered in T; then the walks resume.  A set that is in a stack-relative
// frame list is walked through the lists' byte table instead (list states,
// below), and only its boundary bytes are requested, through the boundary
// table LT.  Every entry is computed by the same advance_byte as the direct
// walk, so verdicts are identical.  A row that needs more than kMemoSets
// distinct sets marks the missing entries "overflow", leaves those tokens
// untouched and is finished by the direct-walk kernel (pda_mask_kernel
// filtered to flagged rows).
constexpr int kMemoThreads = 1024;
constexpr int kMemoSets = 128;
constexpr int kMemoReq = 128;
// tokens a thread walks per tile (1: the walk's registers then fit without
// spilling in the walk loops; 2 and 4 measured 154 and 163 us per mask)
constexpr int kMemoTok = 1;
constexpr int kMemoMaxVocab = 262144;  // verdict bitmap of a row in LDS
constexpr uint8_t kTUnknown = 0xFE;
constexpr uint8_t kTDead = 0xFF;
constexpr uint8_t kTOverflow = 0xFD;
// In the table kept for the commit, an entry with kTExact set is an id whose
// interned set has the raw words the step itself gives; ids stay below
// kMemoIds so that no flagged id reaches the special entries.
constexpr uint8_t kTExact = 0x80;
// bit of a frame-list word above the list id and the saturation flag where
// the depth of the list's common stack starts
constexpr int kListBase = 17;
constexpr int kMemoIds = 125;
// List states of the row-wide walk.  A set that is in a frame list is walked
// through the lists' byte table (BpdPdaFrames::trans) without interning the
// sets it reaches: the walk state is kListState | anchor << 13 | sat << 12 |
// list, where `anchor` is the pool set whose common stack the list sits on
// (every list reached from it sits on the same stack) and `sat` the
// saturation flag.  Only a boundary byte (trans -2: the step needs the
// stack) makes a set with words: the boundary table LT, keyed by
// (anchor, sat, list, byte), holds the pool set it leads to.
constexpr int kListState = 1 << 20;
constexpr int kLT = 512;                 // boundary entries of a row (LDS hash table)
constexpr uint32_t kLTEmpty = 0xFFFFFFFFu;
constexpr int kReqLT = 1 << 30;          // request list: boundary entry `slot` (else set << 8 | byte)
// Direct-mapped LDS cache of the lists' byte table (global, 1 KB per list):
// word = list << 21 | byte << 13 | code, code 0x1FFF empties (-1), 0x1FFE
// boundary (-2), else sat << 11 | list reached (list ids < 2048); an empty
// slot (all ones) names list 2047, which no table has.  One 32-bit word per
// entry, so a reader sees a whole entry whichever thread wrote it last.
constexpr int kLC = 1024;
static_assert(BPD_PDA_MAX_FRAME_LISTS < 2047, "list ids of the byte-table cache are 11 bits");

// (the bytes of one list take distinct slots: 11 is odd)
__device__ __forceinline__ int lc_slot(int l, int byte) {
  return int((uint32_t(l) * 37u + uint32_t(byte) * 11u) & uint32_t(kLC - 1));
}
__device__ __forceinline__ uint32_t lc_entry(int l, int byte, int code) {
  const uint32_t c = code == -1 ? 0x1FFFu
                     : code < 0 ? 0x1FFEu
                                : (uint32_t(code & 0x7FF) | ((code & BPD_PDA_FRAME_SAT) != 0 ? 0x800u : 0u));
  return (uint32_t(l) << 21) | (uint32_t(byte) << 13) | c;
}

__device__ __forceinline__ int list_code(const BpdPdaFrames& f, uint32_t* lcache, int l, int byte) {
  const uint32_t tag = (uint32_t(l) << 21) | (uint32_t(byte) << 13);
  const int slot = lc_slot(l, byte);
  const uint32_t w = lcache[slot];
  if ((w & ~0x1FFFu) == tag) {
    const uint32_t c = w & 0x1FFFu;
    return c == 0x1FFFu ? -1 : c == 0x1FFEu ? -2 : int((c & 0x7FFu) | ((c & 0x800u) != 0u ? BPD_PDA_FRAME_SAT : 0));
  }
  const int code = f.trans[l * 256 + byte];
  lcache[slot] = lc_entry(l, byte, code);
  return code;
}

__device__ __forceinline__ bool walking(int cur) { return cur < 256 || cur >= kListState; }
__device__ __forceinline__ int list_state(int anchor, int sl) {
  // sl: the anchor's frame-list word (list | saturation flag | base << kListBase)
  return kListState | (anchor << 13) | ((sl & BPD_PDA_FRAME_SAT) != 0 ? 1 << 12 : 0) | (sl & 0xFFF);
}
// key of a boundary entry: anchor << 21 | sat << 20 | list << 8 | byte
__device__ __forceinline__ uint32_t lt_key_of(int cur, int byte) {
  return (uint32_t(cur - kListState) << 8) | uint32_t(byte);
}
__device__ __forceinline__ uint32_t lt_hash(uint32_t key) {
  key ^= key >> 15;
  key *= 0x2C1B3C6Du;
  key ^= key >> 12;
  return key;
}

struct MemoWs {
  uint32_t* header;   // [64]: word 0 = generation of the last mask launch on this workspace,
                      // words 2-3 = pack key of the token records it walked (0: none),
                      // word kFinishWord = running count of rows that reached their logits,
                      // word kFinishWord + 1 = its value when the last mask launch began,
                      // words kDeferWord + 2k.. (64 bits) = generation << 32 | row of
                      // deferred write slot k
  int32_t* pool;      // [rows, kMemoSets, kConfigWords]
  int32_t* cand;      // [rows, kMemoReq, kConfigWords]
  int32_t* overflow;  // [rows]
  int32_t* meta;      // [rows, 4]: interned sets (0: dead row), tag low, tag high, generation
  uint32_t* table;    // [rows, kMemoSets * 64]: the row's transition table after the mask
                      // (ids flagged kTExact where the step's raw words are the set's)
  uint4* recs;        // [vocab] first 16 bytes of the token at walk position k, zero padded
  int2* tmeta;        // [vocab] (token id, length) of the token at walk position k
  uint4* trecs;       // [vocab] (length, first 12 bytes) of token t, by token id
  uint2* queue;       // [rows, 2, qcap] paused tokens of the row-wide walk (two buffers)
  int32_t qcap;       // entries per queue buffer (queue_cap)
  uint2* lt;          // [rows, kLT]: the row's boundary table after the mask (key, entry;
                      // entry | kTExact where the step's raw words are the set's)
  int32_t* slist;     // [rows, kMemoSets]: frame-list word of each interned set (-1: none)
  uint32_t* defer;    // [kDefer, kMemoMaxVocab / 32]: verdict bits of the deferred rows
};

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// The last kDefer rows of a logits launch to finish their walk leave the
// logits write to the launch after it (pda_mask_kernel), which spreads each
// row over kDeferBlocks one-wave blocks: one block writes a row at the store
// rate of one CU, and these rows end after every other row has written its
// own.  The slots carry the launch's generation and the finish count runs
// on (the launch after a mask copies it as the next launch's base), so no
// launch has to clear them.
constexpr int kDefer = 4;
constexpr int kDeferBlocks = 128;
constexpr int kFinishWord = 8;
constexpr int kDeferWord = 16;
static_assert(kDeferWord + 2 * kDefer <= 64, "deferred slots in the workspace header");

// Entries of each of a row's two queue buffers: the whole vocab up to 4096
// tokens, a quarter of it above, at most kQueueMax (a row that pauses more
// tokens in one pass starts again in tile mode).  The bench rows pause at
// most 2,692 of 151,936 tokens in their first pass; at kQueueMax the
// buffers take 256 KB of a row's workspace instead of 608 KB at V/4.
constexpr int64_t kQueueMax = 16384;
int32_t queue_cap(int64_t vocab) {
  const int64_t v = vocab > 0 ? vocab : 0;
  int64_t cap = v <= 4096 ? v : std::min<int64_t>((v + 3) / 4, kQueueMax);
  // BPD_PDA_QUEUE_CAP lowers it (tests of the full-queue path; read by the
  // workspace size and the launch alike)
  if (const char* e = std::getenv("BPD_PDA_QUEUE_CAP")) {
    const long q = std::atol(e);
    if (q > 0 && q < cap) cap = q;
  }
  return int32_t(cap);
}

size_t memo_ws_bytes(int64_t rows, int64_t vocab) {
  const size_t r = size_t(rows > 0 ? rows : 0), v = size_t(vocab > 0 ? vocab : 0);
  const size_t sets = r * (kMemoSets + kMemoReq) * kConfigWords * sizeof(int32_t);
  return 256 + sets + align256(r * 4) + align256(r * 16) + r * kMemoSets * 256 + v * sizeof(uint4) +
         v * sizeof(int2) + v * sizeof(uint4) + r * 2 * size_t(queue_cap(vocab)) * sizeof(uint2) +
         r * kLT * sizeof(uint2) +
         align256(r * kMemoSets * sizeof(int32_t)) + size_t(kDefer) * (kMemoMaxVocab / 32) * sizeof(uint32_t);
}

MemoWs memo_ws(void* base, int64_t rows, int64_t vocab) {
  MemoWs w;
  const size_t r = size_t(rows);
  w.header = static_cast<uint32_t*>(base);
  w.pool = reinterpret_cast<int32_t*>(static_cast<char*>(base) + 256);
  w.cand = w.pool + r * kMemoSets * kConfigWords;
  w.overflow = w.cand + r * kMemoReq * kConfigWords;
  char* p = reinterpret_cast<char*>(w.overflow) + align256(r * 4);
  w.meta = reinterpret_cast<int32_t*>(p);
  p += align256(r * 16);
  w.table = reinterpret_cast<uint32_t*>(p);
  p += r * kMemoSets * 256;
  w.recs = reinterpret_cast<uint4*>(p);
  p += size_t(vocab) * sizeof(uint4);
  w.tmeta = reinterpret_cast<int2*>(p);
  p += size_t(vocab) * sizeof(int2);
  w.trecs = reinterpret_cast<uint4*>(p);
  p += size_t(vocab) * sizeof(uint4);
  w.queue = reinterpret_cast<uint2*>(p);
  w.qcap = queue_cap(vocab);
  p += r * 2 * size_t(w.qcap) * sizeof(uint2);
  w.lt = reinterpret_cast<uint2*>(p);
  p += r * kLT * sizeof(uint2);
  w.slist = reinterpret_cast<int32_t*>(p);
  p += align256(r * kMemoSets * sizeof(int32_t));
  w.defer = reinterpret_cast<uint32_t*>(p);
  return w;
}

// Generation of a mask launch: the launch stamps it on every row it writes
// and in the workspace header, and the commit reuses a row's tables only when
// the row's stamp equals the header's -- the rows were written by the last
// mask launch on the workspace.  (The layout depends on the row count, so a
// later launch with fewer rows overwrites parts of a larger batch's pool
// while that batch's row metadata stays intact.)  Process-wide, never 0.
std::atomic<uint32_t> g_mask_generation{1};

uint32_t next_generation() {
  uint32_t g = g_mask_generation.fetch_add(1);
  if (g == 0) g = g_mask_generation.fetch_add(1);
  return g;
}

// Identity of the grammar and token tables a workspace's transition tables
// were built for (the commit reuses them only for the same tables).
uint64_t memo_tag(const BpdPdaTable* g, const BpdTokenBytes* toks, int64_t rows) {
  uint64_t h = 1469598103934665603ull ^ uint64_t(rows);
  auto mix = [&](uint64_t x) { h = (h ^ x) * 1099511628211ull; };
  mix(reinterpret_cast<uintptr_t>(g->edge_offsets));
  mix(reinterpret_cast<uintptr_t>(g->edge_kind));
  mix(reinterpret_cast<uintptr_t>(g->accept));
  mix(uint64_t(uint32_t(g->num_states)));
  mix(uint64_t(uint32_t(g->num_edges)));
  mix(reinterpret_cast<uintptr_t>(toks->offsets));
  mix(reinterpret_cast<uintptr_t>(toks->bytes));
  mix(uint64_t(uint32_t(toks->vocab_size)));
  return h;
}

// Key of the token records a launch packs: the caller's content tag of the
// token tables, the row count (the records' place in the workspace depends
// on it), the vocabulary and whether a walk order is given.  0 (never
// skipped) when the caller gives no tag.
uint64_t pack_key(const BpdTokenBytes* toks, int64_t rows) {
  if (toks->pack_tag == 0) return 0;
  uint64_t h = 1469598103934665603ull ^ toks->pack_tag;
  auto mix = [&](uint64_t x) { h = (h ^ x) * 1099511628211ull; };
  mix(uint64_t(rows));
  mix(uint64_t(uint32_t(toks->vocab_size)));
  mix(toks->order ? 1u : 0u);
  return h ? h : 1;
}

// Record k of the token records below, and token t's record by id.
__device__ __forceinline__ void pack_record(const int32_t* off, const uint8_t* bytes, const int32_t* order, int32_t k,
                                            uint4* recs, int2* meta, uint4* trecs) {
  const int32_t t = order ? order[k] : k;
  const int32_t s = off[t];
  const int32_t len = off[t + 1] - s;
  const int32_t n = min(len, 16);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  for (int i = 0; i < n; ++i) w[i >> 2] |= uint32_t(bytes[s + i]) << ((i & 3) * 8);
  recs[k] = make_uint4(w[0], w[1], w[2], w[3]);
  meta[k] = make_int2(t, len);
  trecs[t] = make_uint4(uint32_t(len), w[0], w[1], w[2]);
}

// Token records in walk order (k -> t = order[k], or t = k): recs[k] = the
// first 16 bytes of t (little-endian words, zero padded), meta[k] = (t,
// length of t), so the walks read them coalesced; trecs[t] = (length of t,
// its first 12 bytes), so the commit has a short token's bytes one read
// after the token id.  Nothing to do when the
// workspace header carries this launch's pack key: the last mask launch on
// the workspace walked records of the same tables at the same place, and
// nothing but a pack writes there (the key is stamped by the launch after
// the mask, once every record is written).
__global__ __launch_bounds__(256) void pack_tokens_kernel(const int32_t* __restrict__ off,
                                                          const uint8_t* __restrict__ bytes,
                                                          const int32_t* __restrict__ order,
                                                          int32_t vocab, uint4* __restrict__ recs,
                                                          int2* __restrict__ meta, uint4* __restrict__ trecs,
                                                          const uint32_t* __restrict__ header,
                                                          uint64_t key) {
  if (key != 0 && header[2] == uint32_t(key) && header[3] == uint32_t(key >> 32)) return;
  for (int32_t k = int32_t(blockIdx.x) * 256 + int32_t(threadIdx.x); k < vocab; k += int32_t(gridDim.x) * 256)
    pack_record(off, bytes, order, k, recs, meta, trecs);
}

__device__ inline int packed_byte(const uint4& p, int i) {
  const uint32_t w = i < 4 ? p.x : (i < 8 ? p.y : (i < 12 ? p.z : p.w));
  return int((w >> ((i & 3) * 8)) & 0xFFu);
}

// FNV-1a over a set's meaningful words.
template <class V>
__device__ uint32_t set_hash(const V& c) {
  uint32_t h = 2166136261u;
  auto mix = [&](uint32_t x) { h = (h ^ x) * 16777619u; };
  const int n = c.n();
  mix(uint32_t(n));
  mix(uint32_t(c.sat()));
  for (int i = 0; i < n; ++i) {
    const int d = c.depth(i);
    mix(uint32_t(d));
    for (int k = 0; k < d; ++k) mix(uint32_t(c.frame(i, k)));
  }
  return h;
}

template <class A, class B>
__device__ bool same_set(const A& x, const B& y) {
  const int n = x.n();
  if (n != y.n() || x.sat() != y.sat()) return false;
  for (int i = 0; i < n; ++i) {
    const int d = x.depth(i);
    if (d != y.depth(i)) return false;
    for (int k = 0; k < d; ++k)
      if (x.frame(i, k) != y.frame(i, k)) return false;
  }
  return true;
}

// ---- wave-cooperative advance_byte (resolution rounds of the memo kernel)
// The same steps as advance_byte / close / prune_dead of pda_core.hpp on
// FlatView sets held in LDS, with the inner work spread over the 64 lanes of
// one wave: holds() compares config j's frames on lanes 8j..8j+7 and ballots,
// append() copies frames lane-parallel, the compaction of prune_dead moves one
// config at a time with its frames lane-parallel.  Control flow is uniform
// across the wave, so every append happens in the sequential order.  LDS
// operations of one wave complete in order, so a wave-scope fence is enough
// between a lane's write and another lane's read.
__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kF = 2 + kMaxConfigs;  // first frame word
constexpr int kSetLoads = (kConfigWords + kWave - 1) / kWave;  // words of a set per lane

__device__ inline bool coop_holds(const int32_t* dst, const int32_t* src, int i, int keep, int x0,
                                  int x1, int nx, int lane) {
  const int D = keep + nx;
  const int n = dst[0];
  const int j = lane >> 3, q = lane & 7;
  bool ok = j < n && dst[2 + j] == D;
  for (int k = q; ok && k < D; k += 8) {
    const int want = k < keep ? src[kF + i * kMaxDepth + k] : (k == keep ? x0 : x1);
    ok = dst[kF + j * kMaxDepth + k] == want;
  }
  uint64_t t = __ballot(ok);
  t &= t >> 1;
  t &= t >> 2;
  t &= t >> 4;
  return (t & 0x0101010101010101ull) != 0;
}

__device__ inline bool coop_append(int32_t* dst, const int32_t* src, int i, int keep, int x0, int x1,
                                   int nx, int lane) {
  const int n = dst[0];
  if (n >= kMaxConfigs) {
    wave_sync();
    if (lane == 0) dst[1] = 1;
    wave_sync();
    return false;
  }
  if (lane < keep) dst[kF + n * kMaxDepth + lane] = src[kF + i * kMaxDepth + lane];
  wave_sync();
  if (lane == 0) {
    if (nx > 0) dst[kF + n * kMaxDepth + keep] = x0;
    if (nx > 1) dst[kF + n * kMaxDepth + keep + 1] = x1;
    dst[2 + n] = keep + nx;
    dst[0] = n + 1;
  }
  wave_sync();
  return true;
}

// Lane i's value of v for a wave-uniform i with every lane active: a scalar
// read of the register (no LDS round trip, unlike a shuffle).
__device__ __forceinline__ int lane_value(int v, int i) { return __builtin_amdgcn_readlane(v, i); }
// v of the first active lane, for a v every active lane holds alike: the
// compiler then keeps it in a scalar register and branches on it as such.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Sum of v over the wave, in every lane (every lane active): DPP exchanges
// within each row of 16 lanes (lane ^ 1, lane ^ 2, then the half-row and row
// mirrors), then the four row sums by scalar lane reads -- no LDS round
// trip, where a shuffle reduction takes six.
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
  uint32_t s = v;
  s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x141, 0xF, 0xF, false));  // row_half_mirror
  s += uint32_t(__builtin_amdgcn_update_dpp(0, int(s), 0x140, 0xF, 0xF, false));  // row_mirror
  return uint32_t(__builtin_amdgcn_readlane(int(s), 0)) + uint32_t(__builtin_amdgcn_readlane(int(s), 16)) +
         uint32_t(__builtin_amdgcn_readlane(int(s), 32)) + uint32_t(__builtin_amdgcn_readlane(int(s), 48));
}

// Closure of c in place.  Lane l < c[0] holds config l's depth (d_l) and
// top state (top_l) on entry; the edge range and accept flag of every top are
// loaded at once, and a config that an append adds gets its own in lane n as
// it is added (the loads complete while earlier configs are visited), so a
// visit waits for no table read before its edges.
__device__ bool coop_close(const PdaTableView& g, int32_t* c, int lane, int d_l, int top_l) {
  // one visit per config in index order, as close() in pda_core.hpp; the
  // top state's edges are loaded lane-parallel and the eps / call edges taken
  // in edge order from the ballot
  int n = c[0];
  int eb_l = 0, ee_l = 0, acc_l = 0;
  if (lane < n && d_l > 0) {
    eb_l = g.edge_offsets[top_l];
    ee_l = g.edge_offsets[top_l + 1];
    acc_l = g.accept[top_l];
  }
  for (int i = 0; i < n; ++i) {
    const int d = lane_value(d_l, i);
    if (d <= 0) continue;
    const int eb = lane_value(eb_l, i), ee = lane_value(ee_l, i);
    // config i's first `keep` frames and x0, x1 (nx of them) unless present;
    // the new config's top is `ntop`
    auto add = [&](int keep, int x0, int x1, int nx, int ntop) {
      if (coop_holds(c, c, i, keep, x0, x1, nx, lane) || !coop_append(c, c, i, keep, x0, x1, nx, lane)) return;
      if (lane == n) {
        d_l = keep + nx;
        top_l = ntop;
        eb_l = g.edge_offsets[ntop];
        ee_l = g.edge_offsets[ntop + 1];
        acc_l = g.accept[ntop];
      }
      ++n;
    };
    if (lane_value(acc_l, i) != 0 && d > 1) add(d - 1, 0, 0, 0, c[kF + i * kMaxDepth + d - 2]);
    for (int base = eb; base < ee; base += kWave) {
      const int e = base + lane;
      int kind = -1, x0 = 0, x1 = 0;
      if (e < ee) {
        kind = g.edge_kind[e];
        x0 = g.edge_dst[e];
        x1 = g.edge_callee[e];
      }
      uint64_t m = __ballot(kind == BPD_PDA_EDGE_EPS || kind == BPD_PDA_EDGE_CALL);
      while (m) {
        const int l = __ffsll(static_cast<unsigned long long>(m)) - 1;
        m &= m - 1;
        const int k = lane_value(kind, l), y0 = lane_value(x0, l), y1 = lane_value(x1, l);
        if (k == BPD_PDA_EDGE_EPS) {
          add(d - 1, y0, 0, 1, y0);
        } else if (d + 1 <= kMaxDepth) {
          add(d - 1, y0, y1, 2, y1);
        } else {
          wave_sync();
          if (lane == 0) c[1] = 1;
          wave_sync();
        }
      }
    }
  }
  // prune_dead: order-preserving compaction, vacated words not cleared (the
  // live flags of every top read at once)
  const uint64_t live = __ballot(lane < n && d_l > 0 && g.live[top_l] != 0);
  int out = 0;
  for (int i = 0; i < n; ++i) {
    if (((live >> i) & 1u) == 0u) continue;
    if (out != i) {
      const int d = lane_value(d_l, i);
      if (lane < d) c[kF + out * kMaxDepth + lane] = c[kF + i * kMaxDepth + lane];
      wave_sync();
      if (lane == 0) c[2 + out] = d;
      wave_sync();
    }
    ++out;
  }
  wave_sync();
  if (lane == 0) c[0] = out;
  wave_sync();
  return out > 0;
}

// next = close(byte step of src) with next freshly zeroed (as
// FlatView::reset_all).  The depth, top and edge range of every config of
// src are read at once (lane l: config l); the configs the step appends to
// next hand their depth and top to coop_close the same way.
__device__ bool coop_advance_byte(const PdaTableView& g, const int32_t* src, int32_t* next, int byte,
                                  int lane) {
  for (int k = lane; k < kConfigWords; k += kWave) next[k] = 0;
  const int n = src[0];
  int sd = 0, seb = 0, see = 0;
  if (lane < n) {
    sd = src[2 + lane];
    if (sd > 0) {
      const int top = src[kF + lane * kMaxDepth + sd - 1];
      seb = g.edge_offsets[top];
      see = g.edge_offsets[top + 1];
    }
  }
  wave_sync();
  int nd = 0, ntop = -1, nn = 0;  // lane l: depth and top of config l of next
  for (int i = 0; i < n; ++i) {
    const int d = lane_value(sd, i);
    if (d <= 0) continue;
    const int eb = lane_value(seb, i), ee = lane_value(see, i);
    for (int base = eb; base < ee; base += kWave) {
      const int e = base + lane;
      bool match = false;
      int x = 0;
      if (e < ee && g.edge_kind[e] == BPD_PDA_EDGE_BYTE) {
        match = byte >= g.edge_lo[e] && byte <= g.edge_hi[e];
        x = g.edge_dst[e];
      }
      uint64_t m = __ballot(match);
      while (m) {
        const int l = __ffsll(static_cast<unsigned long long>(m)) - 1;
        m &= m - 1;
        const int y = lane_value(x, l);
        if (!coop_holds(next, src, i, d - 1, y, 0, 1, lane) && coop_append(next, src, i, d - 1, y, 0, 1, lane)) {
          if (lane == nn) {
            nd = d;
            ntop = y;
          }
          ++nn;
        }
      }
    }
  }
  wave_sync();
  if (lane == 0) next[1] = (next[1] || src[1]) ? 1 : 0;
  wave_sync();
  return coop_close(g, next, lane, nd, ntop);
}

// Is word w of a FlatView set with n configs and depths dep() meaningful?
__device__ inline bool meaningful_word(const int32_t* c, int n, int w) {
  if (w < 2) return true;
  if (w < kF) return w - 2 < n;
  const int i = (w - kF) / kMaxDepth, k = (w - kF) % kMaxDepth;
  return i < n && k < c[2 + i];
}

__device__ inline uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

// Hash of a set's meaningful words (sum of per-word mixes, lane-parallel);
// every lane gets the value.  c must be a well-formed set (n <= 8, depths <= 32).
__device__ uint32_t coop_hash(const int32_t* c, int lane) {
  const int n = c[0];
  uint32_t h = 0;
  for (int w = lane; w < kConfigWords; w += kWave)
    if (meaningful_word(c, n, w)) h += mix32(uint32_t(w) * 0x9E3779B1u ^ uint32_t(c[w]));
  h = wave_sum(h);
  return h;
}

// Equal meaningful words (x in LDS, y anywhere); every lane gets the answer,
// and `raw` whether every word is equal.  One pass over the words: n and the
// saturation flag are words 0 and 1, the depths words 2..9, so a frame is
// compared where it is meaningful in x once those are equal.
__device__ bool coop_same_raw(const int32_t* x, const int32_t* y, int lane, bool& raw) {
  const int n = x[0];
  bool diff = false, rdiff = false;
  for (int w = lane; w < kConfigWords; w += kWave) {
    const bool ne = x[w] != y[w];
    rdiff |= ne;
    if (w < kF) {
      diff |= ne && (w < 2 || w - 2 < n);
    } else {
      const int i = (w - kF) / kMaxDepth, k = (w - kF) % kMaxDepth;
      diff |= ne && i < n && k < x[2 + i];
    }
  }
  raw = __ballot(rdiff) == 0;
  return __ballot(diff) == 0;
}

__device__ inline bool coop_same(const int32_t* x, const int32_t* y, int lane) {
  bool raw;
  return coop_same_raw(x, y, lane, raw);
}

// Elementary byte intervals of a set, from its top states: advance_byte
// of the set depends on a byte c only through which of the tops' byte edges
// contain c, so [0, 255] splits into intervals of equal behaviour.  Bit x of
// `bnd` marks an interval start (x = lo of a byte edge, or hi + 1), bit x of
// `hit` a byte some edge contains.  One wave builds both (lanes over the
// edges, LDS atomics); edges outside [0, 255] clip as they would in a
// byte-by-byte comparison.  The set's transition row `trow` gets "dead" for
// every byte no edge contains (the step empties the set there).
__device__ void coop_set_intervals(const PdaTableView& g, const int32_t* tops, int n, uint32_t* bnd,
                                   uint32_t* hit, uint8_t* trow, int lane) {
  if (lane < 8) {
    bnd[lane] = 0u;
    hit[lane] = 0u;
  }
  wave_sync();
  for (int i = 0; i < n; ++i) {
    const int top = tops[i];
    if (top < 0) continue;
    const int ee = g.edge_offsets[top + 1];
    for (int e = g.edge_offsets[top] + lane; e < ee; e += kWave) {
      if (g.edge_kind[e] != BPD_PDA_EDGE_BYTE) continue;
      const int el = g.edge_lo[e], eh = g.edge_hi[e];
      if (el >= 1 && el <= 255) atomicOr(&bnd[el >> 5], 1u << (el & 31));
      if (eh >= 0 && eh <= 254) atomicOr(&bnd[(eh + 1) >> 5], 1u << ((eh + 1) & 31));
      const int a = el < 0 ? 0 : el, z = eh > 255 ? 255 : eh;
      for (int w = a >> 5; a <= z && w <= (z >> 5); ++w) {
        const int b0 = (a > w * 32 ? a : w * 32) - w * 32, b1 = (z < w * 32 + 31 ? z : w * 32 + 31) - w * 32;
        const uint32_t upto = b1 == 31 ? 0xFFFFFFFFu : ((1u << (b1 + 1)) - 1u);
        atomicOr(&hit[w], upto & ~((1u << b0) - 1u));
      }
    }
  }
  wave_sync();
  for (int c = lane; c < 256; c += kWave)
    if (((hit[c >> 5] >> (c & 31)) & 1u) == 0u) trow[c] = kTDead;
}

// The elementary interval [lo, hi] of `byte` from a set's bitmaps; returns
// whether some byte edge contains it (if none does, the step from the set
// empties it on the whole interval).
__device__ inline bool set_interval(const uint32_t* bnd, const uint32_t* hit, int byte, int& lo, int& hi) {
  const int b = byte & 31;
  const uint32_t le = b == 31 ? 0xFFFFFFFFu : ((2u << b) - 1u);  // bits 0..b
  int w = byte >> 5;
  uint32_t m = bnd[w] & le;
  while (m == 0u && w > 0) m = bnd[--w];
  lo = m ? w * 32 + 31 - __clz(m) : 0;
  w = byte >> 5;
  m = bnd[w] & ~le;
  while (m == 0u && w < 7) m = bnd[++w];
  hi = m ? w * 32 + __ffs(m) - 2 : 255;
  return (hit[byte >> 5] >> b) & 1u;
}

// First byte of the elementary interval of `byte` (as set_interval's lo),
// from the set's interval-start bitmap read as two 16-byte words: the walk
// asks for it on every missing entry, so it avoids set_interval's chain of
// dependent reads.
__device__ inline int interval_start(const uint32_t* bnd, int byte) {
  const uint4 a = reinterpret_cast<const uint4*>(bnd)[0];
  const uint4 b = reinterpret_cast<const uint4*>(bnd)[1];
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  const int bw = byte >> 5, bb = byte & 31;
  const uint32_t le = bb == 31 ? 0xFFFFFFFFu : ((2u << bb) - 1u);  // bits 0..bb
  int lo = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t m = k < bw ? w[k] : (k == bw ? (w[k] & le) : 0u);
    if (m != 0u) lo = k * 32 + 31 - __clz(m);
  }
  return lo;
}

// byte p of the token at walk position k (its first 16 bytes are packed)
__device__ __forceinline__ int long_byte(const MaskArgs& a, int64_t k, int32_t p) {
  const int64_t t = a.order ? a.order[k] : k;
  return a.tok_bytes[a.tok_off[t] + p];
}

__device__ __forceinline__ uint32_t frame_mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7FEB352Du;
  x ^= x >> 15;
  x *= 0x846CA68Bu;
  x ^= x >> 16;
  return x;
}

// The frame list of a set held in LDS (-1: none).  The common stack P is
// tried at the configs' longest common prefix below every top and up to
// BPD_PDA_FRAME_SUFFIX - 1 frames shorter, shortest first, each with every
// suffix at most BPD_PDA_FRAME_SUFFIX frames and P plus that many frames
// within the depth limit.  For each, lane w < BPD_PDA_FRAME_KEY_WORDS builds
// word w of the key the suffixes would have and its term of the key's hash
// (a sum of per-word mixes, grammar/frames.py list_hash); the probe reads the
// slot table (`slots`, staged in LDS) 64 slots at a time up to the first
// empty slot and compares the keys of fingerprint matches lane-parallel.
// Called by the 64 lanes of a wave; every lane gets the answer (and, in
// base_out, the depth of P).  With `codes` (4 per lane), the byte codes of
// the list found are read beside its key: lane l gets those of bytes l,
// 64 + l, 128 + l and 192 + l.
__device__ int frame_list_of(const int32_t* c, const BpdPdaFrames& f, const uint32_t* slots, int lane,
                              int* base_out = nullptr, int32_t* codes = nullptr) {
  if (f.num_lists <= 0) return -1;
  const int n = c[0];
  if (n < 1 || n > kMaxConfigs) return -1;
  int mind = kMaxDepth + 1, maxd = 0;
  for (int i = 0; i < n; ++i) {
    const int d = c[2 + i];
    mind = d < mind ? d : mind;
    maxd = d > maxd ? d : maxd;
  }
  if (mind < 1 || maxd > kMaxDepth) return -1;
  // common prefix: lane k < mind - 1 compares frame k of every config
  bool stop = lane >= mind - 1;
  for (int i = 1; i < n && !stop; ++i) stop = c[kF + i * kMaxDepth + lane] != c[kF + lane];
  const int p = __ffsll(static_cast<unsigned long long>(__ballot(stop))) - 1;
  const int jmax = p < BPD_PDA_FRAME_SUFFIX - 1 ? p : BPD_PDA_FRAME_SUFFIX - 1;
  for (int j = jmax; j >= 0; --j) {
    const int base = p - j;
    if (base + BPD_PDA_FRAME_SUFFIX > kMaxDepth || maxd - base > BPD_PDA_FRAME_SUFFIX) continue;
    int32_t want = 0;
    uint32_t term = 0;
    if (lane == 0) {
      want = n;
      term = frame_mix(0xC2B2AE35u ^ uint32_t(n));
    } else if (lane <= kMaxConfigs) {
      const int i = lane - 1;
      if (i < n) {
        want = c[2 + i] - base;
        term = frame_mix((uint32_t((i << 8) | 0xFF) * 0x85EBCA6Bu) ^ uint32_t(want));
      }
    } else if (lane < 1 + kMaxConfigs + kMaxConfigs * BPD_PDA_FRAME_SUFFIX) {
      const int i = (lane - 1 - kMaxConfigs) / BPD_PDA_FRAME_SUFFIX;
      const int k = (lane - 1 - kMaxConfigs) % BPD_PDA_FRAME_SUFFIX;
      if (i < n && k < c[2 + i] - base) {
        want = c[kF + i * kMaxDepth + base + k];
        term = frame_mix((uint32_t((i << 8) | k) * 0x9E3779B1u) ^ uint32_t(want));
      }
    }
    term = wave_sum(term);
    const uint32_t h = frame_mix(term);
    const uint32_t fp = (h >> 10) & 0xFFFFFu;
    uint32_t at = h;
    for (int w = 0; w < BPD_PDA_FRAME_SLOTS / kWave; ++w, at += kWave) {
      const uint32_t e = slots[(at + uint32_t(lane)) & (BPD_PDA_FRAME_SLOTS - 1)];
      const uint64_t empty = __ballot(e == BPD_PDA_FRAME_EMPTY);
      const int lim = empty != 0u ? __ffsll(static_cast<unsigned long long>(empty)) - 1 : kWave;
      uint64_t m = __ballot(lane < lim && (e >> 12) == fp);
      while (m != 0u) {
        const int k = __ffsll(static_cast<unsigned long long>(m)) - 1;
        m &= m - 1;
        const int id = int(uint32_t(lane_value(int(e), k)) & 0xFFFu);
        if (id < f.num_lists) {
          if (codes) {
#pragma unroll
            for (int q = 0; q < 4; ++q) codes[q] = f.trans[id * 256 + q * kWave + lane];
          }
          const bool diff = lane < BPD_PDA_FRAME_KEY_WORDS && f.keys[id * BPD_PDA_FRAME_KEY_WORDS + lane] != want;
          if (__ballot(diff) == 0u) {
            if (base_out) *base_out = base;
            return id;
          }
        }
      }
      if (empty != 0u) break;
    }
  }
  return -1;
}

// Transition-table row of set `id`, a set in frame list l: a byte whose step
// keeps the list (and, unless the set is already saturated, drops nothing)
// leads back to the set, a byte whose step empties it is dead; the other
// entries stay unknown until a walk requests them.  One wave.
__device__ inline void frame_fill_entry(int32_t code, int l, bool sat, int id, uint8_t* trow, int c) {
  if (code == -1) {
    trow[c] = kTDead;
  } else if (code >= 0 && (code & (BPD_PDA_FRAME_SAT - 1)) == l && (sat || (code & BPD_PDA_FRAME_SAT) == 0)) {
    trow[c] = uint8_t(id);
  }
}

__device__ void frame_fill_row(const BpdPdaFrames& f, int l, bool sat, int id, uint8_t* trow, int lane) {
  const int32_t* tr = f.trans + l * 256;
  for (int c = lane; c < 256; c += kWave) frame_fill_entry(tr[c], l, sat, id, trow, c);
}

// The meaningful words of the set of list `key` over the common stack that
// config 0 of `src` holds in its first `base` frames, written to `dst`
// (words past each depth set to 0; dst may be src).  One wave.
static_assert(BPD_PDA_FRAME_KEY_WORDS <= kWave, "a frame-list key is read one word per lane");
__device__ void compose_list_set(const int32_t* src, int32_t* dst, const int32_t* key, int base, int sat,
                                 int lane) {
  // the key in one load (lane l: word l), read back by lane exchanges
  const int32_t kw = lane < BPD_PDA_FRAME_KEY_WORDS ? key[lane] : 0;
  const int32_t pw = lane < base ? src[kF + lane] : 0;
  const int n = lane_value(kw, 0);
  wave_sync();
  // a lane's frame index k = lane % 32 is the same in every pass, so its
  // common-stack frame is exchanged once; the two configs of a pass (lanes
  // below and above 32) read their suffix lengths by scalar lane reads
  static_assert(kWave == 2 * kMaxDepth, "two configs per pass of the wave");
  const int32_t p = __shfl(pw, (lane & (kMaxDepth - 1)) < base ? (lane & (kMaxDepth - 1)) : 0);
  for (int w = lane; w < kMaxConfigs * kMaxDepth; w += kWave) {
    const int i = w / kMaxDepth, k = w % kMaxDepth;
    const int i0 = (w - lane) / kMaxDepth;  // the pass's first config (wave-uniform)
    const int len0 = lane_value(kw, 1 + i0), len1 = lane_value(kw, 2 + i0);
    const int len = lane < kMaxDepth ? len0 : len1;
    const int f = k - base < 0 ? 0 : (k - base < BPD_PDA_FRAME_SUFFIX ? k - base : BPD_PDA_FRAME_SUFFIX - 1);
    const int32_t sfx = __shfl(kw, 1 + kMaxConfigs + i * BPD_PDA_FRAME_SUFFIX + f);
    int32_t v = 0;
    if (i < n) {
      if (k < base)
        v = p;
      else if (k < base + len)
        v = sfx;
    }
    dst[kF + w] = v;
  }
  const int len_l = __shfl(kw, 1 + (lane & (kMaxConfigs - 1)));
  if (lane < kMaxConfigs) dst[2 + lane] = lane < n ? base + len_l : 0;
  if (lane == 0) {
    dst[0] = n;
    dst[1] = sat;
  }
  wave_sync();
}

// LDS bytes a launch of `kernel` can add to its static arrays on the current
// device (the device's per-workgroup limit less the kernel's own), queried
// once per device and kernel slot.
int lds_room(const void* kernel, int slot, size_t* room) {
  constexpr int kDevices = 64;
  static std::atomic<long long> cache[kDevices][2];  // room + 1; 0: not queried yet
  int dev = 0;
  BPD_HIP(hipGetDevice(&dev));
  if (dev >= 0 && dev < kDevices) {
    const long long c = cache[dev][slot].load(std::memory_order_relaxed);
    if (c > 0) {
      *room = size_t(c - 1);
      return BPD_OK;
    }
  }
  int max_lds = 0;
  BPD_HIP(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
  hipFuncAttributes fa{};
  BPD_HIP(hipFuncGetAttributes(&fa, kernel));
  *room = size_t(max_lds) > fa.sharedSizeBytes ? size_t(max_lds) - fa.sharedSizeBytes : 0;
  if (dev >= 0 && dev < kDevices) cache[dev][slot].store((long long)(*room) + 1, std::memory_order_relaxed);
  return BPD_OK;
}

// Bytes of the grammar tables staged in LDS by stage_tables.
size_t staged_table_bytes(const BpdPdaTable* g) {
  return (size_t(g->num_states) + 1) * 4 + size_t(g->num_edges) * 20 + (size_t(g->num_states) * 2 + 3) / 4 * 4;
}

// Entry tid of each grammar table, read into registers before the workgroup
// fills its LDS arrays so that these loads are in flight meanwhile.
struct TableSlice {
  int32_t eo, ek, elo, ehi, ed, ec;
  uint8_t acc, lv;
};

__device__ TableSlice table_slice(const PdaTableView& src, int tid) {
  TableSlice t{0, 0, 0, 0, 0, 0, 0, 0};
  if (tid <= src.num_states) t.eo = src.edge_offsets[tid];
  if (tid < src.num_edges) {
    t.ek = src.edge_kind[tid];
    t.elo = src.edge_lo[tid];
    t.ehi = src.edge_hi[tid];
    t.ed = src.edge_dst[tid];
    t.ec = src.edge_callee[tid];
  }
  if (tid < src.num_states) {
    t.acc = src.accept[tid];
    t.lv = src.live[tid];
  }
  return t;
}

// Copy of the grammar tables in LDS at `tab` (staged_table_bytes long) made
// by the workgroup's `nthreads` threads (entry tid of each table from the
// thread's slice, the entries past nthreads read here), and a view of it;
// the caller synchronises before the view is read.
__device__ PdaTableView stage_tables(const PdaTableView& src, int32_t* tab, const TableSlice& t, int tid,
                                     int nthreads) {
  const int N = src.num_states, E = src.num_edges;
  int32_t* eo = tab;
  int32_t* ek = eo + N + 1;
  int32_t* elo = ek + E;
  int32_t* ehi = elo + E;
  int32_t* ed = ehi + E;
  int32_t* ec = ed + E;
  uint8_t* acc = reinterpret_cast<uint8_t*>(ec + E);
  uint8_t* lv = acc + N;
  if (tid <= N) eo[tid] = t.eo;
  for (int i = tid + nthreads; i <= N; i += nthreads) eo[i] = src.edge_offsets[i];
  if (tid < E) {
    ek[tid] = t.ek;
    elo[tid] = t.elo;
    ehi[tid] = t.ehi;
    ed[tid] = t.ed;
    ec[tid] = t.ec;
  }
  for (int i = tid + nthreads; i < E; i += nthreads) {
    ek[i] = src.edge_kind[i];
    elo[i] = src.edge_lo[i];
    ehi[i] = src.edge_hi[i];
    ed[i] = src.edge_dst[i];
    ec[i] = src.edge_callee[i];
  }
  if (tid < N) {
    acc[tid] = t.acc;
    lv[tid] = t.lv;
  }
  for (int i = tid + nthreads; i < N; i += nthreads) {
    acc[i] = src.accept[i];
    lv[i] = src.live[i];
  }
  PdaTableView g = src;
  g.edge_offsets = eo;
  g.edge_kind = ek;
  g.edge_lo = elo;
  g.edge_hi = ehi;
  g.edge_dst = ed;
  g.edge_callee = ec;
  g.accept = acc;
  g.live = lv;
  return g;
}

// verdicts of a token in the memoised walk, past every set id
constexpr int kWalkEnd = 256, kAllowed = 256, kRejected = 257, kNone = 258;

// The fill value into the rejected columns [lo, hi) of a logits row of
// E-byte elements (allowed columns: set bits of vb, indexed by column; lo a
// multiple of 64), by the T threads of a block: one column per lane, 64
// consecutive columns per wave and step, eight steps per batch with the
// batch's verdict words read first, so a step is one masked, coalesced store.
// Measured on one row of 151,936 fp32 columns whose 2.5 % allowed columns
// are spread over every 256-column group, by 1024 threads: 9.1 us, where a
// group of four columns per lane with per-column stores in mixed groups
// takes 17.2 us; a row whose destination is not in L2 is bound by the
// stores a wave keeps in flight, so the batch issues them back to back.
template <int E, int T>
__device__ __forceinline__ void write_rejected(uint8_t* rowp, const uint32_t* vb, int lo, int hi, uint32_t fill,
                                               int tid) {
  const int lane = tid & (kWave - 1);
  constexpr int kBatch = 8;
  for (int c0 = lo + tid - lane; c0 < hi; c0 += kBatch * T) {
    uint32_t w[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int c = c0 + u * T + lane;
      w[u] = c < hi ? vb[c >> 5] : 0xFFFFFFFFu;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int c = c0 + u * T + lane;
      if (((w[u] >> (c & 31)) & 1u) == 0u) {
        if (E == 2)
          *reinterpret_cast<uint16_t*>(rowp + c * 2) = uint16_t(fill & 0xFFFFu);
        else
          *reinterpret_cast<uint32_t*>(rowp + c * 4) = fill;
      }
    }
  }
}

// InLds: the grammar tables are staged in LDS (the dynamic array `tab`).  A
// compile-time choice, so that every table read of the walk and of the
// resolution rounds is an LDS read rather than a flat one.
template <bool InLds>
__global__ __launch_bounds__(kMemoThreads) void pda_memo_mask_kernel(MaskArgs a, MemoWs ws, int max_sets,
                                                                     uint64_t tag, uint32_t gen, int row_mode,
                                                                     uint64_t pkey, int lt_cap, int pack_here) {
  extern __shared__ __align__(16) int32_t tab[];  // grammar tables when they fit
  __shared__ int32_t set_tops[kMemoSets][kMaxConfigs];  // top state per config, -1 if empty
  __shared__ int32_t set_n[kMemoSets];
  __shared__ __align__(16) uint32_t set_bnd[kMemoSets][8];  // interval starts of each set's bytes
  __shared__ uint32_t set_hit[kMemoSets][8];  // bytes some top's byte edge contains
  __shared__ int32_t cand_tops[kMemoReq][kMaxConfigs];
  __shared__ int32_t cand_n[kMemoReq];
  __shared__ uint32_t T32[kMemoSets * 256 / 4];
  __shared__ uint32_t vbits[kMemoMaxVocab / 32];  // allowed tokens of the row
  __shared__ uint32_t req[kMemoSets * 8];
  __shared__ uint32_t texact[kMemoSets * 8];  // entries whose step gives the set's raw words
  __shared__ uint32_t pool_hash[kMemoSets];
  __shared__ int32_t req_list[kMemoReq];
  __shared__ uint32_t cand_hash[kMemoReq];
  __shared__ int32_t cand_res[kMemoReq];   // >= 0 pool id, -1 empty, -2 new, -4 duplicate, -5 no edge
  __shared__ int32_t cand_lead[kMemoReq];
  __shared__ uint8_t cand_exact[kMemoReq];  // an existing set with every word of the step's
  // frame list of a new set: l | BPD_PDA_FRAME_SAT (the set's saturation
  // flag) | base << kListBase (the depth of its common stack), -1 none
  __shared__ int32_t cand_list[kMemoReq];
  __shared__ int32_t set_list[kMemoSets];  // the same for the interned sets
  __shared__ int32_t set_ls[kMemoSets];    // list state a walk takes at the set, -1 none
  __shared__ uint32_t lt_key[kLT];         // boundary table: keys (kLTEmpty: free slot)
  __shared__ uint8_t lt_res[kLT];          // ... and entries (pool id, kTDead, kTOverflow, kTUnknown)
  __shared__ uint32_t lt_req[kLT / 32];    // requested boundary entries
  __shared__ uint32_t lt_exact[kLT / 32];  // entries whose step gives the set's raw words
  __shared__ int lt_used;                  // entries inserted in LT
  __shared__ uint32_t lcache[kLC];         // entries of the lists' byte table met so far
  __shared__ uint8_t cand_comp[kMemoReq];  // composed from a list's key: raw words unknown
  __shared__ uint32_t fslots[BPD_PDA_FRAME_SLOTS];  // the frame lists' slot table
  __shared__ int32_t cand_id[kMemoReq];
  __shared__ int16_t cand_lo[kMemoReq];
  __shared__ int16_t cand_hi[kMemoReq];
  __shared__ int32_t row_cfg[kConfigWords];
  __shared__ int32_t work[kMemoThreads / kWave][2][kConfigWords];  // per-wave src / dst
  __shared__ int pool_count, nreq, row_flags, overflowed, qcount, row_fail, loop_n, row_list;
  __shared__ int n_stepped, n_cheap;
  __shared__ int walk_lists;  // the row-wide walk takes list states (not in tile mode)
  __shared__ uint32_t h0_sh;
  __shared__ uint8_t loop0[256];  // T[0][c] == 0: byte c keeps set 0 (row-wide walk)
  // first pass of the row-wide walk: pass index i -> walk position
  __shared__ int32_t grp_pre[258];    // runs: exclusive prefix of the live runs' lengths, then the total
  __shared__ int32_t grp_start[257];  // runs: first walk position of each live run
  __shared__ int pass_mode, pass_list, pass_total, pass_base, run_n, run_top;
  // the first round's idle waves prepare the first pass of a row in a frame
  // list (pre_round: this is that round; pre_pass: they did, pre_s0/pre_s1
  // the list's seed bounds they read)
  __shared__ int pre_round, pre_pass, pre_s0, pre_s1;
  __shared__ uint32_t warm_sink;
  uint8_t* T = reinterpret_cast<uint8_t*>(T32);

  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t row = a.slots ? a.slots[b] : b;
  int32_t* pool = ws.pool + b * kMemoSets * kConfigWords;
  int32_t* cand = ws.cand + b * kMemoReq * kConfigWords;
  // the pack key of the records in the workspace (stamped only by the launch
  // after a mask, so no block of this launch sees another's stamp)
  const uint32_t hdr_key0 = ws.header[2], hdr_key1 = ws.header[3];
  // the finish count when this launch began (copied by the launch after the
  // last mask; a workspace of unknown content only loses the deferral)
  const uint32_t finish_base = ws.header[kFinishWord + 1];

  // the prologue's global reads (the row's set, the frame lists' slot
  // table, the first slice of the grammar tables) are issued first and
  // stored after the LDS fills below, which run while they are in flight
  static_assert(kConfigWords <= kMemoThreads && BPD_PDA_FRAME_SLOTS % kMemoThreads == 0, "prologue slices");
  const int32_t cfg_w = tid < kConfigWords ? a.configs[row * kConfigWords + tid] : 0;
  uint32_t fsv[BPD_PDA_FRAME_SLOTS / kMemoThreads];
#pragma unroll
  for (int q = 0; q < BPD_PDA_FRAME_SLOTS / kMemoThreads; ++q)
    fsv[q] = a.frames.num_lists > 0 ? a.frames.slots[q * kMemoThreads + tid] : BPD_PDA_FRAME_EMPTY;
  const TableSlice tsl = InLds ? table_slice(a.g, tid) : TableSlice{0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = tid; i < kMemoSets * 256 / 4; i += kMemoThreads) T32[i] = 0xFEFEFEFEu;
  const int32_t vwords = (a.vocab + 31) / 32;
  for (int i = tid; i < vwords; i += kMemoThreads) vbits[i] = 0u;
  for (int i = tid; i < kMemoSets * 8; i += kMemoThreads) {
    req[i] = 0;
    texact[i] = 0;
  }
  for (int i = tid; i < kLT; i += kMemoThreads) {
    lt_key[i] = kLTEmpty;
    lt_res[i] = kTUnknown;
    if (i < kLT / 32) {
      lt_req[i] = 0u;
      lt_exact[i] = 0u;
    }
  }
  for (int i = tid; i < kLC; i += kMemoThreads) lcache[i] = 0xFFFFFFFFu;
  if (tid < kConfigWords) row_cfg[tid] = cfg_w;
#pragma unroll
  for (int q = 0; q < BPD_PDA_FRAME_SLOTS / kMemoThreads; ++q) fslots[q * kMemoThreads + tid] = fsv[q];
  const PdaTableView g = InLds ? stage_tables(a.g, tab, tsl, tid, kMemoThreads) : a.g;
  if (tid == 0) {
    pre_round = 0;
    pre_pass = 0;
    pool_count = 1;
    overflowed = 0;
    walk_lists = row_mode != 0 ? 1 : 0;
    lt_used = 0;
    nreq = 0;
  }
  __syncthreads();
  if (tid >= kWave && tid < 2 * kWave) {
    // wave 1: the row's frame list and the entries of T row 0 it fills (the
    // dead entries it writes are ones wave 0 writes too: a byte no top's
    // edge contains empties the list)
    const int lane = tid - kWave;
    const bool dead = (a.broken != nullptr && a.broken[row] != 0) || !config_ok(row_cfg, a.g.num_states, lane);
    int base0 = 0;
    int32_t codes[4] = {-2, -2, -2, -2};
    const int l0 = dead ? -1 : frame_list_of(row_cfg, a.frames, fslots, lane, &base0, codes);
    if (lane == 0) {
      row_list = l0;
      const int sl0 = l0 >= 0 ? (l0 | (row_cfg[1] != 0 ? BPD_PDA_FRAME_SAT : 0) | (base0 << kListBase)) : -1;
      set_list[0] = sl0;
      set_ls[0] = sl0 >= 0 ? list_state(0, sl0) : -1;
    }
    if (l0 >= 0) {
      // T row 0 from the list's codes (read beside its key), which also
      // fill the list's entries of the byte-table cache
      wave_sync();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = q * kWave + lane;
        frame_fill_entry(codes[q], l0, row_cfg[1] != 0, 0, T, c);
        lcache[lc_slot(l0, c)] = lc_entry(l0, c, codes[q]);
      }
    }
  }
  if (tid < kWave) {
    bool dead = a.broken != nullptr && a.broken[row] != 0;
    if (!config_ok(row_cfg, a.g.num_states, tid)) {
      if (tid == 0 && a.err) atomicOr(a.err, BPD_FLAG_STATE_RANGE);
      dead = true;
    }
    const uint32_t h0 = dead ? 0u : coop_hash(row_cfg, tid);
    if (tid == 0) {
      const ConstFlatView C{row_cfg};
      row_flags = dead ? 1 : ((is_complete(a.g, C) ? 2 : 0) | (C.n() > 0 ? 4 : 0));
      pool_hash[0] = h0;
      h0_sh = h0;
    }
    if (tid < kMaxConfigs) {
      const int n = dead ? 0 : row_cfg[0];
      const int d = tid < n ? row_cfg[2 + tid] : 0;
      set_tops[0][tid] = d > 0 ? row_cfg[kF + tid * kMaxDepth + d - 1] : -1;
      if (tid == 0) set_n[0] = n;
    }
    wave_sync();
    coop_set_intervals(g, set_tops[0], set_n[0], set_bnd[0], set_hit[0], T, tid);
  }
  for (int k = tid; k < kConfigWords; k += kMemoThreads) pool[k] = row_cfg[k];
  __syncthreads();
  const int flags = row_flags;
  const bool dead_row = (flags & 1) != 0;

  const int64_t V = a.vocab;

  // Resolve the requested transitions: compact the request bits (T entries,
  // then boundary entries), claim one request per elementary interval,
  // compute each claimed transition (one wave each), intern the new sets and
  // fill T and LT; sets `overflowed` when the pool is full.  A request beyond
  // the first kMemoReq stays unresolved and its token asks again after the
  // next walk.  Called by every thread, between barriers.
  // (nreq is 0 on entry: set so in the prologue and at the end of each call)
  auto resolve = [&]() {
    for (int w = tid; w < kMemoSets * 8 + kLT / 32; w += kMemoThreads) {
      const bool lt = w >= kMemoSets * 8;
      uint32_t* word = lt ? &lt_req[w - kMemoSets * 8] : &req[w];
      uint32_t bits = *word;
      if (bits) {
        *word = 0;
        int at = atomicAdd(&nreq, __popc(bits));
        while (bits) {
          const int bit = __ffs(bits) - 1;
          bits &= bits - 1;
          if (at < kMemoReq)
            req_list[at] = lt ? (kReqLT | ((w - kMemoSets * 8) * 32 + bit)) : (((w >> 3) << 8) | ((w & 7) * 32 + bit));
          ++at;
        }
      }
    }
    __syncthreads();
    const int n = nreq < kMemoReq ? nreq : kMemoReq;
    // with at most one request per wave, request r is computed by wave r and
    // its result stays in that wave's LDS buffer until the round ends (no
    // copy to the workspace's candidate slots)
    const bool in_work = n <= kMemoThreads / kWave;
    auto cand_words = [&](int r) -> const int32_t* { return in_work ? work[r][1] : cand + r * kConfigWords; };
    if (n > kMemoThreads / kWave) {
      // the requests a wave steps (no frame-list composition) first: waves
      // take requests r = wave, wave + 16, ..., so each wave gets at most
      // one more of them than another (with one request per wave at most
      // there is nothing to order)
      uint32_t entry = 0u;
      bool cheap = true;
      if (tid < n) {
        entry = uint32_t(req_list[tid]);
        if (entry >= uint32_t(kReqLT)) {
          cheap = false;  // a boundary entry: always stepped
        } else {
          const int sl = set_list[entry >> 8];
          cheap = sl >= 0 && a.frames.trans[(sl & (BPD_PDA_FRAME_SAT - 1)) * 256 + int(entry & 255u)] != -2;
        }
      }
      if (tid == 0) {
        n_stepped = 0;
        n_cheap = 0;
      }
      __syncthreads();
      int slot = 0;
      if (tid < n && !cheap) slot = atomicAdd(&n_stepped, 1);
      __syncthreads();
      if (tid < n && cheap) slot = n_stepped + atomicAdd(&n_cheap, 1);
      if (tid < n) req_list[slot] = int32_t(entry);
      __syncthreads();
    }
    if (tid < n && req_list[tid] >= kReqLT) {
      cand_lo[tid] = 0;
      cand_hi[tid] = 0;
      cand_res[tid] = 0;  // a boundary entry has its own slot: always computed
    } else if (tid < n) {
      // every byte of the request's elementary interval [lo, hi] shares
      // its result: the first request of an interval computes it and
      // fills the whole interval
      const int set = req_list[tid] >> 8, byte = req_list[tid] & 255;
      int lo, hi;
      const bool hit = set_interval(set_bnd[set], set_hit[set], byte, lo, hi);
      cand_lo[tid] = int16_t(lo);
      cand_hi[tid] = int16_t(hi);
      if (!hit) {
        cand_res[tid] = -5;  // rejected on the whole interval, nothing to compute
      } else {
        const uint32_t bit = 1u << (lo & 31);
        const bool first = (atomicOr(&req[set * 8 + (lo >> 5)], bit) & bit) == 0;
        cand_res[tid] = first ? 0 : -4;
      }
    }
    __syncthreads();
    {
      // one wave per claimed transition, working sets in LDS
      const int lane = tid & (kWave - 1), wave = tid / kWave;
      int32_t* wsrc = work[wave][0];
      int32_t* wdst = work[wave][1];
      // the wave's requests r = wave, wave + 16, ... that compute; the
      // source set of the next one is loaded into registers while the
      // current one is computed (set 0, the row's own set, is in LDS)
      auto next_req = [&](int r) {
        while (r < n && cand_res[r] < -3) r += kMemoThreads / kWave;
        return r;
      };
      // the pool set a request starts from (a boundary entry: its anchor)
      auto req_set = [&](int r) -> int {
        const int e = req_list[r];
        return e >= kReqLT ? int(lt_key[e & (kLT - 1)] >> 21) : e >> 8;
      };
      int32_t words[kSetLoads];
      auto load_src = [&](int r) {
        const int set = r < n ? req_set(r) : 0;
        const int32_t* ps = pool + set * kConfigWords;
#pragma unroll
        for (int q = 0; q < kSetLoads; ++q) {
          const int k = lane + q * kWave;
          words[q] = set != 0 && k < kConfigWords ? ps[k] : 0;
        }
      };
      int r = next_req(wave);
      load_src(r);
      while (r < n) {
        const int e = req_list[r];
        const bool lt = e >= kReqLT;
        const uint32_t lk = lt ? lt_key[e & (kLT - 1)] : 0u;
        const int set = lt ? int(lk >> 21) : e >> 8, byte = lt ? int(lk & 255u) : e & 255;
        if (set != 0) {
#pragma unroll
          for (int q = 0; q < kSetLoads; ++q) {
            const int k = lane + q * kWave;
            if (k < kConfigWords) wsrc[k] = words[q];
          }
          wave_sync();
        }
        const int r_next = next_req(r + kMemoThreads / kWave);
        load_src(r_next);
        // a set in a frame list whose list leads by this byte to a list
        // (over the same common stack): the result is composed from the
        // key instead of stepped
        const int32_t* src = set != 0 ? wsrc : row_cfg;
        const int sl = set_list[set];
        int code = -3;
        if (lt) {
          // a boundary entry steps the list state's set: the anchor's
          // common stack under the list's key
          compose_list_set(src, wsrc, a.frames.keys + int64_t((lk >> 8) & 0xFFFu) * BPD_PDA_FRAME_KEY_WORDS,
                           sl >> kListBase, int((lk >> 20) & 1u), lane);
          src = wsrc;
        } else if (sl >= 0) {
          code = a.frames.trans[(sl & (BPD_PDA_FRAME_SAT - 1)) * 256 + byte];
        }
        bool ok;
        if (code >= 0) {
          const int sat = src[1] != 0 || (code & BPD_PDA_FRAME_SAT) != 0 ? 1 : 0;
          compose_list_set(src, wdst,
                           a.frames.keys + int64_t(code & (BPD_PDA_FRAME_SAT - 1)) * BPD_PDA_FRAME_KEY_WORDS,
                           sl >> kListBase, sat, lane);
          ok = true;
        } else if (code == -1) {
          ok = false;
        } else {
          ok = coop_advance_byte(g, src, wdst, byte, lane);
        }
        if (!ok) {
          if (lane == 0) cand_res[r] = -1;
        } else {
          const uint32_t h = coop_hash(wdst, lane);
          // the first pool set with this hash and these meaningful words;
          // hashes compared 64 at a time
          int found = -2;
          bool raw = false;
          const int pc = pool_count < max_sets ? pool_count : max_sets;
          for (int k0 = 0; k0 < pc && found < 0; k0 += kWave) {
            uint64_t m = __ballot(k0 + lane < pc && pool_hash[k0 + lane] == h);
            while (m != 0u && found < 0) {
              const int k = k0 + __ffsll(static_cast<unsigned long long>(m)) - 1;
              m &= m - 1;
              if (coop_same_raw(wdst, pool + k * kConfigWords, lane, raw)) found = k;
            }
          }
          if (lane < kMaxConfigs) {
            const int nn = wdst[0];
            const int d = lane < nn ? wdst[2 + lane] : 0;
            cand_tops[r][lane] = d > 0 ? wdst[kF + lane * kMaxDepth + d - 1] : -1;
            if (lane == 0) cand_n[r] = nn;
          }
          // a new set is kept in the candidate buffer (its words are needed
          // after this wave's buffer is reused); stored after the pool
          // lookup's loads, which would otherwise wait for these stores
          int lbase = code >= 0 ? (sl >> kListBase) : 0;
          const int lst = found != -2 ? -1
                          : code >= 0 ? (code & (BPD_PDA_FRAME_SAT - 1))
                                      : frame_list_of(wdst, a.frames, fslots, lane, &lbase);
          if (lane == 0) {
            cand_list[r] = lst >= 0 ? (lst | (wdst[1] != 0 ? BPD_PDA_FRAME_SAT : 0) | (lbase << kListBase)) : -1;
            cand_comp[r] = code >= 0 && (code & BPD_PDA_FRAME_RAW) == 0 ? 1 : 0;
          }
          if (found == -2 && !in_work) {
            int32_t* out = cand + r * kConfigWords;
            for (int k = lane; k < kConfigWords; k += kWave) out[k] = wdst[k];
          }
          if (lane == 0) {
            cand_hash[r] = h;
            cand_res[r] = found;
            cand_exact[r] = found >= 0 && raw && (code < 0 || (code & BPD_PDA_FRAME_RAW) != 0) ? 1 : 0;
          }
        }
        wave_sync();
        r = r_next;
      }
      // in the first round of a row in a frame list the waves without a
      // request read the list's verdict bitmap into vbits and its seed
      // bounds, and read the first tile's seed entries and their records
      // once, so that the first pass finds them in L2
      if (pre_round && n < kMemoThreads / kWave && wave >= n) {
        const int idle = kMemoThreads / kWave - n, w = wave - n;
        const int l = row_list;
        const uint32_t* al = a.frames.allowed + int64_t(l) * a.frames.words;
        for (int i = w * kWave + lane; i < vwords; i += idle * kWave) vbits[i] = al[i];
        const int32_t s0 = a.frames.seed_off[l], s1 = a.frames.seed_off[l + 1];
        if (w == 0 && lane == 0) {
          pre_s0 = s0;
          pre_s1 = s1;
          pre_pass = 1;
        }
        uint32_t acc = 0u;
        for (int i = w * kWave + lane; i < kMemoThreads && s0 + i < s1; i += idle * kWave) {
          const int32_t k = a.frames.seeds[s0 + i];
          if (k >= 0 && k < V) acc ^= ws.recs[k].x ^ uint32_t(ws.tmeta[k].x);
        }
        if (acc == 0x9E3779B9u) atomicOr(&warm_sink, 1u);  // (keeps the reads)
      }
    }
    __syncthreads();
    {
      // new sets equal to an earlier candidate of the round: a wave per
      // candidate matches the earlier hashes 64 at a time by ballot and
      // compares meaningful words lane-parallel; the first equal one leads
      const int lane = tid & (kWave - 1), wave = tid / kWave;
      for (int r = wave; r < n; r += kMemoThreads / kWave) {
        if (cand_res[r] != -2) continue;
        const uint32_t h = cand_hash[r];
        const int32_t* mine = cand_words(r);
        int lead = r;
        for (int j0 = 0; j0 < r && lead == r; j0 += kWave) {
          const int j = j0 + lane;
          uint64_t m = __ballot(j < r && cand_res[j] == -2 && cand_hash[j] == h);
          while (m != 0u && lead == r) {
            const int k = j0 + __ffsll(static_cast<unsigned long long>(m)) - 1;
            m &= m - 1;
            if (coop_same(mine, cand_words(k), lane)) lead = k;
          }
        }
        if (lane == 0) cand_lead[r] = lead;
      }
    }
    __syncthreads();
    if (tid < n && cand_res[tid] == -2 && cand_lead[tid] == tid) {
      const int id = atomicAdd(&pool_count, 1);
      if (id < max_sets) {
        pool_hash[id] = cand_hash[tid];
        set_n[id] = cand_n[tid];
        const int cl = cand_list[tid];
        set_list[id] = cl;
        set_ls[id] = cl >= 0 ? list_state(id, cl) : -1;
        for (int i = 0; i < kMaxConfigs; ++i) set_tops[id][i] = cand_tops[tid][i];
        cand_id[tid] = id;
      } else {
        cand_id[tid] = -3;
      }
    }
    __syncthreads();
    {
      // transitions into T, one wave per request with the lanes over the
      // interval's bytes; then new sets into the pool, one wave per set
      const int lane = tid & (kWave - 1), wave = tid / kWave;
      for (int r = wave; r < n; r += kMemoThreads / kWave) {
        const int res = cand_res[r];
        if (res == -4) continue;  // a duplicate of another request's interval
        const int rq = req_list[r];
        const int id = res == -2 ? cand_id[cand_lead[r]] : res;
        uint8_t e;
        if (id == -1 || id == -5) {
          e = kTDead;
        } else if (id == -3) {
          e = kTOverflow;
          if (lane == 0) overflowed = 1;
        } else {
          e = uint8_t(id);
        }
        if (rq >= kReqLT) {
          // a boundary entry: its slot of LT (exact as below; never composed)
          if (lane == 0) {
            const int slot = rq & (kLT - 1);
            lt_res[slot] = e;
            if ((res >= 0 && cand_exact[r]) || (res == -2 && cand_lead[r] == r && id >= 0))
              atomicOr(&lt_exact[slot >> 5], 1u << (slot & 31));
          }
          continue;
        }
        const int set = rq >> 8;
        const int lo = cand_lo[r], hi = cand_hi[r];
        for (int c = lo + lane; c <= hi; c += kWave) T[set * 256 + c] = e;
        // the interval's step gives the set's raw words: a new set (its
        // first computation) or an existing one equal in every word
        const bool exact = (res >= 0 && cand_exact[r]) || (res == -2 && cand_lead[r] == r && id >= 0 && !cand_comp[r]);
        if (exact && lane >= (lo >> 5) && lane <= (hi >> 5)) {
          const int b0 = (lo > lane * 32 ? lo : lane * 32) - lane * 32;
          const int b1 = (hi < lane * 32 + 31 ? hi : lane * 32 + 31) - lane * 32;
          const uint32_t upto = b1 == 31 ? 0xFFFFFFFFu : ((1u << (b1 + 1)) - 1u);
          atomicOr(&texact[set * 8 + lane], upto & ~((1u << b0) - 1u));
        }
        if (lane == 0 && res != -5) atomicAnd(&req[set * 8 + (lo >> 5)], ~(1u << (lo & 31)));
      }
      for (int r = wave; r < n; r += kMemoThreads / kWave) {
        if (cand_res[r] != -2 || cand_lead[r] != r || cand_id[r] < 0) continue;
        // the set's words are loaded first and stored last, so the load
        // waits behind the interval and frame-list work
        const int32_t* src = cand_words(r);
        int32_t* dst = pool + cand_id[r] * kConfigWords;
        int32_t words[kSetLoads];
#pragma unroll
        for (int q = 0; q < kSetLoads; ++q) {
          const int k = lane + q * kWave;
          words[q] = k < kConfigWords ? src[k] : 0;
        }
        // a set in a frame list needs no intervals while lists are walked
        // (its missing entries turn the walk into its list state)
        const int cl = cand_list[r];
        if (cl < 0 || !walk_lists)
          coop_set_intervals(g, cand_tops[r], cand_n[r], set_bnd[cand_id[r]], set_hit[cand_id[r]],
                             T + cand_id[r] * 256, lane);
        if (cl >= 0) {
          wave_sync();
          frame_fill_row(a.frames, cl & (BPD_PDA_FRAME_SAT - 1), (cl & BPD_PDA_FRAME_SAT) != 0, cand_id[r],
                         T + cand_id[r] * 256, lane);
        }
#pragma unroll
        for (int q = 0; q < kSetLoads; ++q) {
          const int k = lane + q * kWave;
          if (k < kConfigWords) dst[k] = words[q];
        }
      }
    }
    if (tid == 0) nreq = 0;  // every thread read it before the claim's barrier
    __syncthreads();
  };

  // Empty the pool back to the row's own set (set 0), T to "unknown" and LT.
  auto reset_pool = [&]() {
    for (int i = tid; i < kMemoSets * 64; i += kMemoThreads) T32[i] = 0xFEFEFEFEu;
    for (int i = tid; i < kMemoSets * 8; i += kMemoThreads) texact[i] = 0u;
    for (int i = tid; i < kLT; i += kMemoThreads) {
      lt_key[i] = kLTEmpty;
      lt_res[i] = kTUnknown;
      if (i < kLT / 32) {
        lt_req[i] = 0u;
        lt_exact[i] = 0u;
      }
    }
    for (int k = tid; k < kConfigWords; k += kMemoThreads) pool[k] = row_cfg[k];
    if (tid < kMaxConfigs) {
      const int n0 = row_cfg[0];
      const int d = tid < n0 ? row_cfg[2 + tid] : 0;
      set_tops[0][tid] = d > 0 ? row_cfg[kF + tid * kMaxDepth + d - 1] : -1;
      if (tid == 0) set_n[0] = n0;
    }
    __syncthreads();
    if (tid < kWave) {
      coop_set_intervals(g, set_tops[0], set_n[0], set_bnd[0], set_hit[0], T, tid);
      if (row_list >= 0) {
        wave_sync();
        frame_fill_row(a.frames, row_list, row_cfg[1] != 0, 0, T, tid);
      }
    }
    if (tid == 0) {
      pool_count = 1;
      pool_hash[0] = h0_sh;
      overflowed = 0;
      lt_used = 0;
    }
    __syncthreads();
  };

  // Row-wide walk.  A first pass walks every token as far as T allows and
  // queues the paused ones (token, set, position, length) in the workspace;
  // each round then resolves all of the row's requests at once and walks the
  // queue again into the other buffer.  A row needs as many rounds as its
  // longest chain of new sets (7 on recursive JSON) rather than that many per
  // tile.  A row whose sets overflow the pool, that pauses a token of 65536
  // bytes or more, or that pauses more tokens in one pass than a queue
  // buffer holds, starts again in tile mode.
  // with no pack launched before this one and records of other tables (or
  // none) in the workspace, every block packs all of them itself before it
  // walks any: blocks write identical values, so a block reads its own
  // writes or equal ones
  if (pack_here && (hdr_key0 != uint32_t(pkey) || hdr_key1 != uint32_t(pkey >> 32))) {
    for (int32_t k = tid; k < a.vocab; k += kMemoThreads) pack_record(a.tok_off, a.tok_bytes, a.order, k, ws.recs, ws.tmeta, ws.trecs);
    __syncthreads();
  }
  bool tiles = row_mode == 0;
  if (!tiles) {
    const int64_t Q = ws.qcap;
    uint2* qin = ws.queue + b * 2 * Q;
    uint2* qout = qin + Q;
    const int lane = tid & (kWave - 1);
    // queue entry e for the lanes with p set (every lane of the wave calls it)
    auto enqueue = [&](bool p, uint2 e, uint2* q) {
      const uint64_t m = __ballot(p);
      if (m == 0u) return;
      const int leader = __ffsll(static_cast<unsigned long long>(m)) - 1;
      int base = 0;
      if (lane == leader) base = atomicAdd(&qcount, __popcll(m));
      base = lane_value(base, leader);
      if (p) {
        const int idx = base + __popcll(m & ((uint64_t(1) << lane) - 1u));
        if (idx < Q)
          q[idx] = e;
        else
          row_fail = 1;  // the buffer is full: the row starts again in tile mode
      }
    };
    // one step of a token by `byte` from its state after the T loop stopped:
    // a pool set's special entry (a missing entry of a set in a frame list
    // turns the state into the set's list state without taking the byte), or
    // a list state (the lists' byte table; a boundary byte takes the entry of
    // LT, inserted when missing).  False when the entry is missing (its
    // interval or LT entry requested, the state unchanged).
    auto step = [&](int& cur, int& pos, int byte) -> bool {
      if (cur < kWalkEnd) {
        const uint8_t nx = T[cur * 256 + byte];
        if (nx == kTUnknown) {
          const int ls = set_ls[cur];
          if (ls >= 0) {
            cur = ls;
            return true;
          }
          if (((set_hit[cur][byte >> 5] >> (byte & 31)) & 1u) == 0u) {
            cur = kRejected;  // no byte edge contains it: the step empties the set
            return true;
          }
          const int lo = interval_start(set_bnd[cur], byte);
          const int w = cur * 8 + (lo >> 5);
          const uint32_t bit = 1u << (lo & 31);
          if ((req[w] & bit) == 0u) atomicOr(&req[w], bit);
          return false;
        }
        if (nx == kTDead || nx == kTOverflow) {
          cur = kRejected;
        } else {
          cur = nx;
          ++pos;
        }
        return true;
      }
      const int code = list_code(a.frames, lcache, cur & 0xFFF, byte);
      if (code >= 0) {
        const int sat = (cur & (1 << 12)) | ((code & BPD_PDA_FRAME_SAT) != 0 ? 1 << 12 : 0);
        cur = (cur & ~0x1FFF) | sat | (code & 0xFFF);
        ++pos;
        return true;
      }
      if (code == -1) {
        cur = kRejected;  // the list (and so the set) empties
        return true;
      }
      const uint32_t key = lt_key_of(cur, byte);
      const uint32_t h = lt_hash(key);
      int slot = -1;
      for (int p = 0; p < kLT && slot < 0; ++p) {
        const int s = int((h + uint32_t(p)) & uint32_t(kLT - 1));
        uint32_t k = lt_key[s];
        if (k == kLTEmpty) {
          k = atomicCAS(&lt_key[s], kLTEmpty, key);
          if (k == kLTEmpty) {
            k = key;
            if (atomicAdd(&lt_used, 1) >= lt_cap) row_fail = 1;  // beyond the cap (tests)
          }
        }
        if (k == key) slot = s;
      }
      if (slot < 0) {
        row_fail = 1;  // LT is full: the row starts again in tile mode
        return false;
      }
      const uint8_t r = lt_res[slot];
      if (r == kTUnknown) {
        const uint32_t bit = 1u << (slot & 31);
        if ((lt_req[slot >> 5] & bit) == 0u) atomicOr(&lt_req[slot >> 5], bit);
        return false;
      }
      if (r == kTDead || r == kTOverflow) {
        cur = kRejected;
      } else {
        cur = r;
        ++pos;
      }
      return true;
    };
    // token t from (cur, pos) until it ends, is rejected or meets a missing
    // entry (requested; returns true).  Its first 16 bytes come from the
    // record in registers: that loop has no memory wait other than the table
    // read, so queue stores still in flight do not stall it; the bytes after
    // them are read from tok_bytes in a second loop.
    // Each T loop takes only entries that are interned sets and stops at the
    // first other one (missing, dead or overflow: entries >= kTOverflow) or
    // at a list state; step() then settles that entry or takes the list
    // state's byte, outside the loop, so the loop body has no branch besides
    // its exit.  Every step() either ends the walk, takes a byte or (turning
    // a pool set into its list state) is followed by one that does.
    auto walk = [&](int& cur, int& pos, int len, uint4 pk, int32_t t) -> bool {
      const int n16 = len < 16 ? len : 16;
      while (pos < n16 && walking(cur)) {
        while (cur < kWalkEnd && pos < n16) {
          const uint8_t nx = T[cur * 256 + packed_byte(pk, pos)];
          if (nx >= kTOverflow) break;
          cur = nx;
          ++pos;
        }
        if (pos < n16 && walking(cur) && !step(cur, pos, packed_byte(pk, pos))) return true;
      }
      if (pos < len && walking(cur)) {
        // the bytes past the record, 16 at a time, each group read with
        // independent loads and packed like a record
        const uint8_t* tb = a.tok_bytes + a.tok_off[t];
        while (pos < len && walking(cur)) {
          uint32_t w4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
          for (int i = 0; i < 16; ++i) w4[i >> 2] |= (pos + i < len ? uint32_t(tb[pos + i]) : 0u) << (8 * (i & 3));
          const uint4 ck = make_uint4(w4[0], w4[1], w4[2], w4[3]);
          const int p0 = pos, pe = len < pos + 16 ? len : pos + 16;
          while (pos < pe && walking(cur)) {
            while (cur < kWalkEnd && pos < pe) {
              const uint8_t nx = T[cur * 256 + packed_byte(ck, pos - p0)];
              if (nx >= kTOverflow) break;
              cur = nx;
              ++pos;
            }
            if (pos < pe && walking(cur) && !step(cur, pos, packed_byte(ck, pos - p0))) return true;
          }
        }
      }
      if (walking(cur)) cur = kAllowed;
      return false;
    };
    // the tail of a token's walk: queue it if paused, else record an accept.
    // A queue entry holds the walk position k (< 2^18) and 14 bits of the
    // state in x, the byte position and the state's other bits in y.
    auto settle = [&](bool paused, int cur, int pos, int len, int32_t k, int32_t t, uint2* q) {
      if (paused && len > 0xFFFF) {
        row_fail = 1;
        paused = false;
      }
      enqueue(paused,
              make_uint2(uint32_t(k) | (uint32_t(cur & 0x3FFF) << 18), uint32_t(pos) | (uint32_t(cur >> 14) << 16)),
              q);
      if (cur == kAllowed) atomicOr(&vbits[t >> 5], 1u << (t & 31));
    };

    if (!dead_row) {
      // every interval of set 0 first, so the first pass already steps past
      // byte 0; of a set in a frame list only the boundary intervals (the
      // others are walked as its list state or were filled from the list)
      // (wave 0: lane l takes bytes l, 64 + l, 128 + l, 192 + l, the list's
      // codes for them from the byte-table cache, which the prologue filled;
      // four ballots are the eight request words, each stored by the thread
      // that collects it)
      if (tid < kWave) {
        int code[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          code[q] = row_list >= 0 ? list_code(a.frames, lcache, row_list, q * kWave + tid) : -2;
        uint64_t m[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = q * kWave + tid;
          const bool start = c == 0 || ((set_bnd[0][c >> 5] >> (c & 31)) & 1u) != 0u;
          bool want = start && ((set_hit[0][c >> 5] >> (c & 31)) & 1u) != 0u;
          if (row_list >= 0) want = want && T[c] == kTUnknown && code[q] == -2;
          m[q] = __ballot(want);
        }
        if (tid < 8) {
          const uint64_t mq = tid < 2 ? m[0] : (tid < 4 ? m[1] : (tid < 6 ? m[2] : m[3]));
          req[tid] = uint32_t(mq >> (32 * (tid & 1)));
        }
        if (tid == 0) pre_round = row_list >= 0 ? 1 : 0;
      }
      resolve();
      if (tid == 0) pre_round = 0;
    }
    if (tid == 0) {
      qcount = 0;
      row_fail = 0;
      loop_n = 0;
      pass_mode = 0;
      pass_list = -1;
      pass_total = dead_row ? 0 : int(V);  // a dead row rejects every token: nothing to walk
      pass_base = 0;
      // Frame lists: a row whose configs share one stack below their tops
      // (depth >= 2) and whose ordered tops are a list's key takes the
      // tokens that stay inside the tops' call-free rule from the list's
      // bitmap and walks only the list's seeds (the tokens that reach the
      // rule's accept state, EOS and the empty tokens).
      if (!dead_row && !overflowed && row_list >= 0) {
        const int l = row_list;
        const int32_t s0 = pre_pass ? pre_s0 : a.frames.seed_off[l], s1 = pre_pass ? pre_s1 : a.frames.seed_off[l + 1];
        pass_list = l;
        pass_mode = 2;
        pass_base = s0;
        pass_total = s1 > s0 ? s1 - s0 : 0;
      }
    }
    __syncthreads();
    if (tid < 256) {
      loop0[tid] = T[tid] == 0 ? 1 : 0;
      if (T[tid] == 0) atomicAdd(&loop_n, 1);
    }
    if (pass_list >= 0) {  // (pass_mode is written below; pass_list is not)
      if (!pre_pass) {
        const uint32_t* al = a.frames.allowed + int64_t(pass_list) * a.frames.words;
        for (int i = tid; i < vwords; i += kMemoThreads) vbits[i] = al[i];
      }
    } else if (a.runs && !dead_row && !overflowed && tid < kWave) {
      // first-byte runs: the run of byte c is walked unless the byte
      // empties set 0 (T[0][c] dead); lane l owns runs 4l..4l+3, lane 63
      // also the run of EOS and the empty tokens.  Only the live runs are
      // listed (the pass searches them), in byte order, then the total.
      int cnt[5], st[5], sum = 0, live = 0;
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        const int c = q < 4 ? 4 * tid + q : 256;
        const int64_t b0 = a.runs[c], b1 = c < 255 ? a.runs[c + 1] : (c == 255 ? a.runs[256] : V);
        const int64_t lo = b0 < 0 ? 0 : (b0 > V ? V : b0);
        const int64_t hi = b1 < lo ? lo : (b1 > V ? V : b1);
        st[q] = int(lo);
        cnt[q] = (q == 4 && tid != kWave - 1) || (c < 256 && T[c] == kTDead) ? 0 : int(hi - lo);
        sum += cnt[q];
        live += cnt[q] > 0 ? 1 : 0;
      }
      int incl = sum, incl_live = live;
      for (int o = 1; o < kWave; o <<= 1) {
        const int y = __shfl_up(incl, o), z = __shfl_up(incl_live, o);
        if (tid >= o) {
          incl += y;
          incl_live += z;
        }
      }
      int ex = incl - sum, li = incl_live - live;
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        if (cnt[q] > 0) {
          grp_pre[li] = ex;
          grp_start[li] = st[q];
          ++li;
          ex += cnt[q];
        }
      }
      if (tid == kWave - 1) {
        grp_pre[li] = ex;
        run_n = li;
        run_top = li > 1 ? 1 << (31 - __clz(li - 1)) : 0;
        pass_total = ex;
        pass_mode = 1;
      }
    }
    __syncthreads();
    // only a set that keeps itself on many bytes (a string or comment loop)
    // is worth the prefix check below
    const bool scan = loop_n >= 32;
    const int mode = pass_mode;
    const int64_t P = pass_total;
    const int rn = run_n, rtop = run_top;
    if (!overflowed) {
      // the records of the next tile are loaded while this one is walked;
      // queue entries are stored after all kMemoTok walks of a tile
      constexpr int64_t kTile = int64_t(kMemoThreads) * kMemoTok;
      int2 nm[kMemoTok];
      uint4 npk[kMemoTok];
      int32_t nk[kMemoTok];
      // walk positions of pass indices base + j * kMemoThreads + tid (-1
      // past the pass or for a seed out of range) and their records.  Over
      // the live runs, the last run whose prefix is <= i is found by binary
      // lifting, the four searches of a thread interleaved (one LDS wait per
      // step); the total after the last run stops every step at it.
      // mode 2: the seed entries (walk positions) are read a tile ahead of
      // the records they index, so a tile's record loads never wait for its
      // seed loads
      int32_t seed_next[kMemoTok];
      auto load_seeds = [&](int64_t base) {
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          const int64_t i = base + int64_t(j) * kMemoThreads + tid;
          seed_next[j] = mode == 2 && i < P ? a.frames.seeds[pass_base + i] : -1;
        }
      };
      auto prefetch = [&](int64_t base) {
        int32_t ii[kMemoTok], lo[kMemoTok];
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          const int64_t i = base + int64_t(j) * kMemoThreads + tid;
          ii[j] = i < P ? int32_t(i) : -1;
          lo[j] = 0;
        }
        if (mode == 1) {
          for (int stp = rtop; stp > 0; stp >>= 1) {
#pragma unroll
            for (int j = 0; j < kMemoTok; ++j) {
              const int m = lo[j] + stp < rn ? lo[j] + stp : rn;
              if (grp_pre[m] <= ii[j]) lo[j] = m;
            }
          }
        }
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          int32_t k = ii[j];
          if (k >= 0 && mode == 1) {
            k = grp_start[lo[j]] + (k - grp_pre[lo[j]]);
          } else if (k >= 0 && mode == 2) {
            k = seed_next[j];
            k = k >= 0 && k < V ? k : -1;
          }
          nk[j] = k;
          nm[j] = k >= 0 ? ws.tmeta[k] : make_int2(-1, 0);
          npk[j] = k >= 0 ? ws.recs[k] : make_uint4(0u, 0u, 0u, 0u);
        }
      };
      load_seeds(0);
      prefetch(0);
      load_seeds(kTile);
      for (int64_t tile = 0; tile < P; tile += kTile) {
        int32_t tt[kMemoTok], pos[kMemoTok], len[kMemoTok], kk[kMemoTok];
        int cur[kMemoTok];
        uint4 pk[kMemoTok];
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          const int2 m = nm[j];
          pk[j] = npk[j];
          kk[j] = nk[j];
          const int32_t t = m.x;
          tt[j] = t;
          pos[j] = len[j] = 0;
          if (t < 0) {
            cur[j] = kNone;
          } else if (dead_row) {
            cur[j] = kRejected;
          } else if (t == a.eos) {
            cur[j] = (flags & 2) ? kAllowed : kRejected;
          } else {
            len[j] = m.y;
            cur[j] = len[j] == 0 ? ((flags & 4) ? kAllowed : kRejected) : 0;
          }
        }
        prefetch(tile + kTile);
        load_seeds(tile + 2 * kTile);
        // the leading bytes that keep set 0 (a string loop's body) are
        // checked together, with independent table reads, and the walk
        // starts at the first other byte
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          if (!scan || cur[j] != 0) continue;
          const int n = len[j] < 16 ? len[j] : 16;
          uint32_t keep = 0u;
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (i < n) keep |= uint32_t(loop0[packed_byte(pk[j], i)]) << i;
          const uint32_t other = ~keep & ((1u << n) - 1u);
          pos[j] = other != 0u ? __ffs(other) - 1 : n;
        }
        bool paused[kMemoTok];
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) paused[j] = walk(cur[j], pos[j], len[j], pk[j], tt[j]);
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) settle(paused[j], cur[j], pos[j], len[j], kk[j], tt[j], qin);
      }
    }
    __syncthreads();
    int qn = qcount;
    while (qn > 0 && !overflowed && !row_fail) {
      resolve();  // its first barrier orders every read of qcount before the reset below
      if (overflowed) break;
      if (tid == 0) qcount = 0;
      __syncthreads();
      for (int i0 = 0; i0 < qn; i0 += kMemoThreads * kMemoTok) {
        uint2 e[kMemoTok];
        uint4 pk[kMemoTok];
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          const int i = i0 + j * kMemoThreads + tid;
          e[j] = i < qn ? qin[i] : make_uint2(0u, 0u);
        }
        int2 tq[kMemoTok];  // (token id, length)
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          const bool valid = i0 + j * kMemoThreads + tid < qn;
          pk[j] = valid ? ws.recs[e[j].x & 0x3FFFFu] : make_uint4(0u, 0u, 0u, 0u);
          tq[j] = valid ? ws.tmeta[e[j].x & 0x3FFFFu] : make_int2(-1, 0);
        }
#pragma unroll
        for (int j = 0; j < kMemoTok; ++j) {
          const bool valid = i0 + j * kMemoThreads + tid < qn;
          const int32_t k = int32_t(e[j].x & 0x3FFFFu);
          int cur = valid ? int((e[j].x >> 18) | ((e[j].y >> 16) << 14)) : kNone;
          int pos = int(e[j].y & 0xFFFFu);
          const int len = tq[j].y;
          const bool paused = walk(cur, pos, len, pk[j], tq[j].x);
          settle(paused, cur, pos, len, k, tq[j].x, qout);
        }
      }
      __syncthreads();
      qn = qcount;
      uint2* q = qin;
      qin = qout;
      qout = q;
    }
    if (overflowed || row_fail) {
      // start again in tile mode from an empty pool, bitmap and request set
      if (tid == 0) walk_lists = 0;
      for (int i = tid; i < vwords; i += kMemoThreads) vbits[i] = 0u;
      for (int i = tid; i < kMemoSets * 8; i += kMemoThreads) req[i] = 0u;
      reset_pool();
      tiles = true;
    }
  }

  bool retry = false;  // the tile is being walked again after a pool reset
  for (int64_t tile = tiles ? 0 : V; tile < V;) {
    // per token: length, position, state and its first 16 bytes; the state
    // is the current set id (< 256) while walking, else kAllowed / kRejected
    // / kNone. Token j of the thread is order[tile + j * kMemoThreads + tid].
    int32_t pos[kMemoTok], len[kMemoTok];
    int cur[kMemoTok];
    uint4 pk[kMemoTok];
#pragma unroll
    for (int j = 0; j < kMemoTok; ++j) {
      const int64_t k = tile + int64_t(j) * kMemoThreads + tid;
      const int2 m = k < V ? ws.tmeta[k] : make_int2(-1, 0);
      pk[j] = k < V ? ws.recs[k] : make_uint4(0u, 0u, 0u, 0u);
      const int32_t t = m.x;
      pos[j] = len[j] = 0;
      if (t < 0) {
        cur[j] = kNone;
      } else if (dead_row) {
        cur[j] = kRejected;
      } else if (t == a.eos) {
        cur[j] = (flags & 2) ? kAllowed : kRejected;
      } else {
        len[j] = m.y;
        cur[j] = len[j] == 0 ? ((flags & 4) ? kAllowed : kRejected) : 0;
      }
    }
    while (true) {
      bool waiting = false;
#pragma unroll
      for (int j = 0; j < kMemoTok; ++j) {
        while (cur[j] < kWalkEnd) {
          if (pos[j] == len[j]) {
            cur[j] = kAllowed;
            break;
          }
          const int byte = pos[j] < 16 ? packed_byte(pk[j], pos[j]) : long_byte(a, tile + int64_t(j) * kMemoThreads + tid, pos[j]);
          const uint8_t nx = T[cur[j] * 256 + byte];
          if (nx == kTUnknown) {
            // request the byte's elementary interval by its first byte; with
            // no byte edge over it the step empties the set
            if (((set_hit[cur[j]][byte >> 5] >> (byte & 31)) & 1u) == 0u) {
              cur[j] = kRejected;
              break;
            }
            const int lo = interval_start(set_bnd[cur[j]], byte);
            atomicOr(&req[cur[j] * 8 + (lo >> 5)], 1u << (lo & 31));
            waiting = true;
            break;
          }
          if (nx == kTDead || nx == kTOverflow) {
            cur[j] = kRejected;  // an overflow entry only exists in a tile that is abandoned
          } else {
            cur[j] = nx;
            ++pos[j];
          }
        }
      }
      if (!__syncthreads_or(waiting)) break;

      resolve();
      if (overflowed) break;
    }
    if (overflowed) {
      // the pool is full: drop every interned set and transition and walk the
      // tile again from an empty pool; a tile that fills the pool twice leaves
      // the whole row to the direct walk
      if (retry) break;
      reset_pool();
      retry = true;
      continue;
    }

    // allowed tokens of the tile into the row's bitmap
#pragma unroll
    for (int j = 0; j < kMemoTok; ++j)
      if (cur[j] == kAllowed) {
        const int64_t k = tile + int64_t(j) * kMemoThreads + tid;
        const int32_t t = int32_t(a.order ? a.order[k] : k);
        atomicOr(&vbits[t >> 5], 1u << (t & 31));
      }
    retry = false;
    tile += int64_t(kMemoThreads) * kMemoTok;
  }
  __syncthreads();
  // keep the transition table for the commit of this step (the rows of the
  // interned sets: the commit reads no other, their count is in the row's
  // metadata)
  uint32_t* tout = ws.table + b * (kMemoSets * 64);
  const int t_rows = pool_count < max_sets ? pool_count : max_sets;
  for (int i = tid; i < t_rows * 64; i += kMemoThreads) {
    const uint32_t v = T32[i];
    const int c = (i & 63) * 4;
    const uint32_t nib = (texact[(i >> 6) * 8 + (c >> 5)] >> (c & 31)) & 0xFu;
    uint32_t m = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (((nib >> j) & 1u) != 0u && ((v >> (8 * j)) & 0xFFu) < kTOverflow) m |= uint32_t(kTExact) << (8 * j);
    tout[i] = v | m;
  }
  // ... the boundary table and the sets' frame-list words (the commit walks
  // list states the same way)
  for (int i = tid; i < kLT; i += kMemoThreads) {
    uint32_t r = lt_res[i];
    if (r < kTOverflow && ((lt_exact[i >> 5] >> (i & 31)) & 1u) != 0u) r |= kTExact;
    ws.lt[b * kLT + i] = make_uint2(lt_key[i], r);
  }
  {
    const int pc = pool_count < max_sets ? pool_count : max_sets;
    for (int i = tid; i < kMemoSets; i += kMemoThreads) ws.slist[b * kMemoSets + i] = i < pc ? set_list[i] : -1;
  }
  if (tid == 0) {
    ws.overflow[b] = overflowed;
    ws.meta[b * 4 + 0] = dead_row ? 0 : (pool_count < max_sets ? pool_count : max_sets);
    ws.meta[b * 4 + 1] = int32_t(uint32_t(tag));
    ws.meta[b * 4 + 2] = int32_t(uint32_t(tag >> 32));
    ws.meta[b * 4 + 3] = int32_t(gen);
    ws.header[0] = gen;
  }
  if (overflowed) return;  // the direct walk writes this row
  if (!a.logits) {
    for (int w = tid; w < vwords && w < a.words; w += kMemoThreads) a.bits[b * a.words + w] = vbits[w];
    return;
  }
  // logits: the rejected columns get the fill value, here or -- for the
  // last kDefer rows of the launch to get here -- by the deferred-write
  // kernel from the row's verdict bits
  __shared__ int defer_slot;
  if (tid == 0) {
    // this row's place among the launch's rows to get here: the running
    // count less its value when the launch began (one atomic add, no retry
    // loop: rows that finish together would serialise on a compare-and-swap)
    const uint32_t order = atomicAdd(&ws.header[kFinishWord], 1u) - finish_base;
    const int64_t first = a.rows > kDefer ? a.rows - kDefer : 0;
    defer_slot = int64_t(order) >= first && int64_t(order) - first < kDefer ? int(int64_t(order) - first) : -1;
  }
  __syncthreads();
  if (defer_slot >= 0) {
    uint32_t* dst = ws.defer + int64_t(defer_slot) * (kMemoMaxVocab / 32);
    for (int i = tid; i < vwords; i += kMemoThreads) dst[i] = vbits[i];
    if (tid == 0)
      *reinterpret_cast<unsigned long long*>(ws.header + kDeferWord + 2 * defer_slot) =
          (static_cast<unsigned long long>(gen) << 32) | static_cast<unsigned long long>(b);
    return;
  }
  uint8_t* rowp = a.logits + b * a.ld_bytes;
  if (a.elem == 2)
    write_rejected<2, kMemoThreads>(rowp, vbits, 0, int(V), a.fill, tid);
  else
    write_rejected<4, kMemoThreads>(rowp, vbits, 0, int(V), a.fill, tid);
}

// Rows of a launch with only_rows set that a block of this kernel checks:
// the flags of the block's rows are one load, so a launch whose rows are
// mostly unflagged is short.
constexpr int kOnlyRowsPerBlock = 16;

// The direct mask: grid (chunks, rows), block (x, b) takes chunk x of row b.
// After a memoised mask (only_rows set): grid (chunks, F + D) with F =
// ceil(rows / kOnlyRowsPerBlock): block (x, y < F) takes chunk x of each
// flagged row among rows [16 y, 16 y + 16), one after another; the blocks
// y >= F, kDeferBlocks per slot in x-major order, write the logits of the
// deferred slots' rows, each block a 64-column-aligned piece; block (0, 0)
// stamps the pack key of the records the mask walked and the finish count
// the next mask launch starts from.
__global__ __launch_bounds__(kWave) void pda_mask_kernel(MaskArgs a) {
  if (!a.only_rows) {
    mask_row_chunk(a, blockIdx.y);
    return;
  }
  const int64_t flag_rows = (a.rows + kOnlyRowsPerBlock - 1) / kOnlyRowsPerBlock;
  if (int64_t(blockIdx.y) >= flag_rows) {
    const int64_t e = (int64_t(blockIdx.y) - flag_rows) * gridDim.x + blockIdx.x;
    const int k = int(e / kDeferBlocks), piece = int(e % kDeferBlocks);
    if (!a.defer_bits || !a.logits || k >= kDefer) return;
    const int V = a.vocab;
    const int per = (V + kDeferBlocks * kWave - 1) / (kDeferBlocks * kWave) * kWave;
    const int lo = piece * per, hi = lo + per < V ? lo + per : V;
    if (lo >= hi) return;
    // the slot's verdict words of the piece's first eight steps are read
    // beside the slot word (the slot's bits exist whether or not it is set)
    const uint32_t* vb = a.defer_bits + int64_t(k) * (kMemoMaxVocab / 32);
    const int lane = int(threadIdx.x);
    uint32_t w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = lo + u * kWave + lane;
      w[u] = c < hi ? vb[c >> 5] : 0xFFFFFFFFu;
    }
    const unsigned long long v = *reinterpret_cast<const unsigned long long*>(a.header + kDeferWord + 2 * k);
    if (uint32_t(v >> 32) != a.gen) return;
    const int64_t b = int64_t(uint32_t(v));
    if (b >= a.rows) return;
    uint8_t* rowp = a.logits + b * a.ld_bytes;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = lo + u * kWave + lane;
      if (((w[u] >> (c & 31)) & 1u) == 0u) {
        if (a.elem == 2)
          *reinterpret_cast<uint16_t*>(rowp + c * 2) = uint16_t(a.fill & 0xFFFFu);
        else
          *reinterpret_cast<uint32_t*>(rowp + c * 4) = a.fill;
      }
    }
    if (lo + 8 * kWave < hi) {
      if (a.elem == 2)
        write_rejected<2, kWave>(rowp, vb, lo + 8 * kWave, hi, a.fill, lane);
      else
        write_rejected<4, kWave>(rowp, vb, lo + 8 * kWave, hi, a.fill, lane);
    }
    return;
  }
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0 && a.header) {
    a.header[2] = uint32_t(a.pkey);
    a.header[3] = uint32_t(a.pkey >> 32);
    a.header[kFinishWord + 1] = a.header[kFinishWord];
  }
  const int64_t b0 = int64_t(blockIdx.y) * kOnlyRowsPerBlock;
  const int64_t bl = b0 + threadIdx.x;
  uint64_t m = __ballot(threadIdx.x < kOnlyRowsPerBlock && bl < a.rows && a.only_rows[bl] != 0);
  while (m != 0u) {
    const int i = __ffsll(static_cast<unsigned long long>(m)) - 1;
    m &= m - 1;
    mask_row_chunk(a, b0 + i);
  }
}

struct AdvanceArgs {
  PdaTableView g;
  const int32_t* tok_off;
  const uint8_t* tok_bytes;
  int32_t vocab;
  int32_t eos;
  int32_t* configs;
  const int64_t* slots;
  const void* tokens;
  int tok_dtype;
  int64_t rows;
  uint8_t* ok;
  uint8_t* broken;
  int32_t* status;
  int32_t* err;
  BpdPdaFrames frames;  // num_lists 0: no frame lists
};

__device__ bool flat_config_ok(const int32_t* c, int32_t num_states) {
  const int n = c[0];
  if (n < 0 || n > kMaxConfigs) return false;
  for (int i = 0; i < n; ++i) {
    const int d = c[2 + i];
    if (d < 0 || d > kMaxDepth) return false;
    for (int k = 0; k < d; ++k) {
      const int v = c[2 + kMaxConfigs + i * kMaxDepth + k];
      if (v < 0 || v >= num_states) return false;
    }
  }
  return true;
}

__global__ __launch_bounds__(kCommitRows) void pda_advance_kernel(AdvanceArgs a) {
  __shared__ int32_t bufs[kCommitRows][2][kConfigWords];
  const int64_t b = int64_t(blockIdx.x) * kCommitRows + threadIdx.x;
  if (b >= a.rows) return;
  const int64_t row = a.slots ? a.slots[b] : b;
  int32_t* cfg = a.configs + row * kConfigWords;
  const int64_t t = read_token(a.tokens, a.tok_dtype, b);
  bool ok;
  if (t < 0 || t >= a.vocab) {
    if (a.err) atomicOr(a.err, BPD_FLAG_TOKEN_RANGE);
    ok = false;
  } else if (!flat_config_ok(cfg, a.g.num_states)) {
    if (a.err) atomicOr(a.err, BPD_FLAG_STATE_RANGE);
    ok = false;
  } else if (t == a.eos) {
    ok = is_complete(a.g, ConstFlatView{cfg});
  } else {
    const int32_t s = a.tok_off[t], e = a.tok_off[t + 1];
    ok = true;
    if (s < e) {
      FlatView x{bufs[threadIdx.x][0]}, y{bufs[threadIdx.x][1]};
      x.reset_all();
      ok = advance_byte(a.g, ConstFlatView{cfg}, x, a.tok_bytes[s]);
      for (int32_t i = s + 1; i < e && ok; ++i) {
        y.reset_all();
        ok = advance_byte(a.g, x, y, a.tok_bytes[i]);
        const FlatView tmp = x;
        x = y;
        y = tmp;
      }
      if (ok)
        for (int k = 0; k < kConfigWords; ++k) cfg[k] = x.w[k];
    }
  }
  if (a.ok) a.ok[b] = ok ? 1 : 0;
  if (a.broken) {
    if (!ok) a.broken[row] = 1;
    if (a.status) a.status[b] = a.broken[row] ? -1 : 1;
  } else if (a.status) {
    a.status[b] = ok ? 1 : -1;
  }
}

// Commit with the mask's transition tables: one wave per row.  When the
// workspace row holds the tables of this config-set (same meaningful words as
// its set 0, same grammar and tokens), the token's bytes but the last are
// walked through the table and the last byte is stepped with advance_byte
// from the interned set reached, so the written config-set has the raw words
// of the direct walk.  Otherwise (or when the table walk meets an entry the
// mask left unresolved) every byte is stepped with advance_byte.
// The memoised commit: one row per workgroup.  All its threads stage the
// row's transition table in LDS with one round of loads (the walk over the
// token's bytes is then a chain of LDS reads, not of global ones); wave 0
// commits the row.
constexpr int kCommitThreads = 256;
static_assert(kCommitThreads == 256, "a thread per byte stages the list's codes");

// InLds: the grammar tables are staged in LDS (the dynamic array `ctab`), so
// the closure of the commit's byte steps reads them from LDS.
template <bool InLds>
__global__ __launch_bounds__(kCommitThreads) void pda_memo_advance_kernel(AdvanceArgs a, MemoWs ws,
                                                                         uint64_t tag, uint64_t pkey) {
  extern __shared__ __align__(16) int32_t ctab[];
  __shared__ int32_t bufs[2][kConfigWords];
  __shared__ uint4 trow[kMemoSets * 16];  // the row's table (256 bytes per set)
  __shared__ int32_t srow[kMemoSets];     // frame-list word of each interned set
  __shared__ int32_t ltrans[256];         // byte codes of the frame list of the row's set (if any)
  __shared__ int32_t lkey[BPD_PDA_FRAME_KEY_WORDS];  // and its key
  __shared__ int row_l0;                  // that list (-1: none)
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t b = blockIdx.x;
  const int64_t row = a.slots ? a.slots[b] : b;
  int32_t* cfg = a.configs + row * kConfigWords;
  int32_t* x = bufs[0];
  int32_t* y = bufs[1];
  // the reads wave 0 needs after the table is staged -- the token, its
  // offsets and record (length and first 12 bytes: one read after the token
  // id, where the bytes themselves are one more), the workspace stamps, the
  // pool's set 0 -- are issued before the staging loads, so their round
  // trips overlap them
  const int64_t t = read_token(a.tokens, a.tok_dtype, b);
  const bool t_in = t >= 0 && t < a.vocab;
  const bool walk_tok = t_in && t != a.eos;
  const uint32_t hk0 = ws.header[2], hk1 = ws.header[3];
  const bool w0 = threadIdx.x < kWave;
  const int32_t s = walk_tok && w0 ? a.tok_off[t] : 0, e = walk_tok && w0 ? a.tok_off[t + 1] : 0;
  const uint4 tr = walk_tok && w0 ? ws.trecs[t] : make_uint4(0u, 0u, 0u, 0u);
  int32_t meta[4] = {0, 0, 0, 0};
  uint32_t hdr = 0;
  int32_t p0[kSetLoads];
  const int32_t* pool = ws.pool ? ws.pool + b * kMemoSets * kConfigWords : nullptr;
  if (threadIdx.x < kWave) {
    for (int k = lane; k < kConfigWords; k += kWave) x[k] = cfg[k];
    if (pool) {
#pragma unroll
      for (int q = 0; q < 4; ++q) meta[q] = ws.meta[b * 4 + q];
      hdr = ws.header[0];
#pragma unroll
      for (int q = 0; q < kSetLoads; ++q) {
        const int k = lane + q * kWave;
        p0[q] = k < kConfigWords ? pool[k] : 0;
      }
    }
  }
  const TableSlice tsl = InLds ? table_slice(a.g, int(threadIdx.x)) : TableSlice{0, 0, 0, 0, 0, 0, 0, 0};
  {
    // T rows of the first 16 sets, then (once the row's set count is read)
    // those of the others the mask interned; the boundary table is probed
    // where it lies (a commit rarely meets a boundary entry)
    static_assert(kCommitThreads == 16 * 16, "one 16-byte piece of the first 16 T rows per thread");
    const uint4* src = reinterpret_cast<const uint4*>(ws.table + b * (kMemoSets * 64));
    const uint4 v = src[threadIdx.x];
    const int32_t pcm = ws.meta[b * 4];
    const int32_t sv = threadIdx.x < kMemoSets ? ws.slist[b * kMemoSets + threadIdx.x] : -1;
    // the list of the row's set (set 0 of the pool), its byte codes and key:
    // the walk's list steps and the composed set mostly use that list
    const int32_t sl0 = a.frames.num_lists > 0 ? ws.slist[b * kMemoSets] : -1;
    const int l0 = sl0 >= 0 && (sl0 & (BPD_PDA_FRAME_SAT - 1)) < a.frames.num_lists ? (sl0 & (BPD_PDA_FRAME_SAT - 1)) : -1;
    const int32_t ltv = l0 >= 0 ? a.frames.trans[int64_t(l0) * 256 + threadIdx.x] : -1;
    const int32_t lkv = l0 >= 0 && threadIdx.x < BPD_PDA_FRAME_KEY_WORDS
                            ? a.frames.keys[int64_t(l0) * BPD_PDA_FRAME_KEY_WORDS + threadIdx.x]
                            : 0;
    trow[threadIdx.x] = v;
    const int pc = pcm < 0 ? 0 : (pcm > kMemoSets ? kMemoSets : pcm);
    for (int q = kCommitThreads + threadIdx.x; q < pc * 16; q += kCommitThreads) trow[q] = src[q];
    if (threadIdx.x < kMemoSets) srow[threadIdx.x] = sv;
    ltrans[threadIdx.x] = ltv;
    if (threadIdx.x < BPD_PDA_FRAME_KEY_WORDS) lkey[threadIdx.x] = lkv;
    if (threadIdx.x == 0) row_l0 = l0;
  }
  const PdaTableView g = InLds ? stage_tables(a.g, ctab, tsl, int(threadIdx.x), kCommitThreads) : a.g;
  __syncthreads();
  if (threadIdx.x >= kWave) return;
  const int own = row_l0;  // the list whose codes and key are staged
  // the record holds the first 12 bytes when the workspace's records are of
  // these tables at this row count (its stamp) and its length is the
  // token's; the bytes past them (all, without it) one per lane, read only
  // for a token that has any
  const int32_t nrec = hk0 == uint32_t(pkey) && hk1 == uint32_t(pkey >> 32) && int32_t(tr.x) == e - s ? 12 : 0;
  int32_t bl = 0;
  if (walk_tok && e - s > nrec) bl = s + lane < e ? int32_t(a.tok_bytes[s + lane]) : 0;
  bool ok;
  if (!t_in) {
    if (lane == 0 && a.err) atomicOr(a.err, BPD_FLAG_TOKEN_RANGE);
    ok = false;
  } else if (!config_ok(x, a.g.num_states, lane)) {
    if (lane == 0 && a.err) atomicOr(a.err, BPD_FLAG_STATE_RANGE);
    ok = false;
  } else if (t == a.eos) {
    ok = is_complete(g, ConstFlatView{x});
  } else {
    ok = true;
    if (s < e) {
      auto byte_at = [&](int32_t i) -> int {
        const int32_t r = i - s;
        if (r < nrec) {
          const uint32_t w = r < 4 ? tr.y : (r < 8 ? tr.z : tr.w);
          return int((w >> ((r & 3) * 8)) & 0xFFu);
        }
        return r < kWave ? __shfl(bl, int(r)) : int(a.tok_bytes[i]);
      };
      // walk the mask's tables while they have the entries, as the mask's
      // walk does: T for interned sets; for a set in a frame list whose T
      // entry is missing, its list state through the lists' byte table and
      // LT at boundary bytes.  A step's raw words depend only on the
      // meaningful words of the set it starts from, so when the last byte's
      // entry is flagged exact the interned set is the written config-set;
      // otherwise the rest (at least the last byte) is stepped with
      // advance_byte from the set reached (a list state's set rebuilt from
      // its anchor's common stack and the list's key)
      int cur = -1, prev = -1;  // -1: no usable table, step every byte from the row's set
      bool exact = false;
      int32_t i = s;
      bool same0 = false;
      if (pool && meta[0] >= 1 && meta[1] == int32_t(uint32_t(tag)) && meta[2] == int32_t(uint32_t(tag >> 32)) &&
          uint32_t(meta[3]) == hdr) {
        // set 0 of the pool against the row's set (coop_same with the pool's
        // words already in registers)
        int32_t* p0l = y;
#pragma unroll
        for (int q = 0; q < kSetLoads; ++q) {
          const int k = lane + q * kWave;
          if (k < kConfigWords) p0l[k] = p0[q];
        }
        wave_sync();
        same0 = coop_same(x, p0l, lane);
      }
      if (same0) {
        // every lane walks alike: the values the walk branches on are made
        // wave-uniform (scalar lane reads), so its control flow is scalar
        const uint8_t* T = reinterpret_cast<const uint8_t*>(trow);
        cur = 0;
        for (; i < e; ++i) {
          const int byte = uniform(byte_at(i));
          if (cur < kListState) {
            const int nx = uniform(T[cur * 256 + byte]);
            if (nx == kTDead) {
              cur = -2;
              break;
            }
            if (nx < kTOverflow) {
              prev = cur;
              cur = nx & (kTExact - 1);
              exact = (nx & kTExact) != 0;
              continue;
            }
            const int sl = a.frames.num_lists > 0 ? uniform(srow[cur]) : -1;
            if (sl < 0) break;  // not resolved by the mask: step from here
            cur = list_state(cur, sl);
          }
          const int code = uniform((cur & 0xFFF) == own ? ltrans[byte] : a.frames.trans[(cur & 0xFFF) * 256 + byte]);
          if (code == -1) {
            cur = -2;
            break;
          }
          if (code >= 0) {
            prev = cur;
            cur = (cur & ~0xFFF) | ((code & BPD_PDA_FRAME_SAT) != 0 ? 1 << 12 : 0) | (code & 0xFFF);
            exact = (code & BPD_PDA_FRAME_RAW) != 0;
            continue;
          }
          // a boundary byte: the mask's LT entry, if it has one
          const uint32_t key = lt_key_of(cur, byte);
          const uint32_t h = lt_hash(key);
          int r = -1;
          for (int p = 0; p < kLT; ++p) {
            const uint2 v = ws.lt[b * kLT + ((h + uint32_t(p)) & uint32_t(kLT - 1))];
            if (uniform(int(v.x)) == int(key)) {
              r = uniform(int(v.y));
              break;
            }
            if (uniform(int(v.x)) == int(kLTEmpty)) break;
          }
          if (r == kTDead) {
            cur = -2;
            break;
          }
          if (r < 0 || r >= kTOverflow) break;  // step from the list state's set
          prev = cur;
          cur = r & (kTExact - 1);
          exact = (r & kTExact) != 0;
        }
      }
      if (cur == -2) {
        ok = false;
      } else if (cur >= 0 && cur < kListState && i == e && exact) {
        for (int k = lane; k < kConfigWords; k += kWave) cfg[k] = pool[cur * kConfigWords + k];
      } else if (cur >= kListState && i == e && exact) {
        // the last byte is a list step whose compaction drops no config: the
        // stepped set is, word for word, the one composed from the anchor's
        // common stack and the list's key
        const int anchor = (cur >> 13) & (kMemoSets - 1);
        if (anchor > 0) {
          for (int k = lane; k < kConfigWords; k += kWave) x[k] = pool[anchor * kConfigWords + k];
          wave_sync();
        }
        compose_list_set(x, cfg, (cur & 0xFFF) == own ? lkey : a.frames.keys + int64_t(cur & 0xFFF) * BPD_PDA_FRAME_KEY_WORDS,
                         srow[anchor] >> kListBase, (cur >> 12) & 1, lane);
      } else {
        if (cur >= 0 && i == e) {
          cur = prev;  // every byte had its entry: step the last one again
          i = e - 1;
        }
        if (cur >= kListState) {
          // the list state's set: its anchor's words under the list's key
          const int anchor = (cur >> 13) & (kMemoSets - 1);
          if (anchor > 0) {
            for (int k = lane; k < kConfigWords; k += kWave) x[k] = pool[anchor * kConfigWords + k];
            wave_sync();
          }
          compose_list_set(x, x, (cur & 0xFFF) == own ? lkey : a.frames.keys + int64_t(cur & 0xFFF) * BPD_PDA_FRAME_KEY_WORDS,
                           srow[anchor] >> kListBase, (cur >> 12) & 1, lane);
        } else if (cur > 0) {
          for (int k = lane; k < kConfigWords; k += kWave) x[k] = pool[cur * kConfigWords + k];
          wave_sync();
        }
        // bytes before the last taken through the frame lists' byte table
        // while the set is in a list: only the set before the last byte
        // needs its words, and only its meaningful ones (the last step
        // zeroes the set it writes), rebuilt from the common stack and the
        // list's key
        if (i < e - 1 && ok && a.frames.num_lists > 0) {
          int base = 0;
          const int l0 = frame_list_of(x, a.frames, a.frames.slots, lane, &base);
          if (l0 >= 0) {
            int l = l0, sat = x[1] != 0 ? 1 : 0, code = 0;
            int32_t j = i;
            for (; j < e - 1; ++j) {
              code = l == own ? ltrans[byte_at(j)] : a.frames.trans[l * 256 + byte_at(j)];
              if (code < 0) break;
              l = code & (BPD_PDA_FRAME_SAT - 1);
              sat |= (code & BPD_PDA_FRAME_SAT) != 0 ? 1 : 0;
            }
            if (j < e - 1 && code == -1) {
              ok = false;  // the list (and so the set) empties at byte j
            } else if (j > i) {
              compose_list_set(x, x, l == own ? lkey : a.frames.keys + int64_t(l) * BPD_PDA_FRAME_KEY_WORDS, base, sat, lane);
              i = j;
            }
          }
        }
        for (; i < e && ok; ++i) {
          ok = coop_advance_byte(g, x, y, byte_at(i), lane);
          int32_t* tmp = x;
          x = y;
          y = tmp;
        }
        if (ok)
          for (int k = lane; k < kConfigWords; k += kWave) cfg[k] = x[k];
      }
    }
  }
  if (lane == 0) {
    if (a.ok) a.ok[b] = ok ? 1 : 0;
    if (a.broken) {
      if (!ok) a.broken[row] = 1;
      if (a.status) a.status[b] = a.broken[row] ? -1 : 1;
    } else if (a.status) {
      a.status[b] = ok ? 1 : -1;
    }
  }
}

// The frame lists of `toks` as a kernel argument (num_lists 0: none).
int frames_arg(const BpdTokenBytes* toks, BpdPdaFrames* out) {
  *out = BpdPdaFrames{};
  if (const BpdPdaFrames* f = toks->frames) {
    BPD_REQUIRE(f->num_lists >= 0 && f->num_lists <= BPD_PDA_MAX_FRAME_LISTS,
                "frame lists: num_lists %d outside [0, %d]", f->num_lists, BPD_PDA_MAX_FRAME_LISTS);
    if (f->num_lists > 0) {
      BPD_REQUIRE(f->words == (toks->vocab_size + 31) / 32, "frame lists: words %d for vocab %d",
                  f->words, toks->vocab_size);
      BPD_REQUIRE(f->keys && f->slots && f->trans && f->allowed && f->seed_off && f->seeds,
                  "frame lists: null array");
      *out = *f;
    }
  }
  return BPD_OK;
}

int check_tables(const BpdPdaTable* g, const BpdTokenBytes* toks) {
  BPD_REQUIRE(g && toks, "null table argument");
  BPD_REQUIRE(g->num_states > 0, "empty PDA table");
  BPD_REQUIRE(g->num_states <= 65536, "PDA tables above 65536 states are not supported");
  BPD_REQUIRE(g->root_start >= 0 && g->root_start < g->num_states, "root_start out of range");
  BPD_REQUIRE(toks->vocab_size >= 0, "negative vocab size");
  return BPD_OK;
}

// ---------------------------------------------------------------- host --
bool host_try_token(const PdaTableView& g, const BpdTokenBytes& tk, const int32_t* cfg,
                    int32_t t, int32_t* x, int32_t* y) {
  if (t == tk.eos_id) return is_complete(g, ConstFlatView{cfg});
  const int32_t s = tk.offsets[t], e = tk.offsets[t + 1];
  if (s == e) return cfg[0] > 0;
  FlatView cur{x}, nxt{y};
  cur.reset_all();
  if (!advance_byte(g, ConstFlatView{cfg}, cur, tk.bytes[s])) return false;
  for (int32_t i = s + 1; i < e; ++i) {
    nxt.reset_all();
    if (!advance_byte(g, cur, nxt, tk.bytes[i])) return false;
    const FlatView tmp = cur;
    cur = nxt;
    nxt = tmp;
  }
  return cur.n() > 0;
}

bool host_config_ok(const int32_t* c, int32_t num_states) {
  const int n = c[0];
  if (n < 0 || n > kMaxConfigs) return false;
  for (int i = 0; i < n; ++i) {
    const int d = c[2 + i];
    if (d < 0 || d > kMaxDepth) return false;
    for (int k = 0; k < d; ++k) {
      const int v = c[2 + kMaxConfigs + i * kMaxDepth + k];
      if (v < 0 || v >= num_states) return false;
    }
  }
  return true;
}

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" size_t bpd_pda_workspace_bytes(int64_t rows, int32_t vocab) {
  return memo_ws_bytes(rows, vocab);
}

namespace {

// bpd_pda_feed's walk: 0 or an error code, whether every byte kept the set
// non-empty in *kept.
int pda_feed_impl(const BpdPdaTable* g, int32_t* config, const uint8_t* data, int64_t n, bool* kept) {
  BPD_REQUIRE(g && config, "null argument");
  BPD_REQUIRE(g->num_states > 0, "empty PDA table");
  BPD_REQUIRE(n >= 0 && (n == 0 || data), "bad byte buffer");
  BPD_REQUIRE(host_config_ok(config, g->num_states), "config-set is malformed");
  const PdaTableView gv = table_view(*g);
  std::vector<int32_t> x(kConfigWords), y(kConfigWords);
  FlatView cur{x.data()}, nxt{y.data()};
  std::copy(config, config + kConfigWords, x.data());
  *kept = false;
  for (int64_t i = 0; i < n; ++i) {
    nxt.reset_all();
    if (!advance_byte(gv, cur, nxt, data[i])) return BPD_OK;
    const FlatView tmp = cur;
    cur = nxt;
    nxt = tmp;
  }
  std::copy(cur.w, cur.w + kConfigWords, config);
  *kept = true;
  return BPD_OK;
}

}  // namespace

extern "C" int bpd_pda_feed(const BpdPdaTable* g, int32_t* config, const uint8_t* data,
                            int64_t n) {
  bool kept = false;
  const int rc = pda_feed_impl(g, config, data, n, &kept);
  return rc != BPD_OK ? -rc : (kept ? 1 : 0);
}

extern "C" int bpd_pda_init(const BpdPdaTable* g, int32_t* config_out) {
  BPD_REQUIRE(g && config_out, "null argument");
  BPD_REQUIRE(g->num_states > 0, "empty PDA table");
  BPD_REQUIRE(g->root_start >= 0 && g->root_start < g->num_states, "root_start out of range");
  init_config(table_view(*g), FlatView{config_out});
  return BPD_OK;
}

// Whether this process launched the pack of key `key` into `workspace`
// before (and records that it has now).
static bool packed_before(const void* workspace, uint64_t key) {
  static std::mutex mu;
  static std::unordered_map<const void*, uint64_t> last;
  std::lock_guard<std::mutex> lock(mu);
  auto it = last.find(workspace);
  if (it != last.end() && it->second == key) return true;
  last[workspace] = key;
  return false;
}

static int launch_pda_mask(const BpdPdaTable* g, const BpdTokenBytes* toks, const int32_t* configs,
                           const int64_t* slots, const uint8_t* broken, int64_t rows,
                           void* logits, int dtype, int64_t ld, double neg_inf, uint32_t* bits,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_tables(g, toks)) return rc;
  BPD_REQUIRE(rows >= 0 && rows < 65536, "rows must lie in [0, 65535]");
  MaskArgs a{};
  a.g = table_view(*g);
  a.tok_off = toks->offsets;
  a.tok_bytes = toks->bytes;
  a.vocab = toks->vocab_size;
  a.eos = toks->eos_id;
  a.configs = configs;
  a.slots = slots;
  a.broken = broken;
  a.rows = rows;
  if (logits) {
    a.elem = elem_bytes(dtype);
    BPD_REQUIRE(a.elem != 0, "unknown logits dtype code %d", dtype);
    BPD_REQUIRE(ld >= toks->vocab_size, "ld smaller than vocab");
    uint32_t fill = 0;
    if (int rc = fill_bits(dtype, neg_inf, &fill)) return rc;
    a.fill = fill;
    a.logits = static_cast<uint8_t*>(logits);
    a.ld_bytes = ld * a.elem;
  } else {
    a.bits = bits;
    a.words = (int64_t(toks->vocab_size) + 31) / 32;
  }
  if (rows == 0 || toks->vocab_size == 0) return BPD_OK;
  // ~16 waves per row keeps >= 4096 waves in flight at serving batch sizes
  const int64_t per_wave_min = 1024;
  int64_t chunks = (int64_t(toks->vocab_size) + per_wave_min - 1) / per_wave_min;
  if (chunks > 16) chunks = 16;
  int64_t per = (int64_t(toks->vocab_size) + chunks - 1) / chunks;
  per = (per + kWave - 1) / kWave * kWave;
  chunks = (int64_t(toks->vocab_size) + per - 1) / per;
  a.chunk_tokens = int32_t(per);
  a.err = nullptr;
  a.only_rows = nullptr;
  a.order = toks->order;
  a.runs = toks->order ? toks->runs : nullptr;
  if (int rc = frames_arg(toks, &a.frames)) return rc;
  if (workspace && toks->vocab_size <= kMemoMaxVocab) {
    const size_t need = memo_ws_bytes(rows, toks->vocab_size);
    BPD_REQUIRE(workspace_bytes >= need, "workspace too small (%zu < %zu bytes)", workspace_bytes, need);
    const MemoWs ws = memo_ws(workspace, rows, toks->vocab_size);
    const uint64_t pkey = pack_key(toks, rows);
    // the records are packed by a launch of their own the first time this
    // process masks with this key on this workspace; after that the mask
    // checks the workspace's stamp itself and, should another key be there
    // (the memory was reused), every block packs the records before walking
    const bool pack_launch = !packed_before(workspace, pkey);
    if (pack_launch) {
      // at most one block per CU
      const int64_t pack_blocks = std::min<int64_t>((int64_t(toks->vocab_size) + 255) / 256, 256);
      pack_tokens_kernel<<<unsigned(pack_blocks), 256, 0, as_stream(stream)>>>(
          toks->offsets, toks->bytes, toks->order, toks->vocab_size, ws.recs, ws.tmeta, ws.trecs, ws.header, pkey);
      BPD_LAUNCHED();
    }
    // BPD_PDA_MEMO_SETS lowers the interned-set limit (tests of the overflow path)
    int max_sets = kMemoIds;
    if (const char* e = std::getenv("BPD_PDA_MEMO_SETS")) {
      const int v = std::atoi(e);
      if (v >= 1 && v < kMemoIds) max_sets = v;
    }
    // BPD_PDA_MEMO_MODE=tile resolves per tile of tokens only (tests of that path)
    const char* mode = std::getenv("BPD_PDA_MEMO_MODE");
    const int row_mode = mode && std::strcmp(mode, "tile") == 0 ? 0 : 1;
    // stage the grammar tables in LDS when they fit beside the static arrays
    const size_t tab_bytes = staged_table_bytes(g);
    size_t room = 0;
    if (int rc = lds_room(reinterpret_cast<const void*>(&pda_memo_mask_kernel<true>), 0, &room)) return rc;
    const uint64_t tag = memo_tag(g, toks, rows);
    const uint32_t gen = next_generation();
    // BPD_PDA_LT_CAP lowers the entries the boundary table takes (tests of a
    // full table: the row starts again in tile mode)
    int lt_cap = kLT;
    if (const char* e = std::getenv("BPD_PDA_LT_CAP")) {
      const int v = std::atoi(e);
      if (v >= 1 && v < kLT) lt_cap = v;
    }
    if (tab_bytes <= room)
      pda_memo_mask_kernel<true><<<unsigned(rows), kMemoThreads, tab_bytes, as_stream(stream)>>>(
          a, ws, max_sets, tag, gen, row_mode, pkey, lt_cap, pack_launch ? 0 : 1);
    else
      pda_memo_mask_kernel<false><<<unsigned(rows), kMemoThreads, 0, as_stream(stream)>>>(
          a, ws, max_sets, tag, gen, row_mode, pkey, lt_cap, pack_launch ? 0 : 1);
    BPD_LAUNCHED();
    a.only_rows = ws.overflow;  // rows that ran out of interned sets
    a.header = ws.header;
    a.defer_bits = a.logits ? ws.defer : nullptr;
    a.gen = gen;
    a.pkey = pkey;
    // rows that overflow are rare: four waves per row keep short a launch
    // whose blocks mostly read their flag and exit
    if (chunks > 4) {
      per = (int64_t(toks->vocab_size) + 3) / 4;
      per = (per + kWave - 1) / kWave * kWave;
      chunks = (int64_t(toks->vocab_size) + per - 1) / per;
      a.chunk_tokens = int32_t(per);
    }
  }
  int64_t grid_rows = rows;
  if (a.only_rows) {
    grid_rows = (rows + kOnlyRowsPerBlock - 1) / kOnlyRowsPerBlock;
    if (a.defer_bits) grid_rows += (int64_t(kDefer) * kDeferBlocks + chunks - 1) / chunks;
  }
  pda_mask_kernel<<<dim3(unsigned(chunks), unsigned(grid_rows)), dim3(kWave), 0, as_stream(stream)>>>(a);
  BPD_LAUNCHED();
  return BPD_OK;
}

extern "C" int bpd_pda_apply_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                                  const int32_t* configs, const int64_t* slots,
                                  const uint8_t* broken, int64_t rows, void* logits, int dtype,
                                  int64_t ld, double neg_inf, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  BPD_REQUIRE(logits || rows == 0, "null logits");
  return launch_pda_mask(g, toks, configs, slots, broken, rows, logits, dtype, ld, neg_inf,
                         nullptr, workspace, workspace_bytes, stream);
}

extern "C" int bpd_pda_compute_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                                    const int32_t* configs, const int64_t* slots, int64_t rows,
                                    uint32_t* bits, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  BPD_REQUIRE(bits || rows == 0, "null bits");
  return launch_pda_mask(g, toks, configs, slots, nullptr, rows, nullptr, 0, 0, 0.0, bits,
                         workspace, workspace_bytes, stream);
}

extern "C" int bpd_pda_advance(const BpdPdaTable* g, const BpdTokenBytes* toks, int32_t* configs,
                               const int64_t* slots, const void* tokens, int token_dtype,
                               int64_t rows, uint8_t* ok, uint8_t* broken, int32_t* status,
                               int32_t* err, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (int rc = check_tables(g, toks)) return rc;
  BPD_REQUIRE(token_dtype_ok(token_dtype), "unknown token dtype code %d", token_dtype);
  BPD_REQUIRE(rows >= 0, "negative row count");
  if (rows == 0) return BPD_OK;
  AdvanceArgs a{};
  a.g = table_view(*g);
  a.tok_off = toks->offsets;
  a.tok_bytes = toks->bytes;
  a.vocab = toks->vocab_size;
  a.eos = toks->eos_id;
  a.configs = configs;
  a.slots = slots;
  a.tokens = tokens;
  a.tok_dtype = token_dtype;
  a.rows = rows;
  a.ok = ok;
  a.broken = broken;
  a.status = status;
  a.err = err;
  if (int rc = frames_arg(toks, &a.frames)) return rc;
  if (workspace) {
    // the mask's workspace of the same batch: reuse its transition tables
    const size_t need = memo_ws_bytes(rows, toks->vocab_size);
    BPD_REQUIRE(workspace_bytes >= need, "workspace too small (%zu < %zu bytes)", workspace_bytes, need);
    const MemoWs ws = memo_ws(workspace, rows, toks->vocab_size);
    // the grammar tables in LDS when they fit beside the static arrays
    const size_t tab_bytes = staged_table_bytes(g);
    size_t room = 0;
    if (int rc = lds_room(reinterpret_cast<const void*>(&pda_memo_advance_kernel<true>), 1, &room)) return rc;
    if (tab_bytes <= room)
      pda_memo_advance_kernel<true><<<unsigned(rows), kCommitThreads, tab_bytes, as_stream(stream)>>>(
          a, ws, memo_tag(g, toks, rows), pack_key(toks, rows));
    else
      pda_memo_advance_kernel<false><<<unsigned(rows), kCommitThreads, 0, as_stream(stream)>>>(
          a, ws, memo_tag(g, toks, rows), pack_key(toks, rows));
    BPD_LAUNCHED();
    return BPD_OK;
  }
  const unsigned blocks = unsigned((rows + kCommitRows - 1) / kCommitRows);
  pda_advance_kernel<<<blocks, kCommitRows, 0, as_stream(stream)>>>(a);
  BPD_LAUNCHED();
  return BPD_OK;
}

static int host_pda_mask(const BpdPdaTable* g, const BpdTokenBytes* toks, const int32_t* configs,
                         const int64_t* slots, const uint8_t* broken, int64_t rows, void* logits,
                         int dtype, int64_t ld, double neg_inf, uint32_t* bits) {
  if (int rc = check_tables(g, toks)) return rc;
  const PdaTableView gv = table_view(*g);
  const int E = logits ? elem_bytes(dtype) : 0;
  uint32_t fill = 0;
  if (logits) {
    BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
    if (int rc = fill_bits(dtype, neg_inf, &fill)) return rc;
  }
  const int64_t words = (int64_t(toks->vocab_size) + 31) / 32;
  std::vector<int32_t> x(kConfigWords), y(kConfigWords);
  for (int64_t b = 0; b < rows; ++b) {
    const int64_t row = slots ? slots[b] : b;
    const int32_t* cfg = configs + row * kConfigWords;
    BPD_REQUIRE(host_config_ok(cfg, g->num_states), "config-set of row %lld is malformed",
                (long long)b);
    const bool dead = broken && broken[row];
    if (bits) std::fill(bits + b * words, bits + (b + 1) * words, 0u);
    for (int32_t t = 0; t < toks->vocab_size; ++t) {
      const bool allow = !dead && host_try_token(gv, *toks, cfg, t, x.data(), y.data());
      if (bits) {
        if (allow) bits[b * words + (t >> 5)] |= 1u << (t & 31);
      } else if (!allow) {
        uint8_t* p = static_cast<uint8_t*>(logits) + (b * ld + t) * E;
        if (E == 2)
          *reinterpret_cast<uint16_t*>(p) = uint16_t(fill);
        else
          *reinterpret_cast<uint32_t*>(p) = fill;
      }
    }
  }
  return BPD_OK;
}

extern "C" int bpd_host_pda_apply_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                                       const int32_t* configs, const int64_t* slots,
                                       const uint8_t* broken, int64_t rows, void* logits,
                                       int dtype, int64_t ld, double neg_inf) {
  return host_pda_mask(g, toks, configs, slots, broken, rows, logits, dtype, ld, neg_inf, nullptr);
}

extern "C" int bpd_host_pda_compute_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                                         const int32_t* configs, const int64_t* slots,
                                         int64_t rows, uint32_t* bits) {
  return host_pda_mask(g, toks, configs, slots, nullptr, rows, nullptr, 0, 0, 0.0, bits);
}

extern "C" int bpd_host_pda_advance(const BpdPdaTable* g, const BpdTokenBytes* toks,
                                    int32_t* configs, const int64_t* slots, const void* tokens,
                                    int token_dtype, int64_t rows, uint8_t* ok, uint8_t* broken,
                                    int32_t* status) {
  if (int rc = check_tables(g, toks)) return rc;
  BPD_REQUIRE(token_dtype_ok(token_dtype), "unknown token dtype code %d", token_dtype);
  const PdaTableView gv = table_view(*g);
  auto token_at = [&](int64_t b) -> int64_t {
    return read_token(tokens, token_dtype, b);
  };
  for (int64_t b = 0; b < rows; ++b) {
    const int64_t t = token_at(b);
    BPD_REQUIRE(t >= 0 && t < toks->vocab_size,
                "index %lld is out of bounds for dimension 0 with size %d", (long long)t,
                toks->vocab_size);
    const int64_t row = slots ? slots[b] : b;
    BPD_REQUIRE(host_config_ok(configs + row * kConfigWords, g->num_states),
                "config-set of row %lld is malformed", (long long)b);
  }
  std::vector<int32_t> x(kConfigWords), y(kConfigWords);
  for (int64_t b = 0; b < rows; ++b) {
    const int64_t row = slots ? slots[b] : b;
    int32_t* cfg = configs + row * kConfigWords;
    const int32_t t = int32_t(token_at(b));
    bool accepted;
    if (t == toks->eos_id) {
      accepted = is_complete(gv, ConstFlatView{cfg});
    } else {
      const int32_t s = toks->offsets[t], e = toks->offsets[t + 1];
      accepted = true;
      if (s < e) {
        FlatView cur{x.data()}, nxt{y.data()};
        cur.reset_all();
        accepted = advance_byte(gv, ConstFlatView{cfg}, cur, toks->bytes[s]);
        for (int32_t i = s + 1; i < e && accepted; ++i) {
          nxt.reset_all();
          accepted = advance_byte(gv, cur, nxt, toks->bytes[i]);
          const FlatView tmp = cur;
          cur = nxt;
          nxt = tmp;
        }
        if (accepted) std::copy(cur.w, cur.w + kConfigWords, cfg);
      }
    }
    if (ok) ok[b] = accepted ? 1 : 0;
    if (broken) {
      if (!accepted) broken[row] = 1;
      if (status) status[b] = broken[row] ? -1 : 1;
    } else if (status) {
      status[b] = accepted ? 1 : -1;
    }
  }
  return BPD_OK;
}
