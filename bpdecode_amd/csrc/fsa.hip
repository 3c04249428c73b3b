// Symbol-class FSA kernels that walk each token through the transition table
// on the fly (no [states, vocab] tok_next table): the device form of the
// reference's non-dense operators for grammars too large to densify.
//
// One block covers kFsaRows rows and kFsaThreads * kFsaTok tokens.  The
// transition table and the live flags are staged in LDS when they fit; each
// token's first 16 symbol classes are loaded once into registers and walked
// from every row state of the block.  Verdicts become fill stores (logits)
// or wave64 ballots (packed bits).

#include <atomic>
#include <cstdlib>
#include <cstring>

#include "bpd_common.hpp"

namespace bpd {
namespace {

constexpr int kFsaThreads = 256;
constexpr int kFsaTok = 4;     // tokens per thread, kFsaThreads apart
constexpr int kFsaRows = 8;    // rows per block
// The table is staged in LDS only when small: every block stages its own
// copy, which for large tables costs more than reading them through L2
// (a 75 KB uint16 copy per block measured 3x slower than L2 reads).
constexpr size_t kFsaMaxLds = 16 * 1024;
constexpr int32_t kNoRow = INT32_MIN;
constexpr int kFsaAdvThreads = 256;
// The fused commit (one block: gather, queued pool writes, walk, scatter)
// stages the transition table in LDS as uint16 up to this size; above it,
// or with 65535 states or more, the walk reads it through L2.
constexpr int kFsaCommitThreads = 1024;
constexpr int kFsaCommitPerThread = 4;
constexpr size_t kFsaCommitLds = 112 * 1024;
// 16-byte loads of the uint16 table per thread when staging: kFsaStage8 * 8 *
// kFsaCommitThreads entries, at least the kFsaCommitLds / 2 a staged table holds.
constexpr int kFsaStage8 = 7;
static_assert(size_t(kFsaStage8) * 8 * kFsaCommitThreads * 2 >= kFsaCommitLds, "staging loads too few");
constexpr uint16_t kReject16 = 0xFFFFu;

struct FsaView {
  const int32_t* trans;
  int32_t S, NS, dead;
  const uint8_t* accept;
  const uint8_t* live;
  const int32_t* off;
  const uint8_t* sym;
  int64_t V;
  int32_t eos;
  const uint16_t* trans16;  // optional: live-filtered uint16 table
  const uint8_t* rec;       // optional: 16-byte token records
};

// Symbol i (< 16) of a load_syms record: one select between the two 64-bit
// halves and a shift (a four-way word select with a loop-uniform index was
// compiled to a scratch store and an indexed scratch load).
__device__ __forceinline__ int packed_sym(const uint4& p, int i) {
  const uint64_t lo = (uint64_t(p.y) << 32) | p.x;
  const uint64_t hi = (uint64_t(p.w) << 32) | p.z;
  return int(((i < 8 ? lo : hi) >> (8 * (i & 7))) & 0xFFu);
}

// The token's first min(len, 16) symbol classes, byte i at bits 8 (i % 4)
// of word i / 4.
__device__ __forceinline__ uint4 load_syms(const uint8_t* __restrict__ p, int32_t len) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  const int n = len < 16 ? int(len) : 16;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (i < n) w[i >> 2] |= uint32_t(p[i]) << (8 * (i & 3));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// step() of mask_cpu.cpp:53-71 for a non-EOS token from a valid state s:
// true iff the walk never leaves the table, never meets `dead` and ends on
// a live state.
__device__ __forceinline__ bool walk_token(const FsaView& f, const int32_t* __restrict__ tr,
                                           const uint8_t* __restrict__ lv, int32_t s, uint4 pk,
                                           const uint8_t* __restrict__ rest, int32_t len) {
  int32_t cur = s;
  for (int32_t i = 0; i < len; ++i) {
    const int k = i < 16 ? packed_sym(pk, i) : int(rest[i]);
    if (k >= f.NS) return false;
    cur = tr[int64_t(cur) * f.NS + k];
    if (cur == f.dead || cur < 0 || cur >= f.S) return false;
  }
  return lv[cur] != 0;
}

// Mask (Bits = false: fill the rejected logits, element size E) or packed
// allow bits (Bits = true).  grid (ceil(V / (kFsaThreads kFsaTok)), ceil(rows / kFsaRows)).
template <int E, bool Bits, bool InLds>
__global__ __launch_bounds__(kFsaThreads) void fsa_mask_kernel(
    FsaView f, const int32_t* __restrict__ states, const int64_t* __restrict__ slots, int64_t rows,
    uint8_t* __restrict__ logits, int64_t ld_bytes, uint32_t fill, uint32_t* __restrict__ bits,
    int64_t words, int32_t* __restrict__ err) {
  extern __shared__ __align__(16) int32_t lds[];
  __shared__ int32_t rs[kFsaRows];
  const int tid = threadIdx.x;
  const int32_t* tr = f.trans;
  const uint8_t* lv = f.live;
  if (InLds) {
    const int64_t n = int64_t(f.S) * f.NS;
    for (int64_t i = tid; i < n; i += kFsaThreads) lds[i] = f.trans[i];
    uint8_t* l8 = reinterpret_cast<uint8_t*>(lds + n);
    for (int32_t i = tid; i < f.S; i += kFsaThreads) l8[i] = f.live[i];
    tr = lds;
    lv = l8;
  }
  const int64_t r0 = int64_t(blockIdx.y) * kFsaRows;
  if (tid < kFsaRows) {
    const int64_t r = r0 + tid;
    int32_t s = kNoRow;
    if (r < rows) {
      s = states[slots ? slots[r] : r];
      if (s >= f.S) {
        if (err) atomicOr(err, BPD_FLAG_STATE_RANGE);
        s = -1;  // the whole row is masked
      }
    }
    rs[tid] = s;
  }
  __syncthreads();
  const int64_t t0 = int64_t(blockIdx.x) * (kFsaThreads * kFsaTok);
#pragma unroll
  for (int j = 0; j < kFsaTok; ++j) {
    const int64_t t = t0 + int64_t(j) * kFsaThreads + tid;
    const bool on = t < f.V;
    const bool is_eos = t == f.eos;
    int32_t len = 0;
    uint4 pk = make_uint4(0u, 0u, 0u, 0u);
    const uint8_t* rest = f.sym;
    if (on && !is_eos) {
      const int32_t b = f.off[t];
      len = f.off[t + 1] - b;
      rest = f.sym + b;
      pk = load_syms(rest, len);
    }
    for (int r = 0; r < kFsaRows; ++r) {
      const int32_t s = rs[r];
      if (s == kNoRow) break;  // rows past the batch come last
      bool ok = false;
      if (on && s >= 0) ok = is_eos ? f.accept[s] != 0 : walk_token(f, tr, lv, s, pk, rest, len);
      if (Bits) {
        const uint64_t m = __ballot(ok);
        const int64_t tw = t - (tid & 63);  // first token of the wave, a multiple of 64
        if ((tid & 63) == 0 && tw < f.V) {
          uint32_t* out = bits + (r0 + r) * words + (tw >> 5);
          out[0] = uint32_t(m);
          if ((tw >> 5) + 1 < words) out[1] = uint32_t(m >> 32);
        }
      } else if (on && !ok) {
        uint8_t* p = logits + (r0 + r) * ld_bytes + t * E;
        if (E == 2)
          *reinterpret_cast<uint16_t*>(p) = uint16_t(fill);
        else
          *reinterpret_cast<uint32_t*>(p) = fill;
      }
    }
  }
}

// advance: one thread per row (mask_cpu.cpp:53-71 with the range handling
// of the dense commit: token ids wrap once like torch indexing, ids still
// out of range and states >= S give -1 and set the error flags).
__global__ __launch_bounds__(kFsaAdvThreads) void fsa_advance_kernel(
    FsaView f, const int32_t* __restrict__ states, const int64_t* __restrict__ slots,
    const void* __restrict__ tokens, int tok_dtype, int64_t rows, int32_t* __restrict__ next_out,
    int32_t* __restrict__ err) {
  const int64_t b = int64_t(blockIdx.x) * kFsaAdvThreads + threadIdx.x;
  if (b >= rows) return;
  const int32_t s = states[slots ? slots[b] : b];
  int64_t t = read_token(tokens, tok_dtype, b);
  if (t < 0) t += f.V;
  int32_t res = -1;
  if (t < 0 || t >= f.V) {
    if (err) atomicOr(err, BPD_FLAG_TOKEN_RANGE);
  } else if (s >= f.S) {
    if (err) atomicOr(err, BPD_FLAG_STATE_RANGE);
  } else if (s >= 0) {
    if (t == f.eos) {
      res = f.accept[s] ? s : -1;
    } else {
      const int32_t b0 = f.off[t], len = f.off[t + 1] - b0;
      int32_t cur = s;
      bool ok = true;
      for (int32_t i = 0; i < len && ok; ++i) {
        const int k = f.sym[b0 + i];
        if (k >= f.NS) {
          ok = false;
        } else {
          cur = f.trans[int64_t(cur) * f.NS + k];
          ok = cur != f.dead && cur >= 0 && cur < f.S;
        }
      }
      res = ok && f.live[cur] ? cur : -1;
    }
  }
  next_out[b] = res;
}

// Commit of up to kFsaCommitThreads * kFsaCommitPerThread rows in one block.
// Every global load whose address is known is issued before the first wait:
// each thread's rows' slot and token, then (InLds) its share of the uint16
// table (trans16) as 16-byte loads held in registers; then the rows' states
// and token records (the table goes to LDS while they are in flight).  So
// the staging costs one memory round trip, and a token's symbols one load.
// InLds: every walk step is one LDS read of the live-filtered table, whose
// 0xFFFF entries (outside the table, `dead` or not live) reject; a walk of
// at least one step that never meets one ends live.  Without the records,
// the token's offsets and symbols are read as in the other kernels.  The
// queued pool writes land after the walks have read the pool and before
// the rows write back -- the order of the calls, as in the dense commit.
template <bool InLds>
__global__ __launch_bounds__(kFsaCommitThreads) void fsa_advance_block_kernel(
    FsaView f, int32_t* __restrict__ states, const int64_t* __restrict__ slots,
    const int64_t* __restrict__ pending, int32_t num_pending, const void* __restrict__ tokens,
    int tok_dtype, int64_t rows, int32_t* __restrict__ next_out, int write_back,
    int32_t* __restrict__ err) {
  extern __shared__ __align__(16) uint16_t tr16[];
  __shared__ int64_t pslot[BPD_MAX_FUSED_PENDING];
  __shared__ int32_t pval[BPD_MAX_FUSED_PENDING];
  const int tid = threadIdx.x;
  int64_t slot[kFsaCommitPerThread], tk[kFsaCommitPerThread];
#pragma unroll
  for (int i = 0; i < kFsaCommitPerThread; ++i) {
    const int64_t b = int64_t(i) * kFsaCommitThreads + tid;
    slot[i] = -1;
    tk[i] = 0;
    if (b < rows) {
      slot[i] = slots ? slots[b] : b;
      tk[i] = read_token(tokens, tok_dtype, b);
    }
  }
  const int64_t n = int64_t(f.S) * f.NS;
  const int64_t n8 = n >> 3;
  int4 tv[InLds ? kFsaStage8 : 1];
  uint16_t tail = kReject16;
  if (InLds) {
    const int4* t8 = reinterpret_cast<const int4*>(f.trans16);
#pragma unroll
    for (int k = 0; k < kFsaStage8; ++k) {
      const int64_t j = int64_t(k) * kFsaCommitThreads + tid;
      tv[k] = j < n8 ? t8[j] : make_int4(0, 0, 0, 0);
    }
    if (tid < n - 8 * n8) tail = f.trans16[8 * n8 + tid];
  }
  for (int32_t i = tid; i < num_pending; i += kFsaCommitThreads) {
    pslot[i] = pending[i];
    pval[i] = int32_t(pending[num_pending + i]);
  }
  int32_t st[kFsaCommitPerThread], b0[kFsaCommitPerThread], len[kFsaCommitPerThread];
  uint4 pk[kFsaCommitPerThread];
#pragma unroll
  for (int i = 0; i < kFsaCommitPerThread; ++i) {
    st[i] = -1;
    b0[i] = 0;
    len[i] = 0;
    pk[i] = make_uint4(0u, 0u, 0u, 0u);
    if (slot[i] < 0) continue;
    st[i] = states[slot[i]];
    int64_t t = tk[i];
    if (t < 0) t += f.V;
    tk[i] = t;
    if (t >= 0 && t < f.V && t != f.eos) {
      if (f.rec) {
        pk[i] = reinterpret_cast<const uint4*>(f.rec)[t];
      } else {
        b0[i] = f.off[t];
        len[i] = f.off[t + 1] - b0[i];
      }
    }
  }
  if (InLds) {
    int4* l8 = reinterpret_cast<int4*>(tr16);
#pragma unroll
    for (int k = 0; k < kFsaStage8; ++k) {
      const int64_t j = int64_t(k) * kFsaCommitThreads + tid;
      if (j < n8) l8[j] = tv[k];
    }
    if (tid < n - 8 * n8) tr16[8 * n8 + tid] = tail;
  }
  // the symbols: from the record (bytes 0-14, length in byte 15; a longer
  // token reads the rest through its offset) or from the offsets
  const int inline_syms = f.rec ? 15 : 16;
#pragma unroll
  for (int i = 0; i < kFsaCommitPerThread; ++i) {
    if (f.rec) {
      len[i] = int32_t(pk[i].w >> 24);
      if (len[i] > 15) {
        b0[i] = f.off[tk[i]];
        if (len[i] == 255) len[i] = f.off[tk[i] + 1] - b0[i];
      }
    } else {
      pk[i] = load_syms(f.sym + b0[i], len[i]);
    }
  }
  __syncthreads();
  // one row's walk (its symbols passed by value, so they stay in registers)
  auto walk = [&](int i, const uint4 sy) __attribute__((always_inline)) -> int32_t {
    const int64_t b = int64_t(i) * kFsaCommitThreads + tid;
    if (b >= rows) return -1;
    int32_t s = st[i];
    for (int32_t k = 0; k < num_pending; ++k)
      if (pslot[k] == slot[i]) s = pval[k];
    const int64_t t = tk[i];
    int32_t res = -1;
    if (t < 0 || t >= f.V) {
      if (err) atomicOr(err, BPD_FLAG_TOKEN_RANGE);
    } else if (s >= f.S) {
      if (err) atomicOr(err, BPD_FLAG_STATE_RANGE);
    } else if (s >= 0) {
      if (t == f.eos) {
        res = f.accept[s] ? s : -1;
      } else if (len[i] == 0) {
        res = f.live[s] ? s : -1;
      } else {
        const uint8_t* rest = f.sym + b0[i];
        int32_t cur = s;
        bool ok = true;
        for (int32_t j = 0; j < len[i] && ok; ++j) {
          const int k = j < inline_syms ? packed_sym(sy, j) : int(rest[j]);
          if (k >= f.NS) {
            ok = false;
          } else if (InLds) {
            const uint16_t v = tr16[cur * f.NS + k];
            ok = v != kReject16;
            cur = v;
          } else {
            cur = f.trans[int64_t(cur) * f.NS + k];
            ok = cur != f.dead && cur >= 0 && cur < f.S;
          }
        }
        if (InLds)
          res = ok ? cur : -1;  // every state the filtered table names is live
        else
          res = ok && f.live[cur] ? cur : -1;
      }
    }
    if (next_out) next_out[b] = res;
    return res;
  };
  static_assert(kFsaCommitPerThread == 4, "one walk call per row below");
  int32_t nxt[kFsaCommitPerThread];
  nxt[0] = walk(0, pk[0]);
  nxt[1] = walk(1, pk[1]);
  nxt[2] = walk(2, pk[2]);
  nxt[3] = walk(3, pk[3]);
  __syncthreads();
  for (int32_t i = tid; i < num_pending; i += kFsaCommitThreads) states[pslot[i]] = pval[i];
  if (!write_back) return;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kFsaCommitPerThread; ++i)
    if (slot[i] >= 0) states[slot[i]] = nxt[i];
}

__global__ void fsa_scatter_kernel(int32_t* __restrict__ states, const int64_t* __restrict__ slots,
                                   const int32_t* __restrict__ next, int64_t rows) {
  const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= rows) return;
  states[slots ? slots[b] : b] = next[b];
}

// Dynamic LDS the fused commit may take on the current device: the device's
// per-block limit less the kernel's static arrays (queried once per device).
int commit_lds_room(size_t* room) {
  constexpr int kDevices = 64;
  static std::atomic<long long> cache[kDevices];  // room + 1; 0: not queried yet
  int dev = 0;
  BPD_HIP(hipGetDevice(&dev));
  const bool cached = dev >= 0 && dev < kDevices;
  if (cached) {
    const long long c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *room = size_t(c - 1);
      return BPD_OK;
    }
  }
  int max_lds = 0;
  BPD_HIP(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
  hipFuncAttributes fa{};
  BPD_HIP(hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(&fsa_advance_block_kernel<true>)));
  *room = size_t(max_lds) > fa.sharedSizeBytes ? size_t(max_lds) - fa.sharedSizeBytes : 0;
  if (cached) cache[dev].store((long long)(*room) + 1, std::memory_order_relaxed);
  return BPD_OK;
}

int check_fsa(const BpdFsaTable* t) {
  BPD_REQUIRE(t, "null table argument");
  BPD_REQUIRE(t->num_states > 0 && t->num_symbols > 0 && t->vocab >= 0, "bad FSA table shape");
  BPD_REQUIRE(t->dead >= 0 && t->dead < t->num_states, "dead state out of range");
  BPD_REQUIRE(t->vocab < (int64_t(1) << 31), "vocab too large");
  BPD_REQUIRE(t->trans && t->accept && t->live && t->tok_offsets && t->tok_symbols, "null table array");
  return BPD_OK;
}

FsaView view_of(const BpdFsaTable& t) {
  return FsaView{t.trans, t.num_states, t.num_symbols, t.dead, t.accept, t.live,
                 t.tok_offsets, t.tok_symbols, t.vocab, t.eos_id, t.trans16, t.tok_records};
}

size_t fsa_lds_bytes(const BpdFsaTable& t) {
  return size_t(t.num_states) * size_t(t.num_symbols) * 4 + size_t(t.num_states);
}

template <int E, bool Bits>
int launch_fsa_mask(const BpdFsaTable& t, const int32_t* states, const int64_t* slots, int64_t rows,
                    void* logits, int64_t ld_bytes, uint32_t fill, uint32_t* bits, int64_t words,
                    int32_t* err, hipStream_t s) {
  const size_t lds = fsa_lds_bytes(t);
  bool in_lds = lds <= kFsaMaxLds;
  // BPD_FSA_TABLE=global forces the global-memory form (tests cover both
  // forms on small grammars with it)
  if (const char* e = std::getenv("BPD_FSA_TABLE"))
    if (std::strcmp(e, "global") == 0) in_lds = false;
  const int64_t gx = (t.vocab + kFsaThreads * kFsaTok - 1) / (kFsaThreads * kFsaTok);
  const int64_t gy = (rows + kFsaRows - 1) / kFsaRows;
  BPD_REQUIRE(gy < 65536, "at most %d rows per launch", 65535 * kFsaRows);
  const dim3 grid = dim3(unsigned(gx), unsigned(gy));
  uint8_t* lg = static_cast<uint8_t*>(logits);
  if (in_lds)
    fsa_mask_kernel<E, Bits, true><<<grid, kFsaThreads, lds, s>>>(view_of(t), states, slots, rows, lg,
                                                                   ld_bytes, fill, bits, words, err);
  else
    fsa_mask_kernel<E, Bits, false><<<grid, kFsaThreads, 0, s>>>(view_of(t), states, slots, rows, lg,
                                                                  ld_bytes, fill, bits, words, err);
  BPD_LAUNCHED();
  return BPD_OK;
}

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" int bpd_fsa_apply_mask(const BpdFsaTable* table, void* logits, int dtype, int64_t rows,
                                  int64_t ld, const int32_t* states, const int64_t* slots, double neg_inf,
                                  int32_t* err, void* stream) {
  if (int rc = check_fsa(table)) return rc;
  const int E = elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && ld >= table->vocab, "bad logits shape rows=%lld ld=%lld", (long long)rows,
              (long long)ld);
  uint32_t fill = 0;
  if (int rc = fill_bits(dtype, neg_inf, &fill)) return rc;
  if (rows == 0 || table->vocab == 0) return BPD_OK;
  BPD_REQUIRE(logits && states, "null pointer argument");
  hipStream_t s = as_stream(stream);
  if (E == 2) return launch_fsa_mask<2, false>(*table, states, slots, rows, logits, ld * E, fill, nullptr, 0, err, s);
  return launch_fsa_mask<4, false>(*table, states, slots, rows, logits, ld * E, fill, nullptr, 0, err, s);
}

extern "C" int bpd_fsa_compute_mask(const BpdFsaTable* table, const int32_t* states, const int64_t* slots,
                                    int64_t rows, uint32_t* bits, int32_t* err, void* stream) {
  if (int rc = check_fsa(table)) return rc;
  BPD_REQUIRE(rows >= 0, "negative row count");
  const int64_t words = (table->vocab + 31) / 32;
  if (rows == 0 || words == 0) return BPD_OK;
  BPD_REQUIRE(states && bits, "null pointer argument");
  return launch_fsa_mask<4, true>(*table, states, slots, rows, nullptr, 0, 0u, bits, words, err,
                                  as_stream(stream));
}

extern "C" int bpd_fsa_advance(const BpdFsaTable* table, int32_t* states, const int64_t* slots,
                               const int64_t* pending, int64_t num_pending, const void* tokens,
                               int token_dtype, int64_t rows, int32_t* next_out, int write_back,
                               int32_t* err, void* stream) {
  if (int rc = check_fsa(table)) return rc;
  BPD_REQUIRE(token_dtype_ok(token_dtype), "unknown token dtype code %d", token_dtype);
  BPD_REQUIRE(table->vocab > 0, "empty vocabulary");
  BPD_REQUIRE(rows >= 0, "negative row count");
  BPD_REQUIRE(num_pending >= 0 && num_pending <= BPD_MAX_FUSED_PENDING,
              "at most %d queued pool writes per launch (got %lld)", BPD_MAX_FUSED_PENDING,
              (long long)num_pending);
  BPD_REQUIRE(num_pending == 0 || (pending && slots && write_back),
              "queued writes need a slot map and write_back");
  BPD_REQUIRE(rows > 0 || num_pending == 0, "queued writes need at least one row");
  if (rows == 0) return BPD_OK;
  BPD_REQUIRE(states && tokens, "null pointer argument");
  BPD_REQUIRE(next_out || write_back, "advance with neither next_out nor write_back");
  hipStream_t s = as_stream(stream);
  const FsaView v = view_of(*table);
  if (rows <= int64_t(kFsaCommitThreads) * kFsaCommitPerThread) {
    const size_t lds = size_t(table->num_states) * size_t(table->num_symbols) * 2;  // uint16 table
    size_t room = 0;
    if (int rc = commit_lds_room(&room)) return rc;
    const bool staged = table->trans16 && reinterpret_cast<uintptr_t>(table->trans16) % 16 == 0;
    BPD_REQUIRE(!table->tok_records || reinterpret_cast<uintptr_t>(table->tok_records) % 16 == 0,
                "token records must be 16-byte aligned");
    if (staged && table->num_states < 65535 && lds <= kFsaCommitLds && lds <= room)
      fsa_advance_block_kernel<true><<<1, kFsaCommitThreads, lds, s>>>(
          v, states, slots, pending, int32_t(num_pending), tokens, token_dtype, rows, next_out,
          write_back, err);
    else
      fsa_advance_block_kernel<false><<<1, kFsaCommitThreads, 0, s>>>(
          v, states, slots, pending, int32_t(num_pending), tokens, token_dtype, rows, next_out,
          write_back, err);
    BPD_LAUNCHED();
    return BPD_OK;
  }
  BPD_REQUIRE(next_out, "batches above %d rows need next_out", kFsaCommitThreads * kFsaCommitPerThread);
  BPD_REQUIRE(num_pending == 0, "batches above %d rows take no queued writes",
              kFsaCommitThreads * kFsaCommitPerThread);
  const unsigned g = unsigned((rows + kFsaAdvThreads - 1) / kFsaAdvThreads);
  fsa_advance_kernel<<<g, kFsaAdvThreads, 0, s>>>(v, states, slots, tokens, token_dtype, rows, next_out, err);
  BPD_LAUNCHED();
  if (write_back) {
    fsa_scatter_kernel<<<g, kFsaAdvThreads, 0, s>>>(states, slots, next_out, rows);
    BPD_LAUNCHED();
  }
  return BPD_OK;
}
