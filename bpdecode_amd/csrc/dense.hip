// Dense tok_next path for gfx950: the mask over a [rows, vocab] logits batch
// (from the packed allow-bit table or from tok_next itself), the commit
// gather/advance/scatter, the packed allow-bit kernel and the device-side
// table builder.
//
// The mask is HBM-bound byte work that writes only what it must: the
// rejected logits.  A wave owns one row and 2048 columns; for each group of
// 64 columns the allowed/rejected verdicts select the lanes that store the
// fill value, one element per lane, so a group is one store instruction over
// 64 consecutive elements and allowed logits are neither read nor written.
// Measured on MI355X (B = 256, V = 151,936 bf16, email DFA) this matches a
// plain copy of the logits: with ~5 % of the tokens allowed and scattered,
// nearly every 128-byte line mixes kept and filled elements, so the memory
// side merges each partial line (a read and a write per line), the same
// traffic a kernel that reads, blends and rewrites the logits produces --
// but without the round trip through the CUs.  Non-temporal stores were
// slower (33 against 27 us).
//
// The queued state-pool writes of ConstraintBatch.add/evict/reset ride in
// the mask and commit launches (`pending`): rows read the queued value of
// their slot and one wave stores the queued values, so continuous batching
// costs no launch of its own.
#include <algorithm>

#include "bpd_common.hpp"

namespace bpd {
namespace {

constexpr int kXcds = 8;
constexpr int kFillWaves = 4;                 // waves per block: one row, 4 chunks
constexpr int kFillThreads = 64 * kFillWaves;
constexpr int kFillGroups = 32;               // 64-column groups per chunk (one wave)
constexpr int64_t kChunkCols = int64_t(kFillGroups) * 64;

// Block index -> logical block, numbered so that consecutive logical blocks
// run on one XCD (workgroups are dealt round-robin to the 8 XCDs).
// gridDim.x is a multiple of kXcds.
__device__ __forceinline__ uint32_t logical_block() {
  const uint32_t nb = gridDim.x;
  const uint32_t hw = blockIdx.x;
  return (hw % kXcds) * (nb / kXcds) + hw / kXcds;
}

template <int E> struct Elem;
template <> struct Elem<2> { using T = uint16_t; };
template <> struct Elem<4> { using T = uint32_t; };
template <> struct Elem<8> { using T = uint64_t; };

// Wave-uniform state of row r: the pool entry at its slot, or the value of a
// queued write to that slot (`pending` = num_pending slots, then as many
// values; slots are distinct).
__device__ __forceinline__ int32_t wave_row_state(const int32_t* states, const int64_t* slots,
                                                  const int64_t* pending, int32_t num_pending,
                                                  uint32_t r, int lane) {
  const int64_t slot = slots ? slots[r] : int64_t(r);
  int32_t s = __builtin_amdgcn_readfirstlane(states[slot]);
  for (int32_t base = 0; base < num_pending; base += 64) {
    const int32_t i = base + lane;
    const bool hit = i < num_pending && pending[i] == slot;
    const uint64_t m = __ballot(hit);
    if (m) {
      const int src = __builtin_ctzll(m);
      const int32_t v = hit ? int32_t(pending[num_pending + i]) : 0;
      s = __builtin_amdgcn_readlane(v, src);
    }
  }
  return s;
}

// Dense mask, write-only.  A wave owns one row and a chunk of 2048 columns
// (32 groups of 64); for each group the 64 verdicts of its columns decide
// which lanes store the fill value (one 2/4/8-byte store per lane, the
// group's store instruction covering 64 consecutive elements); allowed
// elements are never read or written.  Kernel `Bits`: the verdicts come from
// the packed allow-bit table, one uint32 word per lane holding the chunk's
// 64 words, broadcast per group with readlane; otherwise from the int32
// tok_next row (one coalesced load per group and lane).  A block holds one
// row and 4 consecutive chunks; logical blocks are numbered column-group
// major, so one XCD's L2 serves a contiguous band of table columns to every
// row.  The block with logical index 0 also applies the queued pool writes.
template <int E, bool Bits>
__global__ __launch_bounds__(kFillThreads) void dense_fill_kernel(
    uint8_t* __restrict__ logits, int64_t ld_bytes, const void* __restrict__ table,
    int64_t table_ld, int64_t vocab, int32_t num_states, int32_t* states,
    const int64_t* __restrict__ slots, const int64_t* __restrict__ pending, int32_t num_pending,
    uint32_t rows, uint32_t chunks, uint64_t fill, int32_t* __restrict__ err) {
  using T = typename Elem<E>::T;
  const uint32_t lb = logical_block();
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const uint32_t cg = lb / rows;
  const uint32_t r = lb - cg * rows;
  const uint32_t chunk = cg * kFillWaves + wave;
  if (lb == 0 && wave == 0)
    for (int32_t i = lane; i < num_pending; i += 64) states[pending[i]] = int32_t(pending[num_pending + i]);
  if (chunk >= chunks) return;
  const int32_t s = wave_row_state(states, slots, pending, num_pending, r, lane);
  const bool live = s >= 0 && s < num_states;
  if (s >= num_states && err && lane == 0 && chunk == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
  const int64_t c0 = int64_t(chunk) * kChunkCols;
  const bool tail = c0 + kChunkCols > vocab;
  const int64_t lim = vocab - c0 - lane;  // columns left for this lane
  T* p = reinterpret_cast<T*>(logits + int64_t(r) * ld_bytes) + c0 + lane;
  const T f = T(fill);
  if (Bits) {
    const uint32_t* bw = static_cast<const uint32_t*>(table);
    const int64_t w = c0 / 32 + lane;
    const uint32_t mine = (live && w < table_ld) ? bw[int64_t(s) * table_ld + w] : 0u;
    const uint32_t lanebit = 1u << (lane & 31);
#pragma unroll
    for (int j = 0; j < kFillGroups; ++j) {
      const uint32_t lo = __builtin_amdgcn_readlane(mine, 2 * j);
      const uint32_t hi = __builtin_amdgcn_readlane(mine, 2 * j + 1);
      const uint32_t word = lane < 32 ? lo : hi;
      const int c = j * 64;
      if (!(word & lanebit) && (!tail || c < lim)) p[c] = f;
    }
  } else {
    const int32_t* tn = static_cast<const int32_t*>(table) + (live ? int64_t(s) * table_ld : 0) + c0 + lane;
    int32_t v[kFillGroups];
#pragma unroll
    for (int j = 0; j < kFillGroups; ++j) v[j] = (live && (!tail || j * 64 < lim)) ? tn[j * 64] : -1;
#pragma unroll
    for (int j = 0; j < kFillGroups; ++j) {
      const int c = j * 64;
      if (v[j] == -1 && (!tail || c < lim)) p[c] = f;
    }
  }
}

// Token id of row b: int32, int64, or int64 read as its low 32 bits (what
// tensor.to(torch.int32) keeps); a negative id indexes from the end, as
// torch advanced indexing does.  False when the id is out of range.
__device__ __forceinline__ int32_t row_state(const int32_t* __restrict__ states,
                                             const int64_t* __restrict__ slots, int64_t r) {
  return states[slots ? slots[r] : r];
}

__device__ __forceinline__ bool token_index(const void* tokens, int tok_dtype, int64_t b,
                                            int64_t vocab, int64_t* out) {
  int64_t t = read_token(tokens, tok_dtype, b);
  if (t < 0) t += vocab;
  *out = t;
  return t >= 0 && t < vocab;
}

__device__ __forceinline__ int32_t advance_one(const int32_t* __restrict__ tok_next,
                                               int32_t num_states, int64_t vocab, int32_t s,
                                               const void* tokens, int tok_dtype, int64_t b,
                                               int32_t* __restrict__ err) {
  int64_t t;
  const bool t_ok = token_index(tokens, tok_dtype, b, vocab, &t);
  if (!t_ok) {
    if (err) atomicOr(err, BPD_FLAG_TOKEN_RANGE);
    return -1;
  }
  if (s >= num_states) {
    if (err) atomicOr(err, BPD_FLAG_STATE_RANGE);
    return -1;
  }
  if (s < 0) return -1;
  return tok_next[int64_t(s) * vocab + t];
}

// advance_one with the token id already read (raw: negative ids index from
// the end)
__device__ __forceinline__ int32_t advance_tok(const int32_t* __restrict__ tok_next, int32_t num_states,
                                               int64_t vocab, int32_t s, int64_t t, int32_t* __restrict__ err) {
  if (t < 0) t += vocab;
  if (t < 0 || t >= vocab) {
    if (err) atomicOr(err, BPD_FLAG_TOKEN_RANGE);
    return -1;
  }
  if (s >= num_states) {
    if (err) atomicOr(err, BPD_FLAG_STATE_RANGE);
    return -1;
  }
  if (s < 0) return -1;
  return tok_next[int64_t(s) * vocab + t];
}

constexpr int kAdvThreads = 1024;
constexpr int kAdvPerThread = 4;

// rows <= kAdvThreads * kAdvPerThread: one block.  The queued pool writes are
// staged in LDS.  Every pool read happens before the second barrier, the
// queued writes land between the second and third and the rows' write-backs
// after the third -- the order of the calls: the queued writes were made
// before the commit, and a row reads the queued value of its slot.
__global__ __launch_bounds__(kAdvThreads) void dense_advance_block_kernel(
    const int32_t* __restrict__ tok_next, int32_t num_states, int64_t vocab,
    int32_t* __restrict__ states, const int64_t* __restrict__ slots,
    const int64_t* __restrict__ pending, int32_t num_pending, const void* __restrict__ tokens,
    int tok_dtype, int64_t rows, int32_t* __restrict__ next_out, int write_back,
    int32_t* __restrict__ err) {
  __shared__ int64_t pslot[BPD_MAX_FUSED_PENDING];
  __shared__ int32_t pval[BPD_MAX_FUSED_PENDING];
  // every load that does not need the queued writes is issued before they
  // are staged: each row's slot and token, then the slot's state (one chain
  // of two dependent loads beside the staging instead of after it)
  int64_t slot[kAdvPerThread], tk[kAdvPerThread];
#pragma unroll
  for (int i = 0; i < kAdvPerThread; ++i) {
    const int64_t b = int64_t(i) * kAdvThreads + threadIdx.x;
    slot[i] = b < rows ? (slots ? slots[b] : b) : -1;
    tk[i] = b < rows ? read_token(tokens, tok_dtype, b) : 0;
  }
  int32_t st[kAdvPerThread];
#pragma unroll
  for (int i = 0; i < kAdvPerThread; ++i) st[i] = slot[i] >= 0 ? states[slot[i]] : 0;
  for (int32_t i = threadIdx.x; i < num_pending; i += kAdvThreads) {
    pslot[i] = pending[i];
    pval[i] = int32_t(pending[num_pending + i]);
  }
  __syncthreads();
  int32_t nxt[kAdvPerThread];
#pragma unroll
  for (int i = 0; i < kAdvPerThread; ++i) {
    const int64_t b = int64_t(i) * kAdvThreads + threadIdx.x;
    nxt[i] = -1;
    if (b < rows) {
      int32_t s = st[i];
      for (int32_t k = 0; k < num_pending; ++k)
        if (pslot[k] == slot[i]) s = pval[k];
      nxt[i] = advance_tok(tok_next, num_states, vocab, s, tk[i], err);
      if (next_out) next_out[b] = nxt[i];
    }
  }
  __syncthreads();
  for (int32_t i = threadIdx.x; i < num_pending; i += kAdvThreads) states[pslot[i]] = pval[i];
  if (!write_back) return;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kAdvPerThread; ++i)
    if (slot[i] >= 0) states[slot[i]] = nxt[i];
}

__global__ void dense_advance_gather_kernel(const int32_t* __restrict__ tok_next,
                                            int32_t num_states, int64_t vocab,
                                            const int32_t* __restrict__ states,
                                            const int64_t* __restrict__ slots,
                                            const void* __restrict__ tokens, int tok_dtype,
                                            int64_t rows, int32_t* __restrict__ next_out,
                                            int32_t* __restrict__ err) {
  const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= rows) return;
  const int64_t slot = slots ? slots[b] : b;
  next_out[b] = advance_one(tok_next, num_states, vocab, states[slot], tokens, tok_dtype, b, err);
}

__global__ void dense_scatter_kernel(int32_t* __restrict__ states, const int64_t* __restrict__ slots,
                                     const int32_t* __restrict__ next, int64_t rows) {
  const int64_t b = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (b >= rows) return;
  states[slots ? slots[b] : b] = next[b];
}

// One thread per token; each wave64 packs its 64 verdicts with a ballot into
// two consecutive uint32 words (LSB-first), written by lane 0.
__global__ __launch_bounds__(256) void dense_bits_kernel(
    const int32_t* __restrict__ tok_next, int32_t num_states, int64_t vocab,
    const int32_t* __restrict__ states, const int64_t* __restrict__ slots, int64_t rows,
    uint32_t* __restrict__ bits, int64_t words, int32_t* __restrict__ err) {
  const int64_t r = blockIdx.y;
  if (r >= rows) return;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int32_t s = row_state(states, slots, r);
  const bool live_row = s >= 0 && s < num_states;
  if (s >= num_states && err && t == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
  const bool allowed = live_row && t < vocab && tok_next[int64_t(s) * vocab + t] != -1;
  const uint64_t m = __ballot(allowed);
  if ((threadIdx.x & 63) == 0) {
    const int64_t w0 = t >> 5;
    if (w0 < words) bits[r * words + w0] = uint32_t(m);
    if (w0 + 1 < words) bits[r * words + w0 + 1] = uint32_t(m >> 32);
  }
}

// tok_next builder: one thread per (row, token); walks the token's symbol
// classes through the dense symbol-class table.
__global__ __launch_bounds__(256) void build_tok_next_kernel(
    const int32_t* __restrict__ trans, int32_t num_states, int32_t num_symbols, int32_t dead,
    const uint8_t* __restrict__ accept, const uint8_t* __restrict__ live,
    const int32_t* __restrict__ offsets, const uint8_t* __restrict__ syms, int64_t vocab,
    int32_t eos_id, const int32_t* __restrict__ row_states, int32_t num_rows,
    int32_t* __restrict__ out) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int32_t r = blockIdx.y;
  if (t >= vocab || r >= num_rows) return;
  const int32_t s0 = row_states ? row_states[r] : r;
  int32_t res = -1;
  if (s0 < 0 || s0 >= num_states) {
    res = -1;
  } else if (t == eos_id) {
    res = accept[s0] ? s0 : -1;
  } else {
    int32_t cur = s0;
    const int32_t b = offsets[t], e = offsets[t + 1];
    bool ok = true;
    for (int32_t i = b; i < e && cur != dead; ++i) {
      const int32_t k = syms[i];
      if (k >= num_symbols) {
        ok = false;
        break;
      }
      cur = trans[int64_t(cur) * num_symbols + k];
      if (cur < 0 || cur >= num_states) {
        ok = false;
        break;
      }
    }
    res = (ok && live[cur]) ? cur : -1;
  }
  out[int64_t(r) * vocab + t] = res;
}

// Reachability (the live set of a DFA): live[s] = 1 iff an accepting state
// is reachable from s.  One workgroup sweeps the states in place over LDS
// flags until a sweep changes nothing (monotone, so at most num_states + 1
// sweeps); the flag is read by every thread between two barriers, so every
// wave takes the same exit.
constexpr int kReachThreads = 1024;
constexpr int kReachMaxStates = 65536;  // LDS flags

__global__ __launch_bounds__(kReachThreads) void reachability_kernel(
    const int32_t* __restrict__ trans, int32_t num_states, int32_t num_symbols,
    const uint8_t* __restrict__ accept, uint8_t* __restrict__ live_out) {
  __shared__ uint8_t live[kReachMaxStates];
  __shared__ int changed;
  const int tid = threadIdx.x;
  for (int32_t s = tid; s < num_states; s += kReachThreads) live[s] = accept[s] ? 1 : 0;
  for (int32_t sweep = 0; sweep <= num_states; ++sweep) {
    if (tid == 0) changed = 0;
    __syncthreads();
    for (int32_t s = tid; s < num_states; s += kReachThreads) {
      if (live[s]) continue;
      const int32_t* row = trans + int64_t(s) * num_symbols;
      for (int32_t k = 0; k < num_symbols; ++k) {
        const int32_t t = row[k];
        if (t >= 0 && t < num_states && live[t]) {
          live[s] = 1;
          changed = 1;
          break;
        }
      }
    }
    __syncthreads();
    const int more = changed;
    __syncthreads();  // every thread has read the flag before it is reset
    if (!more) break;
  }
  for (int32_t s = tid; s < num_states; s += kReachThreads) live_out[s] = live[s];
}

}  // namespace
}  // namespace bpd

using namespace bpd;

namespace {

// Shared launch of the write-only mask (both table forms).
int launch_fill(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld, const void* table,
                int64_t table_ld, bool bits, int32_t num_states, int32_t* states,
                const int64_t* slots, const int64_t* pending, int64_t num_pending, double neg_inf,
                int32_t* err, void* stream) {
  const int E = dense_elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && vocab >= 0 && ld >= vocab, "bad logits shape rows=%lld vocab=%lld ld=%lld",
              (long long)rows, (long long)vocab, (long long)ld);
  BPD_REQUIRE(num_states > 0, "empty grammar table");
  BPD_REQUIRE(num_pending >= 0 && num_pending <= BPD_MAX_FUSED_PENDING,
              "at most %d queued pool writes per launch (got %lld)", BPD_MAX_FUSED_PENDING,
              (long long)num_pending);
  BPD_REQUIRE(num_pending == 0 || (pending && slots), "queued writes need a slot map");
  uint64_t fill = 0;
  if (int rc = fill_bits64(dtype, neg_inf, &fill)) return rc;
  BPD_REQUIRE(rows > 0 || num_pending == 0, "queued writes need at least one row");
  if (rows == 0) return BPD_OK;
  BPD_REQUIRE(logits && table && states, "null pointer argument");
  BPD_REQUIRE(reinterpret_cast<uintptr_t>(logits) % E == 0, "logits are not aligned to their element size");
  BPD_REQUIRE(rows < (int64_t(1) << 31), "too many rows for one launch");
  const int64_t chunks = vocab == 0 ? 1 : (vocab + kChunkCols - 1) / kChunkCols;
  int64_t blocks = (chunks + kFillWaves - 1) / kFillWaves * rows;
  blocks = (blocks + kXcds - 1) / kXcds * kXcds;
  BPD_REQUIRE(blocks < (int64_t(1) << 31), "batch too large for one launch");
  hipStream_t s = as_stream(stream);
  uint8_t* lg = static_cast<uint8_t*>(logits);
  const int32_t np = int32_t(num_pending);
#define BPD_FILL(EB, BITS)                                                                      \
  dense_fill_kernel<EB, BITS><<<dim3(unsigned(blocks)), dim3(kFillThreads), 0, s>>>(            \
      lg, ld * EB, table, table_ld, vocab, num_states, states, slots, pending, np,              \
      uint32_t(rows), uint32_t(chunks), fill, err)
  if (bits) {
    if (E == 2) BPD_FILL(2, true);
    else if (E == 4) BPD_FILL(4, true);
    else BPD_FILL(8, true);
  } else {
    if (E == 2) BPD_FILL(2, false);
    else if (E == 4) BPD_FILL(4, false);
    else BPD_FILL(8, false);
  }
#undef BPD_FILL
  BPD_LAUNCHED();
  return BPD_OK;
}

}  // namespace

extern "C" int bpd_dense_apply_mask(void* logits, int dtype, int64_t rows, int64_t vocab,
                                    int64_t ld, const int32_t* tok_next, int32_t num_states,
                                    int32_t* states, const int64_t* slots,
                                    const int64_t* pending, int64_t num_pending, double neg_inf,
                                    int32_t* err, void* stream) {
  return launch_fill(logits, dtype, rows, vocab, ld, tok_next, vocab, false, num_states, states,
                     slots, pending, num_pending, neg_inf, err, stream);
}

extern "C" int bpd_dense_apply_mask_bits(void* logits, int dtype, int64_t rows, int64_t vocab,
                                         int64_t ld, const uint32_t* allow_bits, int64_t words,
                                         int32_t num_states, int32_t* states,
                                         const int64_t* slots, const int64_t* pending,
                                         int64_t num_pending, double neg_inf, int32_t* err,
                                         void* stream) {
  BPD_REQUIRE(words == (vocab + 31) / 32, "allow-bit rows must hold ceil(vocab/32) words");
  return launch_fill(logits, dtype, rows, vocab, ld, allow_bits, words, true, num_states, states,
                     slots, pending, num_pending, neg_inf, err, stream);
}

extern "C" int bpd_dense_advance(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                                 int32_t* states, const int64_t* slots, const int64_t* pending,
                                 int64_t num_pending, const void* tokens, int token_dtype,
                                 int64_t rows, int32_t* next_out, int write_back, int32_t* err,
                                 void* stream) {
  BPD_REQUIRE(token_dtype_ok(token_dtype), "unknown token dtype code %d", token_dtype);
  BPD_REQUIRE(num_states > 0 && vocab > 0, "empty tok_next table");
  BPD_REQUIRE(rows >= 0, "negative row count");
  BPD_REQUIRE(num_pending >= 0 && num_pending <= BPD_MAX_FUSED_PENDING,
              "at most %d queued pool writes per launch (got %lld)", BPD_MAX_FUSED_PENDING,
              (long long)num_pending);
  BPD_REQUIRE(num_pending == 0 || (pending && slots && write_back),
              "queued writes need a slot map and write_back");
  BPD_REQUIRE(rows > 0 || num_pending == 0, "queued writes need at least one row");
  if (rows == 0) return BPD_OK;
  BPD_REQUIRE(tok_next && states && tokens, "null pointer argument");
  BPD_REQUIRE(next_out || write_back, "advance with neither next_out nor write_back");
  hipStream_t s = as_stream(stream);
  if (rows <= int64_t(kAdvThreads) * kAdvPerThread) {
    dense_advance_block_kernel<<<1, kAdvThreads, 0, s>>>(tok_next, num_states, vocab, states,
                                                         slots, pending, int32_t(num_pending),
                                                         tokens, token_dtype, rows, next_out,
                                                         write_back, err);
    BPD_LAUNCHED();
    return BPD_OK;
  }
  BPD_REQUIRE(next_out, "batches above %d rows need next_out", kAdvThreads * kAdvPerThread);
  BPD_REQUIRE(num_pending == 0, "batches above %d rows take no queued writes",
              kAdvThreads * kAdvPerThread);
  const unsigned g = unsigned((rows + 255) / 256);
  dense_advance_gather_kernel<<<g, 256, 0, s>>>(tok_next, num_states, vocab, states, slots,
                                                tokens, token_dtype, rows, next_out, err);
  BPD_LAUNCHED();
  if (write_back) {
    dense_scatter_kernel<<<g, 256, 0, s>>>(states, slots, next_out, rows);
    BPD_LAUNCHED();
  }
  return BPD_OK;
}

extern "C" int bpd_dense_compute_mask(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                                      const int32_t* states, const int64_t* slots, int64_t rows,
                                      uint32_t* bits, int32_t* err, void* stream) {
  BPD_REQUIRE(num_states > 0 && vocab >= 0 && rows >= 0, "bad shape");
  const int64_t words = (vocab + 31) / 32;
  if (rows == 0 || words == 0) return BPD_OK;
  BPD_REQUIRE(rows < 65536, "at most 65535 rows");
  BPD_REQUIRE(tok_next && states && bits, "null pointer argument");
  const dim3 grid = dim3(unsigned((vocab + 255) / 256), unsigned(rows));
  dense_bits_kernel<<<grid, 256, 0, as_stream(stream)>>>(tok_next, num_states, vocab, states,
                                                          slots, rows, bits, words, err);
  BPD_LAUNCHED();
  return BPD_OK;
}

extern "C" int bpd_build_tok_next(const int32_t* trans, int32_t num_states, int32_t num_symbols,
                                  int32_t dead, const uint8_t* accept, const uint8_t* live,
                                  const int32_t* tok_offsets, const uint8_t* tok_symbols,
                                  int64_t vocab, int32_t eos_id, const int32_t* row_states,
                                  int32_t num_rows, int32_t* out, void* stream) {
  BPD_REQUIRE(num_states > 0 && num_symbols > 0 && vocab >= 0 && num_rows >= 0, "bad shape");
  BPD_REQUIRE(dead >= 0 && dead < num_states, "dead state out of range");
  if (vocab == 0 || num_rows == 0) return BPD_OK;
  BPD_REQUIRE(num_rows < 65536, "at most 65535 table rows per launch");
  const dim3 grid = dim3(unsigned((vocab + 255) / 256), unsigned(num_rows));
  build_tok_next_kernel<<<grid, 256, 0, as_stream(stream)>>>(
      trans, num_states, num_symbols, dead, accept, live, tok_offsets, tok_symbols, vocab,
      eos_id, row_states, num_rows, out);
  BPD_LAUNCHED();
  return BPD_OK;
}

extern "C" int bpd_build_reachability(const int32_t* trans, int32_t num_states, int32_t num_symbols,
                                      const uint8_t* accept, uint8_t* live, void* stream) {
  BPD_REQUIRE(num_states >= 0 && num_symbols > 0, "bad table shape");
  BPD_REQUIRE(num_states <= kReachMaxStates, "at most %d states on the device", kReachMaxStates);
  if (num_states == 0) return BPD_OK;
  BPD_REQUIRE(trans && accept && live, "null pointer argument");
  reachability_kernel<<<1, kReachThreads, 0, as_stream(stream)>>>(trans, num_states, num_symbols,
                                                                   accept, live);
  BPD_LAUNCHED();
  return BPD_OK;
}
