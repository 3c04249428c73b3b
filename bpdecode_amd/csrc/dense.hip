// Dense tok_next path for gfx950: gather+mask over a [rows, vocab] logits
// batch, the commit gather/scatter, the packed allow-bit mask, and the
// device-side table builder.
//
// apply_mask is HBM-bound integer work: per row it streams the logits row
// once (read + write, unit stride) and the int32 tok_next row of that row's
// state.  A 256-thread block owns a 2048-column slab of a few rows; each lane
// handles 8 consecutive columns with 16-byte vector accesses, issuing all
// loads of its rows before any store.  Blocks are numbered so that all
// row-slabs of one column slab run on the same XCD (workgroups are dealt
// round-robin to the 8 XCDs), so each (state, column slab) tile of the table
// is fetched from HBM into one L2 and re-read from there by the other rows in
// that state.
//
// The mask only needs "tok_next[s, t] != -1", so the serving path masks from
// a packed allow-bit table (1 bit per (state, token), LSB-first uint32 words,
// built once per grammar from tok_next by the bit kernel below): a lane's 8
// verdicts are one byte, and table traffic drops 32x against the int32 rows.
// Measured on MI355X the logits stream then sets the pace; plain (temporal)
// global loads/stores beat non-temporal ones for this read-modify-write
// pattern.
#include <algorithm>

#include "bpd_common.hpp"

namespace bpd {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kVec = 8;                          // columns per lane
constexpr int64_t kSlab = int64_t(kThreads) * kVec;  // columns per block
constexpr int kRows = 2;                         // rows per block (int32 table)
// rows per block (bit table): 2, or 4 from 512 rows on, which keeps about
// 9,600 blocks at V = 151,936 (measured best at 256 and 512 rows)
constexpr int kBitRowsSmall = 2, kBitRowsLarge = 4, kBitRowsLargeFrom = 512;
constexpr int kXcds = 8;

__device__ __forceinline__ int32_t row_state(const int32_t* __restrict__ states,
                                             const int64_t* __restrict__ slots, int64_t r) {
  const int64_t slot = slots ? slots[r] : r;
  return states[slot];
}

// Block index -> (column slab, row slab) with all row slabs of a column slab
// on one XCD.  gridDim.x is a multiple of kXcds.
__device__ __forceinline__ uint32_t logical_block() {
  const uint32_t nb = gridDim.x;
  const uint32_t hw = blockIdx.x;
  return (hw % kXcds) * (nb / kXcds) + hw / kXcds;
}

// Replace the 2-byte lanes of `v` whose tok_next entry is -1.
__device__ __forceinline__ uint32_t pick16(uint32_t word, int32_t t0, int32_t t1, uint32_t fill) {
  const uint32_t lo = (t0 == -1) ? fill : (word & 0xFFFFu);
  const uint32_t hi = (t1 == -1) ? fill : (word >> 16);
  return lo | (hi << 16);
}

template <int E>
__global__ __launch_bounds__(kThreads) void dense_mask_vec_kernel(
    uint8_t* __restrict__ logits, int64_t ld_bytes, const int32_t* __restrict__ tok_next,
    int64_t vocab, int32_t num_states, const int32_t* __restrict__ states,
    const int64_t* __restrict__ slots, int64_t rows, uint32_t row_slabs, uint32_t col_slabs,
    uint32_t fill, int32_t* __restrict__ err) {
  const uint32_t lb = logical_block();
  const uint32_t cs = lb / row_slabs;
  const uint32_t rs = lb - cs * row_slabs;
  if (cs >= col_slabs) return;
  const int64_t col = int64_t(cs) * kSlab + int64_t(threadIdx.x) * kVec;
  if (col >= vocab) return;  // vocab % kVec == 0 on this path
  const int64_t r0 = int64_t(rs) * kRows;

  // Issue order: the logits loads (independent of the states) first, then
  // the slot and state lookups of all rows, then the tok_next loads.
  int32_t st[kRows];
  int64_t slot[kRows];
  u32x4 lg[kRows][E / 2];
  i32x4 tn[kRows][2];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int64_t r = r0 + i;
    if (r < rows) {
      const u32x4* p = reinterpret_cast<const u32x4*>(logits + r * ld_bytes + col * E);
#pragma unroll
      for (int k = 0; k < E / 2; ++k) lg[i][k] = p[k];
    }
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int64_t r = r0 + i;
    slot[i] = (r < rows) ? (slots ? slots[r] : r) : -1;
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) st[i] = (slot[i] >= 0) ? states[slot[i]] : -1;
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    if (st[i] >= 0 && st[i] < num_states) {
      const i32x4* q = reinterpret_cast<const i32x4*>(tok_next + int64_t(st[i]) * vocab + col);
      tn[i][0] = q[0];
      tn[i][1] = q[1];
    }
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int64_t r = r0 + i;
    if (r >= rows) break;
    u32x4* p = reinterpret_cast<u32x4*>(logits + r * ld_bytes + col * E);
    const int32_t s = st[i];
    if (s < 0 || s >= num_states) {
      if (s >= num_states && err && threadIdx.x == 0 && cs == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
      const u32x4 f = (E == 2) ? u32x4{fill | (fill << 16), fill | (fill << 16),
                                       fill | (fill << 16), fill | (fill << 16)}
                               : u32x4{fill, fill, fill, fill};
#pragma unroll
      for (int k = 0; k < E / 2; ++k) p[k] = f;
      continue;
    }
    if (E == 2) {
      u32x4 v = lg[i][0];
      v.x = pick16(v.x, tn[i][0].x, tn[i][0].y, fill);
      v.y = pick16(v.y, tn[i][0].z, tn[i][0].w, fill);
      v.z = pick16(v.z, tn[i][1].x, tn[i][1].y, fill);
      v.w = pick16(v.w, tn[i][1].z, tn[i][1].w, fill);
      *p = v;
    } else {
      u32x4 a = lg[i][0], b = lg[i][E / 2 - 1];
      a.x = tn[i][0].x == -1 ? fill : a.x;
      a.y = tn[i][0].y == -1 ? fill : a.y;
      a.z = tn[i][0].z == -1 ? fill : a.z;
      a.w = tn[i][0].w == -1 ? fill : a.w;
      b.x = tn[i][1].x == -1 ? fill : b.x;
      b.y = tn[i][1].y == -1 ? fill : b.y;
      b.z = tn[i][1].z == -1 ? fill : b.z;
      b.w = tn[i][1].w == -1 ? fill : b.w;
      p[0] = a;
      p[1] = b;
    }
  }
}

// Mask from the packed allow-bit table: byte (col / 8) of a state's bit row
// holds the verdicts of the lane's 8 columns.  The verdicts come first: a
// lane whose 8 columns are all rejected writes the fill without reading
// them, one whose columns are all allowed touches nothing, and only the
// mixed ones read, blend and write (the result is the same; on a DFA that
// allows a few percent of the vocab most logits are never read).
template <int E, int kBitRows>
__global__ __launch_bounds__(kThreads) void dense_mask_bits_kernel(
    uint8_t* __restrict__ logits, int64_t ld_bytes, const uint8_t* __restrict__ bits,
    int64_t row_bytes, int64_t vocab, int32_t num_states, const int32_t* __restrict__ states,
    const int64_t* __restrict__ slots, int64_t rows, uint32_t row_slabs, uint32_t col_slabs,
    uint32_t fill, int32_t* __restrict__ err) {
  const uint32_t lb = logical_block();
  const uint32_t cs = lb / row_slabs;
  const uint32_t rs = lb - cs * row_slabs;
  if (cs >= col_slabs) return;
  const int64_t col = int64_t(cs) * kSlab + int64_t(threadIdx.x) * kVec;
  if (col >= vocab) return;  // vocab % kVec == 0 on this path
  const int64_t r0 = int64_t(rs) * kBitRows;
  u32x4 lg[kBitRows][E / 2];
  int64_t slot[kBitRows];
  int32_t st[kBitRows];
  uint32_t m[kBitRows];
#pragma unroll
  for (int i = 0; i < kBitRows; ++i) {
    const int64_t r = r0 + i;
    slot[i] = (r < rows) ? (slots ? slots[r] : r) : -1;
  }
#pragma unroll
  for (int i = 0; i < kBitRows; ++i) st[i] = (slot[i] >= 0) ? states[slot[i]] : -1;
#pragma unroll
  for (int i = 0; i < kBitRows; ++i)
    m[i] = (st[i] >= 0 && st[i] < num_states) ? uint32_t(bits[int64_t(st[i]) * row_bytes + (col >> 3)]) : 0u;
#pragma unroll
  for (int i = 0; i < kBitRows; ++i) {
    const int64_t r = r0 + i;
    if (r < rows && m[i] != 0u && m[i] != 0xFFu) {
      const u32x4* p = reinterpret_cast<const u32x4*>(logits + r * ld_bytes + col * E);
#pragma unroll
      for (int k = 0; k < E / 2; ++k) lg[i][k] = p[k];
    }
  }
#pragma unroll
  for (int i = 0; i < kBitRows; ++i) {
    const int64_t r = r0 + i;
    if (r >= rows) break;
    if (st[i] >= num_states && err && threadIdx.x == 0 && cs == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
    const uint32_t mm = m[i];
    if (mm == 0xFFu) continue;
    u32x4* p = reinterpret_cast<u32x4*>(logits + r * ld_bytes + col * E);
    if (mm == 0u) {
      const u32x4 f = (E == 2) ? u32x4{fill | (fill << 16), fill | (fill << 16),
                                       fill | (fill << 16), fill | (fill << 16)}
                               : u32x4{fill, fill, fill, fill};
#pragma unroll
      for (int k = 0; k < E / 2; ++k) p[k] = f;
      continue;
    }
    if (E == 2) {
      u32x4 v = lg[i][0];
      v.x = ((mm & 1u) ? (v.x & 0xFFFFu) : fill) | (((mm & 2u) ? (v.x >> 16) : fill) << 16);
      v.y = ((mm & 4u) ? (v.y & 0xFFFFu) : fill) | (((mm & 8u) ? (v.y >> 16) : fill) << 16);
      v.z = ((mm & 16u) ? (v.z & 0xFFFFu) : fill) | (((mm & 32u) ? (v.z >> 16) : fill) << 16);
      v.w = ((mm & 64u) ? (v.w & 0xFFFFu) : fill) | (((mm & 128u) ? (v.w >> 16) : fill) << 16);
      *p = v;
    } else {
      u32x4 a = lg[i][0], b = lg[i][E / 2 - 1];
      a.x = (mm & 1u) ? a.x : fill;
      a.y = (mm & 2u) ? a.y : fill;
      a.z = (mm & 4u) ? a.z : fill;
      a.w = (mm & 8u) ? a.w : fill;
      b.x = (mm & 16u) ? b.x : fill;
      b.y = (mm & 32u) ? b.y : fill;
      b.z = (mm & 64u) ? b.z : fill;
      b.w = (mm & 128u) ? b.w : fill;
      p[0] = a;
      p[1] = b;
    }
  }
}

// Any alignment / vocab, bit table: one element per lane per step.
template <int E>
__global__ __launch_bounds__(kThreads) void dense_mask_bits_scalar_kernel(
    uint8_t* __restrict__ logits, int64_t ld_bytes, const uint32_t* __restrict__ bits,
    int64_t words, int64_t vocab, int32_t num_states, const int32_t* __restrict__ states,
    const int64_t* __restrict__ slots, int64_t rows, uint32_t fill, int32_t* __restrict__ err) {
  const int64_t r = blockIdx.y;
  if (r >= rows) return;
  const int32_t s = row_state(states, slots, r);
  const bool whole = s < 0 || s >= num_states;
  if (s >= num_states && err && threadIdx.x == 0 && blockIdx.x == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
  uint8_t* row = logits + r * ld_bytes;
  const uint32_t* bw = bits + (whole ? 0 : int64_t(s) * words);
  for (int64_t t = int64_t(blockIdx.x) * kThreads + threadIdx.x; t < vocab;
       t += int64_t(gridDim.x) * kThreads) {
    if (whole || !((bw[t >> 5] >> (t & 31)) & 1u)) {
      if (E == 2)
        *reinterpret_cast<uint16_t*>(row + t * 2) = static_cast<uint16_t>(fill);
      else
        *reinterpret_cast<uint32_t*>(row + t * 4) = fill;
    }
  }
}

// Any alignment / vocab: one element per lane per step, grid-stride over the
// columns of each row.
template <int E>
__global__ __launch_bounds__(kThreads) void dense_mask_scalar_kernel(
    uint8_t* __restrict__ logits, int64_t ld_bytes, const int32_t* __restrict__ tok_next,
    int64_t vocab, int32_t num_states, const int32_t* __restrict__ states,
    const int64_t* __restrict__ slots, int64_t rows, uint32_t fill, int32_t* __restrict__ err) {
  const int64_t r = blockIdx.y;
  if (r >= rows) return;
  const int32_t s = row_state(states, slots, r);
  const bool whole = s < 0 || s >= num_states;
  if (s >= num_states && err && threadIdx.x == 0 && blockIdx.x == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
  uint8_t* row = logits + r * ld_bytes;
  const int32_t* tn = tok_next + (whole ? 0 : int64_t(s) * vocab);
  for (int64_t t = int64_t(blockIdx.x) * kThreads + threadIdx.x; t < vocab;
       t += int64_t(gridDim.x) * kThreads) {
    if (whole || tn[t] == -1) {
      if (E == 2)
        *reinterpret_cast<uint16_t*>(row + t * 2) = static_cast<uint16_t>(fill);
      else
        *reinterpret_cast<uint32_t*>(row + t * 4) = fill;
    }
  }
}

__device__ __forceinline__ bool token_index(const void* tokens, int tok_dtype, int64_t b,
                                            int64_t vocab, int64_t* out) {
  int64_t t = (tok_dtype == BPD_INDEX_I64)
                  ? int64_t(int32_t(reinterpret_cast<const int64_t*>(tokens)[b]))
                  : int64_t(reinterpret_cast<const int32_t*>(tokens)[b]);
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

constexpr int kAdvThreads = 1024;
constexpr int kAdvPerThread = 4;

// rows <= kAdvThreads * kAdvPerThread: one block; every pool read happens
// before the barrier, every write-back after it.
__global__ __launch_bounds__(kAdvThreads) void dense_advance_block_kernel(
    const int32_t* __restrict__ tok_next, int32_t num_states, int64_t vocab,
    int32_t* __restrict__ states, const int64_t* __restrict__ slots,
    const void* __restrict__ tokens, int tok_dtype, int64_t rows, int32_t* __restrict__ next_out,
    int write_back, int32_t* __restrict__ err) {
  int32_t nxt[kAdvPerThread];
  int64_t slot[kAdvPerThread];
#pragma unroll
  for (int i = 0; i < kAdvPerThread; ++i) {
    const int64_t b = int64_t(i) * kAdvThreads + threadIdx.x;
    nxt[i] = -1;
    slot[i] = -1;
    if (b < rows) {
      slot[i] = slots ? slots[b] : b;
      nxt[i] = advance_one(tok_next, num_states, vocab, states[slot[i]], tokens, tok_dtype, b, err);
      if (next_out) next_out[b] = nxt[i];
    }
  }
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

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" int bpd_dense_apply_mask(void* logits, int dtype, int64_t rows, int64_t vocab,
                                    int64_t ld, const int32_t* tok_next, int32_t num_states,
                                    const int32_t* states, const int64_t* slots, double neg_inf,
                                    int32_t* err, void* stream) {
  const int E = elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && vocab >= 0 && ld >= vocab, "bad logits shape rows=%lld vocab=%lld ld=%lld",
              (long long)rows, (long long)vocab, (long long)ld);
  BPD_REQUIRE(num_states > 0, "empty tok_next table");
  uint32_t fill = 0;
  if (int rc = fill_bits(dtype, neg_inf, &fill)) return rc;
  if (rows == 0 || vocab == 0) return BPD_OK;
  BPD_REQUIRE(logits && tok_next && states, "null pointer argument");
  hipStream_t s = as_stream(stream);
  const int64_t ld_bytes = ld * E;
  const bool aligned = (vocab % kVec == 0) && (ld_bytes % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(logits) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(tok_next) % 16 == 0);
  if (aligned) {
    const int64_t col_slabs = (vocab + kSlab - 1) / kSlab;
    const int64_t row_slabs = (rows + kRows - 1) / kRows;
    int64_t blocks = col_slabs * row_slabs;
    blocks = (blocks + kXcds - 1) / kXcds * kXcds;
    BPD_REQUIRE(blocks < (int64_t(1) << 31), "batch too large for one launch");
    if (E == 2)
      dense_mask_vec_kernel<2><<<dim3(unsigned(blocks)), dim3(kThreads), 0, s>>>(
          static_cast<uint8_t*>(logits), ld_bytes, tok_next, vocab, num_states, states, slots,
          rows, uint32_t(row_slabs), uint32_t(col_slabs), fill, err);
    else
      dense_mask_vec_kernel<4><<<dim3(unsigned(blocks)), dim3(kThreads), 0, s>>>(
          static_cast<uint8_t*>(logits), ld_bytes, tok_next, vocab, num_states, states, slots,
          rows, uint32_t(row_slabs), uint32_t(col_slabs), fill, err);
  } else {
    BPD_REQUIRE(rows < 65536, "unaligned path supports at most 65535 rows");
    const int64_t gx = std::min<int64_t>((vocab + kThreads - 1) / kThreads, 1024);
    const dim3 grid = dim3(unsigned(gx), unsigned(rows));
    if (E == 2)
      dense_mask_scalar_kernel<2><<<grid, dim3(kThreads), 0, s>>>(
          static_cast<uint8_t*>(logits), ld_bytes, tok_next, vocab, num_states, states, slots,
          rows, fill, err);
    else
      dense_mask_scalar_kernel<4><<<grid, dim3(kThreads), 0, s>>>(
          static_cast<uint8_t*>(logits), ld_bytes, tok_next, vocab, num_states, states, slots,
          rows, fill, err);
  }
  BPD_LAUNCHED();
  return BPD_OK;
}

extern "C" int bpd_dense_advance(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                                 int32_t* states, const int64_t* slots, const void* tokens,
                                 int token_dtype, int64_t rows, int32_t* next_out,
                                 int write_back, int32_t* err, void* stream) {
  BPD_REQUIRE(token_dtype == BPD_INDEX_I32 || token_dtype == BPD_INDEX_I64,
              "unknown token dtype code %d", token_dtype);
  BPD_REQUIRE(num_states > 0 && vocab > 0, "empty tok_next table");
  BPD_REQUIRE(rows >= 0, "negative row count");
  if (rows == 0) return BPD_OK;
  BPD_REQUIRE(tok_next && states && tokens, "null pointer argument");
  BPD_REQUIRE(next_out || write_back, "advance with neither next_out nor write_back");
  hipStream_t s = as_stream(stream);
  if (rows <= int64_t(kAdvThreads) * kAdvPerThread) {
    dense_advance_block_kernel<<<1, kAdvThreads, 0, s>>>(tok_next, num_states, vocab, states,
                                                         slots, tokens, token_dtype, rows,
                                                         next_out, write_back, err);
    BPD_LAUNCHED();
    return BPD_OK;
  }
  BPD_REQUIRE(next_out, "batches above %d rows need next_out", kAdvThreads * kAdvPerThread);
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

extern "C" int bpd_dense_apply_mask_bits(void* logits, int dtype, int64_t rows, int64_t vocab,
                                         int64_t ld, const uint32_t* allow_bits, int64_t words,
                                         int32_t num_states, const int32_t* states,
                                         const int64_t* slots, double neg_inf, int32_t* err,
                                         void* stream) {
  const int E = elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && vocab >= 0 && ld >= vocab, "bad logits shape rows=%lld vocab=%lld ld=%lld",
              (long long)rows, (long long)vocab, (long long)ld);
  BPD_REQUIRE(num_states > 0, "empty allow-bit table");
  BPD_REQUIRE(words == (vocab + 31) / 32, "allow-bit rows must hold ceil(vocab/32) words");
  uint32_t fill = 0;
  if (int rc = fill_bits(dtype, neg_inf, &fill)) return rc;
  if (rows == 0 || vocab == 0) return BPD_OK;
  BPD_REQUIRE(logits && allow_bits && states, "null pointer argument");
  hipStream_t s = as_stream(stream);
  const int64_t ld_bytes = ld * E;
  const bool aligned = (vocab % kVec == 0) && (ld_bytes % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(logits) % 16 == 0);
  if (aligned) {
    const int64_t col_slabs = (vocab + kSlab - 1) / kSlab;
    const int R = rows >= kBitRowsLargeFrom ? kBitRowsLarge : kBitRowsSmall;
    const int64_t row_slabs = (rows + R - 1) / R;
    int64_t blocks = col_slabs * row_slabs;
    blocks = (blocks + kXcds - 1) / kXcds * kXcds;
    BPD_REQUIRE(blocks < (int64_t(1) << 31), "batch too large for one launch");
    const uint8_t* b8 = reinterpret_cast<const uint8_t*>(allow_bits);
#define BPD_MASK_BITS(EB, RB)                                                                     \
  dense_mask_bits_kernel<EB, RB><<<dim3(unsigned(blocks)), dim3(kThreads), 0, s>>>(              \
      static_cast<uint8_t*>(logits), ld_bytes, b8, words * 4, vocab, num_states, states, slots,  \
      rows, uint32_t(row_slabs), uint32_t(col_slabs), fill, err)
    if (E == 2 && R == kBitRowsSmall) BPD_MASK_BITS(2, kBitRowsSmall);
    else if (E == 2) BPD_MASK_BITS(2, kBitRowsLarge);
    else if (R == kBitRowsSmall) BPD_MASK_BITS(4, kBitRowsSmall);
    else BPD_MASK_BITS(4, kBitRowsLarge);
#undef BPD_MASK_BITS
  } else {
    BPD_REQUIRE(rows < 65536, "unaligned path supports at most 65535 rows");
    const int64_t gx = std::min<int64_t>((vocab + kThreads - 1) / kThreads, 1024);
    const dim3 grid = dim3(unsigned(gx), unsigned(rows));
    if (E == 2)
      dense_mask_bits_scalar_kernel<2><<<grid, dim3(kThreads), 0, s>>>(
          static_cast<uint8_t*>(logits), ld_bytes, allow_bits, words, vocab, num_states, states,
          slots, rows, fill, err);
    else
      dense_mask_bits_scalar_kernel<4><<<grid, dim3(kThreads), 0, s>>>(
          static_cast<uint8_t*>(logits), ld_bytes, allow_bits, words, vocab, num_states, states,
          slots, rows, fill, err);
  }
  BPD_LAUNCHED();
  return BPD_OK;
}
