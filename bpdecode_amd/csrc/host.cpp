// Host side of libbpdecode_hip: error state and the CPU-tensor forms of the
// dense entry points.  Same contracts as the device entry points in
// dense.hip; they run on the calling thread.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>
#include <thread>
#include <vector>

#include "bpd_common.hpp"

namespace bpd {
namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

namespace {

inline int64_t host_token(const void* tokens, int dtype, int64_t b) {
  return read_token(tokens, dtype, b);
}

// One row's mask: a select per element (rejected -> fill, else the element
// itself), with no branch in the loop so the compiler vectorises it.
// Work units of the host masks: a span of kHostSpan columns of one row.
constexpr int64_t kHostElemsPerWorker = int64_t(1) << 20;
constexpr int64_t kHostSpan = int64_t(1) << 13;

template <typename T>
void mask_span(T* __restrict__ row, const int32_t* __restrict__ tn, int64_t n, const T fill) {
  for (int64_t t = 0; t < n; ++t) row[t] = tn[t] == -1 ? fill : row[t];
}

// Runs task(k) for k in [0, tasks) on the calling thread, or spread over up
// to 16 host threads, one per kHostElemsPerWorker elements of the batch (a
// thread costs tens of microseconds to start, more while torch's own pool
// still spins after an operator, so small batches stay on the caller).
template <typename F>
void for_tasks(int64_t tasks, int64_t elems, F&& task) {
  // hardware_concurrency reads a sysfs file: asked once per process
  static const unsigned hw = std::thread::hardware_concurrency();
  const int64_t workers =
      std::min<int64_t>({hw ? int64_t(hw) : 1, 16, tasks, elems / kHostElemsPerWorker});
  if (workers <= 1) {
    for (int64_t k = 0; k < tasks; ++k) task(k);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(size_t(workers - 1));
  for (int64_t w = 1; w < workers; ++w)
    pool.emplace_back([&, w] {
      for (int64_t k = w; k < tasks; k += workers) task(k);
    });
  for (int64_t k = 0; k < tasks; k += workers) task(k);  // the calling thread takes a share
  for (auto& th : pool) th.join();
}

template <typename T>
void mask_rows(T* logits, int64_t rows, int64_t vocab, int64_t ld, const int32_t* tok_next,
               const int32_t* states, const int64_t* slots, T fill) {
  const int64_t spans = vocab == 0 ? 0 : (vocab + kHostSpan - 1) / kHostSpan;
  for_tasks(rows * spans, rows * vocab, [=](int64_t task) {
    const int64_t b = task / spans, c0 = (task - b * spans) * kHostSpan;
    const int64_t n = std::min(kHostSpan, vocab - c0);
    const int32_t s = states[slots ? slots[b] : b];
    T* row = logits + b * ld + c0;
    if (s < 0)
      std::fill(row, row + n, fill);
    else
      mask_span(row, tok_next + int64_t(s) * vocab + c0, n, fill);
  });
}

// The same mask from the packed allow bits over columns [c0, c1) of one row:
// a word with no allowed token is 32 plain fill stores (its logits are not
// read), a word with all allowed is skipped, a mixed word keeps its few
// allowed elements aside around a fill or fills its few rejected ones.
// Arguments by value and restrict pointers, so the fill loops vectorise.
template <typename T>
void mask_span_bits(T* __restrict__ row, const uint32_t* __restrict__ rb, int64_t c0, int64_t c1,
                    const T fill) {
  for (int64_t w = c0 >> 5; w << 5 < c1; ++w) {
    const uint32_t m = rb[w];
    T* __restrict__ p = row + (w << 5);
    const int n = int(std::min<int64_t>(32, c1 - (w << 5)));
    if (n < 32) {
      for (int i = 0; i < n; ++i) p[i] = ((m >> i) & 1u) ? p[i] : fill;
    } else if (m == 0u) {
      for (int i = 0; i < 32; ++i) p[i] = fill;
    } else if (m == 0xFFFFFFFFu) {
      continue;
    } else if (__builtin_popcount(m) <= 16) {
      T keep[32];
      for (uint32_t r = m; r; r &= r - 1) keep[__builtin_ctz(r)] = p[__builtin_ctz(r)];
      for (int i = 0; i < 32; ++i) p[i] = fill;
      for (uint32_t r = m; r; r &= r - 1) p[__builtin_ctz(r)] = keep[__builtin_ctz(r)];
    } else {
      for (uint32_t r = ~m; r; r &= r - 1) p[__builtin_ctz(r)] = fill;
    }
  }
}

template <typename T>
void mask_rows_bits(T* logits, int64_t rows, int64_t vocab, int64_t ld, const uint32_t* bits,
                    int64_t words, const int32_t* states, const int64_t* slots, T fill) {
  const int64_t spans = vocab == 0 ? 0 : (vocab + kHostSpan - 1) / kHostSpan;
  for_tasks(rows * spans, rows * vocab, [=](int64_t task) {
    const int64_t b = task / spans, c0 = (task - b * spans) * kHostSpan;
    const int64_t c1 = std::min(c0 + kHostSpan, vocab);
    const int32_t s = states[slots ? slots[b] : b];
    if (s < 0)
      std::fill(logits + b * ld + c0, logits + b * ld + c1, fill);
    else
      mask_span_bits(logits + b * ld, bits + int64_t(s) * words, c0, c1, fill);
  });
}

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" const char* bpd_last_error(void) { return g_error; }

extern "C" int bpd_abi_version(void) { return 9; }

extern "C" int bpd_host_dense_apply_mask(void* logits, int dtype, int64_t rows, int64_t vocab,
                                         int64_t ld, const int32_t* tok_next,
                                         int32_t num_states, const int32_t* states,
                                         const int64_t* slots, double neg_inf) {
  const int E = dense_elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && vocab >= 0 && ld >= vocab, "bad logits shape");
  BPD_REQUIRE(num_states > 0, "empty tok_next table");
  uint64_t fill = 0;
  if (int rc = fill_bits64(dtype, neg_inf, &fill)) return rc;
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s = states[slots ? slots[b] : b];
    BPD_REQUIRE(s < num_states, "index %d is out of bounds for dimension 0 with size %d", s,
                num_states);
  }
  if (E == 8)
    mask_rows(static_cast<uint64_t*>(logits), rows, vocab, ld, tok_next, states, slots, fill);
  else if (E == 4)
    mask_rows(static_cast<uint32_t*>(logits), rows, vocab, ld, tok_next, states, slots,
              static_cast<uint32_t>(fill));
  else
    mask_rows(static_cast<uint16_t*>(logits), rows, vocab, ld, tok_next, states, slots,
              static_cast<uint16_t>(fill));
  return BPD_OK;
}

extern "C" int bpd_host_dense_apply_mask_bits(void* logits, int dtype, int64_t rows,
                                              int64_t vocab, int64_t ld,
                                              const uint32_t* allow_bits, int64_t words,
                                              int32_t num_states, const int32_t* states,
                                              const int64_t* slots, double neg_inf) {
  const int E = dense_elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && vocab >= 0 && ld >= vocab, "bad logits shape");
  BPD_REQUIRE(num_states > 0, "empty grammar table");
  BPD_REQUIRE(words == (vocab + 31) / 32, "allow-bit rows must hold ceil(vocab/32) words");
  uint64_t fill = 0;
  if (int rc = fill_bits64(dtype, neg_inf, &fill)) return rc;
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s = states[slots ? slots[b] : b];
    BPD_REQUIRE(s < num_states, "index %d is out of bounds for dimension 0 with size %d", s,
                num_states);
  }
  if (E == 8)
    mask_rows_bits(static_cast<uint64_t*>(logits), rows, vocab, ld, allow_bits, words, states,
                   slots, fill);
  else if (E == 4)
    mask_rows_bits(static_cast<uint32_t*>(logits), rows, vocab, ld, allow_bits, words, states,
                   slots, static_cast<uint32_t>(fill));
  else
    mask_rows_bits(static_cast<uint16_t*>(logits), rows, vocab, ld, allow_bits, words, states,
                   slots, static_cast<uint16_t>(fill));
  return BPD_OK;
}

extern "C" int bpd_host_dense_advance(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                                      int32_t* states, const int64_t* slots, const void* tokens,
                                      int token_dtype, int64_t rows, int32_t* next_out,
                                      int write_back) {
  BPD_REQUIRE(token_dtype_ok(token_dtype), "unknown token dtype code %d", token_dtype);
  BPD_REQUIRE(num_states > 0 && vocab > 0 && rows >= 0, "bad shape");
  BPD_REQUIRE(next_out || write_back, "advance with neither next_out nor write_back");
  // validate everything before any write, as an indexing error in the
  // reference raises before the state pool is touched
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s = states[slots ? slots[b] : b];
    BPD_REQUIRE(s < num_states, "index %d is out of bounds for dimension 0 with size %d", s,
                num_states);
    const int64_t t = host_token(tokens, token_dtype, b);
    BPD_REQUIRE(t >= -vocab && t < vocab,
                "index %lld is out of bounds for dimension 1 with size %lld", (long long)t,
                (long long)vocab);
  }
  int32_t* out = next_out;
  std::vector<int32_t> tmp;
  if (!out) {
    tmp.resize(size_t(rows));
    out = tmp.data();
  }
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s = states[slots ? slots[b] : b];
    int64_t t = host_token(tokens, token_dtype, b);
    if (t < 0) t += vocab;
    out[b] = s < 0 ? -1 : tok_next[int64_t(s) * vocab + t];
  }
  if (write_back)
    for (int64_t b = 0; b < rows; ++b) states[slots ? slots[b] : b] = out[b];
  return BPD_OK;
}

extern "C" int bpd_host_dense_compute_mask(const int32_t* tok_next, int32_t num_states,
                                           int64_t vocab, const int32_t* states,
                                           const int64_t* slots, int64_t rows, uint32_t* bits) {
  BPD_REQUIRE(num_states > 0 && vocab >= 0 && rows >= 0, "bad shape");
  const int64_t words = (vocab + 31) / 32;
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s = states[slots ? slots[b] : b];
    BPD_REQUIRE(s < num_states, "index %d is out of bounds for dimension 0 with size %d", s,
                num_states);
    uint32_t* row = bits + b * words;
    std::fill(row, row + words, 0u);
    if (s < 0) continue;
    const int32_t* tn = tok_next + int64_t(s) * vocab;
    for (int64_t t = 0; t < vocab; ++t)
      if (tn[t] != -1) row[t >> 5] |= 1u << (t & 31);
  }
  return BPD_OK;
}

extern "C" int bpd_host_build_tok_next(const int32_t* trans, int32_t num_states,
                                       int32_t num_symbols, int32_t dead, const uint8_t* accept,
                                       const uint8_t* live, const int32_t* tok_offsets,
                                       const uint8_t* tok_symbols, int64_t vocab, int32_t eos_id,
                                       const int32_t* row_states, int32_t num_rows,
                                       int32_t* out) {
  BPD_REQUIRE(num_states > 0 && num_symbols > 0 && vocab >= 0 && num_rows >= 0, "bad shape");
  BPD_REQUIRE(dead >= 0 && dead < num_states, "dead state out of range");
  for (int32_t r = 0; r < num_rows; ++r) {
    const int32_t s0 = row_states ? row_states[r] : r;
    BPD_REQUIRE(s0 >= 0 && s0 < num_states, "row state %d out of range", s0);
    int32_t* o = out + int64_t(r) * vocab;
    for (int64_t t = 0; t < vocab; ++t) {
      int32_t cur = s0;
      bool ok = true;
      for (int32_t i = tok_offsets[t]; i < tok_offsets[t + 1] && cur != dead; ++i) {
        const int32_t k = tok_symbols[i];
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
      o[t] = (ok && live[cur]) ? cur : -1;
    }
    if (eos_id >= 0 && eos_id < vocab) o[eos_id] = accept[s0] ? s0 : -1;
  }
  return BPD_OK;
}

extern "C" int bpd_host_build_reachability(const int32_t* trans, int32_t num_states,
                                           int32_t num_symbols, const uint8_t* accept,
                                           uint8_t* live) {
  BPD_REQUIRE(num_states >= 0 && num_symbols > 0, "bad table shape");
  if (num_states == 0) return BPD_OK;
  BPD_REQUIRE(trans && accept && live, "null pointer argument");
  // reverse edges (CSR), then a breadth-first search back from the accepting states
  std::vector<int32_t> cnt(size_t(num_states) + 1, 0);
  const int64_t nt = int64_t(num_states) * num_symbols;
  for (int64_t i = 0; i < nt; ++i) {
    const int32_t t = trans[i];
    if (t >= 0 && t < num_states) ++cnt[size_t(t) + 1];
  }
  for (int32_t s = 0; s < num_states; ++s) cnt[size_t(s) + 1] += cnt[size_t(s)];
  std::vector<int32_t> pred(static_cast<size_t>(cnt[static_cast<size_t>(num_states)]));
  std::vector<int32_t> fill(cnt.begin(), cnt.end() - 1);
  for (int64_t i = 0; i < nt; ++i) {
    const int32_t t = trans[i];
    if (t >= 0 && t < num_states) pred[size_t(fill[size_t(t)]++)] = int32_t(i / num_symbols);
  }
  std::vector<int32_t> todo;
  for (int32_t s = 0; s < num_states; ++s) {
    live[s] = accept[s] ? 1 : 0;
    if (live[s]) todo.push_back(s);
  }
  for (size_t h = 0; h < todo.size(); ++h) {
    const int32_t t = todo[h];
    for (int32_t j = cnt[size_t(t)]; j < cnt[size_t(t) + 1]; ++j) {
      const int32_t p = pred[size_t(j)];
      if (!live[p]) {
        live[p] = 1;
        todo.push_back(p);
      }
    }
  }
  return BPD_OK;
}

// Every (frame list, token) walk of the PDA mask's frame lists, split over
// `threads` host threads by list.  trans[l][c]: the list byte c leads to
// (or-ed with the saturation and raw-words flags), -1 when the step empties the set, -2 at
// a boundary.  A token is inside list l when every byte leads to a list;
// its bit in allowed[l] is set unless it is EOS or empty.  The seeds of l are
// the walk positions whose token meets a boundary, or is EOS or empty.
extern "C" int bpd_host_frame_classify(const int32_t* trans, int32_t num_lists, const int32_t* tok_offsets,
                                       const uint8_t* tok_bytes, int32_t vocab_size, int32_t eos_id,
                                       const int32_t* order, uint32_t* allowed, int32_t* seed_count,
                                       const int32_t* seed_off, int32_t* seeds, int32_t threads) {
  BPD_REQUIRE(num_lists >= 0 && vocab_size >= 0, "bad shape");
  if (num_lists == 0) return BPD_OK;
  BPD_REQUIRE(trans && tok_offsets && order && allowed && seed_count, "null pointer argument");
  BPD_REQUIRE((seed_off != nullptr) == (seeds != nullptr), "seeds and seed_off go together");
  for (int64_t i = 0; i < int64_t(num_lists) * 256; ++i) {
    const int32_t c = trans[i];
    BPD_REQUIRE(c == -1 || c == -2 || (c >= 0 && (c & (BPD_PDA_FRAME_SAT - 1)) < num_lists &&
                                       (c & ~(BPD_PDA_FRAME_RAW | BPD_PDA_FRAME_SAT | (BPD_PDA_FRAME_SAT - 1))) == 0),
                "frame transition %d out of range", c);
  }
  BPD_REQUIRE(tok_offsets[0] == 0, "token offsets start at %d", tok_offsets[0]);
  for (int32_t t = 0; t < vocab_size; ++t)
    BPD_REQUIRE(tok_offsets[t + 1] >= tok_offsets[t], "token offsets decrease at %d", t);
  BPD_REQUIRE(tok_offsets[vocab_size] == 0 || tok_bytes, "null token bytes");
  for (int32_t k = 0; k < vocab_size; ++k)
    BPD_REQUIRE(order[k] >= 0 && order[k] < vocab_size, "walk order entry %d out of range", order[k]);
  if (seed_off) {
    BPD_REQUIRE(seed_off[0] == 0, "seed offsets start at %d", seed_off[0]);
    for (int32_t l = 0; l < num_lists; ++l)
      BPD_REQUIRE(seed_off[l + 1] >= seed_off[l] && int64_t(seed_off[l + 1]) - seed_off[l] <= vocab_size,
                  "seed offsets out of range at list %d", l);
  }
  const int64_t words = (int64_t(vocab_size) + 31) / 32;
  auto work = [&](int32_t first, int32_t step) {
    for (int32_t l = first; l < num_lists; l += step) {
      uint32_t* al = allowed + int64_t(l) * words;
      std::fill(al, al + words, 0u);
      int32_t n = 0;
      const int32_t cap = seed_off ? seed_off[l + 1] - seed_off[l] : 0;
      int32_t* out = seeds ? seeds + seed_off[l] : nullptr;
      for (int32_t k = 0; k < vocab_size; ++k) {
        const int32_t t = order[k];
        const int32_t s = tok_offsets[t], e = tok_offsets[t + 1];
        int32_t cur = l;
        for (int32_t i = s; i < e && cur >= 0; ++i) {
          const int32_t c = trans[int64_t(cur) * 256 + tok_bytes[i]];
          cur = c >= 0 ? (c & (BPD_PDA_FRAME_SAT - 1)) : c;
        }
        const bool special = e == s || t == eos_id;
        if (special || cur == -2) {
          if (out && n < cap) out[n] = k;
          ++n;
        } else if (cur >= 0) {
          al[t >> 5] |= 1u << (t & 31);
        }
      }
      seed_count[l] = n;
    }
  };
  const int32_t nt = std::max<int32_t>(1, std::min<int32_t>(threads, std::min<int32_t>(num_lists, 64)));
  std::vector<std::thread> pool;
  for (int32_t i = 1; i < nt; ++i) pool.emplace_back(work, i, nt);
  work(0, nt);
  for (auto& th : pool) th.join();
  if (seed_off)
    for (int32_t l = 0; l < num_lists; ++l)
      BPD_REQUIRE(seed_count[l] == seed_off[l + 1] - seed_off[l], "list %d has %d seeds, not %d", l,
                  seed_count[l], seed_off[l + 1] - seed_off[l]);
  return BPD_OK;
}
