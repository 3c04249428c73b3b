// Host side of libbpdecode_hip: error state and the CPU-tensor forms of the
// dense entry points.  Same contracts as the device entry points in
// dense.hip; they run on the calling thread.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>
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

template <typename T>
void mask_rows(T* logits, int64_t rows, int64_t vocab, int64_t ld, const int32_t* tok_next,
               const int32_t* states, const int64_t* slots, T fill) {
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s = states[slots ? slots[b] : b];
    T* row = logits + b * ld;
    if (s < 0) {
      std::fill(row, row + vocab, fill);
      continue;
    }
    const int32_t* tn = tok_next + int64_t(s) * vocab;
    for (int64_t t = 0; t < vocab; ++t)
      if (tn[t] == -1) row[t] = fill;
  }
}

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" const char* bpd_last_error(void) { return g_error; }

extern "C" int bpd_abi_version(void) { return 7; }

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
