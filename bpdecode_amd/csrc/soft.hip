// Soft lookahead on gfx950: the uniform-count bias table of build_lookahead
// (ops.py:200-236) and the in-place bias-and-mask of apply_soft_
// (ops.py:239-259).
//
// Table build: k-1 rounds of logZ(s) = logsumexp_t logZ(tok_next[s, t])
// (logaddexp with 0 for accepting s, -inf off the live set).  One block per
// state reduces the whole vocab row with an online (max, sum-exp) pair per
// thread and a tree merge in LDS; logZ of the previous round sits in LDS so
// the gather is an LDS read.  Rounds ping-pong two logZ vectors in the
// caller's workspace.  A last pass writes out[s, t] = logZ(tok_next[s, t]).
#include <cmath>
#include <vector>

#include "bpd_common.hpp"

namespace bpd {
namespace {

constexpr int kSoftThreads = 1024;
constexpr int kMaxLdsStates = 8192;

struct Lse {
  float m, s;  // value = m + log(s); m = -inf <=> empty
};

__host__ __device__ inline Lse lse_push(Lse a, float x) {
  if (x == -INFINITY) return a;
  if (x > a.m) {
    a.s = (a.m == -INFINITY ? 0.0f : a.s * expf(a.m - x)) + 1.0f;
    a.m = x;
  } else {
    a.s += expf(x - a.m);
  }
  return a;
}

__host__ __device__ inline Lse lse_merge(Lse a, Lse b) {
  if (b.m == -INFINITY) return a;
  if (a.m == -INFINITY) return b;
  if (a.m >= b.m) return Lse{a.m, a.s + b.s * expf(b.m - a.m)};
  return Lse{b.m, b.s + a.s * expf(a.m - b.m)};
}

__host__ __device__ inline float lse_value(Lse a) {
  return a.m == -INFINITY ? -INFINITY : a.m + logf(a.s);
}

// torch.logaddexp(a, b) for float.
__host__ __device__ inline float log_add_exp(float a, float b) {
  if (a == b && (a == INFINITY || a == -INFINITY)) return a;
  const float m = fmaxf(a, b);
  return m + log1pf(expf(-fabsf(a - b)));
}

__global__ __launch_bounds__(kSoftThreads) void soft_round_kernel(
    const int32_t* __restrict__ tok_next, int32_t S, int64_t V, const uint8_t* __restrict__ accept,
    const uint8_t* __restrict__ live, const float* __restrict__ logz_in,
    float* __restrict__ logz_out) {
  __shared__ float lz[kMaxLdsStates];
  __shared__ float red_m[kSoftThreads];
  __shared__ float red_s[kSoftThreads];
  for (int i = threadIdx.x; i < S; i += kSoftThreads) lz[i] = logz_in[i];
  __syncthreads();
  const int32_t s = blockIdx.x;
  const int32_t* row = tok_next + int64_t(s) * V;
  Lse acc{-INFINITY, 0.0f};
  for (int64_t t = threadIdx.x; t < V; t += kSoftThreads) {
    const int32_t d = row[t];
    if (d >= 0 && d < S) acc = lse_push(acc, lz[d]);
  }
  red_m[threadIdx.x] = acc.m;
  red_s[threadIdx.x] = acc.s;
  __syncthreads();
  for (int w = kSoftThreads / 2; w > 0; w >>= 1) {
    if (int(threadIdx.x) < w) {
      const Lse r = lse_merge(Lse{red_m[threadIdx.x], red_s[threadIdx.x]},
                              Lse{red_m[threadIdx.x + w], red_s[threadIdx.x + w]});
      red_m[threadIdx.x] = r.m;
      red_s[threadIdx.x] = r.s;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float nxt = lse_value(Lse{red_m[0], red_s[0]});
    if (accept[s]) nxt = log_add_exp(nxt, 0.0f);
    logz_out[s] = live[s] ? nxt : -INFINITY;
  }
}

__global__ void soft_init_kernel(const uint8_t* __restrict__ live, int32_t S, float* __restrict__ logz) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < S) logz[i] = live[i] ? 0.0f : -INFINITY;
}

__global__ __launch_bounds__(256) void soft_table_kernel(const int32_t* __restrict__ tok_next,
                                                         int32_t S, int64_t V,
                                                         const uint8_t* __restrict__ accept,
                                                         int32_t eos, const float* __restrict__ logz,
                                                         float* __restrict__ out) {
  __shared__ float lz[kMaxLdsStates];
  for (int i = threadIdx.x; i < S; i += blockDim.x) lz[i] = logz[i];
  __syncthreads();
  const int32_t s = blockIdx.y;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= V) return;
  float v;
  if (t == eos) {
    v = accept[s] ? 0.0f : -INFINITY;
  } else {
    const int32_t d = tok_next[int64_t(s) * V + t];
    v = (d >= 0 && d < S) ? lz[d] : -INFINITY;
  }
  out[int64_t(s) * V + t] = v;
}

__device__ inline float load_as_float(const uint8_t* p, int D) {
  if (D == BPD_DTYPE_F32) return *reinterpret_cast<const float*>(p);
  const uint16_t h = *reinterpret_cast<const uint16_t*>(p);
  if (D == BPD_DTYPE_BF16) return __uint_as_float(uint32_t(h) << 16);
  _Float16 x;
  __builtin_memcpy(&x, &h, 2);
  return float(x);
}

__device__ inline void store_from_float(uint8_t* p, int D, float v) {
  if (D == BPD_DTYPE_F32) {
    *reinterpret_cast<float*>(p) = v;
    return;
  }
  uint16_t h;
  if (D == BPD_DTYPE_BF16) {
    const uint32_t u = __float_as_uint(v);
    h = isnan(v) ? uint16_t(0x7FC0) : uint16_t((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  } else {
    const _Float16 x = _Float16(v);
    __builtin_memcpy(&h, &x, 2);
  }
  *reinterpret_cast<uint16_t*>(p) = h;
}

// logits[b, t] += alpha * bias on finite bias entries (computed in float,
// stored in the logits dtype), -inf where the bias is -inf or the row's
// state is negative.
template <int D>
__global__ __launch_bounds__(256) void soft_apply_kernel(uint8_t* __restrict__ logits, int64_t ld_bytes,
                                                         int64_t V, const float* __restrict__ la,
                                                         int32_t S, const int32_t* __restrict__ states,
                                                         const int64_t* __restrict__ slots,
                                                         float alpha, uint32_t neg_inf_bits,
                                                         int32_t* __restrict__ err) {
  constexpr int E = D == BPD_DTYPE_F32 ? 4 : 2;
  const int64_t b = blockIdx.y;
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= V) return;
  const int32_t s = states[slots ? slots[b] : b];
  if (s >= S && err && t == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
  const float bias = (s < 0 || s >= S) ? -INFINITY : la[int64_t(s) * V + t];
  uint8_t* p = logits + b * ld_bytes + t * E;
  if (bias == -INFINITY) {
    if (E == 4)
      *reinterpret_cast<uint32_t*>(p) = neg_inf_bits;
    else
      *reinterpret_cast<uint16_t*>(p) = uint16_t(neg_inf_bits);
  } else if (alpha != 0.0f) {
    store_from_float(p, D, fmaf(alpha, bias, load_as_float(p, D)));
  }
}

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" size_t bpd_soft_workspace_bytes(int64_t rows, int32_t num_states, int32_t k) {
  (void)rows;
  (void)k;
  return size_t(2) * size_t(num_states > 0 ? num_states : 0) * sizeof(float);
}

extern "C" int bpd_soft_build_lookahead(const int32_t* tok_next, int32_t S, int64_t V,
                                        const uint8_t* accept, const uint8_t* live, int32_t eos,
                                        int32_t k, float* out, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  BPD_REQUIRE(S > 0 && V >= 0, "bad table shape");
  BPD_REQUIRE(S <= kMaxLdsStates, "at most %d states", kMaxLdsStates);
  BPD_REQUIRE(workspace_bytes >= bpd_soft_workspace_bytes(0, S, k), "workspace too small");
  BPD_REQUIRE(S < 65536, "at most 65535 states");
  hipStream_t st = as_stream(stream);
  float* a = static_cast<float*>(workspace);
  float* b = a + S;
  soft_init_kernel<<<(S + 255) / 256, 256, 0, st>>>(live, S, a);
  BPD_LAUNCHED();
  for (int j = 0; j < k - 1; ++j) {
    soft_round_kernel<<<S, kSoftThreads, 0, st>>>(tok_next, S, V, accept, live, a, b);
    BPD_LAUNCHED();
    float* tmp = a;
    a = b;
    b = tmp;
  }
  if (V == 0) return BPD_OK;
  const dim3 grid = dim3(unsigned((V + 255) / 256), unsigned(S));
  soft_table_kernel<<<grid, 256, 0, st>>>(tok_next, S, V, accept, eos, a, out);
  BPD_LAUNCHED();
  return BPD_OK;
}

extern "C" int bpd_soft_apply(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                              const float* lookahead, int32_t num_states, const int32_t* states,
                              const int64_t* slots, float alpha, int32_t* err, void* stream) {
  const int E = elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && vocab >= 0 && ld >= vocab, "bad logits shape");
  BPD_REQUIRE(num_states > 0, "empty lookahead table");
  uint32_t ninf = 0;
  if (int rc = fill_bits(dtype, -INFINITY, &ninf)) return rc;
  if (rows == 0 || vocab == 0) return BPD_OK;
  BPD_REQUIRE(rows < 65536, "at most 65535 rows");
  const dim3 grid = dim3(unsigned((vocab + 255) / 256), unsigned(rows));
  uint8_t* lg = static_cast<uint8_t*>(logits);
  hipStream_t st = as_stream(stream);
  if (dtype == BPD_DTYPE_F32)
    soft_apply_kernel<BPD_DTYPE_F32><<<grid, 256, 0, st>>>(lg, ld * E, vocab, lookahead, num_states,
                                                           states, slots, alpha, ninf, err);
  else if (dtype == BPD_DTYPE_F16)
    soft_apply_kernel<BPD_DTYPE_F16><<<grid, 256, 0, st>>>(lg, ld * E, vocab, lookahead, num_states,
                                                           states, slots, alpha, ninf, err);
  else
    soft_apply_kernel<BPD_DTYPE_BF16><<<grid, 256, 0, st>>>(lg, ld * E, vocab, lookahead,
                                                            num_states, states, slots, alpha, ninf,
                                                            err);
  BPD_LAUNCHED();
  return BPD_OK;
}

// ---------------------------------------------------------------- host --
namespace {

float host_load(const uint8_t* p, int dtype) {
  if (dtype == BPD_DTYPE_F32) {
    float f;
    std::memcpy(&f, p, 4);
    return f;
  }
  uint16_t h;
  std::memcpy(&h, p, 2);
  if (dtype == BPD_DTYPE_BF16) {
    const uint32_t u = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
  }
  _Float16 x;
  std::memcpy(&x, &h, 2);
  return float(x);
}

void host_store(uint8_t* p, int dtype, float v) {
  if (dtype == BPD_DTYPE_F32) {
    std::memcpy(p, &v, 4);
    return;
  }
  const uint16_t h = dtype == BPD_DTYPE_BF16 ? bf16_bits_rne(v) : f16_bits_rne(v);
  std::memcpy(p, &h, 2);
}

}  // namespace

extern "C" int bpd_host_soft_build_lookahead(const int32_t* tok_next, int32_t S, int64_t V,
                                             const uint8_t* accept, const uint8_t* live,
                                             int32_t eos, int32_t k, float* out) {
  BPD_REQUIRE(S > 0 && V >= 0, "bad table shape");
  std::vector<float> a(static_cast<size_t>(S)), b(static_cast<size_t>(S));
  for (int32_t s = 0; s < S; ++s) a[size_t(s)] = live[s] ? 0.0f : -INFINITY;
  for (int j = 0; j < k - 1; ++j) {
    for (int32_t s = 0; s < S; ++s) {
      Lse acc{-INFINITY, 0.0f};
      const int32_t* row = tok_next + int64_t(s) * V;
      for (int64_t t = 0; t < V; ++t)
        if (row[t] >= 0) acc = lse_push(acc, a[size_t(row[t])]);
      float nxt = lse_value(acc);
      if (accept[s]) nxt = log_add_exp(nxt, 0.0f);
      b[size_t(s)] = live[s] ? nxt : -INFINITY;
    }
    a.swap(b);
  }
  for (int32_t s = 0; s < S; ++s) {
    const int32_t* row = tok_next + int64_t(s) * V;
    float* o = out + int64_t(s) * V;
    for (int64_t t = 0; t < V; ++t) o[t] = row[t] >= 0 ? a[size_t(row[t])] : -INFINITY;
    if (eos >= 0 && eos < V) o[eos] = accept[s] ? 0.0f : -INFINITY;
  }
  return BPD_OK;
}

extern "C" int bpd_host_soft_apply(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                                   const float* lookahead, int32_t num_states,
                                   const int32_t* states, const int64_t* slots, float alpha) {
  const int E = elem_bytes(dtype);
  BPD_REQUIRE(E != 0, "unknown logits dtype code %d", dtype);
  BPD_REQUIRE(rows >= 0 && vocab >= 0 && ld >= vocab, "bad logits shape");
  uint32_t ninf = 0;
  if (int rc = fill_bits(dtype, -INFINITY, &ninf)) return rc;
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s = states[slots ? slots[b] : b];
    BPD_REQUIRE(s < num_states, "index %d is out of bounds for dimension 0 with size %d", s,
                num_states);
    uint8_t* row = static_cast<uint8_t*>(logits) + b * ld * E;
    for (int64_t t = 0; t < vocab; ++t) {
      const float bias = s < 0 ? -INFINITY : lookahead[int64_t(s) * vocab + t];
      uint8_t* p = row + t * E;
      if (bias == -INFINITY)
        std::memcpy(p, &ninf, size_t(E));
      else if (alpha != 0.0f)
        host_store(p, dtype, std::fmaf(alpha, bias, host_load(p, dtype)));
    }
  }
  return BPD_OK;
}
