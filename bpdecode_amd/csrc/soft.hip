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
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <unordered_map>
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

// ------------------------------------------------------- prior-weighted --
// Soft lookahead weighted by each row's own model prior.  With
// logpi_b = log_softmax(logits_b) and k-1 rounds of
//   logZ_0(s)     = 0 on live s, -inf elsewhere
//   logZ_{j+1}(s) = logsumexp_t [logpi_b(t) + logZ_j(tok_next[s, t])]
//                   (logaddexp with logpi_b(eos) for accepting s), -inf off live
// the output is out[b, t] = logpi_b(t) + alpha * logZ_{k-1}(tok_next[s_b, t])
// on allowed tokens, logpi_b(eos) / -inf in the EOS column, -inf elsewhere.
// With logpi == 0 the recurrence is the uniform one above.  Logits are
// expected finite or -inf.
//
// Token classes make the per-row work independent of the vocab size: tokens
// whose tok_next columns are equal behave identically in every state, so a
// round needs only logsumexp_{t in class} logpi_b(t) per class.  Classes are
// built once per grammar on the host (bpd_host_soft_classes).  One call is
// three kernels:
//   stats:  grid (G, rows), block g streams tokens [8192 g, 8192 (g+1)) of
//           its row with their class ids and leaves the chunk's logsumexp
//           and, per class, (max, sum exp(x - max)) of its members: a
//           class-max pass and a class-sum pass through LDS atomics.  Above
//           kLdsClasses classes the class sums come from gathers over class
//           pieces of <= 256 members instead (one wave per piece).
//   rounds: one block per row merges the partials, runs the k-1 rounds with
//           logZ, the class sums and the (class, next) pairs in LDS, and
//           writes zcls[b, c] = logZ(next of class c from s_b) and lse[b].
//   out:    one streaming pass, out = x - lse + alpha * zcls[b, class(t)].
// The kernel boundaries order the cross-block hand-offs; an in-kernel
// last-block hand-off needs agent-scope release fences, which write back the
// whole L2 of each XCD on this part and cost far more than a launch.
namespace bpd {
namespace {

constexpr int kPriorThreads = 256;
constexpr int kPriorOutThreads = 256;
constexpr int kPriorMaxStates = 4096;
constexpr int kPieceMembers = 256;
constexpr int kLdsClasses = 1024;                          // class-atomic stats up to this many classes
constexpr int kStatLoads = 4;                              // float4 loads per thread (class-atomic stats)
constexpr int64_t kStatChunk = kPriorThreads * 4 * kStatLoads;  // tokens per block
constexpr size_t kPriorMaxLds = 60 * 1024;
constexpr float kLog2e = 1.4426950408889634f;
typedef float F4v __attribute__((ext_vector_type(4)));  // float4 for the non-temporal builtins

// 2^x by the hardware exponential (v_exp_f32); used for x <= 0.
__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// exp(x - m) for x <= m: the difference is formed first (exact for x close
// to m), so the result keeps full precision however large m is
__device__ inline float exp_shift(float x, float m) { return exp2_fast((x - m) * kLog2e); }

// Order-preserving int image of a float (and back: the map is an involution).
__device__ inline int32_t ord_of(float x) {
  const int32_t i = __float_as_int(x);
  return i >= 0 ? i : i ^ 0x7FFFFFFF;
}
__device__ inline float float_of_ord(int32_t i) { return __int_as_float(i >= 0 ? i : i ^ 0x7FFFFFFF); }

// lse_merge by the hardware exponential (the prior kernels' reductions)
__device__ inline Lse lse_merge_fast(Lse a, Lse b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return Lse{m, 0.0f};
  return Lse{m, a.s * exp_shift(a.m, m) + b.s * exp_shift(b.m, m)};
}

// Wave reductions with every lane active, the result in every lane: DPP
// exchanges within each row of 16 lanes (lane ^ 1, lane ^ 2, the half-row
// mirror, the row mirror), then the four row results by scalar lane reads --
// no LDS round trip, where a shuffle butterfly takes six.
template <int Ctrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_max_f(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum_f(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ inline Lse wave_lse(Lse a) {
  a = lse_merge_fast(a, Lse{dpp_f<0xB1>(a.m), dpp_f<0xB1>(a.s)});
  a = lse_merge_fast(a, Lse{dpp_f<0x4E>(a.m), dpp_f<0x4E>(a.s)});
  a = lse_merge_fast(a, Lse{dpp_f<0x141>(a.m), dpp_f<0x141>(a.s)});
  a = lse_merge_fast(a, Lse{dpp_f<0x140>(a.m), dpp_f<0x140>(a.s)});
  const Lse r0 = lse_merge_fast(Lse{lane_f(a.m, 0), lane_f(a.s, 0)}, Lse{lane_f(a.m, 16), lane_f(a.s, 16)});
  const Lse r1 = lse_merge_fast(Lse{lane_f(a.m, 32), lane_f(a.s, 32)}, Lse{lane_f(a.m, 48), lane_f(a.s, 48)});
  return lse_merge_fast(r0, r1);
}

// Block-wide merge of one Lse per thread; the result is valid in every thread.
template <int kThreads>
__device__ inline Lse block_lse(Lse a) {
  __shared__ float wm[kThreads / 64];
  __shared__ float ws[kThreads / 64];
  a = wave_lse(a);
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) {
    wm[w] = a.m;
    ws[w] = a.s;
  }
  __syncthreads();
  Lse r{-INFINITY, 0.0f};
  for (int i = 0; i < kThreads / 64; ++i) r = lse_merge_fast(r, Lse{wm[i], ws[i]});
  __syncthreads();
  return r;
}

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Launch geometry of one call.
constexpr int kWideLoads = 8;                                   // float4 groups per thread (wave-shift stats)
constexpr int64_t kWideChunk = kPriorThreads * 4 * kWideLoads;  // 8192 tokens per block

struct PriorPlan {
  bool class_stats;  // class-atomic stats (else pieces)
  bool wide;         // wave-shift stats over 16384-token chunks (class_stats only)
  int G;             // chunk blocks per row
  int Gp;            // piece blocks per row (pieces path)
};

PriorPlan prior_plan(int64_t rows, int64_t vocab, int32_t C, int32_t P, bool force_pieces, bool wide) {
  PriorPlan pl;
  pl.class_stats = !force_pieces && C <= kLdsClasses;
  pl.wide = pl.class_stats && wide;
  if (pl.class_stats) {
    const int64_t chunk = pl.wide ? kWideChunk : kStatChunk;
    pl.G = int((vocab + chunk - 1) / chunk);
    pl.Gp = 0;
  } else {
    const int64_t g = rows > 0 ? (1024 + rows - 1) / rows : 1;
    pl.G = int(g < 1 ? 1 : (g > 64 ? 64 : g));
    pl.Gp = (P + 2 * (kPriorThreads / 64) - 1) / (2 * (kPriorThreads / 64));
  }
  return pl;
}

struct PriorWs {
  float* part;   // [rows, G, 2] chunk logsumexp partials
  float* mid;    // class-atomic: [rows, G, C, 2] class partials; pieces: [rows, P, 2]
  float* lse;    // [rows]
  float* zcls;   // [rows, C]
};

size_t prior_mid_floats(int64_t rows, const PriorPlan& pl, int32_t C, int32_t P) {
  return pl.class_stats ? size_t(rows) * pl.G * C * 2 : size_t(rows) * P * 2;
}

PriorWs prior_ws(void* base, int64_t rows, const PriorPlan& pl, int32_t C, int32_t P) {
  char* p = static_cast<char*>(base);
  PriorWs w;
  w.part = reinterpret_cast<float*>(p);
  p += align256(size_t(rows) * pl.G * 8);
  w.mid = reinterpret_cast<float*>(p);
  p += align256(prior_mid_floats(rows, pl, C, P) * 4);
  w.lse = reinterpret_cast<float*>(p);
  p += align256(size_t(rows) * 4);
  w.zcls = reinterpret_cast<float*>(p);
  return w;
}

size_t prior_ws_bytes(int64_t rows, const PriorPlan& pl, int32_t C, int32_t P) {
  return align256(size_t(rows) * pl.G * 8) + align256(prior_mid_floats(rows, pl, C, P) * 4) +
         align256(size_t(rows) * 4) + align256(size_t(rows) * C * 4);
}

size_t prior_lds_bytes(int32_t S, int32_t C, int32_t P, int64_t pairs, bool pairs_in_lds, bool pieces) {
  size_t n = size_t(C) * 4 + size_t(S) * 8 + size_t(S + 3) / 4 * 4 + size_t(S + 1) * 4;
  if (pairs_in_lds) n += size_t(pairs) * 4;
  n = (n + 7) / 8 * 8;
  return pieces ? n + size_t(P) * 8 : n;
}

__device__ inline int32_t narrow_class(uint32_t c) { return c == 0xFFFFu ? -1 : int32_t(c); }

// Class-atomic stats, grid (G, rows): block g takes tokens
// [kStatChunk g, kStatChunk (g+1)) of its row.  Narrow: the class map is read
// as uint16 (0xFFFF: no class).
template <bool Vec, bool Narrow>
__global__ __launch_bounds__(kPriorThreads) void prior_stats_classes_kernel(
    const float* __restrict__ logits, int64_t ld, int64_t V, const int32_t* __restrict__ token_class,
    const uint16_t* __restrict__ token_class16, int32_t C, PriorWs ws) {
  __shared__ int32_t cmax[kLdsClasses];
  __shared__ float csum[kLdsClasses];
  constexpr int kE = 4 * kStatLoads;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int64_t b = blockIdx.y;
  const float* row = logits + b * ld;
  const int64_t base = int64_t(g) * kStatChunk;
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    cmax[c] = ord_of(-INFINITY);
    csum[c] = 0.0f;
  }
  float x[kE];
  int32_t k[kE];
  if (Vec) {
#pragma unroll
    for (int u = 0; u < kStatLoads; ++u) {
      const int64_t t = base + (int64_t(u) * kPriorThreads + threadIdx.x) * 4;
      float4 xv = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      int4 kv = make_int4(-1, -1, -1, -1);
      if (t < V) {
        xv = *reinterpret_cast<const float4*>(row + t);
        if (Narrow) {
          const uint2 n = *reinterpret_cast<const uint2*>(token_class16 + t);
          kv = make_int4(narrow_class(n.x & 0xFFFFu), narrow_class(n.x >> 16), narrow_class(n.y & 0xFFFFu),
                         narrow_class(n.y >> 16));
        } else {
          kv = *reinterpret_cast<const int4*>(token_class + t);
        }
      }
      x[4 * u] = xv.x;
      x[4 * u + 1] = xv.y;
      x[4 * u + 2] = xv.z;
      x[4 * u + 3] = xv.w;
      k[4 * u] = kv.x;
      k[4 * u + 1] = kv.y;
      k[4 * u + 2] = kv.z;
      k[4 * u + 3] = kv.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < kE; ++e) {
      const int64_t t = base + int64_t(e) * kPriorThreads + threadIdx.x;
      x[e] = t < V ? row[t] : -INFINITY;
      k[e] = t < V ? (Narrow ? narrow_class(token_class16[t]) : token_class[t]) : -1;
    }
  }
  // chunk logsumexp
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < kE; ++e) m = fmaxf(m, x[e]);
  Lse acc{-INFINITY, 0.0f};
  if (m != -INFINITY) {
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < kE; ++e) sum += exp_shift(x[e], m);
    acc = Lse{m, sum};
  }
  acc = block_lse<kPriorThreads>(acc);  // its barriers also publish the LDS init
  if (threadIdx.x == 0) {
    ws.part[(b * G + g) * 2] = acc.m;
    ws.part[(b * G + g) * 2 + 1] = acc.s;
  }
  // per-class max, then per-class sum of exp(x - max)
#pragma unroll
  for (int e = 0; e < kE; ++e)
    if (k[e] >= 0 && x[e] != -INFINITY) atomicMax(&cmax[k[e]], ord_of(x[e]));
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    if (k[e] >= 0 && x[e] != -INFINITY) {
      const float cm = float_of_ord(cmax[k[e]]);
      atomicAdd(&csum[k[e]], exp_shift(x[e], cm));
    }
  }
  __syncthreads();
  float* out = ws.mid + (b * G + g) * int64_t(C) * 2;
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    out[2 * c] = float_of_ord(cmax[c]);
    out[2 * c + 1] = csum[c];
  }
}

// Class statistics from the chunk's member list instead of the per-token
// class map: the chunk is staged in LDS while its row logsumexp is formed,
// then only the classed tokens (Cap fixed slots per chunk, (offset << 16 |
// class), 0xFFFFFFFF empty; loaded with the logits) take part in the class
// max and sum.  Same per-class arithmetic as prior_stats_classes_kernel.
// Dynamic LDS: kStatChunk floats, then C class maxima and C sums.
template <int Cap>
__global__ __launch_bounds__(kPriorThreads) void prior_stats_members_kernel(
    const float* __restrict__ logits, int64_t ld, int64_t V, const uint32_t* __restrict__ members,
    int32_t C, PriorWs ws) {
  static_assert(kStatChunk == BPD_SOFT_MEMBER_CHUNK, "member lists are cut at the statistics chunk");
  extern __shared__ __align__(16) float smem[];
  float4* xs = reinterpret_cast<float4*>(smem);
  int32_t* cmax = reinterpret_cast<int32_t*>(smem + kStatChunk);
  float* csum = smem + kStatChunk + C;
  constexpr int kE = 4 * kStatLoads;
  constexpr int kM = Cap / kPriorThreads;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int64_t b = blockIdx.y;
  const float* row = logits + b * ld;
  const int64_t base = int64_t(g) * kStatChunk;
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    cmax[c] = ord_of(-INFINITY);
    csum[c] = 0.0f;
  }
  float x[kE];
#pragma unroll
  for (int u = 0; u < kStatLoads; ++u) {
    const int64_t t = base + (int64_t(u) * kPriorThreads + threadIdx.x) * 4;
    float4 xv = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    if (t < V) xv = *reinterpret_cast<const float4*>(row + t);
    xs[u * kPriorThreads + threadIdx.x] = xv;
    x[4 * u] = xv.x;
    x[4 * u + 1] = xv.y;
    x[4 * u + 2] = xv.z;
    x[4 * u + 3] = xv.w;
  }
  uint32_t mm[kM];
#pragma unroll
  for (int j = 0; j < kM; ++j) mm[j] = members[int64_t(g) * Cap + j * kPriorThreads + threadIdx.x];
  // chunk logsumexp
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < kE; ++e) m = fmaxf(m, x[e]);
  Lse acc{-INFINITY, 0.0f};
  if (m != -INFINITY) {
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < kE; ++e) sum += exp_shift(x[e], m);
    acc = Lse{m, sum};
  }
  acc = block_lse<kPriorThreads>(acc);  // its barriers also publish the staged chunk and the LDS init
  if (threadIdx.x == 0) {
    ws.part[(b * G + g) * 2] = acc.m;
    ws.part[(b * G + g) * 2 + 1] = acc.s;
  }
  // per-class max, then per-class sum of exp(x - max), over the members only
  const float* xf = smem;
  float v[kM];
#pragma unroll
  for (int j = 0; j < kM; ++j) {
    v[j] = mm[j] != 0xFFFFFFFFu ? xf[mm[j] >> 16] : -INFINITY;
    if (v[j] != -INFINITY) atomicMax(&cmax[mm[j] & 0xFFFFu], ord_of(v[j]));
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kM; ++j) {
    if (v[j] != -INFINITY) {
      const int32_t c = int32_t(mm[j] & 0xFFFFu);
      atomicAdd(&csum[c], exp_shift(v[j], float_of_ord(cmax[c])));
    }
  }
  __syncthreads();
  float* out = ws.mid + (b * G + g) * int64_t(C) * 2;
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    out[2 * c] = float_of_ord(cmax[c]);
    out[2 * c + 1] = csum[c];
  }
}

// Wave-shift statistics, grid (G, rows): block g takes tokens
// [16384 g, 16384 (g + 1)) of its row, 64 per thread (16 float4 groups in
// flight, each group coalesced), and the uint16 class map of the same tokens
// (shared by every row, so it stays in L2).  Each wave shifts by its own
// maximum M_w: the chunk logsumexp and, per class, sum exp(x - M_w) over the
// wave's classed tokens go to the wave's own LDS array, so the block needs
// no class-maximum pass and a single barrier.  The class partials written
// are (max_w M_w over waves with a non-zero sum, the sums rescaled to it),
// the same (max, sum) form the rounds kernel merges.  A class member more
// than 80 below its wave maximum could underflow there; a block that has one
// takes the exact per-class maximum instead (class-max pass, then the sums).
// Dynamic LDS: 4 * C wave sums, then C class maxima and C sums (exact path).
__global__ __launch_bounds__(kPriorThreads) void prior_stats_wave_kernel(
    const float* __restrict__ logits, int64_t ld, int64_t V, const uint16_t* __restrict__ token_class16,
    int32_t C, PriorWs ws) {
  extern __shared__ __align__(16) float smem[];
  constexpr int kWaves = kPriorThreads / 64;
  float* wsum = smem;                                               // [kWaves][C]
  int32_t* cmax = reinterpret_cast<int32_t*>(smem + kWaves * C);    // [C] exact path
  float* esum = smem + kWaves * C + C;                              // [C] exact path
  __shared__ float wm[kWaves], wl[kWaves];
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x / 64;
  const float* row = logits + b * ld;
  const int64_t base = int64_t(g) * kWideChunk;
  for (int32_t c = lane; c < C; c += 64) wsum[w * C + c] = 0.0f;
  float4 x[kWideLoads];
  uint2 k[kWideLoads];
#pragma unroll
  for (int u = 0; u < kWideLoads; ++u) {
    const int64_t t = base + (int64_t(u) * kPriorThreads + threadIdx.x) * 4;
    if (t < V) {
      x[u] = *reinterpret_cast<const float4*>(row + t);
      k[u] = *reinterpret_cast<const uint2*>(token_class16 + t);
    } else {
      x[u] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      k[u] = make_uint2(0xFFFFFFFFu, 0xFFFFFFFFu);
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < kWideLoads; ++u) m = fmaxf(m, fmaxf(fmaxf(x[u].x, x[u].y), fmaxf(x[u].z, x[u].w)));
  m = wave_max_f(m);
  // the wave's own class sums: only this wave writes them, and LDS
  // operations of one wave complete in order, so a wave fence orders the
  // zeroing above before the atomics
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float sum = 0.0f;
  bool under = false;
  if (m != -INFINITY) {
    auto one = [&](float v, uint32_t kc) {
      const float e = exp_shift(v, m);
      sum += e;
      if (kc != 0xFFFFu && v != -INFINITY) {
        under = under || v - m < -80.0f;
        atomicAdd(&wsum[w * C + int32_t(kc)], e);
      }
    };
#pragma unroll
    for (int u = 0; u < kWideLoads; ++u) {
      one(x[u].x, k[u].x & 0xFFFFu);
      one(x[u].y, k[u].x >> 16);
      one(x[u].z, k[u].y & 0xFFFFu);
      one(x[u].w, k[u].y >> 16);
    }
  }
  sum = wave_sum_f(sum);
  if (lane == 0) {
    wm[w] = m;
    wl[w] = sum;
  }
  const bool exact = __syncthreads_or(under);
  if (threadIdx.x == 0) {
    Lse r{-INFINITY, 0.0f};
#pragma unroll
    for (int i = 0; i < kWaves; ++i) r = lse_merge_fast(r, Lse{wm[i], wl[i]});
    ws.part[(b * G + g) * 2] = r.m;
    ws.part[(b * G + g) * 2 + 1] = r.s;
  }
  float* out = ws.mid + (b * G + g) * int64_t(C) * 2;
  if (!exact) {
    for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
      float cm = -INFINITY;
#pragma unroll
      for (int i = 0; i < kWaves; ++i)
        if (wsum[i * C + c] > 0.0f) cm = fmaxf(cm, wm[i]);
      float cs = 0.0f;
      if (cm != -INFINITY) {
#pragma unroll
        for (int i = 0; i < kWaves; ++i)
          if (wsum[i * C + c] > 0.0f) cs += wsum[i * C + c] * exp_shift(wm[i], cm);
      }
      out[2 * c] = cm;
      out[2 * c + 1] = cs;
    }
    return;
  }
  // exact path: per-class maximum, then the sums, from the values in registers
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    cmax[c] = ord_of(-INFINITY);
    esum[c] = 0.0f;
  }
  __syncthreads();
  auto cls_max = [&](float v, uint32_t kc) {
    if (kc != 0xFFFFu && v != -INFINITY) atomicMax(&cmax[int32_t(kc)], ord_of(v));
  };
#pragma unroll
  for (int u = 0; u < kWideLoads; ++u) {
    cls_max(x[u].x, k[u].x & 0xFFFFu);
    cls_max(x[u].y, k[u].x >> 16);
    cls_max(x[u].z, k[u].y & 0xFFFFu);
    cls_max(x[u].w, k[u].y >> 16);
  }
  __syncthreads();
  auto cls_sum = [&](float v, uint32_t kc) {
    if (kc != 0xFFFFu && v != -INFINITY) {
      const int32_t c = int32_t(kc);
      atomicAdd(&esum[c], exp_shift(v, float_of_ord(cmax[c])));
    }
  };
#pragma unroll
  for (int u = 0; u < kWideLoads; ++u) {
    cls_sum(x[u].x, k[u].x & 0xFFFFu);
    cls_sum(x[u].y, k[u].x >> 16);
    cls_sum(x[u].z, k[u].y & 0xFFFFu);
    cls_sum(x[u].w, k[u].y >> 16);
  }
  __syncthreads();
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    out[2 * c] = float_of_ord(cmax[c]);
    out[2 * c + 1] = esum[c];
  }
}

// Member-list statistics, grid (G, rows): block g takes tokens [8192 g,
// 8192 (g + 1)) of its row, 32 per thread (eight float4 groups in flight),
// and stages them in LDS.  Each wave shifts by its own maximum M_w: the
// chunk logsumexp as in prior_stats_wave_kernel.  The class sums come from
// the member lists of the block's two 4096-token chunks alone (no per-token
// class test): member o of class c adds exp(x_o - M_w) to the class sum of
// the wave w that loaded token o ((o >> 8) & 3 in this layout).  Partials,
// the exact path for members more than 80 below their wave's maximum and
// the outputs are those of prior_stats_wave_kernel.  Dynamic LDS: the 8192
// logits, 4 * C wave sums, C class maxima and C sums (exact path).
template <int Cap>
__global__ __launch_bounds__(kPriorThreads) void prior_stats_list_kernel(
    const float* __restrict__ logits, int64_t ld, int64_t V, const uint32_t* __restrict__ members,
    int32_t C, PriorWs ws) {
  static_assert(kWideChunk == 2 * BPD_SOFT_MEMBER_CHUNK, "a block covers two member chunks");
  extern __shared__ __align__(16) float smem[];
  constexpr int kWaves = kPriorThreads / 64;
  constexpr int kHalf = Cap / kPriorThreads;  // member slots per thread and chunk
  float4* xs = reinterpret_cast<float4*>(smem);                   // [kWideChunk / 4]
  float* wsum = smem + kWideChunk;                                // [kWaves][C]
  int32_t* cmax = reinterpret_cast<int32_t*>(wsum + kWaves * C);  // [C] exact path
  float* esum = wsum + kWaves * C + C;                            // [C] exact path
  __shared__ float wm[kWaves], wl[kWaves];
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x / 64;
  const float* row = logits + b * ld;
  const int64_t base = int64_t(g) * kWideChunk;
  const int64_t nchunks = (V + BPD_SOFT_MEMBER_CHUNK - 1) / BPD_SOFT_MEMBER_CHUNK;
  // the member entries first: loads complete in issue order, so waiting for
  // them does not wait for the logits
  uint32_t mm[2 * kHalf];
#pragma unroll
  for (int j = 0; j < 2 * kHalf; ++j) {
    const int64_t ch = 2 * int64_t(g) + j / kHalf;
    mm[j] = ch < nchunks ? members[ch * Cap + (j % kHalf) * kPriorThreads + threadIdx.x] : 0xFFFFFFFFu;
  }
  float4 x[kWideLoads];
#pragma unroll
  for (int u = 0; u < kWideLoads; ++u) {
    const int64_t t = base + (int64_t(u) * kPriorThreads + threadIdx.x) * 4;
    x[u] = t < V ? *reinterpret_cast<const float4*>(row + t)
                 : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  }
  for (int32_t c = threadIdx.x; c < kWaves * C; c += kPriorThreads) wsum[c] = 0.0f;
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < kWideLoads; ++u) m = fmaxf(m, fmaxf(fmaxf(x[u].x, x[u].y), fmaxf(x[u].z, x[u].w)));
  m = wave_max_f(m);
  float sum = 0.0f;
  if (m != -INFINITY) {
#pragma unroll
    for (int u = 0; u < kWideLoads; ++u)
      sum += (exp_shift(x[u].x, m) + exp_shift(x[u].y, m)) + (exp_shift(x[u].z, m) + exp_shift(x[u].w, m));
  }
  sum = wave_sum_f(sum);
#pragma unroll
  for (int u = 0; u < kWideLoads; ++u) xs[u * kPriorThreads + threadIdx.x] = x[u];
  if (lane == 0) {
    wm[w] = m;
    wl[w] = sum;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Lse r{-INFINITY, 0.0f};
#pragma unroll
    for (int i = 0; i < kWaves; ++i) r = lse_merge_fast(r, Lse{wm[i], wl[i]});
    ws.part[(b * G + g) * 2] = r.m;
    ws.part[(b * G + g) * 2 + 1] = r.s;
  }
  const float* xf = smem;
  float v[2 * kHalf];
  bool under = false;
#pragma unroll
  for (int j = 0; j < 2 * kHalf; ++j) {
    v[j] = -INFINITY;
    if (mm[j] != 0xFFFFFFFFu) {
      const int o = int(mm[j] >> 16) + (j / kHalf) * BPD_SOFT_MEMBER_CHUNK;
      const int ow = (o >> 8) & (kWaves - 1);
      v[j] = xf[o];
      if (v[j] != -INFINITY) {
        const float mw = wm[ow];
        under = under || v[j] - mw < -80.0f;
        atomicAdd(&wsum[ow * C + int32_t(mm[j] & 0xFFFFu)], exp_shift(v[j], mw));
      }
    }
  }
  const bool exact = __syncthreads_or(under);
  float* out = ws.mid + (b * G + g) * int64_t(C) * 2;
  if (!exact) {
    for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
      float cm = -INFINITY;
#pragma unroll
      for (int i = 0; i < kWaves; ++i)
        if (wsum[i * C + c] > 0.0f) cm = fmaxf(cm, wm[i]);
      float cs = 0.0f;
      if (cm != -INFINITY) {
#pragma unroll
        for (int i = 0; i < kWaves; ++i)
          if (wsum[i * C + c] > 0.0f) cs += wsum[i * C + c] * exp_shift(wm[i], cm);
      }
      out[2 * c] = cm;
      out[2 * c + 1] = cs;
    }
    return;
  }
  // exact path: per-class maximum over the members, then the sums
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    cmax[c] = ord_of(-INFINITY);
    esum[c] = 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2 * kHalf; ++j)
    if (v[j] != -INFINITY) atomicMax(&cmax[int32_t(mm[j] & 0xFFFFu)], ord_of(v[j]));
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2 * kHalf; ++j) {
    if (v[j] != -INFINITY) {
      const int32_t c = int32_t(mm[j] & 0xFFFFu);
      atomicAdd(&esum[c], exp_shift(v[j], float_of_ord(cmax[c])));
    }
  }
  __syncthreads();
  for (int32_t c = threadIdx.x; c < C; c += kPriorThreads) {
    out[2 * c] = float_of_ord(cmax[c]);
    out[2 * c + 1] = esum[c];
  }
}

// Pieces stats, grid (G + Gp, rows): block g < G takes vocab chunk g
// (partial row logsumexp), blocks G.. the class pieces (one wave per piece,
// unnormalised piece logsumexp).
template <bool Vec>
__global__ __launch_bounds__(kPriorThreads) void prior_stats_pieces_kernel(
    const float* __restrict__ logits, int64_t ld, int64_t V, int64_t chunk, int G,
    BpdSoftClasses cls, PriorWs ws) {
  const int g = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int32_t P = cls.num_pieces;
  const float* row = logits + b * ld;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x / 64;
  constexpr int kWaves = kPriorThreads / 64;
  if (g >= G) {
    const int nw = (int(gridDim.x) - G) * kWaves;
    for (int32_t p = (g - G) * kWaves + wave; p < P; p += nw) {
      const int32_t m0 = cls.piece_off[p], m1 = cls.piece_off[p + 1];
      int32_t idx[kPieceMembers / 64];
#pragma unroll
      for (int j = 0; j < kPieceMembers / 64; ++j) {
        const int32_t i = m0 + lane + 64 * j;
        idx[j] = i < m1 ? cls.class_tok[i] : -1;
      }
      float v[kPieceMembers / 64];
#pragma unroll
      for (int j = 0; j < kPieceMembers / 64; ++j) v[j] = idx[j] >= 0 ? row[idx[j]] : -INFINITY;
      Lse a{-INFINITY, 0.0f};
#pragma unroll
      for (int j = 0; j < kPieceMembers / 64; ++j) a = lse_push(a, v[j]);
      a = wave_lse(a);
      if (lane == 0) {
        ws.mid[(b * P + p) * 2] = a.m;
        ws.mid[(b * P + p) * 2 + 1] = a.s;
      }
    }
    return;
  }
  const int64_t lo = g * chunk;
  const int64_t hi = lo + chunk < V ? lo + chunk : V;
  Lse acc{-INFINITY, 0.0f};
  if (Vec) {
    const float4* row4 = reinterpret_cast<const float4*>(row);
    const int64_t q1 = hi / 4;
    for (int64_t q = lo / 4 + threadIdx.x; q < q1; q += int64_t(kPriorThreads) * kStatLoads) {
      float4 x[kStatLoads];
#pragma unroll
      for (int u = 0; u < kStatLoads; ++u) {
        const int64_t qq = q + int64_t(u) * kPriorThreads;
        x[u] = qq < q1 ? row4[qq] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      }
      float m = -INFINITY;
#pragma unroll
      for (int u = 0; u < kStatLoads; ++u) m = fmaxf(m, fmaxf(fmaxf(x[u].x, x[u].y), fmaxf(x[u].z, x[u].w)));
      if (m != -INFINITY) {
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < kStatLoads; ++u)
          sum += (exp_shift(x[u].x, m) + exp_shift(x[u].y, m)) + (exp_shift(x[u].z, m) + exp_shift(x[u].w, m));
        acc = lse_merge(acc, Lse{m, sum});
      }
    }
  } else {
    for (int64_t t = lo + threadIdx.x; t < hi; t += kPriorThreads) acc = lse_push(acc, row[t]);
  }
  acc = block_lse<kPriorThreads>(acc);
  if (threadIdx.x == 0) {
    ws.part[(b * G + g) * 2] = acc.m;
    ws.part[(b * G + g) * 2 + 1] = acc.s;
  }
}

// One block per row: merge the partials into lse[b] and the class sums, run
// the k-1 rounds with logZ, the class sums and (when they fit) the
// (class, next) pairs in LDS, and write zcls[b, c] = logZ(next state of
// class c from s_b) and lse[b].  The global loads of the prologue are all
// issued before the first wait.  In a round, a quad of lanes takes one
// state: each lane folds every fourth pair of the state into a running
// (max, sum of exp(v - max)), and the quad merges the four by DPP exchanges.
constexpr int kRoundThreads = 1024;
constexpr int kPairRegs = 8;     // pairs per thread held in registers while they load

// DPP quad permutations: lane i reads lane i ^ 1, lane i ^ 2 of its quad;
// row_half_mirror: lane i of each aligned group of eight reads lane 7 - i
// (a lane of the other quad: after a quad reduction, that quad's result)
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;

template <int Ctrl>
__device__ inline float quad_read(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), Ctrl, 0xF, 0xF, false));
}

// (m, s) <- merge of (m, s) with the pair held by the lane Ctrl names
template <int Ctrl>
__device__ inline void quad_lse_step(float& m, float& s) {
  const float mo = quad_read<Ctrl>(m), so = quad_read<Ctrl>(s);
  const float nm = fmaxf(m, mo);
  if (nm != -INFINITY) {
    s = s * exp_shift(m, nm) + so * exp_shift(mo, nm);
  }
  m = nm;
}

// max / sum over the eight lanes of an aligned group (quad DPP, then the
// other quad); every lane of the group gets the result
__device__ inline float group8_max(float x) {
  x = fmaxf(x, quad_read<kDppQuadXor1>(x));
  x = fmaxf(x, quad_read<kDppQuadXor2>(x));
  return fmaxf(x, quad_read<kDppHalfMirror>(x));
}
__device__ inline float group8_sum(float x) {
  x += quad_read<kDppQuadXor1>(x);
  x += quad_read<kDppQuadXor2>(x);
  return x + quad_read<kDppHalfMirror>(x);
}

template <bool PairsInLds>
__device__ inline uint32_t prior_pair(const uint32_t* pr, const BpdSoftClasses& cls, int32_t i) {
  if (PairsInLds) return pr[i];
  return (uint32_t(cls.pair_class[i]) << 16) | uint32_t(cls.pair_next[i]);
}

__device__ inline float prior_value(float x, float lse, int64_t t, float z, bool acc_s, int32_t eos,
                                    float alpha) {
  const float lp = x - lse;
  if (t == eos) return acc_s ? lp : -INFINITY;
  if (z == -INFINITY) return -INFINITY;
  return alpha != 0.0f ? fmaf(alpha, z, lp) : lp;
}

// The rounds and the epilogue of the prior lookahead for row b, by the
// kRoundThreads threads of its block: lc holds the class logsumexps of the
// row (LDS, reused for zcls), z0 / z1 the state values (z0 initialised: 0
// for live states, -inf else), flag / so the state flags and pair offsets,
// pr the pairs (PairsInLds); writes zcls[b] and lse[b] to the workspace.
template <bool PairsInLds>
__device__ __forceinline__ void prior_rounds_tail(float* lc, float* z0, float* z1, const uint8_t* flag,
                                                  const int32_t* so, const uint32_t* pr,
                                                  const BpdSoftClasses& cls, int32_t S, int32_t rounds,
                                                  float lse, float lp_eos, int32_t sb, int64_t b,
                                                  const PriorWs& ws) {
  const int tid = threadIdx.x;
  const int32_t C = cls.num_classes;
  // eight lanes per state: lane l folds pairs l, l + 8, ... of its state
  constexpr int kLanes = 8;
  constexpr int kGroups = kRoundThreads / kLanes;
  constexpr int kRegPairs = 16;  // pairs per lane kept in registers across the rounds
  const int grp = tid / kLanes, gl = tid % kLanes;
  float* zc = z0;
  float* zn = z1;
  // the fold of one (value, ...) into a running (max, sum of exp(v - max))
  auto fold = [](float& m, float& sm, float x) {
    if (x == -INFINITY) return;
    if (x > m) {
      sm = (m == -INFINITY ? 0.0f : sm * exp_shift(m, x)) + 1.0f;
      m = x;
    } else {
      sm += exp_shift(x, m);
    }
  };
  // the group's (max, sum) into zn[s]
  auto finish = [&](int32_t s, bool on, float m, float sm) {
    quad_lse_step<kDppQuadXor1>(m, sm);
    quad_lse_step<kDppQuadXor2>(m, sm);
    {
      // the two quads of the state
      const float mo = quad_read<kDppHalfMirror>(m), so4 = quad_read<kDppHalfMirror>(sm);
      const float nm = fmaxf(m, mo);
      if (nm != -INFINITY) sm = sm * exp_shift(m, nm) + so4 * exp_shift(mo, nm);
      m = nm;
    }
    if (on && gl == 0) {
      const uint8_t f = flag[s];
      float v = m == -INFINITY ? -INFINITY : m + logf(sm) - lse;
      if (f & 2) v = log_add_exp(v, lp_eos);
      zn[s] = (f & 1) ? v : -INFINITY;
    }
  };
  if (S <= kGroups) {
    // one state per group; a lane's first kRegPairs pairs are gathered once
    // as (class logsumexp, next state), so a round reads only zc for them
    const int32_t s = grp;
    const bool on = s < S;
    const int32_t i0 = on ? so[s] : 0, i1 = on ? so[s + 1] : 0;
    float w[kRegPairs];
    int32_t nx[kRegPairs];
#pragma unroll
    for (int u = 0; u < kRegPairs; ++u) {
      const int32_t i = i0 + gl + kLanes * u;
      const uint32_t p = i < i1 ? prior_pair<PairsInLds>(pr, cls, i) : 0u;
      w[u] = i < i1 ? lc[p >> 16] : -INFINITY;
      nx[u] = i < i1 ? int32_t(p & 0xFFFFu) : 0;
    }
    const int32_t i_rest = i0 + kLanes * kRegPairs;
    for (int32_t j = 0; j < rounds; ++j) {
      float v[kRegPairs];
#pragma unroll
      for (int u = 0; u < kRegPairs; ++u) v[u] = w[u] + zc[nx[u]];  // zc is never +inf
      float m = v[0];
#pragma unroll
      for (int u = 1; u < kRegPairs; ++u) m = fmaxf(m, v[u]);
      float sm = 0.0f;
      if (m != -INFINITY) {
        // pairwise: four dependent adds instead of sixteen
        float e[kRegPairs];
#pragma unroll
        for (int u = 0; u < kRegPairs; ++u) e[u] = exp_shift(v[u], m);
#pragma unroll
        for (int w = kRegPairs / 2; w > 0; w /= 2) {
#pragma unroll
          for (int u = 0; u < w; ++u) e[u] += e[u + w];
        }
        sm = e[0];
      }
      for (int32_t i = i_rest + gl; i < i1; i += kLanes) {
        const uint32_t p = prior_pair<PairsInLds>(pr, cls, i);
        fold(m, sm, lc[p >> 16] + zc[p & 0xFFFFu]);
      }
      finish(s, on, m, sm);
      __syncthreads();
      float* t = zc;
      zc = zn;
      zn = t;
    }
  } else {
    for (int32_t j = 0; j < rounds; ++j) {
      for (int32_t s0 = 0; s0 < S; s0 += kGroups) {
        const int32_t s = s0 + grp;
        const bool on = s < S;
        const int32_t i1 = on ? so[s + 1] : 0;
        float m = -INFINITY, sm = 0.0f;
        for (int32_t i = (on ? so[s] : 0) + gl; i < i1; i += kLanes) {
          const uint32_t p = prior_pair<PairsInLds>(pr, cls, i);
          fold(m, sm, lc[p >> 16] + zc[p & 0xFFFFu]);
        }
        finish(s, on, m, sm);
      }
      __syncthreads();
      float* t = zc;
      zc = zn;
      zn = t;
    }
  }

  // zcls[b, c] = logZ(next state of class c from s_b), -inf when rejected
  for (int32_t c = tid; c < C; c += kRoundThreads) lc[c] = -INFINITY;
  __syncthreads();
  if (sb >= 0 && sb < S) {
    for (int32_t i = so[sb] + tid; i < so[sb + 1]; i += kRoundThreads) {
      const uint32_t p = prior_pair<PairsInLds>(pr, cls, i);
      lc[p >> 16] = zc[p & 0xFFFFu];
    }
  }
  __syncthreads();
  for (int32_t c = tid; c < C; c += kRoundThreads) ws.zcls[b * C + c] = lc[c];
  if (tid == 0) ws.lse[b] = lse;
}

template <bool PairsInLds, bool ClassStats>
__global__ __launch_bounds__(kRoundThreads) void prior_rounds_kernel(
    const float* __restrict__ logits, int64_t ld, int32_t S, int G, BpdSoftClasses cls,
    const uint8_t* __restrict__ accept, const uint8_t* __restrict__ live, int32_t eos,
    const int32_t* __restrict__ states, const int64_t* __restrict__ slots, int32_t rounds,
    PriorWs ws) {
  extern __shared__ __align__(16) float lds[];
  __shared__ float lse_sh;
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t C = cls.num_classes, P = cls.num_pieces, NP = cls.num_pairs;
  float* lc = lds;                                        // [C] class logsumexp, later zcls
  float* z0 = lc + C;                                     // [S]
  float* z1 = z0 + S;                                     // [S]
  uint8_t* flag = reinterpret_cast<uint8_t*>(z1 + S);     // [S] bit 0 live, bit 1 accept
  int32_t* so = reinterpret_cast<int32_t*>(z1 + S + (S + 3) / 4);  // [S + 1]
  uint32_t* pr = reinterpret_cast<uint32_t*>(so + S + 1); // [pairs] class << 16 | next (PairsInLds)

  // global loads: the EOS logit, the pairs, the class partials, the row
  // partials, the state flags and offsets
  const float x_eos = eos >= 0 ? logits[b * ld + eos] : -INFINITY;
  uint32_t pv[kPairRegs];
  if (PairsInLds) {
#pragma unroll
    for (int u = 0; u < kPairRegs; ++u) {
      const int32_t j = tid + u * kRoundThreads;
      pv[u] = j < NP ? (uint32_t(cls.pair_class[j]) << 16) | uint32_t(cls.pair_next[j]) : 0u;
    }
  }
  const float* mid = ws.mid + b * int64_t(G) * C * 2;  // [G][C] (max, sum)
  // class partials: eight lanes per class, lane q takes chunks q, q + 8, ...;
  // those of the first 128 classes and 32 chunks are loaded here
  constexpr int kMergeLanes = 8, kMergeRegs = 4;
  const int mc = tid / kMergeLanes, mq = tid % kMergeLanes;
  float2 mv[kMergeRegs];
  if (ClassStats) {
#pragma unroll
    for (int u = 0; u < kMergeRegs; ++u) {
      const int g = mq + kMergeLanes * u;
      mv[u] = mc < C && g < G ? *reinterpret_cast<const float2*>(mid + (int64_t(g) * C + mc) * 2)
                              : make_float2(-INFINITY, 0.0f);
    }
  }
  // the row's state, needed only at the end, loaded with the rest
  const int32_t sb = states[slots ? slots[b] : b];
  Lse part{-INFINITY, 0.0f};
  if (tid < 64 && tid < G) part = Lse{ws.part[(b * G + tid) * 2], ws.part[(b * G + tid) * 2 + 1]};
  const uint8_t lv0 = tid < S ? live[tid] : 0;
  const uint8_t ac0 = tid < S ? accept[tid] : 0;
  const int32_t so0 = tid <= S ? cls.state_off[tid] : 0;

  if (tid < 64) {
    for (int i = tid + 64; i < G; i += 64) part = lse_merge(part, Lse{ws.part[(b * G + i) * 2], ws.part[(b * G + i) * 2 + 1]});
    part = wave_lse(part);
    if (tid == 0) lse_sh = lse_value(part);
  }
  for (int32_t s = tid; s < S; s += kRoundThreads) {
    const bool lv = (s == tid ? lv0 : live[s]) != 0;
    const bool ac = (s == tid ? ac0 : accept[s]) != 0;
    flag[s] = uint8_t((lv ? 1 : 0) | (ac ? 2 : 0));
    z0[s] = lv ? 0.0f : -INFINITY;
  }
  for (int32_t s = tid; s <= S; s += kRoundThreads) so[s] = s == tid ? so0 : cls.state_off[s];
  if (PairsInLds) {
#pragma unroll
    for (int u = 0; u < kPairRegs; ++u) {
      const int32_t j = tid + u * kRoundThreads;
      if (j < NP) pr[j] = pv[u];
    }
    for (int32_t j = tid + kPairRegs * kRoundThreads; j < NP; j += kRoundThreads)
      pr[j] = (uint32_t(cls.pair_class[j]) << 16) | uint32_t(cls.pair_next[j]);
  }
  __syncthreads();
  if (ClassStats) {
    // class c: the maximum of its G chunk partials over the group's lanes,
    // then the rescaled sum (every lane runs the same loop: the group
    // exchanges need all of them)
    for (int32_t c0 = 0; c0 < C; c0 += kRoundThreads / kMergeLanes) {
      const int32_t c = c0 + mc;
      float2 v[kMergeRegs];
#pragma unroll
      for (int u = 0; u < kMergeRegs; ++u) {
        const int g = mq + kMergeLanes * u;
        v[u] = c0 == 0 ? mv[u]
                       : (c < C && g < G ? *reinterpret_cast<const float2*>(mid + (int64_t(g) * C + c) * 2)
                                         : make_float2(-INFINITY, 0.0f));
      }
      float cm = -INFINITY;
#pragma unroll
      for (int u = 0; u < kMergeRegs; ++u) cm = fmaxf(cm, v[u].x);
      for (int g = mq + kMergeLanes * kMergeRegs; c < C && g < G; g += kMergeLanes)
        cm = fmaxf(cm, mid[(int64_t(g) * C + c) * 2]);
      cm = group8_max(cm);
      float csum = 0.0f;
      if (cm != -INFINITY) {
#pragma unroll
        for (int u = 0; u < kMergeRegs; ++u)
          if (v[u].x != -INFINITY) csum += v[u].y * exp_shift(v[u].x, cm);
        for (int g = mq + kMergeLanes * kMergeRegs; c < C && g < G; g += kMergeLanes) {
          const float2 w = *reinterpret_cast<const float2*>(mid + (int64_t(g) * C + c) * 2);
          if (w.x != -INFINITY) csum += w.y * exp_shift(w.x, cm);
        }
      }
      csum = group8_sum(csum);
      if (mq == 0 && c < C) lc[c] = csum > 0.0f ? cm + logf(csum) : -INFINITY;
    }
  } else {
    // [P] piece (max, sum) pairs, 8-byte aligned after the pairs
    // (offsets from the LDS base rather than an integer address, so that the
    // accesses stay LDS ones)
    const size_t pc_at = size_t(reinterpret_cast<char*>(pr + (PairsInLds ? NP : 0)) - reinterpret_cast<char*>(lds));
    float2* pc = reinterpret_cast<float2*>(reinterpret_cast<char*>(lds) + ((pc_at + 7) & ~size_t(7)));
    for (int32_t p = tid; p < P; p += kRoundThreads)
      pc[p] = make_float2(ws.mid[(b * P + p) * 2], ws.mid[(b * P + p) * 2 + 1]);
    __syncthreads();
    for (int32_t c = tid; c < C; c += kRoundThreads) {
      Lse a{-INFINITY, 0.0f};
      for (int32_t p = cls.class_piece[c]; p < cls.class_piece[c + 1]; ++p) a = lse_merge(a, Lse{pc[p].x, pc[p].y});
      lc[c] = lse_value(a);
    }
  }
  __syncthreads();
  const float lse = lse_sh;
  const float lp_eos = eos >= 0 ? x_eos - lse : -INFINITY;
  prior_rounds_tail<PairsInLds>(lc, z0, z1, flag, so, pr, cls, S, rounds, lse, lp_eos, sb, b, ws);
}

constexpr int kOutLoads = 4;          // float4 loads in flight per thread (prior_out_kernel)
constexpr int kOutLdsClasses = 4096;  // zcls rows up to this size are staged in LDS

// grid (ceil(V / (16 * 256)), rows); each thread rewrites 16 tokens, four
// float4 groups 256 * 4 tokens apart (coalesced per group).  Narrow: the
// class ids come from the uint16 map (half the bytes; 0xFFFF: no class).
template <bool Vec, bool ZInLds, bool Narrow>
__global__ __launch_bounds__(kPriorOutThreads) void prior_out_kernel(
    float* __restrict__ logits, int64_t ld, int64_t V, const int32_t* __restrict__ token_class,
    const uint16_t* __restrict__ token_class16, int32_t C, const float* __restrict__ lse_in, const float* __restrict__ zcls, int32_t S,
    const uint8_t* __restrict__ accept, int32_t eos, const int32_t* __restrict__ states,
    const int64_t* __restrict__ slots, float alpha, int32_t* __restrict__ err) {
  __shared__ float zs[ZInLds ? kOutLdsClasses : 1];
  const int64_t b = blockIdx.y;
  const int64_t base = int64_t(blockIdx.x) * kPriorOutThreads * 4 * kOutLoads;
  const int32_t s = states[slots ? slots[b] : b];
  float* row = logits + b * ld;
  if (s < 0 || s >= S) {
    if (s >= S && err && blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
    for (int u = 0; u < 4 * kOutLoads; ++u) {
      const int64_t t = base + int64_t(u) * kPriorOutThreads + threadIdx.x;
      if (t < V) row[t] = -INFINITY;
    }
    return;
  }
  const float* zrow = zcls + b * C;
  if (ZInLds) {
    for (int32_t c = threadIdx.x; c < C; c += kPriorOutThreads) zs[c] = zrow[c];
    __syncthreads();
  }
  const float* z = ZInLds ? zs : zrow;
  const float lse = lse_in[b];
  const bool acc_s = accept[s] != 0;
  auto zof = [&](int32_t c) { return c >= 0 ? z[c] : -INFINITY; };
  if (Vec) {
    // class ids first (the map is shared by every row and stays in L2),
    // then the logits only of the groups of four that hold a token with a
    // finite lookahead value or EOS: every other output is -inf whatever the
    // logit, so those reads are skipped (a line of rejected tokens is only
    // written)
    int4 c[kOutLoads];
#pragma unroll
    for (int u = 0; u < kOutLoads; ++u) {
      const int64_t t = base + (int64_t(u) * kPriorOutThreads + threadIdx.x) * 4;
      if (Narrow) {
        const uint2 n = t < V ? *reinterpret_cast<const uint2*>(token_class16 + t) : make_uint2(~0u, ~0u);
        c[u] = make_int4(narrow_class(n.x & 0xFFFFu), narrow_class(n.x >> 16), narrow_class(n.y & 0xFFFFu),
                         narrow_class(n.y >> 16));
      } else {
        c[u] = t < V ? *reinterpret_cast<const int4*>(token_class + t) : make_int4(-1, -1, -1, -1);
      }
    }
    float4 zv[kOutLoads];
    float4 x[kOutLoads];
#pragma unroll
    for (int u = 0; u < kOutLoads; ++u) {
      const int64_t t = base + (int64_t(u) * kPriorOutThreads + threadIdx.x) * 4;
      zv[u] = make_float4(zof(c[u].x), zof(c[u].y), zof(c[u].z), zof(c[u].w));
      const bool need = t < V && (zv[u].x != -INFINITY || zv[u].y != -INFINITY || zv[u].z != -INFINITY ||
                                  zv[u].w != -INFINITY || (eos >= t && eos < t + 4));
      x[u] = need ? *reinterpret_cast<const float4*>(row + t) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int u = 0; u < kOutLoads; ++u) {
      const int64_t t = base + (int64_t(u) * kPriorOutThreads + threadIdx.x) * 4;
      if (t < V) {
        float4 o;
        o.x = prior_value(x[u].x, lse, t, zv[u].x, acc_s, eos, alpha);
        o.y = prior_value(x[u].y, lse, t + 1, zv[u].y, acc_s, eos, alpha);
        o.z = prior_value(x[u].z, lse, t + 2, zv[u].z, acc_s, eos, alpha);
        o.w = prior_value(x[u].w, lse, t + 3, zv[u].w, acc_s, eos, alpha);
        *reinterpret_cast<float4*>(row + t) = o;
      }
    }
  } else {
    for (int u = 0; u < 4 * kOutLoads; ++u) {
      const int64_t t = base + int64_t(u) * kPriorOutThreads + threadIdx.x;
      if (t < V) row[t] = prior_value(row[t], lse, t, zof(token_class[t]), acc_s, eos, alpha);
    }
  }
}


// Member-list output, grid (ceil(V / 4096), rows): block g rewrites the
// 4096-token member chunk g of its row.  The chunk is staged in LDS as -inf;
// the threads take the chunk's member list (Cap slots, 0xFFFFFFFF empty),
// gather the logits of the members whose class has a finite lookahead value
// from the row's state and write x - lse + alpha * z there (EOS: its log
// softmax when the state accepts); the chunk then goes out as coalesced
// float4 non-temporal stores (every 128-byte line written whole; nothing
// reads the rows again in this call).  Needs vocab, ld and the logits
// aligned to 4 floats.
template <int Cap>
__global__ __launch_bounds__(kPriorOutThreads) void prior_out_list_kernel(
    float* __restrict__ logits, int64_t ld, int64_t V, const uint32_t* __restrict__ members, int32_t C,
    const float* __restrict__ lse_in, const float* __restrict__ zcls, int32_t S,
    const uint8_t* __restrict__ accept, int32_t eos, const int32_t* __restrict__ states,
    const int64_t* __restrict__ slots, float alpha, int32_t* __restrict__ err) {
  constexpr int kSlots = Cap / kPriorOutThreads;
  constexpr int kGroups = BPD_SOFT_MEMBER_CHUNK / 4 / kPriorOutThreads;  // float4 groups per thread
  __shared__ float4 outs[BPD_SOFT_MEMBER_CHUNK / 4];
  __shared__ float zs[kLdsClasses];
  const int64_t b = blockIdx.y;
  const int64_t base = int64_t(blockIdx.x) * BPD_SOFT_MEMBER_CHUNK;
  const int32_t s = states[slots ? slots[b] : b];
  float* row = logits + b * ld;
  const float4 ninf = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  if (s < 0 || s >= S) {
    if (s >= S && err && blockIdx.x == 0 && threadIdx.x == 0) atomicOr(err, BPD_FLAG_STATE_RANGE);
#pragma unroll
    for (int q = 0; q < kGroups; ++q) {
      const int64_t t = base + (int64_t(q) * kPriorOutThreads + threadIdx.x) * 4;
      if (t < V) *reinterpret_cast<float4*>(row + t) = ninf;
    }
    return;
  }
  uint32_t mm[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) mm[j] = members[int64_t(blockIdx.x) * Cap + j * kPriorOutThreads + threadIdx.x];
  const float* zrow = zcls + b * C;
  for (int32_t c = threadIdx.x; c < C; c += kPriorOutThreads) zs[c] = zrow[c];
#pragma unroll
  for (int q = 0; q < kGroups; ++q) outs[q * kPriorOutThreads + threadIdx.x] = ninf;
  const float lse = lse_in[b];
  const bool acc_s = accept[s] != 0;
  __syncthreads();
  // gathers of the members that keep a finite value (all issued, then used)
  float xv[kSlots], zv[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    zv[j] = -INFINITY;
    if (mm[j] != 0xFFFFFFFFu) {
      const int64_t t = base + int64_t(mm[j] >> 16);
      if (t != eos) zv[j] = zs[mm[j] & 0xFFFFu];
    }
    xv[j] = zv[j] != -INFINITY ? row[base + int64_t(mm[j] >> 16)] : 0.0f;
  }
  float* of = reinterpret_cast<float*>(outs);
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    if (zv[j] != -INFINITY) {
      const float lp = xv[j] - lse;
      of[mm[j] >> 16] = alpha != 0.0f ? fmaf(alpha, zv[j], lp) : lp;
    }
  }
  if (threadIdx.x == 0 && eos >= base && eos < base + BPD_SOFT_MEMBER_CHUNK && eos < V)
    of[eos - base] = acc_s ? row[eos] - lse : -INFINITY;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kGroups; ++q) {
    const int64_t t = base + (int64_t(q) * kPriorOutThreads + threadIdx.x) * 4;
    if (t < V) {
      const float4 o = outs[q * kPriorOutThreads + threadIdx.x];
      __builtin_nontemporal_store(F4v{o.x, o.y, o.z, o.w}, reinterpret_cast<F4v*>(row + t));
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool force_pieces() {
  const char* e = std::getenv("BPD_SOFT_PRIOR_PIECES");
  return e && *e && std::strcmp(e, "0") != 0;
}

// BPD_SOFT_STATS=wave selects the wave-shift statistics over the class map
// (with the class-map output pass), members / classes the 4096-token class
// statistics (the member lists / the class map) instead of the member-list
// statistics and output (tests of those paths); BPD_SOFT_MEMBERS=0 selects
// the class map too
const char* stats_choice() {
  const char* e = std::getenv("BPD_SOFT_STATS");
  if (e && *e) return e;
  const char* me = std::getenv("BPD_SOFT_MEMBERS");
  if (me && std::strcmp(me, "0") == 0) return "classes";
  return "list";
}

}  // namespace
}  // namespace bpd

using namespace bpd;

extern "C" size_t bpd_soft_prior_workspace_bytes(int64_t rows, int64_t vocab, int32_t num_classes,
                                                 int32_t num_pieces) {
  if (rows <= 0 || vocab <= 0) return 0;
  const int32_t C = num_classes > 0 ? num_classes : 0, P = num_pieces > 0 ? num_pieces : 0;
  // room for every stats path
  const size_t a = prior_ws_bytes(rows, prior_plan(rows, vocab, C, P, false, false), C, P);
  const size_t b = prior_ws_bytes(rows, prior_plan(rows, vocab, C, P, true, false), C, P);
  const size_t w = prior_ws_bytes(rows, prior_plan(rows, vocab, C, P, false, true), C, P);
  const size_t m = a > b ? a : b;
  return m > w ? m : w;
}

namespace {

// The prior lookahead on a caller-provided workspace (both entry points).
int soft_prior_impl(float* logits, int64_t rows, int64_t vocab, int64_t ld, int32_t num_states,
                    const uint8_t* accept, const uint8_t* live, int32_t eos_id,
                    const int32_t* states, const int64_t* slots, const BpdSoftClasses* classes,
                    int32_t k, float alpha, void* workspace, size_t workspace_bytes, int32_t* err,
                    void* stream) {
  BPD_REQUIRE(rows >= 0 && vocab > 0 && ld >= vocab, "bad logits shape");
  BPD_REQUIRE(num_states > 0 && num_states <= kPriorMaxStates, "1..%d states", kPriorMaxStates);
  BPD_REQUIRE(classes, "null classes");
  const BpdSoftClasses cls = *classes;
  BPD_REQUIRE(cls.num_classes >= 0 && cls.num_pieces >= 0 && cls.num_pairs >= 0, "bad class counts");
  BPD_REQUIRE(k >= 1, "k must be >= 1");
  BPD_REQUIRE(eos_id < vocab, "eos id out of range");
  if (rows == 0) return BPD_OK;
  BPD_REQUIRE(rows < 65536, "at most 65535 rows");
  BPD_REQUIRE(workspace_bytes >= bpd_soft_prior_workspace_bytes(rows, vocab, cls.num_classes, cls.num_pieces),
              "workspace too small");
  BPD_REQUIRE(logits && accept && live && states && workspace && cls.class_off && cls.class_piece &&
                  cls.piece_off && cls.state_off && cls.token_class,
              "null pointer argument");
  const char* choice = stats_choice();
  // member lists: statistics over each 8192-token block's members and the
  // output pass over each 4096-token chunk's members (the default)
  const bool list_ok = std::strcmp(choice, "list") == 0 && cls.chunk_members != nullptr &&
                       cls.num_classes < 65535 &&
                       (cls.chunk_cap == 256 || cls.chunk_cap == 512 || cls.chunk_cap == 1024) &&
                       vocab % 4 == 0 && ld % 4 == 0 && aligned16(logits);
  const bool wide_ok = (std::strcmp(choice, "wave") == 0 && cls.token_class16 != nullptr &&
                        cls.num_classes < 65535 && vocab % 4 == 0 && ld % 4 == 0 && aligned16(logits) &&
                        (reinterpret_cast<uintptr_t>(cls.token_class16) & 7u) == 0) ||
                       list_ok;
  const PriorPlan pl = prior_plan(rows, vocab, cls.num_classes, cls.num_pieces, force_pieces(), wide_ok);
  const bool pieces = !pl.class_stats;
  const bool pairs_in_lds =
      cls.num_classes < 65536 &&
      prior_lds_bytes(num_states, cls.num_classes, cls.num_pieces, cls.num_pairs, true, pieces) <= kPriorMaxLds;
  const size_t lds = prior_lds_bytes(num_states, cls.num_classes, cls.num_pieces, cls.num_pairs, pairs_in_lds, pieces);
  BPD_REQUIRE(lds <= kPriorMaxLds, "%d states and %d classes exceed the LDS budget", num_states,
              cls.num_classes);
  hipStream_t st = as_stream(stream);
  const PriorWs ws = prior_ws(workspace, rows, pl, cls.num_classes, cls.num_pieces);
  const bool vec = vocab % 4 == 0 && ld % 4 == 0 && aligned16(logits) && aligned16(cls.token_class);
  if (pl.class_stats) {
    const dim3 grid = dim3(unsigned(pl.G), unsigned(rows));
    const bool narrow = cls.token_class16 != nullptr && cls.num_classes < 65535;
    const bool nvec = vocab % 4 == 0 && ld % 4 == 0 && aligned16(logits) &&
                      (reinterpret_cast<uintptr_t>(cls.token_class16) & 7u) == 0;
#define BPD_PRIOR_STATS(VEC, NARROW)                                                            \
  prior_stats_classes_kernel<VEC, NARROW><<<grid, kPriorThreads, 0, st>>>(logits, ld, vocab,    \
                                                                         cls.token_class,       \
                                                                         cls.token_class16,     \
                                                                         cls.num_classes, ws)
    const bool members = vocab % 4 == 0 && ld % 4 == 0 && aligned16(logits) && cls.chunk_members != nullptr &&
                         cls.num_classes < 65535 && std::strcmp(choice, "classes") != 0 &&
                         (cls.chunk_cap == 256 || cls.chunk_cap == 512 || cls.chunk_cap == 1024);
    const size_t mlds = size_t(kStatChunk) * sizeof(float) + size_t(cls.num_classes) * 8;
    const size_t llds = (size_t(kWideChunk) + size_t(kPriorThreads / 64 + 2) * cls.num_classes) * 4;
    if (pl.wide && list_ok && cls.chunk_cap == 256)
      prior_stats_list_kernel<256><<<grid, kPriorThreads, llds, st>>>(logits, ld, vocab, cls.chunk_members,
                                                                      cls.num_classes, ws);
    else if (pl.wide && list_ok && cls.chunk_cap == 512)
      prior_stats_list_kernel<512><<<grid, kPriorThreads, llds, st>>>(logits, ld, vocab, cls.chunk_members,
                                                                      cls.num_classes, ws);
    else if (pl.wide && list_ok)
      prior_stats_list_kernel<1024><<<grid, kPriorThreads, llds, st>>>(logits, ld, vocab, cls.chunk_members,
                                                                       cls.num_classes, ws);
    else if (pl.wide)
      prior_stats_wave_kernel<<<grid, kPriorThreads, size_t(cls.num_classes) * (kPriorThreads / 64 + 2) * 4, st>>>(
          logits, ld, vocab, cls.token_class16, cls.num_classes, ws);
    else if (members && cls.chunk_cap == 256)
      prior_stats_members_kernel<256><<<grid, kPriorThreads, mlds, st>>>(logits, ld, vocab, cls.chunk_members, cls.num_classes, ws);
    else if (members && cls.chunk_cap == 512)
      prior_stats_members_kernel<512><<<grid, kPriorThreads, mlds, st>>>(logits, ld, vocab, cls.chunk_members, cls.num_classes, ws);
    else if (members)
      prior_stats_members_kernel<1024><<<grid, kPriorThreads, mlds, st>>>(logits, ld, vocab, cls.chunk_members, cls.num_classes, ws);
    else if (narrow && nvec) BPD_PRIOR_STATS(true, true);
    else if (narrow) BPD_PRIOR_STATS(false, true);
    else if (vec) BPD_PRIOR_STATS(true, false);
    else BPD_PRIOR_STATS(false, false);
#undef BPD_PRIOR_STATS
  } else {
    int64_t chunk = (vocab + pl.G - 1) / pl.G;
    chunk = (chunk + 3) / 4 * 4;
    const dim3 grid = dim3(unsigned(pl.G + pl.Gp), unsigned(rows));
    if (vec) {
      prior_stats_pieces_kernel<true><<<grid, kPriorThreads, 0, st>>>(logits, ld, vocab, chunk, pl.G, cls, ws);
    } else {
      prior_stats_pieces_kernel<false><<<grid, kPriorThreads, 0, st>>>(logits, ld, vocab, chunk, pl.G, cls, ws);
    }
  }
  BPD_LAUNCHED();
#define BPD_PRIOR_ROUNDS(LDSP, CLS)                                                                  \
  prior_rounds_kernel<LDSP, CLS><<<unsigned(rows), kRoundThreads, lds, st>>>(                       \
      logits, ld, num_states, pl.G, cls, accept, live, eos_id, states, slots, k - 1, ws)
  if (pairs_in_lds && pl.class_stats) BPD_PRIOR_ROUNDS(true, true);
  else if (pairs_in_lds) BPD_PRIOR_ROUNDS(true, false);
  else if (pl.class_stats) BPD_PRIOR_ROUNDS(false, true);
  else BPD_PRIOR_ROUNDS(false, false);
#undef BPD_PRIOR_ROUNDS
  BPD_LAUNCHED();
  const dim3 ogrid = dim3(unsigned((vocab + 4 * kOutLoads * kPriorOutThreads - 1) /
                                   (4 * kOutLoads * kPriorOutThreads)),
                          unsigned(rows));
  const bool z_lds = cls.num_classes <= kOutLdsClasses;
  const bool onarrow = vec && cls.token_class16 != nullptr && cls.num_classes < 65535 &&
                       (reinterpret_cast<uintptr_t>(cls.token_class16) & 7u) == 0;
#define BPD_PRIOR_OUT(VEC, ZL, NW)                                                                \
  prior_out_kernel<VEC, ZL, NW><<<ogrid, kPriorOutThreads, 0, st>>>(                            \
      logits, ld, vocab, cls.token_class, cls.token_class16, cls.num_classes, ws.lse, ws.zcls,   \
      num_states, accept, eos_id, states, slots, alpha, err)
  const dim3 lgrid = dim3(unsigned((vocab + BPD_SOFT_MEMBER_CHUNK - 1) / BPD_SOFT_MEMBER_CHUNK), unsigned(rows));
#define BPD_PRIOR_OUT_LIST(CAP)                                                                      \
  prior_out_list_kernel<CAP><<<lgrid, kPriorOutThreads, 0, st>>>(                                   \
      logits, ld, vocab, cls.chunk_members, cls.num_classes, ws.lse, ws.zcls, num_states, accept, eos_id, \
      states, slots, alpha, err)
  if (list_ok && pl.class_stats && cls.chunk_cap == 256) BPD_PRIOR_OUT_LIST(256);
  else if (list_ok && pl.class_stats && cls.chunk_cap == 512) BPD_PRIOR_OUT_LIST(512);
  else if (list_ok && pl.class_stats) BPD_PRIOR_OUT_LIST(1024);
  else if (onarrow && z_lds) BPD_PRIOR_OUT(true, true, true);
  else if (onarrow) BPD_PRIOR_OUT(true, false, true);
  else if (vec && z_lds) BPD_PRIOR_OUT(true, true, false);
  else if (vec) BPD_PRIOR_OUT(true, false, false);
  else if (z_lds) BPD_PRIOR_OUT(false, true, false);
  else BPD_PRIOR_OUT(false, false, false);
#undef BPD_PRIOR_OUT
#undef BPD_PRIOR_OUT_LIST
  BPD_LAUNCHED();
  return BPD_OK;
}

}  // namespace

extern "C" int bpd_soft_prior(float* logits, int64_t rows, int64_t vocab, int64_t ld,
                              int32_t num_states, const uint8_t* accept, const uint8_t* live,
                              int32_t eos_id, const int32_t* states, const int64_t* slots,
                              const BpdSoftClasses* classes, int32_t k, float alpha,
                              void* workspace, size_t workspace_bytes, int32_t* err, void* stream) {
  return soft_prior_impl(logits, rows, vocab, ld, num_states, accept, live, eos_id, states, slots,
                         classes, k, alpha, workspace, workspace_bytes, err, stream);
}

// Workspace of the allocation-free entry point: a file-scope device array,
// one copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel or a copy: its device address comes from
// hipGetSymbolAddress, once per device, on the first call there.
static __device__ __align__(256) unsigned char scratch[BPD_SOFT_PRIOR_SCRATCH_BYTES];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

// Device address of `scratch` on the device `stream` belongs to.
int scratch_address(void* stream, void** out) {
  hipDevice_t dev = 0;
  BPD_HIP(hipStreamGetDevice(as_stream(stream), &dev));
  BPD_REQUIRE(dev >= 0 && dev < kScratchDevices, "device %d out of range", int(dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = 0;
    BPD_HIP(hipGetDevice(&cur));
    if (cur != dev) BPD_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) BPD_HIP(hipSetDevice(cur));
    if (e != hipSuccess)
      BPD_FAIL(BPD_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    BPD_REQUIRE(p != nullptr, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BPD_OK;
}
}  // namespace

extern "C" int bpd_soft_prior_noalloc(float* logits, int64_t rows, int64_t vocab, int64_t ld,
                                      int32_t num_states, const uint8_t* accept,
                                      const uint8_t* live, int32_t eos_id, const int32_t* states,
                                      const int64_t* slots, const BpdSoftClasses* classes,
                                      int32_t k, float alpha, int32_t* err, void* stream) {
  BPD_REQUIRE(classes, "null classes");
  BPD_REQUIRE(rows >= 0 && vocab > 0, "bad logits shape");
  const size_t need = bpd_soft_prior_workspace_bytes(rows, vocab, classes->num_classes,
                                                     classes->num_pieces);
  BPD_REQUIRE(need <= size_t(BPD_SOFT_PRIOR_SCRATCH_BYTES),
              "%lld rows x %d classes need %zu bytes of workspace, more than the %d-byte scratch of "
              "the allocation-free entry point",
              (long long)rows, classes->num_classes, need, BPD_SOFT_PRIOR_SCRATCH_BYTES);
  if (rows == 0) return BPD_OK;
  void* ws = nullptr;
  if (int rc = scratch_address(stream, &ws)) return rc;
  return soft_prior_impl(logits, rows, vocab, ld, num_states, accept, live, eos_id, states, slots,
                         classes, k, alpha, ws, size_t(BPD_SOFT_PRIOR_SCRATCH_BYTES), err, stream);
}

// Token classes of the prior recurrence (once per grammar, host side).
// Class c holds the tokens whose tok_next columns are equal once every entry
// outside [0, S) reads as "rejected"; tokens rejected in every state form no
// class (token_class -1).  Classes are numbered by their smallest token,
// members are listed in increasing token order and cut into pieces of at most
// 256 members; the (class, next) pairs of state s are listed in class order.
extern "C" int bpd_host_soft_classes(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                                     BpdSoftClasses* out) {
  BPD_REQUIRE(tok_next && out, "null pointer argument");
  BPD_REQUIRE(num_states > 0 && vocab > 0 && vocab < (int64_t(1) << 31), "bad table shape");
  const int32_t S = num_states;
  const int64_t V = vocab;
  auto norm = [&](int32_t d) { return (d >= 0 && d < S) ? d : -1; };
  std::vector<uint64_t> h(size_t(V), 1469598103934665603ull);
  std::vector<uint8_t> any(size_t(V), 0);
  for (int32_t s = 0; s < S; ++s) {
    const int32_t* r = tok_next + int64_t(s) * V;
    for (int64_t t = 0; t < V; ++t) {
      const int32_t d = norm(r[t]);
      h[size_t(t)] = (h[size_t(t)] ^ uint32_t(d)) * 1099511628211ull;
      any[size_t(t)] |= uint8_t(d >= 0);
    }
  }
  std::unordered_map<uint64_t, std::vector<int32_t>> by_hash;
  std::vector<int32_t> rep, cls(size_t(V), -1);
  for (int64_t t = 0; t < V; ++t) {
    if (!any[size_t(t)]) continue;
    auto& cands = by_hash[h[size_t(t)]];
    int32_t found = -1;
    for (const int32_t c : cands) {
      const int64_t u = rep[size_t(c)];
      bool same = true;
      for (int32_t s = 0; s < S && same; ++s)
        same = norm(tok_next[int64_t(s) * V + t]) == norm(tok_next[int64_t(s) * V + u]);
      if (same) {
        found = c;
        break;
      }
    }
    if (found < 0) {
      found = int32_t(rep.size());
      rep.push_back(int32_t(t));
      cands.push_back(found);
    }
    cls[size_t(t)] = found;
  }
  const int64_t C = int64_t(rep.size());
  std::vector<int64_t> size(size_t(C), 0);
  for (int64_t t = 0; t < V; ++t)
    if (cls[size_t(t)] >= 0) ++size[size_t(cls[size_t(t)])];
  int64_t members = 0, pieces = 0, pairs = 0;
  for (int64_t c = 0; c < C; ++c) {
    members += size[size_t(c)];
    pieces += (size[size_t(c)] + kPieceMembers - 1) / kPieceMembers;
  }
  for (int32_t s = 0; s < S; ++s)
    for (int64_t c = 0; c < C; ++c) pairs += norm(tok_next[int64_t(s) * V + rep[size_t(c)]]) >= 0;
  BPD_REQUIRE(pairs < (int64_t(1) << 31), "too many (class, next) pairs");
  const bool fill = out->class_off && out->class_tok && out->class_piece && out->piece_off &&
                    out->state_off && out->pair_class && out->pair_next && out->token_class;
  if (fill) {
    BPD_REQUIRE(out->num_classes == C && out->num_members == members && out->num_pieces == pieces &&
                    out->num_pairs == pairs,
                "class buffers were sized for another table (counts differ)");
  }
  out->num_classes = int32_t(C);
  out->num_members = int32_t(members);
  out->num_pieces = int32_t(pieces);
  out->num_pairs = int32_t(pairs);
  if (!fill) return BPD_OK;
  int64_t m = 0, p = 0;
  std::vector<int64_t> pos(size_t(C), 0);
  for (int64_t c = 0; c < C; ++c) {
    out->class_off[c] = int32_t(m);
    out->class_piece[c] = int32_t(p);
    pos[size_t(c)] = m;
    for (int64_t i = 0; i < size[size_t(c)]; i += kPieceMembers) out->piece_off[p++] = int32_t(m + i);
    m += size[size_t(c)];
  }
  out->class_off[C] = int32_t(m);
  out->class_piece[C] = int32_t(p);
  out->piece_off[p] = int32_t(m);
  for (int64_t t = 0; t < V; ++t) {
    out->token_class[t] = cls[size_t(t)];
    if (cls[size_t(t)] >= 0) out->class_tok[pos[size_t(cls[size_t(t)])]++] = int32_t(t);
  }
  int64_t q = 0;
  for (int32_t s = 0; s < S; ++s) {
    out->state_off[s] = int32_t(q);
    for (int64_t c = 0; c < C; ++c) {
      const int32_t d = norm(tok_next[int64_t(s) * V + rep[size_t(c)]]);
      if (d >= 0) {
        out->pair_class[q] = int32_t(c);
        out->pair_next[q] = d;
        ++q;
      }
    }
  }
  out->state_off[S] = int32_t(q);
  if (out->token_class16 && C < 65535)
    for (int64_t t = 0; t < V; ++t)
      out->token_class16[t] = cls[size_t(t)] < 0 ? uint16_t(0xFFFF) : uint16_t(cls[size_t(t)]);
  out->chunk_cap = 0;
  if (out->chunk_members && C < 65535) {
    const int64_t G = (V + BPD_SOFT_MEMBER_CHUNK - 1) / BPD_SOFT_MEMBER_CHUNK;
    int64_t most = 0;
    for (int64_t g = 0; g < G; ++g) {
      int64_t n = 0;
      for (int64_t t = g * BPD_SOFT_MEMBER_CHUNK; t < V && t < (g + 1) * BPD_SOFT_MEMBER_CHUNK; ++t)
        n += cls[size_t(t)] >= 0;
      most = n > most ? n : most;
    }
    const int32_t cap = most <= 256 ? 256 : most <= 512 ? 512 : most <= BPD_SOFT_MEMBER_CAP_MAX ? 1024 : 0;
    if (cap) {
      for (int64_t g = 0; g < G; ++g) {
        uint32_t* row = out->chunk_members + g * cap;
        int32_t n = 0;
        for (int64_t t = g * BPD_SOFT_MEMBER_CHUNK; t < V && t < (g + 1) * BPD_SOFT_MEMBER_CHUNK; ++t)
          if (cls[size_t(t)] >= 0)
            row[n++] = (uint32_t(t - g * BPD_SOFT_MEMBER_CHUNK) << 16) | uint32_t(cls[size_t(t)]);
        for (; n < cap; ++n) row[n] = 0xFFFFFFFFu;
      }
      out->chunk_cap = cap;
    }
  }
  return BPD_OK;
}

// Host form of bpd_soft_prior: direct sums over the vocab, accumulated in
// double (float32 logits in and out).
namespace {
struct LseD {
  double m, s;
};
inline LseD lse_push_d(LseD a, double x) {
  if (x == -INFINITY) return a;
  if (x > a.m) {
    a.s = (a.m == -INFINITY ? 0.0 : a.s * std::exp(a.m - x)) + 1.0;
    a.m = x;
  } else {
    a.s += std::exp(x - a.m);
  }
  return a;
}
inline double lse_value_d(LseD a) { return a.m == -INFINITY ? -INFINITY : a.m + std::log(a.s); }
inline double log_add_exp_d(double a, double b) {
  if (a == b && (a == INFINITY || a == -INFINITY)) return a;
  return std::fmax(a, b) + std::log1p(std::exp(-std::fabs(a - b)));
}
}  // namespace

extern "C" int bpd_host_soft_prior(float* logits, int64_t rows, int64_t vocab, int64_t ld,
                                   const int32_t* tok_next, int32_t num_states,
                                   const uint8_t* accept, const uint8_t* live, int32_t eos_id,
                                   const int32_t* states, const int64_t* slots, int32_t k,
                                   float alpha) {
  BPD_REQUIRE(rows >= 0 && vocab > 0 && ld >= vocab, "bad logits shape");
  BPD_REQUIRE(num_states > 0 && k >= 1 && eos_id < vocab, "bad arguments");
  const int32_t S = num_states;
  std::vector<double> cur(static_cast<size_t>(S)), nxt(static_cast<size_t>(S));
  for (int64_t b = 0; b < rows; ++b) {
    const int32_t s_b = states[slots ? slots[b] : b];
    if (s_b >= S) BPD_FAIL(BPD_ERR_INVALID, "index %d is out of bounds for dimension 0 with size %d", s_b, S);
  }
  for (int64_t b = 0; b < rows; ++b) {
    float* row = logits + b * ld;
    LseD r{-INFINITY, 0.0};
    for (int64_t t = 0; t < vocab; ++t) r = lse_push_d(r, row[t]);
    const double lse = lse_value_d(r);
    const double lp_eos = eos_id >= 0 ? row[eos_id] - lse : -INFINITY;
    for (int32_t s = 0; s < S; ++s) cur[size_t(s)] = live[s] ? 0.0 : -INFINITY;
    for (int32_t j = 0; j + 1 < k; ++j) {
      for (int32_t s = 0; s < S; ++s) {
        LseD a{-INFINITY, 0.0};
        const int32_t* tn = tok_next + int64_t(s) * vocab;
        for (int64_t t = 0; t < vocab; ++t) {
          const int32_t d = tn[t];
          if (d >= 0 && d < S && cur[size_t(d)] != -INFINITY) a = lse_push_d(a, row[t] + cur[size_t(d)]);
        }
        double v = lse_value_d(a);
        v = v == -INFINITY ? v : v - lse;
        if (accept[s]) v = log_add_exp_d(v, lp_eos);
        nxt[size_t(s)] = live[s] ? v : -INFINITY;
      }
      cur.swap(nxt);
    }
    const int32_t s_b = states[slots ? slots[b] : b];
    for (int64_t t = 0; t < vocab; ++t) {
      if (s_b < 0) {
        row[t] = -INFINITY;
        continue;
      }
      const double lp = row[t] - lse;
      double v;
      if (t == eos_id) {
        v = accept[s_b] ? lp : -INFINITY;
      } else {
        const int32_t d = tok_next[int64_t(s_b) * vocab + t];
        const double z = (d >= 0 && d < S) ? cur[size_t(d)] : -INFINITY;
        v = z == -INFINITY ? -INFINITY : (alpha != 0.0f ? lp + double(alpha) * z : lp);
      }
      row[t] = float(v);
    }
  }
  return BPD_OK;
}
