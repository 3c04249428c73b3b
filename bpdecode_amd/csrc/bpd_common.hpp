// Shared helpers for the libbpdecode_hip translation units: error reporting,
// logits element handling and the scalar fill conversion.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>

#include "bpdecode_hip.h"

namespace bpd {

// Thread-local message behind bpd_last_error().
void set_error(const char* fmt, ...);

#define BPD_FAIL(code, ...)        \
  do {                             \
    ::bpd::set_error(__VA_ARGS__); \
    return (code);                 \
  } while (0)

#define BPD_REQUIRE(cond, ...)                                 \
  do {                                                         \
    if (!(cond)) BPD_FAIL(BPD_ERR_INVALID, __VA_ARGS__);       \
  } while (0)

#define BPD_HIP(call)                                                            \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess)                                                        \
      BPD_FAIL(BPD_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_));            \
  } while (0)

// Launch-error check after a <<<>>> launch.
#define BPD_LAUNCHED()                                                           \
  do {                                                                           \
    hipError_t e_ = hipGetLastError();                                           \
    if (e_ != hipSuccess)                                                        \
      BPD_FAIL(BPD_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e_)); \
  } while (0)

// Element size of the logits dtypes every kernel takes (0: not one of them).
inline int elem_bytes(int dtype) {
  switch (dtype) {
    case BPD_DTYPE_F32: return 4;
    case BPD_DTYPE_F16: return 2;
    case BPD_DTYPE_BF16: return 2;
    default: return 0;
  }
}

// The dense tok_next mask also takes float64 (the reference's masked_fill_
// path accepts any float dtype).
inline int dense_elem_bytes(int dtype) { return dtype == BPD_DTYPE_F64 ? 8 : elem_bytes(dtype); }

// float -> bfloat16 bits, round to nearest even; NaN -> 0x7FC0 (the
// conversion c10::BFloat16 applies).
inline uint16_t bf16_bits_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if (std::isnan(f)) return 0x7FC0;
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return static_cast<uint16_t>(u >> 16);
}

// float -> IEEE half bits, round to nearest even (hardware conversion of the
// host compiler's _Float16).
inline uint16_t f16_bits_rne(float f) {
  _Float16 h = static_cast<_Float16>(f);
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

// The bit pattern masked_fill_ stores for a Python float `v` in a tensor of
// `dtype`: ATen converts the double scalar with an overflow check (finite
// values outside [lowest, max] of the target type raise) and then casts
// double -> float -> target (double stays double).  Returns BPD_ERR_OVERFLOW
// on the raising case.
inline int fill_bits64(int dtype, double v, uint64_t* out) {
  double lo, hi;
  const char* name;
  switch (dtype) {
    case BPD_DTYPE_F64:
      std::memcpy(out, &v, 8);
      return BPD_OK;
    case BPD_DTYPE_F32:
      lo = -static_cast<double>(std::numeric_limits<float>::max());
      hi = static_cast<double>(std::numeric_limits<float>::max());
      name = "float";
      break;
    case BPD_DTYPE_F16:
      lo = -65504.0;
      hi = 65504.0;
      name = "c10::Half";
      break;
    case BPD_DTYPE_BF16:
      lo = -3.3895313892515355e38;
      hi = 3.3895313892515355e38;
      name = "c10::BFloat16";
      break;
    default:
      BPD_FAIL(BPD_ERR_INVALID, "unknown logits dtype code %d", dtype);
  }
  if (std::isfinite(v) && (v < lo || v > hi))
    BPD_FAIL(BPD_ERR_OVERFLOW, "value cannot be converted to type %s without overflow", name);
  const float f = static_cast<float>(v);
  uint32_t u = 0;
  if (dtype == BPD_DTYPE_F32) {
    std::memcpy(&u, &f, 4);
  } else if (dtype == BPD_DTYPE_F16) {
    u = f16_bits_rne(f);
  } else {
    u = bf16_bits_rne(f);
  }
  *out = u;
  return BPD_OK;
}

// The same for the 2- and 4-byte dtypes (float64 is refused).
inline int fill_bits(int dtype, double v, uint32_t* out) {
  if (elem_bytes(dtype) == 0) BPD_FAIL(BPD_ERR_INVALID, "unknown logits dtype code %d", dtype);
  uint64_t f = 0;
  if (int rc = fill_bits64(dtype, v, &f)) return rc;
  *out = static_cast<uint32_t>(f);
  return BPD_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool token_dtype_ok(int d) {
  return d == BPD_INDEX_I32 || d == BPD_INDEX_I64 || d == BPD_INDEX_I64_LOW32;
}

// Token id b of `tokens` as an int64: int32 ids, int64 ids, or int64 ids read
// as their low 32 bits (two's complement), which is what tensor.to(int32)
// keeps.  Range checks are the caller's.
__host__ __device__ __forceinline__ int64_t read_token(const void* tokens, int dtype, int64_t b) {
  if (dtype == BPD_INDEX_I64) return static_cast<const int64_t*>(tokens)[b];
  if (dtype == BPD_INDEX_I64_LOW32)
    return int64_t(int32_t(uint32_t(static_cast<const uint64_t*>(tokens)[b])));
  return static_cast<const int32_t*>(tokens)[b];
}

}  // namespace bpd
