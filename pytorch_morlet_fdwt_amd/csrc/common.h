// Shared device/host helpers of the fdwt HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/fdwt_hip.h"

namespace fdwt {

// ------------------------------------------------------------------ storage types
struct bf16_t {
  uint16_t bits;
};

template <typename S>
struct Storage;
template <>
struct Storage<float> {
  __device__ static float load(const float* p, int64_t i) { return p[i]; }
  __device__ static void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Storage<double> {
  __device__ static double load(const double* p, int64_t i) { return p[i]; }
  __device__ static void store(double* p, int64_t i, double v) { p[i] = v; }
};
template <>
struct Storage<__half> {
  __device__ static float load(const __half* p, int64_t i) { return __half2float(p[i]); }
  __device__ static void store(__half* p, int64_t i, float v) { p[i] = __float2half(v); }
};
template <>
struct Storage<bf16_t> {
  __device__ static float load(const bf16_t* p, int64_t i) {
    return __uint_as_float(static_cast<uint32_t>(p[i].bits) << 16);
  }
  __device__ static void store(bf16_t* p, int64_t i, float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) {
      p[i].bits = static_cast<uint16_t>((u >> 16) | 0x40u);  // keep NaN a NaN
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
      p[i].bits = static_cast<uint16_t>(u >> 16);
    }
  }
};

// ------------------------------------------------------------------ boundary extension
// Modes of the reference (kernels/dwt.py:30-49): the period of the extended signal and the
// map of an extended position p onto [0, n).  `valid` is false only for zero padding.
__host__ __device__ inline int mode_period(int mode, int n) {
  switch (mode) {
    case FDWT_MODE_PERIODIC: return n;
    case FDWT_MODE_SYMMETRIC: return 2 * n;
    case FDWT_MODE_REFLECT: return 2 * n - 2;
    case FDWT_MODE_PERIODIZATION: return n + (n & 1);
    default: return 1;
  }
}

__host__ __device__ inline int normalize_mode(int mode, int n) {
  return (mode == FDWT_MODE_REFLECT && n == 1) ? FDWT_MODE_PERIODIC : mode;
}

__device__ inline int ext_index(int p, int n, int mode, int P, bool& valid) {
  if (mode == FDWT_MODE_ZERO) {
    valid = (p >= 0) && (p < n);
    return p;
  }
  valid = true;
  int q = p % P;
  if (q < 0) q += P;
  if (mode == FDWT_MODE_PERIODIC) return q;
  if (mode == FDWT_MODE_SYMMETRIC) return q < n ? q : P - 1 - q;
  if (mode == FDWT_MODE_REFLECT) return q < n ? q : P - q;
  return q < n ? q : n - 1;  // periodization of an odd signal repeats the last sample
}

// ------------------------------------------------------------------ misc
__host__ __device__ constexpr inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int dtype_size(int dtype) {
  switch (dtype) {
    case FDWT_F64: return 8;
    case FDWT_F16:
    case FDWT_BF16: return 2;
    default: return 4;
  }
}

}  // namespace fdwt

#define FDWT_CHECK_LAUNCH()                   \
  do {                                        \
    hipError_t e_ = hipGetLastError();        \
    if (e_ != hipSuccess) return (int)e_;     \
  } while (0)
