// Shared helpers for the gfx950 kernels of libcacheslide_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>

#include "../../include/cacheslide_hip.h"

namespace cs {

// ---------------------------------------------------------------- errors
void set_error(const char* fmt, ...);

#define CS_REQUIRE(cond, ...)            \
  do {                                   \
    if (!(cond)) {                       \
      ::cs::set_error(__VA_ARGS__);      \
      return CS_EINVAL;                  \
    }                                    \
  } while (0)

#define CS_LAUNCH_CHECK(what)                                                  \
  do {                                                                         \
    hipError_t err_ = hipGetLastError();                                       \
    if (err_ != hipSuccess) {                                                  \
      ::cs::set_error("%s: %s", what, hipGetErrorString(err_));                \
      return CS_ELAUNCH;                                                       \
    }                                                                          \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool present(const cs_view* v) { return v != nullptr && v->data != nullptr; }

inline int dtype_size(int dt) {
  switch (dt) {
    case CS_F32: return 4;
    case CS_F16: return 2;
    case CS_BF16: return 2;
    case CS_F64: return 8;
    case CS_I32: return 4;
    case CS_I64: return 8;
    case CS_U8: return 1;
    default: return 0;
  }
}

inline bool is_float_dtype(int dt) {
  return dt == CS_F32 || dt == CS_F16 || dt == CS_BF16 || dt == CS_F64;
}

// --------------------------------------------------------- numeric types
// bf16 and f16 are carried as raw 16-bit patterns; conversions are explicit so
// every rounding step is visible.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __host__ inline float bf16_to_float(uint16_t b) {
  union { uint32_t u; float f; } x;
  x.u = static_cast<uint32_t>(b) << 16;
  return x.f;
}

// Round-to-nearest-even float -> bf16 (NaN stays NaN), as torch's .to(bfloat16).
__device__ __host__ inline uint16_t float_to_bf16(float f) {
  union { uint32_t u; float f; } x;
  x.f = f;
  if ((x.u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((x.u >> 16) | 0x40u);
  uint32_t lsb = (x.u >> 16) & 1u;
  x.u += 0x7fffu + lsb;
  return static_cast<uint16_t>(x.u >> 16);
}

__device__ inline float f16_to_float(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return static_cast<float>(v);
}

__device__ inline uint16_t float_to_f16(float f) {
  _Float16 v = static_cast<_Float16>(f);
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// double -> bf16 / f16 as torch's CPU copy kernel does it: the double is first
// rounded to float, then the float is rounded to the 16-bit type (two roundings).
__device__ inline uint16_t double_to_bf16(double d) { return float_to_bf16(static_cast<float>(d)); }
__device__ inline uint16_t double_to_f16(double d) { return float_to_f16(static_cast<float>(d)); }

// Any non-finite element in a 16-byte word of KIND 0 bf16, 1 f16, 2 f32, 3 f64
// (exponent field all ones).
template <int KIND>
__device__ inline bool word_nonfinite(uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  bool bad = false;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if constexpr (KIND == 0) {
      bad |= ((w[q] & 0x7f80u) == 0x7f80u) || ((w[q] & 0x7f800000u) == 0x7f800000u);
    } else if constexpr (KIND == 1) {
      bad |= ((w[q] & 0x7c00u) == 0x7c00u) || ((w[q] & 0x7c000000u) == 0x7c000000u);
    } else if constexpr (KIND == 2) {
      bad |= (w[q] & 0x7f800000u) == 0x7f800000u;
    } else {
      if (q & 1) bad |= (w[q] & 0x7ff00000u) == 0x7ff00000u;
    }
  }
  return bad;
}

// Dynamic-dtype scalar loads/stores (small tensors only: tables, positions).
__device__ inline double load_as_double(const void* p, int dt, int64_t i) {
  switch (dt) {
    case CS_F32: return static_cast<double>(static_cast<const float*>(p)[i]);
    case CS_F64: return static_cast<const double*>(p)[i];
    case CS_BF16: return static_cast<double>(bf16_to_float(static_cast<const uint16_t*>(p)[i]));
    case CS_F16: return static_cast<double>(f16_to_float(static_cast<const uint16_t*>(p)[i]));
    case CS_I32: return static_cast<double>(static_cast<const int32_t*>(p)[i]);
    case CS_I64: return static_cast<double>(static_cast<const int64_t*>(p)[i]);
    case CS_U8: return static_cast<double>(static_cast<const uint8_t*>(p)[i]);
  }
  return 0.0;
}

__device__ inline void store_from_double(void* p, int dt, int64_t i, double v) {
  switch (dt) {
    case CS_F32: static_cast<float*>(p)[i] = static_cast<float>(v); break;
    case CS_F64: static_cast<double*>(p)[i] = v; break;
    case CS_BF16: static_cast<uint16_t*>(p)[i] = double_to_bf16(v); break;
    case CS_F16: static_cast<uint16_t*>(p)[i] = double_to_f16(v); break;
    default: break;
  }
}

// Typed element access for templated kernels.
template <typename T> struct elem;
template <> struct elem<float> {
  using acc = float;
  using storage = float;
  __device__ static float load(const float* p, int64_t i) { return p[i]; }
  __device__ static void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct elem<double> {
  using acc = double;
  using storage = double;
  __device__ static double load(const double* p, int64_t i) { return p[i]; }
  __device__ static void store(double* p, int64_t i, double v) { p[i] = v; }
};
template <> struct elem<bf16_t> {
  using acc = float;
  using storage = uint16_t;
  __device__ static float load(const uint16_t* p, int64_t i) { return bf16_to_float(p[i]); }
  __device__ static void store(uint16_t* p, int64_t i, float v) { p[i] = float_to_bf16(v); }
};
template <> struct elem<f16_t> {
  using acc = float;
  using storage = uint16_t;
  __device__ static float load(const uint16_t* p, int64_t i) { return f16_to_float(p[i]); }
  __device__ static void store(uint16_t* p, int64_t i, float v) { p[i] = float_to_f16(v); }
};

// Device-side copy of a view's addressing (kernels take it by value).
struct dview {
  void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t shape[6];
  int64_t stride[6];
};

inline dview to_dview(const cs_view* v) {
  dview d{};
  if (v == nullptr) return d;
  d.data = v->data;
  d.dtype = v->dtype;
  d.ndim = v->ndim;
  for (int i = 0; i < 6; ++i) {
    d.shape[i] = v->shape[i];
    d.stride[i] = v->stride[i];
  }
  return d;
}

// Wavefront helpers (wave64).
__device__ inline float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline double wave_max(double v) {
  for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ inline double wave_sum(double v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace cs
