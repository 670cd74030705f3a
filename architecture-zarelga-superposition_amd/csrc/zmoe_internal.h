// Internal helpers shared by the gfx950 kernels of libzmoe_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "zmoe.h"

namespace zmoe {

// ---------------------------------------------------------------- vector types
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- element traits
// Storage types: bf16 is carried as uint16_t bit patterns, f32 as float.
template <int DT> struct Elem;
template <> struct Elem<ZMOE_DTYPE_BF16> {
  using T = uint16_t;
  static constexpr int VEC = 8;  // elements per 16-byte chunk
};
template <> struct Elem<ZMOE_DTYPE_F32> {
  using T = float;
  static constexpr int VEC = 4;
};

__device__ __forceinline__ float to_f32(uint16_t v) { return __uint_as_float(((uint32_t)v) << 16); }
__device__ __forceinline__ float to_f32(float v) { return v; }

// float -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}
// Two floats -> packed bf16 pair (lo = a, hi = b).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return bf16_bits(v); }

// 16-byte chunk <-> 8 (bf16) or 4 (f32) floats.
__device__ __forceinline__ void unpack_chunk(const uint4& c, float* out, uint16_t) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    out[2 * q] = __uint_as_float(w[q] << 16);
    out[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack_chunk(const uint4& c, float* out, float) {
  out[0] = __uint_as_float(c.x);
  out[1] = __uint_as_float(c.y);
  out[2] = __uint_as_float(c.z);
  out[3] = __uint_as_float(c.w);
}
__device__ __forceinline__ uint4 pack_chunk(const float* v, uint16_t) {
  uint4 c;
  c.x = pack_bf16x2(v[0], v[1]);
  c.y = pack_bf16x2(v[2], v[3]);
  c.z = pack_bf16x2(v[4], v[5]);
  c.w = pack_bf16x2(v[6], v[7]);
  return c;
}
__device__ __forceinline__ uint4 pack_chunk(const float* v, float) {
  uint4 c;
  c.x = __float_as_uint(v[0]);
  c.y = __float_as_uint(v[1]);
  c.z = __float_as_uint(v[2]);
  c.w = __float_as_uint(v[3]);
  return c;
}

// sigmoid(g) = 1 / (1 + e^-g) from the hardware exp2 and reciprocal (v_exp_f32 of g log2 e,
// v_rcp_f32): within ~1e-6 relative for |g| < 20, far inside the bf16 rounding of every
// value computed from it, at a third of the instructions of a correctly rounded divide.
// 1 + e^-g >= 1, so the reciprocal never sees a denormal; below g = -88.8 (e^-g overflows)
// it returns 0 (silu -0), above g = 17 exactly 1, and NaN stays NaN.
__device__ __forceinline__ float sigmoid_fast(float g) { return __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_fast(g); }

// ---------------------------------------------------------------- wave helpers
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ---------------------------------------------------------------- grouped GEMM, Newton-Schulz epilogue
// C rows [R, N] (bf16; expert e owns rows offsets[e-1] .. offsets[e] - 1) = A rows [R, K] @ B_e,
// where B_e sits at B + e * b_estride elements as [N][K] (K contiguous; b_kn false) or
// [K][N] (N contiguous; b_kn true). Epilogue (t = bf16(acc)): C = bf16(t + bf16(beta * D))
// when D is given, else t; C2 = bf16(gamma * t) when C2 is given. D and C2 share C's rows.
struct NsGemm {
  const void* A;
  int64_t lda;
  const void* B;
  int64_t b_estride, ldb;
  bool b_kn;
  const int64_t* offsets;
  int64_t R;
  int K, N, E;
  void* C;
  int64_t ldc;
  const void* D;
  int64_t ldd;
  float beta;
  void* C2;
  int64_t ldc2;
  float gamma;
  int sym_m;  // > 0: each expert's output is a symmetric sym_m x sym_m matrix (N == sym_m, uniform
              // rows): only the tiles on or above the diagonal run and they write their mirror
};
int ns_gemm(const NsGemm& g, hipStream_t s);

// ---------------------------------------------------------------- host helpers
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline int dtype_size(int dt) { return dt == ZMOE_DTYPE_BF16 ? 2 : 4; }
inline bool dtype_ok(int dt) { return dt == ZMOE_DTYPE_BF16 || dt == ZMOE_DTYPE_F32; }
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t align_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }

}  // namespace zmoe

#define ZMOE_REQUIRE(cond, code, ...)                  \
  do {                                                 \
    if (!(cond)) return ::zmoe::set_error((code), __VA_ARGS__); \
  } while (0)
