// HBM-bound row kernels of the MoE path: dispatch gather (ops.py:449-529), the
// weighted combine (parallel_experts.py:50-52 + moe_layer.py:53), its backward
// (parallel_experts.py:80-97), the k-reduction of the input grad
// (parallel_experts.py:125), rowwise_sum_product (ops.py:9-80) and stand-alone
// SwiGLU (mlp.py:86).
//
// Layout: a row of d elements is d/VEC 16-byte chunks (VEC = 8 bf16 or 4 f32).
// A group of TPR threads (64, 128 or 256; a whole number of waves) owns one row
// and strides over its chunks, so every load and store is a coalesced 16-byte
// access; a 256-thread block holds 256/TPR rows.
#include <type_traits>

#include "zmoe_internal.h"

namespace zmoe {

constexpr int kRowThreads = 256;
constexpr int kMaxFanOut = 32;

struct RowMap {
  int tpr;    // threads per row
  int rpb;    // rows per block
};

inline RowMap row_map(int64_t nchunks) {
  int tpr = nchunks <= 64 ? 64 : (nchunks <= 128 ? 128 : 256);
  return RowMap{tpr, kRowThreads / tpr};
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// Rows read exactly once (slot rows of Y / dXe, the addends, H in the SwiGLU passes):
// non-temporal loads, so the stream does not evict lines that other rows still use
// (measured: combine 0.267 -> 0.232 ms at C3).
typedef unsigned v4u32_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_stream(const void* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const v4u32_t*>(p)));
}
__device__ __forceinline__ void st16(void* p, const uint4& v) { *reinterpret_cast<uint4*>(p) = v; }

template <typename T> struct V { static constexpr int N = 16 / sizeof(T); };

// ------------------------------------------------------------------ group
template <typename T, typename CT>
__global__ __launch_bounds__(kRowThreads) void group_kernel(const T* __restrict__ A, int64_t lda, int64_t nch,
                                                            const int64_t* __restrict__ idx, int64_t N,
                                                            int fan_out, const CT* __restrict__ coeff,
                                                            T* __restrict__ Y, int64_t ldy, int tpr) {
  constexpr int VN = V<T>::N;
  const int rpb = kRowThreads / tpr;
  const int64_t n = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
  if (n >= N) return;
  const int lt = threadIdx.x % tpr;
  const int64_t src = idx[n];
  const T* a = A + (src / fan_out) * lda;
  T* y = Y + n * ldy;
  const float c = coeff ? to_f32(coeff[src]) : 1.f;
  for (int64_t ch = lt; ch < nch; ch += tpr) {
    uint4 v = ld16(a + ch * VN);
    if (coeff) {
      float f[VN];
      unpack_chunk(v, f, T{});
#pragma unroll
      for (int q = 0; q < VN; ++q) f[q] *= c;
      v = pack_chunk(f, T{});
    }
    st16(y + ch * VN, v);
  }
}

// The k-way row kernels below come in two forms: KF > 0 is compiled for exactly k = KF
// (every slot row of a chunk is loaded before any is used, so k loads are in flight
// per thread), KF = 0 loops over a runtime k.

// ------------------------------------------------------------------ combine
// out_rows (optional): token t's output row (the re-pad of moe_layer.py:55-56 folded in);
// a row outside [0, out_total) is not written.
template <typename T, int KF>
__global__ __launch_bounds__(kRowThreads) void combine_kernel(const T* __restrict__ Y, const float* __restrict__ g,
                                                              const T* __restrict__ add, int64_t T_, int k_rt,
                                                              int64_t d, T* __restrict__ out,
                                                              const int64_t* __restrict__ out_rows, int64_t out_total,
                                                              int tpr) {
  constexpr int VN = V<T>::N;
  const int k = KF > 0 ? KF : k_rt;
  const int rpb = kRowThreads / tpr;
  const int64_t t = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
  if (t >= T_) return;
  const int lt = threadIdx.x % tpr;
  const int64_t nch = d / VN;
  const int64_t orow = out_rows ? out_rows[t] : t;
  if (orow < 0 || orow >= out_total) return;
  for (int64_t ch = lt; ch < nch; ch += tpr) {
    float acc[VN];
    if (add) {
      unpack_chunk(ld16_stream(add + t * d + ch * VN), acc, T{});
    } else {
#pragma unroll
      for (int q = 0; q < VN; ++q) acc[q] = 0.f;
    }
    float part[VN];
#pragma unroll
    for (int q = 0; q < VN; ++q) part[q] = 0.f;
    if constexpr (KF > 0) {
      uint4 yv[KF];
#pragma unroll
      for (int j = 0; j < KF; ++j) yv[j] = ld16_stream(Y + (t * KF + j) * d + ch * VN);
#pragma unroll
      for (int j = 0; j < KF; ++j) {
        const float w = g ? g[t * KF + j] : 1.f;
        float y[VN];
        unpack_chunk(yv[j], y, T{});
#pragma unroll
        for (int q = 0; q < VN; ++q) part[q] = fmaf(w, y[q], part[q]);
      }
    } else {
      for (int j = 0; j < k; ++j) {
        const float w = g ? g[t * k + j] : 1.f;
        float y[VN];
        unpack_chunk(ld16_stream(Y + (t * k + j) * d + ch * VN), y, T{});
#pragma unroll
        for (int q = 0; q < VN; ++q) part[q] = fmaf(w, y[q], part[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < VN; ++q) acc[q] += part[q];
    st16(out + orow * d + ch * VN, pack_chunk(acc, T{}));
  }
}

// ------------------------------------------------------------------ combine backward
// d_gates[t,j] = <Y[t*k+j], dout[t]>; grouped[inverse[t*k+j]] = g[t,j] * dout[t].
// KM: a compile-time bound on k (slot arrays sized KM; slots j >= k are skipped).
// dout_rows (optional): token t's row of dout (the padded layout's gradient read in place);
// a row outside [0, dout_total) reads as zero. DOTS = false: the grouped rows only (no Y).
template <typename T, int KM, bool DOTS>
__global__ __launch_bounds__(kRowThreads) void combine_backward_kernel(
    const T* __restrict__ Y, const T* __restrict__ dout, const int64_t* __restrict__ dout_rows, int64_t dout_total,
    const float* __restrict__ g, const int32_t* __restrict__ inverse, int64_t T_, int k, int64_t d,
    float* __restrict__ d_gates, T* __restrict__ grouped, int tpr) {
  constexpr int VN = V<T>::N;
  __shared__ float red[kRowThreads / 64][KM];
  const int rpb = kRowThreads / tpr;
  const int64_t t = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
  const bool live = t < T_;
  const int lt = threadIdx.x % tpr;
  const int64_t nch = d / VN;
  float dot[KM];
#pragma unroll
  for (int j = 0; j < KM; ++j) dot[j] = 0.f;
  if (live) {
    int32_t dst[KM];
    float w[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
      // slots past k repeat slot k - 1 (their results are dropped), so every load stays in bounds
      const int jj = j < k ? j : k - 1;
      dst[j] = inverse[t * k + jj];
      w[j] = g[t * k + jj];
    }
    const int64_t drow = dout_rows ? dout_rows[t] : t;
    const bool drow_ok = drow >= 0 && drow < dout_total;
    for (int64_t ch = lt; ch < nch; ch += tpr) {
      float go[VN];
      if (drow_ok) {
        unpack_chunk(ld16_stream(dout + drow * d + ch * VN), go, T{});
      } else {
#pragma unroll
        for (int q = 0; q < VN; ++q) go[q] = 0.f;
      }
      uint4 yv[KM];
      if constexpr (DOTS) {
#pragma unroll
        for (int j = 0; j < KM; ++j) yv[j] = ld16_stream(Y + (t * k + (j < k ? j : k - 1)) * d + ch * VN);
      }
#pragma unroll
      for (int j = 0; j < KM; ++j) {
        float sv[VN];
#pragma unroll
        for (int q = 0; q < VN; ++q) sv[q] = w[j] * go[q];
        if constexpr (DOTS) {
          float y[VN];
          unpack_chunk(yv[j], y, T{});
          float acc = 0.f;
#pragma unroll
          for (int q = 0; q < VN; ++q) acc = fmaf(y[q], go[q], acc);
          dot[j] += acc;
        }
        if (j < k) st16(grouped + (int64_t)dst[j] * d + ch * VN, pack_chunk(sv, T{}));
      }
    }
  }
  if constexpr (!DOTS) return;
  // reduce the partial dots over the row's threads (whole waves)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < KM; ++j) {
    const float sj = wave_sum(dot[j]);
    if (lane == 0) red[wave][j] = sj;
  }
  __syncthreads();
  const int wpr = tpr / 64;  // waves per row
  if (live && lt < k) {
    const int w0 = (threadIdx.x / tpr) * wpr;
    float sum = 0.f;
    for (int w2 = 0; w2 < wpr; ++w2) sum += red[w0 + w2][lt];
    d_gates[t * k + lt] = sum;
  }
}

// ------------------------------------------------------------------ k-sum
// TO: the output type (T, or float for bf16 rows: the fp32 sum unrounded, the input grad of an
// fp32 residual stream under bf16 autocast)
template <typename T, int KF, typename TO = T>
__global__ __launch_bounds__(kRowThreads) void sum_k_kernel(const T* __restrict__ Xe, int64_t T_, int k_rt, int64_t d,
                                                            const T* __restrict__ a0, const T* __restrict__ a1,
                                                            TO* __restrict__ out, int tpr) {
  constexpr int VN = V<T>::N;
  const int k = KF > 0 ? KF : k_rt;
  const int rpb = kRowThreads / tpr;
  const int64_t t = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
  if (t >= T_) return;
  const int lt = threadIdx.x % tpr;
  const int64_t nch = d / VN;
  for (int64_t ch = lt; ch < nch; ch += tpr) {
    float acc[VN], x[VN];
#pragma unroll
    for (int q = 0; q < VN; ++q) acc[q] = 0.f;
    if constexpr (KF > 0) {
      uint4 xv[KF];
#pragma unroll
      for (int j = 0; j < KF; ++j) xv[j] = ld16_stream(Xe + (t * KF + j) * d + ch * VN);
#pragma unroll
      for (int j = 0; j < KF; ++j) {
        unpack_chunk(xv[j], x, T{});
#pragma unroll
        for (int q = 0; q < VN; ++q) acc[q] += x[q];
      }
    } else {
      for (int j = 0; j < k; ++j) {
        unpack_chunk(ld16_stream(Xe + (t * k + j) * d + ch * VN), x, T{});
#pragma unroll
        for (int q = 0; q < VN; ++q) acc[q] += x[q];
      }
    }
    if (a0) {
      unpack_chunk(ld16_stream(a0 + t * d + ch * VN), x, T{});
#pragma unroll
      for (int q = 0; q < VN; ++q) acc[q] += x[q];
    }
    if (a1) {
      unpack_chunk(ld16_stream(a1 + t * d + ch * VN), x, T{});
#pragma unroll
      for (int q = 0; q < VN; ++q) acc[q] += x[q];
    }
    if constexpr (sizeof(TO) == sizeof(T)) {
      st16(out + t * d + ch * VN, pack_chunk(acc, T{}));
    } else {
#pragma unroll
      for (int h = 0; h < VN / 4; ++h) st16(out + t * d + ch * VN + 4 * h, pack_chunk(acc + 4 * h, float{}));
    }
  }
}

// ------------------------------------------------------------------ fp32 -> bf16 copies
// dst[i] = bf16(src[i]), round to nearest even (NaN stays NaN): one 8-element chunk per
// thread (two 16-byte streaming loads, one 16-byte store), one thread per chunk; the last
// n % 8 elements by the first lanes of block 0. (Measured on the C3 W1 stack, 402M elements:
// 6.1 TB/s; grid-stride loops over fewer blocks 4.7-5.6 TB/s.)
__global__ __launch_bounds__(256) void cast_f32_bf16_kernel(const float* __restrict__ src, int64_t n,
                                                            uint16_t* __restrict__ dst) {
  const int64_t nv = n / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < nv) {
    float v[8];
    unpack_chunk(ld16_stream(src + 8 * i), v, float{});
    unpack_chunk(ld16_stream(src + 8 * i + 4), v + 4, float{});
    st16(dst + 8 * i, pack_chunk(v, uint16_t{}));
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 8 * nv) dst[8 * nv + threadIdx.x] = bf16_bits(src[8 * nv + threadIdx.x]);
}

// ------------------------------------------------------------------ rowwise_sum_product
// One wave per (t, j): out[t,j] = sum_h A[t,j,h] * B[t,h]; scalar loads so any
// H and mixed dtypes work.
template <typename TA, typename TB, typename TO>
__global__ __launch_bounds__(kRowThreads) void rowwise_kernel(const TA* __restrict__ A, const TB* __restrict__ B,
                                                              int64_t T_, int F, int64_t H, TO* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (r >= T_ * F) return;
  const int lane = threadIdx.x & 63;
  const int64_t t = r / F;
  const TA* a = A + r * H;
  const TB* b = B + t * H;
  float acc = 0.f;
  for (int64_t h = lane; h < H; h += 64) acc = fmaf(to_f32(a[h]), to_f32(b[h]), acc);
  acc = wave_sum(acc);
  if (lane == 0) out[r] = from_f32<TO>(acc);
}

// ------------------------------------------------------------------ swiglu
template <typename T>
__global__ __launch_bounds__(kRowThreads) void swiglu_kernel(const T* __restrict__ H, int64_t R, int64_t f,
                                                             T* __restrict__ A) {
  constexpr int VN = V<T>::N;
  const int64_t nch = f / VN;
  const int64_t i = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
  if (i >= R * nch) return;
  const int64_t r = i / nch, ch = i % nch;
  float h[VN], g[VN], a[VN];
  unpack_chunk(ld16_stream(H + r * 2 * f + ch * VN), h, T{});
  unpack_chunk(ld16_stream(H + r * 2 * f + f + ch * VN), g, T{});
#pragma unroll
  for (int q = 0; q < VN; ++q) a[q] = silu_f(g[q]) * h[q];
  st16(A + r * f + ch * VN, pack_chunk(a, T{}));
}

template <typename T>
__global__ __launch_bounds__(kRowThreads) void swiglu_backward_kernel(const T* __restrict__ dA,
                                                                      const T* __restrict__ H, int64_t R,
                                                                      int64_t f, T* __restrict__ dH, int64_t ld) {
  constexpr int VN = V<T>::N;
  const int64_t nch = f / VN;
  const int64_t i = (int64_t)blockIdx.x * kRowThreads + threadIdx.x;
  if (i >= R * nch) return;
  const int64_t r = i / nch, ch = i % nch;
  float h[VN], g[VN], da[VN], dh[VN], dg[VN];
  unpack_chunk(ld16_stream(H + r * 2 * f + ch * VN), h, T{});
  unpack_chunk(ld16_stream(H + r * 2 * f + f + ch * VN), g, T{});
  unpack_chunk(ld16_stream(dA + r * f + ch * VN), da, T{});
#pragma unroll
  for (int q = 0; q < VN; ++q) {
    const float s = sigmoid_fast(g[q]);
    dh[q] = da[q] * g[q] * s;
    dg[q] = da[q] * h[q] * s * (1.f + g[q] * (1.f - s));
  }
  st16(dH + r * ld + ch * VN, pack_chunk(dh, T{}));
  st16(dH + r * ld + f + ch * VN, pack_chunk(dg, T{}));
}

// SwiGLU backward of gate-scaled rows with the gates' grad: one wave per sorted row r,
//   dA = row_scale[r] * dAu[r];  dH[r] = [dA * g * s | dA * h * s * (1 + g (1 - s))];
//   d_gates[slot[r]] = sum_c dAu[r, c] * silu(g) * h      (s = sigmoid(g), [h | g] = H[r])
template <typename T>
__global__ __launch_bounds__(kRowThreads) void swiglu_backward_gates_kernel(
    const T* __restrict__ dAu, const T* __restrict__ H, int64_t R, int64_t f, const float* __restrict__ row_scale,
    const int64_t* __restrict__ slot, T* __restrict__ dH, float* __restrict__ d_gates) {
  constexpr int VN = V<T>::N;
  const int64_t r = (int64_t)blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (r >= R) return;  // whole waves
  const int lane = threadIdx.x & 63;
  const int64_t nch = f / VN;
  const float sc = row_scale[r];
  float dot = 0.f;
  for (int64_t ch = lane; ch < nch; ch += 64) {
    float da[VN], h[VN], g[VN], dh[VN], dg[VN];
    unpack_chunk(ld16_stream(dAu + r * f + ch * VN), da, T{});
    unpack_chunk(ld16_stream(H + r * 2 * f + ch * VN), h, T{});
    unpack_chunk(ld16_stream(H + r * 2 * f + f + ch * VN), g, T{});
#pragma unroll
    for (int q = 0; q < VN; ++q) {
      const float s = sigmoid_fast(g[q]);
      dot = fmaf(da[q], g[q] * s * h[q], dot);
      const float d = sc * da[q];
      dh[q] = d * g[q] * s;
      dg[q] = d * h[q] * s * (1.f + g[q] * (1.f - s));
    }
    st16(dH + r * 2 * f + ch * VN, pack_chunk(dh, T{}));
    st16(dH + r * 2 * f + f + ch * VN, pack_chunk(dg, T{}));
  }
  dot = wave_sum(dot);
  if (lane == 0) d_gates[slot[r]] = dot;
}

}  // namespace zmoe

using namespace zmoe;

namespace {

int vec_of(int dtype) { return dtype == ZMOE_DTYPE_BF16 ? 8 : 4; }

bool rows_aligned(int dtype, const void* p, int64_t ld) {
  return p == nullptr || (aligned16(p) && (ld % vec_of(dtype)) == 0);
}

}  // namespace

extern "C" int zmoe_group(const void* A, int64_t lda, int64_t K, int dtype, const int64_t* sorted_idxs, int64_t N,
                          int fan_out, const void* coeff, int coeff_dtype, void* Y, int64_t ldy, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype) && dtype_ok(coeff_dtype), ZMOE_ERR_DTYPE, "group: dtype");
  ZMOE_REQUIRE(N >= 0 && K >= 0 && fan_out >= 1, ZMOE_ERR_SHAPE, "group: bad sizes");
  if (N == 0 || K == 0) return ZMOE_OK;
  ZMOE_REQUIRE(A && sorted_idxs && Y, ZMOE_ERR_NULL, "group: null pointer");
  ZMOE_REQUIRE(K % vec_of(dtype) == 0 && rows_aligned(dtype, A, lda) && rows_aligned(dtype, Y, ldy), ZMOE_ERR_ALIGN,
               "group: K (%lld) and row strides must be multiples of %d elements, pointers 16-byte aligned",
               (long long)K, vec_of(dtype));
  const int64_t nch = K / vec_of(dtype);
  const RowMap m = row_map(nch);
  const dim3 grid((unsigned)cdiv(N, m.rpb)), block(kRowThreads);
  hipStream_t s = as_stream(stream);
#define ZMOE_GROUP_LAUNCH(T, CT)                                                                                  \
  hipLaunchKernelGGL((group_kernel<T, CT>), grid, block, 0, s, (const T*)A, lda, nch, sorted_idxs, N, fan_out, \
                     (const CT*)coeff, (T*)Y, ldy, m.tpr)
  if (dtype == ZMOE_DTYPE_BF16) {
    if (coeff_dtype == ZMOE_DTYPE_BF16) ZMOE_GROUP_LAUNCH(uint16_t, uint16_t);
    else ZMOE_GROUP_LAUNCH(uint16_t, float);
  } else {
    if (coeff_dtype == ZMOE_DTYPE_BF16) ZMOE_GROUP_LAUNCH(float, uint16_t);
    else ZMOE_GROUP_LAUNCH(float, float);
  }
#undef ZMOE_GROUP_LAUNCH
  return check_launch("group");
}

namespace {

int combine_impl(const void* Y, const float* gates, const void* addend, int64_t T, int k, int64_t d, int dtype,
                 const int64_t* out_rows, int64_t out_total, void* out, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "combine: dtype");
  ZMOE_REQUIRE(T >= 0 && k >= 1 && d >= 0, ZMOE_ERR_SHAPE, "combine: bad sizes");
  if (T == 0 || d == 0) return ZMOE_OK;
  ZMOE_REQUIRE(Y && out, ZMOE_ERR_NULL, "combine: null pointer");
  ZMOE_REQUIRE(d % vec_of(dtype) == 0 && rows_aligned(dtype, Y, d) && rows_aligned(dtype, out, d) &&
                   rows_aligned(dtype, addend, d),
               ZMOE_ERR_ALIGN, "combine: d must be a multiple of %d, pointers 16-byte aligned", vec_of(dtype));
  const RowMap m = row_map(d / vec_of(dtype));
  const dim3 grid((unsigned)cdiv(T, m.rpb)), block(kRowThreads);
  auto launch = [&](auto kf, auto tt) {
    using TT = decltype(tt);
    hipLaunchKernelGGL((combine_kernel<TT, decltype(kf)::value>), grid, block, 0, as_stream(stream), (const TT*)Y,
                       gates, (const TT*)addend, T, k, d, (TT*)out, out_rows, out_total, m.tpr);
  };
  auto by_k = [&](auto tt) {
    if (k == 8) launch(std::integral_constant<int, 8>{}, tt);
    else if (k == 2) launch(std::integral_constant<int, 2>{}, tt);
    else if (k == 4) launch(std::integral_constant<int, 4>{}, tt);
    else if (k == 6) launch(std::integral_constant<int, 6>{}, tt);
    else launch(std::integral_constant<int, 0>{}, tt);
  };
  if (dtype == ZMOE_DTYPE_BF16) by_k(uint16_t{});
  else by_k(float{});
  return check_launch("combine");
}

int combine_backward_impl(const void* Y, const void* grad_out, const int64_t* grad_rows, int64_t grad_total,
                          const float* gates, const int32_t* inverse, int64_t T, int k, int64_t d, int dtype,
                          float* d_gates, void* grouped_grad_out, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "combine_backward: dtype");
  ZMOE_REQUIRE(T >= 0 && k >= 1 && k <= kMaxFanOut && d >= 0, ZMOE_ERR_SHAPE,
               "combine_backward: need 1 <= k <= %d", kMaxFanOut);
  if (T == 0) return ZMOE_OK;
  ZMOE_REQUIRE(grad_out && gates && inverse && grouped_grad_out && (Y != nullptr) == (d_gates != nullptr),
               ZMOE_ERR_NULL, "combine_backward: null pointer");
  ZMOE_REQUIRE(d % vec_of(dtype) == 0 && (Y == nullptr || rows_aligned(dtype, Y, d)) &&
                   rows_aligned(dtype, grad_out, d) &&
                   rows_aligned(dtype, grouped_grad_out, d),
               ZMOE_ERR_ALIGN, "combine_backward: d must be a multiple of %d, pointers 16-byte aligned",
               vec_of(dtype));
  const RowMap m = row_map(d / vec_of(dtype));
  const dim3 grid((unsigned)cdiv(T, m.rpb)), block(kRowThreads);
  auto launch = [&](auto km, auto tt) {
    using TT = decltype(tt);
    if (Y != nullptr)
      hipLaunchKernelGGL((combine_backward_kernel<TT, decltype(km)::value, true>), grid, block, 0,
                         as_stream(stream), (const TT*)Y, (const TT*)grad_out, grad_rows, grad_total, gates, inverse,
                         T, k, d, d_gates, (TT*)grouped_grad_out, m.tpr);
    else
      hipLaunchKernelGGL((combine_backward_kernel<TT, decltype(km)::value, false>), grid, block, 0,
                         as_stream(stream), (const TT*)Y, (const TT*)grad_out, grad_rows, grad_total, gates, inverse,
                         T, k, d, d_gates, (TT*)grouped_grad_out, m.tpr);
  };
  auto by_k = [&](auto tt) {
    if (k <= 2) launch(std::integral_constant<int, 2>{}, tt);
    else if (k <= 4) launch(std::integral_constant<int, 4>{}, tt);
    else if (k <= 8) launch(std::integral_constant<int, 8>{}, tt);
    else if (k <= 16) launch(std::integral_constant<int, 16>{}, tt);
    else launch(std::integral_constant<int, kMaxFanOut>{}, tt);
  };
  if (dtype == ZMOE_DTYPE_BF16) by_k(uint16_t{});
  else by_k(float{});
  return check_launch("combine_backward");
}

}  // namespace

extern "C" int zmoe_combine(const void* Y, const float* gates, const void* addend, int64_t T, int k, int64_t d,
                            int dtype, void* out, void* stream) {
  return combine_impl(Y, gates, addend, T, k, d, dtype, nullptr, T, out, stream);
}

extern "C" int zmoe_combine_rows(const void* Y, const float* gates, const void* addend, int64_t T, int k, int64_t d,
                                 int dtype, const int64_t* out_rows, int64_t out_total, void* out, void* stream) {
  ZMOE_REQUIRE(T == 0 || out_rows, ZMOE_ERR_NULL, "combine_rows: null out_rows");
  ZMOE_REQUIRE(out_total >= 0, ZMOE_ERR_SHAPE, "combine_rows: out_total < 0");
  return combine_impl(Y, gates, addend, T, k, d, dtype, out_rows, out_total, out, stream);
}

extern "C" int zmoe_combine_backward(const void* Y, const void* grad_out, const float* gates, const int32_t* inverse,
                                     int64_t T, int k, int64_t d, int dtype, float* d_gates, void* grouped_grad_out,
                                     void* stream) {
  return combine_backward_impl(Y, grad_out, nullptr, T, gates, inverse, T, k, d, dtype, d_gates, grouped_grad_out,
                               stream);
}

extern "C" int zmoe_combine_backward_rows(const void* Y, const void* grad_out, const int64_t* grad_rows,
                                          int64_t grad_total, const float* gates, const int32_t* inverse, int64_t T,
                                          int k, int64_t d, int dtype, float* d_gates, void* grouped_grad_out,
                                          void* stream) {
  ZMOE_REQUIRE(T == 0 || grad_rows, ZMOE_ERR_NULL, "combine_backward_rows: null grad_rows");
  ZMOE_REQUIRE(grad_total >= 0, ZMOE_ERR_SHAPE, "combine_backward_rows: grad_total < 0");
  return combine_backward_impl(Y, grad_out, grad_rows, grad_total, gates, inverse, T, k, d, dtype, d_gates,
                               grouped_grad_out, stream);
}

extern "C" int zmoe_sum_k(const void* Xe, int64_t T, int k, int64_t d, int dtype, const void* add0, const void* add1,
                          int out_dtype, void* out, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "sum_k: dtype");
  ZMOE_REQUIRE(out_dtype == dtype || (dtype == ZMOE_DTYPE_BF16 && out_dtype == ZMOE_DTYPE_F32), ZMOE_ERR_DTYPE,
               "sum_k: out_dtype %d with rows of dtype %d", out_dtype, dtype);
  ZMOE_REQUIRE(T >= 0 && k >= 1 && d >= 0, ZMOE_ERR_SHAPE, "sum_k: bad sizes");
  if (T == 0 || d == 0) return ZMOE_OK;
  ZMOE_REQUIRE(Xe && out, ZMOE_ERR_NULL, "sum_k: null pointer");
  ZMOE_REQUIRE(d % vec_of(dtype) == 0 && rows_aligned(dtype, Xe, d) && rows_aligned(out_dtype, out, d) &&
                   rows_aligned(dtype, add0, d) && rows_aligned(dtype, add1, d),
               ZMOE_ERR_ALIGN, "sum_k: d must be a multiple of %d, pointers 16-byte aligned", vec_of(dtype));
  const RowMap m = row_map(d / vec_of(dtype));
  const dim3 grid((unsigned)cdiv(T, m.rpb)), block(kRowThreads);
  auto launch = [&](auto kf, auto tt, auto to) {
    using TT = decltype(tt);
    using TO = decltype(to);
    hipLaunchKernelGGL((sum_k_kernel<TT, decltype(kf)::value, TO>), grid, block, 0, as_stream(stream),
                       (const TT*)Xe, T, k, d, (const TT*)add0, (const TT*)add1, (TO*)out, m.tpr);
  };
  auto by_k = [&](auto tt, auto to) {
    if (k == 8) launch(std::integral_constant<int, 8>{}, tt, to);
    else if (k == 2) launch(std::integral_constant<int, 2>{}, tt, to);
    else if (k == 4) launch(std::integral_constant<int, 4>{}, tt, to);
    else if (k == 6) launch(std::integral_constant<int, 6>{}, tt, to);
    else launch(std::integral_constant<int, 0>{}, tt, to);
  };
  if (dtype == ZMOE_DTYPE_BF16 && out_dtype == ZMOE_DTYPE_F32) by_k(uint16_t{}, float{});
  else if (dtype == ZMOE_DTYPE_BF16) by_k(uint16_t{}, uint16_t{});
  else by_k(float{}, float{});
  return check_launch("sum_k");
}

extern "C" int zmoe_cast_f32_bf16(const float* src, int64_t n, void* dst, void* stream) {
  ZMOE_REQUIRE(n >= 0, ZMOE_ERR_SHAPE, "cast_f32_bf16: n < 0");
  if (n == 0) return ZMOE_OK;
  ZMOE_REQUIRE(src && dst, ZMOE_ERR_NULL, "cast_f32_bf16: null pointer");
  ZMOE_REQUIRE(aligned16(src) && aligned16(dst), ZMOE_ERR_ALIGN, "cast_f32_bf16: pointers must be 16-byte aligned");
  const int64_t blocks = cdiv(n / 8 > 0 ? n / 8 : 1, 256);
  ZMOE_REQUIRE(blocks < (int64_t)0x7fffffff, ZMOE_ERR_SHAPE, "cast_f32_bf16: n too large");
  hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream), src, n,
                     (uint16_t*)dst);
  return check_launch("cast_f32_bf16");
}

extern "C" int zmoe_rowwise_sum_product(const void* A, int a_dtype, const void* B, int b_dtype, int64_t T, int F,
                                        int64_t H, void* out, int out_dtype, void* stream) {
  ZMOE_REQUIRE(dtype_ok(a_dtype) && dtype_ok(b_dtype) && dtype_ok(out_dtype), ZMOE_ERR_DTYPE,
               "rowwise_sum_product: dtype");
  ZMOE_REQUIRE(T >= 0 && F >= 0 && H >= 0, ZMOE_ERR_SHAPE, "rowwise_sum_product: bad sizes");
  if (T == 0 || F == 0) return ZMOE_OK;
  ZMOE_REQUIRE(A && B && out, ZMOE_ERR_NULL, "rowwise_sum_product: null pointer");
  const dim3 grid((unsigned)cdiv(T * F, kRowThreads / 64)), block(kRowThreads);
  hipStream_t s = as_stream(stream);
#define ZMOE_RW(TA, TB, TO) \
  hipLaunchKernelGGL((rowwise_kernel<TA, TB, TO>), grid, block, 0, s, (const TA*)A, (const TB*)B, T, F, H, (TO*)out)
#define ZMOE_RW_O(TA, TB) \
  if (out_dtype == ZMOE_DTYPE_BF16) ZMOE_RW(TA, TB, uint16_t); else ZMOE_RW(TA, TB, float)
  if (a_dtype == ZMOE_DTYPE_BF16) {
    if (b_dtype == ZMOE_DTYPE_BF16) { ZMOE_RW_O(uint16_t, uint16_t); } else { ZMOE_RW_O(uint16_t, float); }
  } else {
    if (b_dtype == ZMOE_DTYPE_BF16) { ZMOE_RW_O(float, uint16_t); } else { ZMOE_RW_O(float, float); }
  }
#undef ZMOE_RW_O
#undef ZMOE_RW
  return check_launch("rowwise_sum_product");
}

extern "C" int zmoe_swiglu(const void* H, int64_t R, int64_t f, int dtype, void* A, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "swiglu: dtype");
  ZMOE_REQUIRE(R >= 0 && f >= 0, ZMOE_ERR_SHAPE, "swiglu: bad sizes");
  if (R == 0 || f == 0) return ZMOE_OK;
  ZMOE_REQUIRE(H && A, ZMOE_ERR_NULL, "swiglu: null pointer");
  ZMOE_REQUIRE(f % vec_of(dtype) == 0 && aligned16(H) && aligned16(A), ZMOE_ERR_ALIGN,
               "swiglu: f must be a multiple of %d", vec_of(dtype));
  const int64_t n = R * (f / vec_of(dtype));
  const dim3 grid((unsigned)cdiv(n, kRowThreads)), block(kRowThreads);
  if (dtype == ZMOE_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_kernel<uint16_t>, grid, block, 0, as_stream(stream), (const uint16_t*)H, R, f,
                       (uint16_t*)A);
  else
    hipLaunchKernelGGL(swiglu_kernel<float>, grid, block, 0, as_stream(stream), (const float*)H, R, f, (float*)A);
  return check_launch("swiglu");
}

extern "C" int zmoe_swiglu_backward_gates(const void* dA, const void* H, int64_t R, int64_t f, const float* row_scale,
                                          const int64_t* slot_of_row, int dtype, void* dH, float* d_gates,
                                          void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "swiglu_backward_gates: dtype");
  ZMOE_REQUIRE(R >= 0 && f >= 1, ZMOE_ERR_SHAPE, "swiglu_backward_gates: bad sizes");
  if (R == 0) return ZMOE_OK;
  ZMOE_REQUIRE(dA && H && dH && row_scale && slot_of_row && d_gates, ZMOE_ERR_NULL,
               "swiglu_backward_gates: null pointer");
  ZMOE_REQUIRE(f % vec_of(dtype) == 0 && aligned16(H) && aligned16(dA) && aligned16(dH), ZMOE_ERR_ALIGN,
               "swiglu_backward_gates: f must be a multiple of %d", vec_of(dtype));
  const dim3 grid((unsigned)cdiv(R, kRowThreads / 64)), block(kRowThreads);
  if (dtype == ZMOE_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_backward_gates_kernel<uint16_t>, grid, block, 0, as_stream(stream),
                       (const uint16_t*)dA, (const uint16_t*)H, R, f, row_scale, slot_of_row, (uint16_t*)dH, d_gates);
  else
    hipLaunchKernelGGL(swiglu_backward_gates_kernel<float>, grid, block, 0, as_stream(stream), (const float*)dA,
                       (const float*)H, R, f, row_scale, slot_of_row, (float*)dH, d_gates);
  return check_launch("swiglu_backward_gates");
}

extern "C" int zmoe_swiglu_backward(const void* dA, const void* H, int64_t R, int64_t f, int dtype, void* dH,
                                    int64_t ld_dh, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "swiglu_backward: dtype");
  ZMOE_REQUIRE(R >= 0 && f >= 0 && f < (1 << 30) && ld_dh >= 2 * f, ZMOE_ERR_SHAPE, "swiglu_backward: bad sizes");
  if (R == 0 || f == 0) return ZMOE_OK;
  ZMOE_REQUIRE(dA && H && dH, ZMOE_ERR_NULL, "swiglu_backward: null pointer");
  ZMOE_REQUIRE(f % vec_of(dtype) == 0 && ld_dh % vec_of(dtype) == 0 && aligned16(H) && aligned16(dA) &&
                   aligned16(dH),
               ZMOE_ERR_ALIGN, "swiglu_backward: f and the dH row stride must be multiples of %d", vec_of(dtype));
  const int64_t n = R * (f / vec_of(dtype));
  const dim3 grid((unsigned)cdiv(n, kRowThreads)), block(kRowThreads);
  if (dtype == ZMOE_DTYPE_BF16)
    hipLaunchKernelGGL(swiglu_backward_kernel<uint16_t>, grid, block, 0, as_stream(stream), (const uint16_t*)dA,
                       (const uint16_t*)H, R, f, (uint16_t*)dH, ld_dh);
  else
    hipLaunchKernelGGL(swiglu_backward_kernel<float>, grid, block, 0, as_stream(stream), (const float*)dA,
                       (const float*)H, R, f, (float*)dH, ld_dh);
  return check_launch("swiglu_backward");
}
