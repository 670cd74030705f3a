// ZeroCenteredRMSNorm (modeling/zRMSNorm.py:10-17) fused with the unpad gather in front of
// the MoE layer (modeling/moe_layer.py:39-42, flash_attn's index_first_axis):
//   Y[i] = X[rows[i]] * rsqrt(mean(X[rows[i]]^2) + eps) * (1 + w)      (fp32, stored as X's dtype)
// one pass that reads each selected row once, and its backward
//   dX[rows[i]] = r (1 + w) dy - X r^3 / d * sum_j dy_j (1 + w_j) X_j     (r = the saved rstd)
//   dw          = sum_i dy_i * X[rows[i]] * r_i                           (fixed-order, deterministic)
// Layout: a group of TPR threads (64, 128 or 256) owns a row and holds up to kMaxChunks
// 16-byte chunks of it in registers (d <= TPR * kMaxChunks * 16 / sizeof(T)).
#include "zmoe_internal.h"

namespace zmoe {

constexpr int kNormThreads = 256;
constexpr int kNormMaxChunks = 8;
constexpr int kNormMaxPartials = 512;

struct NormMap {
  int tpr, rpb;
};

inline NormMap norm_map(int64_t nch) {
  const int tpr = nch <= 64 ? 64 : (nch <= 128 ? 128 : 256);
  return NormMap{tpr, kNormThreads / tpr};
}

template <typename TW> __device__ __forceinline__ float load_w(const TW* w, int64_t c) { return to_f32(w[c]); }

// Sum over the TPR threads of one row (whole waves), via LDS across the row's waves.
__device__ __forceinline__ float row_sum(float v, int tpr, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, wpr = tpr >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  const int w0 = (wave / wpr) * wpr;
  float t = 0.f;
  for (int q = 0; q < wpr; ++q) t += red[w0 + q];
  __syncthreads();
  return t;
}

template <typename T, typename TW>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_rows_kernel(const T* __restrict__ X, int64_t ldx,
                                                                    int64_t x_rows, const int64_t* __restrict__ rows,
                                                                    int64_t n, int64_t d, const TW* __restrict__ w,
                                                                    float eps, T* __restrict__ Y,
                                                                    float* __restrict__ rstd, int tpr) {
  constexpr int VN = 16 / sizeof(T);
  __shared__ float red[kNormThreads / 64];
  const int rpb = kNormThreads / tpr;
  const int64_t i = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
  const int lt = threadIdx.x % tpr;
  const int64_t nch = d / VN;
  int64_t src = -1;
  if (i < n) {
    src = rows ? rows[i] : i;
    if (src < 0 || src >= x_rows) src = -1;  // out-of-range row: written as zeros
  }
  uint4 c[kNormMaxChunks];
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q) {
    const int64_t ch = lt + (int64_t)q * tpr;
    c[q] = make_uint4(0, 0, 0, 0);
    if (src >= 0 && ch < nch) {
      c[q] = *reinterpret_cast<const uint4*>(X + src * ldx + ch * VN);
      float v[VN];
      unpack_chunk(c[q], v, T{});
#pragma unroll
      for (int u = 0; u < VN; ++u) ss = fmaf(v[u], v[u], ss);
    }
  }
  const float tot = row_sum(ss, tpr, red);  // every thread of the block reaches the barriers
  if (i >= n) return;
  const float r = src >= 0 ? rsqrtf(tot / (float)d + eps) : 0.f;
  if (rstd && lt == 0) rstd[i] = r;
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q) {
    const int64_t ch = lt + (int64_t)q * tpr;
    if (ch < nch) {
      float v[VN];
      unpack_chunk(c[q], v, T{});
#pragma unroll
      for (int u = 0; u < VN; ++u) v[u] = (v[u] * r) * (1.0f + load_w(w, ch * VN + u));
      *reinterpret_cast<uint4*>(Y + i * d + ch * VN) = pack_chunk(v, T{});
    }
  }
}

// One block per partial: grid-stride over rows, every thread accumulating dw for its own
// columns in registers; the block's row slots are summed in slot order through LDS.
template <typename T, typename TW>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_rows_backward_kernel(
    const T* __restrict__ dY, const T* __restrict__ X, int64_t ldx, int64_t x_rows, const int64_t* __restrict__ rows,
    int64_t n, int64_t d, const float* __restrict__ rstd, const TW* __restrict__ w, T* __restrict__ dX,
    int64_t lddx, float* __restrict__ partial, int tpr) {
  constexpr int VN = 16 / sizeof(T);
  extern __shared__ float slot_dw[];  // [rpb][d]
  __shared__ float red[kNormThreads / 64];
  const int rpb = kNormThreads / tpr;
  const int slot = threadIdx.x / tpr, lt = threadIdx.x % tpr;
  const int64_t nch = d / VN;
  float acc[kNormMaxChunks][VN];
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q)
#pragma unroll
    for (int u = 0; u < VN; ++u) acc[q][u] = 0.f;
  const float inv_d = 1.0f / (float)d;
  const int64_t step = (int64_t)gridDim.x * rpb;
  const int64_t n_iter = (n + step - 1) / step;  // same trip count for every thread (barriers inside)
  for (int64_t it = 0; it < n_iter; ++it) {
    const int64_t i = it * step + (int64_t)blockIdx.x * rpb + slot;
    int64_t src = -1;
    float r = 0.f;
    if (i < n) {
      src = rows ? rows[i] : i;
      if (src < 0 || src >= x_rows) src = -1;
      r = rstd[i];
    }
    uint4 xc[kNormMaxChunks], gc[kNormMaxChunks];
    float dot = 0.f;
#pragma unroll
    for (int q = 0; q < kNormMaxChunks; ++q) {
      const int64_t ch = lt + (int64_t)q * tpr;
      xc[q] = make_uint4(0, 0, 0, 0);
      gc[q] = make_uint4(0, 0, 0, 0);
      if (src >= 0 && ch < nch) {
        xc[q] = *reinterpret_cast<const uint4*>(X + src * ldx + ch * VN);
        gc[q] = *reinterpret_cast<const uint4*>(dY + i * d + ch * VN);
        float xv[VN], gv[VN];
        unpack_chunk(xc[q], xv, T{});
        unpack_chunk(gc[q], gv, T{});
#pragma unroll
        for (int u = 0; u < VN; ++u) {
          dot = fmaf(gv[u] * (1.0f + load_w(w, ch * VN + u)), xv[u], dot);
          acc[q][u] = fmaf(gv[u] * xv[u], r, acc[q][u]);
        }
      }
    }
    const float tot = row_sum(dot, tpr, red);
    if (src < 0) continue;
    const float coef = r * r * r * tot * inv_d;
#pragma unroll
    for (int q = 0; q < kNormMaxChunks; ++q) {
      const int64_t ch = lt + (int64_t)q * tpr;
      if (ch < nch) {
        float xv[VN], gv[VN];
        unpack_chunk(xc[q], xv, T{});
        unpack_chunk(gc[q], gv, T{});
#pragma unroll
        for (int u = 0; u < VN; ++u) gv[u] = r * gv[u] * (1.0f + load_w(w, ch * VN + u)) - xv[u] * coef;
        *reinterpret_cast<uint4*>(dX + src * lddx + ch * VN) = pack_chunk(gv, T{});
      }
    }
  }
  // one row slot per block (rpb == 1): the partial is this thread's accumulators; otherwise
  // (d <= 1024 elements) the slots are summed in slot order through LDS
  float* dst = rpb == 1 ? partial + (int64_t)blockIdx.x * d : slot_dw + (int64_t)slot * d;
#pragma unroll
  for (int q = 0; q < kNormMaxChunks; ++q) {
    const int64_t ch = lt + (int64_t)q * tpr;
    if (ch < nch)
#pragma unroll
      for (int u = 0; u < VN; ++u) dst[ch * VN + u] = acc[q][u];
  }
  if (rpb == 1) return;
  __syncthreads();
  for (int64_t col = threadIdx.x; col < d; col += kNormThreads) {
    float t = 0.f;
    for (int s2 = 0; s2 < rpb; ++s2) t += slot_dw[(int64_t)s2 * d + col];
    partial[(int64_t)blockIdx.x * d + col] = t;
  }
}

// dw[c] = sum over partials p (in order) of partial[p][c], rounded once to the weight's dtype.
template <typename TW>
__global__ __launch_bounds__(256) void rmsnorm_dw_reduce_kernel(const float* __restrict__ partial, int P, int64_t d,
                                                                TW* __restrict__ dw) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= d) return;
  float t = 0.f;
  for (int p = 0; p < P; ++p) t += partial[(int64_t)p * d + c];
  dw[c] = from_f32<TW>(t);
}

int norm_partials(int64_t n, int rpb) {
  const int64_t want = cdiv(n > 0 ? n : 1, rpb);
  return (int)(want < kNormMaxPartials ? want : kNormMaxPartials);
}

template <typename T, typename TW>
int launch_norm_fwd(const void* X, int64_t ldx, int64_t x_rows, const int64_t* rows, int64_t n, int64_t d,
                    const void* w, float eps, void* Y, float* rstd, hipStream_t s) {
  const NormMap m = norm_map(d / (16 / (int64_t)sizeof(T)));
  hipLaunchKernelGGL((rmsnorm_rows_kernel<T, TW>), dim3((unsigned)cdiv(n, m.rpb)), dim3(kNormThreads), 0, s,
                     static_cast<const T*>(X), ldx, x_rows, rows, n, d, static_cast<const TW*>(w), eps,
                     static_cast<T*>(Y), rstd, m.tpr);
  return check_launch("rmsnorm_rows");
}

template <typename T, typename TW>
int launch_norm_bwd(const void* dY, const void* X, int64_t ldx, int64_t x_rows, const int64_t* rows, int64_t n,
                    int64_t d, const float* rstd, const void* w, void* dX, int64_t lddx, void* dw, float* partial,
                    hipStream_t s) {
  const NormMap m = norm_map(d / (16 / (int64_t)sizeof(T)));
  const int P = norm_partials(n, m.rpb);
  const size_t lds = m.rpb == 1 ? 0 : (size_t)m.rpb * (size_t)d * sizeof(float);  // rpb > 1: d <= 1024
  hipLaunchKernelGGL((rmsnorm_rows_backward_kernel<T, TW>), dim3((unsigned)P), dim3(kNormThreads), lds, s,
                     static_cast<const T*>(dY), static_cast<const T*>(X), ldx, x_rows, rows, n, d, rstd,
                     static_cast<const TW*>(w), static_cast<T*>(dX), lddx, partial, m.tpr);
  int rc = check_launch("rmsnorm_rows_backward");
  if (rc) return rc;
  hipLaunchKernelGGL((rmsnorm_dw_reduce_kernel<TW>), dim3((unsigned)cdiv(d, 256)), dim3(256), 0, s, partial, P, d,
                     static_cast<TW*>(dw));
  return check_launch("rmsnorm_rows_backward dw");
}

int norm_shape_checks(int64_t x_stride, int64_t x_rows, int64_t n, int64_t d, int w_dtype, int dtype,
                      const char* name) {
  ZMOE_REQUIRE(dtype_ok(dtype) && dtype_ok(w_dtype), ZMOE_ERR_DTYPE, "%s: dtype %d / weight dtype %d", name, dtype,
               w_dtype);
  const int64_t vec = 16 / dtype_size(dtype);
  ZMOE_REQUIRE(n >= 0 && x_rows >= 0 && d >= 1, ZMOE_ERR_SHAPE, "%s: bad sizes (n=%lld d=%lld)", name,
               (long long)n, (long long)d);
  ZMOE_REQUIRE(d <= 256 * kNormMaxChunks * vec, ZMOE_ERR_SHAPE, "%s: d=%lld above the row kernel's %lld", name,
               (long long)d, (long long)(256 * kNormMaxChunks * vec));
  ZMOE_REQUIRE(d % vec == 0 && x_stride % vec == 0 && x_stride >= d, ZMOE_ERR_ALIGN,
               "%s: d and the row stride must be multiples of %lld elements", name, (long long)vec);
  return ZMOE_OK;
}

}  // namespace zmoe

using namespace zmoe;

extern "C" int zmoe_rmsnorm_rows(const void* X, int64_t x_stride, int64_t x_rows, const int64_t* rows, int64_t n,
                                 int64_t d, const void* weight, int w_dtype, float eps, int dtype, void* Y,
                                 float* rstd, void* stream) {
  int rc = norm_shape_checks(x_stride, x_rows, n, d, w_dtype, dtype, "rmsnorm_rows");
  if (rc) return rc;
  if (n == 0) return ZMOE_OK;
  ZMOE_REQUIRE(X && weight && Y, ZMOE_ERR_NULL, "rmsnorm_rows: null pointer");
  ZMOE_REQUIRE(aligned16(X) && aligned16(Y), ZMOE_ERR_ALIGN, "rmsnorm_rows: X and Y must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  if (dtype == ZMOE_DTYPE_BF16)
    return w_dtype == ZMOE_DTYPE_BF16
               ? launch_norm_fwd<uint16_t, uint16_t>(X, x_stride, x_rows, rows, n, d, weight, eps, Y, rstd, s)
               : launch_norm_fwd<uint16_t, float>(X, x_stride, x_rows, rows, n, d, weight, eps, Y, rstd, s);
  return w_dtype == ZMOE_DTYPE_BF16
             ? launch_norm_fwd<float, uint16_t>(X, x_stride, x_rows, rows, n, d, weight, eps, Y, rstd, s)
             : launch_norm_fwd<float, float>(X, x_stride, x_rows, rows, n, d, weight, eps, Y, rstd, s);
}

extern "C" size_t zmoe_rmsnorm_rows_backward_workspace_bytes(int64_t n, int64_t d, int dtype) {
  if (d < 1 || !dtype_ok(dtype)) return 0;
  const NormMap m = norm_map(d / (16 / dtype_size(dtype)));
  return (size_t)norm_partials(n, m.rpb) * (size_t)d * sizeof(float);
}

extern "C" int zmoe_rmsnorm_rows_backward(const void* dY, const void* X, int64_t x_stride, int64_t x_rows,
                                          const int64_t* rows, int64_t n, int64_t d, const float* rstd,
                                          const void* weight, int w_dtype, int dtype, void* dX, int64_t dx_stride,
                                          void* dweight, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = norm_shape_checks(x_stride, x_rows, n, d, w_dtype, dtype, "rmsnorm_rows_backward");
  if (rc) return rc;
  const int64_t vec = 16 / dtype_size(dtype);
  ZMOE_REQUIRE(dx_stride % vec == 0 && dx_stride >= d, ZMOE_ERR_ALIGN,
               "rmsnorm_rows_backward: dX row stride must be a multiple of %lld elements", (long long)vec);
  ZMOE_REQUIRE(weight && dweight && workspace, ZMOE_ERR_NULL, "rmsnorm_rows_backward: null pointer");
  ZMOE_REQUIRE(n == 0 || (dY && X && rstd && dX), ZMOE_ERR_NULL, "rmsnorm_rows_backward: null operand");
  const size_t need = zmoe_rmsnorm_rows_backward_workspace_bytes(n, d, dtype);
  ZMOE_REQUIRE(workspace_bytes >= need, ZMOE_ERR_WORKSPACE, "rmsnorm_rows_backward: workspace %zu < %zu bytes",
               workspace_bytes, need);
  ZMOE_REQUIRE((n == 0 || (aligned16(dY) && aligned16(X) && aligned16(dX))) && aligned16(workspace), ZMOE_ERR_ALIGN,
               "rmsnorm_rows_backward: operands must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  float* partial = static_cast<float*>(workspace);
  if (dtype == ZMOE_DTYPE_BF16)
    return w_dtype == ZMOE_DTYPE_BF16
               ? launch_norm_bwd<uint16_t, uint16_t>(dY, X, x_stride, x_rows, rows, n, d, rstd, weight, dX, dx_stride,
                                                     dweight, partial, s)
               : launch_norm_bwd<uint16_t, float>(dY, X, x_stride, x_rows, rows, n, d, rstd, weight, dX, dx_stride,
                                                  dweight, partial, s);
  return w_dtype == ZMOE_DTYPE_BF16
             ? launch_norm_bwd<float, uint16_t>(dY, X, x_stride, x_rows, rows, n, d, rstd, weight, dX, dx_stride,
                                                dweight, partial, s)
             : launch_norm_bwd<float, float>(dY, X, x_stride, x_rows, rows, n, d, rstd, weight, dX, dx_stride,
                                             dweight, partial, s);
}
