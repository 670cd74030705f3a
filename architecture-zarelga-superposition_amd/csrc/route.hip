// Aux-loss-free sigmoid routing (modeling/moe_gate.py:27-34), its backward, and
// the aux-loss-free bias update (main.py:161-175).
//
// One 64-lane wave owns one token row. Lane l holds experts l, l+64, ... so a
// row of E <= 1024 scores sits in registers; k rounds of a wave-wide max
// (xor-shuffle butterfly over packed (score, expert) keys) pick the slots in the
// contract order (score desc, expert asc, NaN first).
#include <type_traits>

#include "zmoe_internal.h"

namespace zmoe {

constexpr int kRouteMaxPerLane = 16;  // E <= 1024

// Sort key of a routing candidate; a larger key takes an earlier slot. The high word is
// a monotone image of the biased score (every NaN canonicalised above +inf, -0 folded
// into +0), the low word the inverted expert id, so equal scores go to the lower expert.
__device__ __forceinline__ uint64_t route_key(float s, int e) {
  uint32_t b = __float_as_uint(s);
  if (s != s) b = 0x7fffffffu;
  else if (s == 0.f) b = 0u;
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)b << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}
// key 0 is below every candidate's key (the high word of a real key is at least 0x007fffff)
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o, 64);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}

// sigmoid evaluated in double, rounded once to float
__device__ __forceinline__ float sigmoid_f64(float z) { return (float)(1.0 / (1.0 + exp(-(double)z))); }

// One wave per token; lane l holds experts l + 64 q (q < PL). The score is the sigmoid
// evaluated in double and rounded once to float (then to bf16 when the gate ran in
// bf16, as autocast stores it); k rounds of a wave-wide max over route_key pick the
// slots in contract order.
template <int PL, typename LT>
__global__ __launch_bounds__(256) void route_topk_kernel(const LT* __restrict__ logits, int64_t T, int E,
                                                         int k, const float* __restrict__ bias,
                                                         int round_bf16, int64_t* __restrict__ out_idx,
                                                         float* __restrict__ out_w,
                                                         float* __restrict__ out_p) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  const LT* row = logits + t * (int64_t)E;

  float p[PL];
  uint64_t key[PL];
#pragma unroll
  for (int q = 0; q < PL; ++q) {
    const int e = lane + 64 * q;
    p[q] = 0.f;
    key[q] = 0;  // padding never wins
    if (e < E) {
      const float z = to_f32(row[e]);
      float pv = sigmoid_f64(z);
      if (round_bf16) pv = to_f32(bf16_bits(pv));
      p[q] = pv;
      key[q] = route_key(pv + bias[e], e);
    }
  }

  int my_e = 0;  // slot owned by this lane (lane j keeps slot j)
  float my_p = 0.f;
  for (int j = 0; j < k; ++j) {
    uint64_t best = key[0];
#pragma unroll
    for (int q = 1; q < PL; ++q) best = key[q] > best ? key[q] : best;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const uint64_t other = shfl_xor_u64(best, o);
      best = other > best ? other : best;
    }
    const int be = (int)(0xffffffffu - (uint32_t)best);  // uniform across the wave
    const int owner = be & 63, oq = be >> 6;
    float pw = p[0];
#pragma unroll
    for (int q = 1; q < PL; ++q) pw = q == oq ? p[q] : pw;
    pw = __shfl(pw, owner, 64);
    if (lane == owner) {
#pragma unroll
      for (int q = 0; q < PL; ++q) key[q] = q == oq ? 0 : key[q];
    }
    if (lane == j) {
      my_e = be;
      my_p = pw;
    }
  }

  const float sum = wave_sum(lane < k ? fabsf(my_p) : 0.f);
  const float denom = sum < 1e-12f ? 1e-12f : sum;  // NaN propagates
  if (lane < k) {
    out_idx[t * k + lane] = my_e;
    out_w[t * k + lane] = my_p / denom;
    if (out_p) out_p[t * k + lane] = my_p;
  }
}

template <typename GT>
__global__ __launch_bounds__(256) void route_topk_backward_kernel(const float* __restrict__ dw,
                                                                  const float* __restrict__ prob,
                                                                  const int64_t* __restrict__ idx,
                                                                  int64_t T, int E, int k,
                                                                  GT* __restrict__ dlogits, int64_t ld) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;
  float pj = 0.f, dwj = 0.f;
  int ej = -1;
  if (lane < k) {
    pj = prob[t * k + lane];
    dwj = dw[t * k + lane];
    ej = (int)idx[t * k + lane];
  }
  const float S_raw = wave_sum(fabsf(pj));
  const float S = S_raw < 1e-12f ? 1e-12f : S_raw;
  const float inner = wave_sum(dwj * (pj / S));
  const float sgn = pj > 0.f ? 1.f : (pj < 0.f ? -1.f : 0.f);
  const float dp = S_raw > 1e-12f ? (dwj - inner * sgn) / S : dwj / S;
  const float dz = dp * pj * (1.f - pj);
  GT* row = dlogits + t * ld;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    float v = 0.f;
    for (int j = 0; j < k; ++j) {
      const int ek = __shfl(ej, j, 64);
      const float vk = __shfl(dz, j, 64);
      if (ek == e) v = vk;
    }
    if (e < E) row[e] = from_f32<GT>(v);
  }
}

__global__ void bias_update_kernel(const int64_t* __restrict__ offsets, int E, float rate,
                                   float* __restrict__ bias) {
  const int e = threadIdx.x;
  if (e >= E) return;
  const int64_t R = offsets[E - 1];
  if (R <= 0) return;  // no routed tokens this step: no update (main.py:170-171)
  const float count = (float)(offsets[e] - (e ? offsets[e - 1] : 0));
  const float mean = (float)R / (float)E;
  const float err = mean - count;
  const float sgn = err > 0.f ? 1.f : (err < 0.f ? -1.f : 0.f);
  bias[e] = bias[e] + rate * sgn;
}

}  // namespace zmoe

using namespace zmoe;

extern "C" int zmoe_route_topk(const void* logits, int logits_dtype, int64_t T, int E, int k,
                               const float* expert_biases, int round_probs_bf16, int64_t* topk_idx,
                               float* topk_weight, float* topk_prob, void* stream) {
  ZMOE_REQUIRE(dtype_ok(logits_dtype), ZMOE_ERR_DTYPE, "route_topk: logits dtype %d", logits_dtype);
  ZMOE_REQUIRE(T >= 0 && E >= 1 && E <= 64 * kRouteMaxPerLane, ZMOE_ERR_SHAPE,
               "route_topk: need 1 <= E <= %d (E=%d)", 64 * kRouteMaxPerLane, E);
  ZMOE_REQUIRE(k >= 1 && k <= E && k <= 64, ZMOE_ERR_SHAPE, "route_topk: need 1 <= k <= min(E, 64) (k=%d, E=%d)", k, E);
  if (T == 0) return ZMOE_OK;
  ZMOE_REQUIRE(logits && expert_biases && topk_idx && topk_weight, ZMOE_ERR_NULL, "route_topk: null pointer");
  const dim3 grid((unsigned)cdiv(T, 4)), block(256);
  const int per_lane = (E + 63) / 64;
  auto launch = [&](auto pl, auto lt) {
    using LT = decltype(lt);
    hipLaunchKernelGGL((route_topk_kernel<decltype(pl)::value, LT>), grid, block, 0, as_stream(stream),
                       (const LT*)logits, T, E, k, expert_biases, round_probs_bf16, topk_idx, topk_weight,
                       topk_prob);
  };
  auto by_width = [&](auto lt) {
    if (per_lane <= 1) launch(std::integral_constant<int, 1>{}, lt);
    else if (per_lane <= 2) launch(std::integral_constant<int, 2>{}, lt);
    else if (per_lane <= 4) launch(std::integral_constant<int, 4>{}, lt);
    else if (per_lane <= 8) launch(std::integral_constant<int, 8>{}, lt);
    else launch(std::integral_constant<int, 16>{}, lt);
  };
  if (logits_dtype == ZMOE_DTYPE_BF16) by_width(uint16_t{});
  else by_width(float{});
  return check_launch("route_topk");
}

extern "C" int zmoe_route_topk_backward(const float* d_weight, const float* topk_prob,
                                        const int64_t* topk_idx, int64_t T, int E, int k, void* d_logits,
                                        int64_t ld_d_logits, int d_logits_dtype, void* stream) {
  ZMOE_REQUIRE(dtype_ok(d_logits_dtype), ZMOE_ERR_DTYPE, "route_topk_backward: dtype %d", d_logits_dtype);
  ZMOE_REQUIRE(T >= 0 && E >= 1 && k >= 1 && k <= E && k <= 64, ZMOE_ERR_SHAPE,
               "route_topk_backward: bad sizes (E=%d, k=%d)", E, k);
  ZMOE_REQUIRE(ld_d_logits >= E, ZMOE_ERR_SHAPE, "route_topk_backward: row stride %lld below E=%d",
               (long long)ld_d_logits, E);
  if (T == 0) return ZMOE_OK;
  ZMOE_REQUIRE(d_weight && topk_prob && topk_idx && d_logits, ZMOE_ERR_NULL, "route_topk_backward: null pointer");
  const dim3 grid((unsigned)cdiv(T, 4)), block(256);
  if (d_logits_dtype == ZMOE_DTYPE_BF16)
    hipLaunchKernelGGL(route_topk_backward_kernel<uint16_t>, grid, block, 0, as_stream(stream), d_weight,
                       topk_prob, topk_idx, T, E, k, (uint16_t*)d_logits, ld_d_logits);
  else
    hipLaunchKernelGGL(route_topk_backward_kernel<float>, grid, block, 0, as_stream(stream), d_weight,
                       topk_prob, topk_idx, T, E, k, (float*)d_logits, ld_d_logits);
  return check_launch("route_topk_backward");
}

extern "C" int zmoe_bias_update(const int64_t* expert_offsets, int E, float update_rate, float* expert_biases,
                                void* stream) {
  ZMOE_REQUIRE(E >= 1 && E <= 1024, ZMOE_ERR_SHAPE, "bias_update: need 1 <= E <= 1024 (E=%d)", E);
  ZMOE_REQUIRE(expert_offsets && expert_biases, ZMOE_ERR_NULL, "bias_update: null pointer");
  hipLaunchKernelGGL(bias_update_kernel, dim3(1), dim3(1024), 0, as_stream(stream), expert_offsets, E,
                     update_rate, expert_biases);
  return check_launch("bias_update");
}
