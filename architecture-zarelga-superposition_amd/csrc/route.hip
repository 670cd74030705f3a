// Aux-loss-free sigmoid routing (modeling/moe_gate.py:27-34), its backward, and
// the aux-loss-free bias update (main.py:161-175).
//
// Slots come in the contract order (score desc, expert asc, NaN first), picked in
// k rounds of a max over the token's score keys. For bf16 logits with E % 8 == 0,
// E <= 256 and k <= 16 a wave routes 4 or 8 tokens at once, one per row of 16 or 8
// lanes, each lane holding 8 or 16 consecutive experts, with bf16 probabilities
// read from a table the build writes (route_topk_rows_kernel). Otherwise one
// 64-lane wave owns one token row: lane l holds experts l, l+64, ... (E <= 1024)
// and each round is a wave-wide max (route_topk_kernel).
#include <type_traits>

#include "zmoe_internal.h"

namespace zmoe {

constexpr int kRouteMaxPerLane = 16;  // E <= 1024

// Sort key of a routing candidate's score; a larger key takes an earlier slot. A monotone
// image of the biased score: every NaN canonicalised above +inf, -0 folded into +0. Equal
// scores go to the lower expert. Key 0 marks a taken (or padding) candidate: a real
// score's key is at least 0x007fffff (that of -inf).
__device__ __forceinline__ uint32_t score_key(float s) {
  uint32_t b = __float_as_uint(s);
  b = s != s ? 0x7fffffffu : b;  // selects, not branches
  b = s == 0.f ? 0u : b;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Logits at or below this value give probability 0: there torch's sigmoid, which forms
// 1 / (1 + exp(-z)) in fp32, overflows exp(-z) to inf (fp32 exp overflows from
// 88.72283935546875 up; the true probabilities, below 2.9e-39, would be subnormal).
constexpr float kSigmoidZeroBelow = -88.72283935546875f;

// Below this |z| the probability comes from p = 0.5 + z/4 - z^3/48 + ...: 0.5 + z/4 is
// exact in double, and the cubic term cannot move it across an fp32 rounding midpoint
// unless it lies exactly on one (its distance from a midpoint is a multiple of z's last
// bit / 4, more than |z|^3/48 here).
constexpr float kSigmoidSeriesBelow = 0x1p-12f;

// sigmoid correctly rounded to float: for |z| < kSigmoidSeriesBelow, 0.5 + z/4 rounded to
// nearest with an exact tie going to the side the cubic term puts the true value on (down
// for z > 0, up for z < 0; many small bf16 logits land on such ties, where a double
// evaluation's rounding would hang on the last bit of its exp); otherwise
// 1 / (1 + exp(-z)) in double, rounded once; 0 at or below kSigmoidZeroBelow.
__device__ __forceinline__ float sigmoid_f64(float z) {
  if (z <= kSigmoidZeroBelow) return 0.f;
  if (fabsf(z) < kSigmoidSeriesBelow) {
    const double s = 0.5 + 0.25 * (double)z;
    const float f = (float)s;
    const double fd = (double)f;
    if (fd != s) {  // f > 0: its other neighbour around s is one bit pattern up or down
      const float o = __uint_as_float(__float_as_uint(f) + (fd < s ? 1u : 0xffffffffu));
      if (fabs(s - fd) == fabs((double)o - s)) return z > 0.f ? fminf(f, o) : fmaxf(f, o);
    }
    return f;
  }
  return (float)(1.0 / (1.0 + exp(-(double)z)));
}

// bf16(sigmoid_f64(z)) (the probability a bf16 gate stores) from fp32 arithmetic where that
// is provably the same value: the fp32 estimate is within a few fp32 ulps of the true
// sigmoid (expf within 1 ulp, one add, v_rcp_f32 within 1 ulp), and so is sigmoid_f64's
// fp32 rounding, so both round to the same bf16 unless they lie within 16 fp32 ulps of a
// bf16 rounding midpoint (low 16 bits near 0x8000). Those lanes (about 1 score in 2000),
// saturated arguments (|z| >= 80, where expf overflows) and NaN take the double
// evaluation. (1 + expf(-z) lies in [1, 6e34] here, so the reciprocal is a normal float.)
__device__ __forceinline__ float sigmoid_bf16(float z) {
  if (fabsf(z) < 80.f) {  // false for NaN
    const float s = __builtin_amdgcn_rcpf(1.0f + expf(-z));
    const uint32_t low = __float_as_uint(s) & 0xffffu;
    const uint32_t dist = low > 0x8000u ? low - 0x8000u : 0x8000u - low;
    if (dist > 16u) return to_f32(bf16_bits(s));
  }
  return to_f32(bf16_bits(sigmoid_f64(z)));
}

// bf16(fp32(sigmoid_f64(z))) for every bf16 logit z, indexed by z's bits: the value
// sigmoid_bf16 returns, read instead of evaluated when the logits themselves are bf16.
// The build writes the entries (float64 sigmoid, one rounding to float, then to bf16 by
// round to nearest even; 0 at or below kSigmoidZeroBelow; NaN logits give 0x7fc0). 128 KB,
// read through the caches.
__device__ const uint16_t kSigmoidBf16[65536] = {
#include "zmoe_sigmoid_bf16.inc"
};

// The stored probability of a logit when the gate rounds to bf16: looked up for bf16
// logits, evaluated for fp32 ones.
__device__ __forceinline__ float sigmoid_bf16_of(uint16_t zb) { return to_f32(kSigmoidBf16[zb]); }
__device__ __forceinline__ float sigmoid_bf16_of(float z) { return sigmoid_bf16(z); }

// Wave-wide max of a 32-bit key, the same value in every lane: DPP within rows of 16
// (xor 1, xor 2, half mirror, mirror: no LDS round trip), then the four row maxima
// through readlane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x140, 0xF, 0xF, false));  // row_mirror
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(r0, r1), max(r2, r3));
}

// Waves stride over tokens (each wave one token at a time, the next row's logits loaded
// before the current one is ranked); lane l holds experts l + 64 q (q < PL). The score is
// the sigmoid evaluated in double and rounded once to float (then to bf16 when the gate
// ran in bf16, as autocast stores it). k rounds each take the wave max of the score keys
// and the lowest expert holding it (ballots in expert order), so slots come in contract
// order: score desc, expert asc, NaN first.
template <int PL, typename LT>
__global__ __launch_bounds__(256) void route_topk_kernel(const LT* __restrict__ logits, int64_t T, int E,
                                                         int k, const float* __restrict__ bias,
                                                         int round_bf16, int64_t* __restrict__ out_idx,
                                                         float* __restrict__ out_w,
                                                         float* __restrict__ out_p) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
  int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  float bq[PL];
  LT nxt[PL];
#pragma unroll
  for (int q = 0; q < PL; ++q) {
    const int e = lane + 64 * q;
    bq[q] = e < E ? bias[e] : 0.f;
    nxt[q] = LT{};
    if (t < T && e < E) nxt[q] = logits[t * (int64_t)E + e];
  }
  for (; t < T; t += nwaves) {
    LT cur[PL];
#pragma unroll
    for (int q = 0; q < PL; ++q) {
      const int e = lane + 64 * q;
      cur[q] = nxt[q];
      if (t + nwaves < T && e < E) nxt[q] = logits[(t + nwaves) * (int64_t)E + e];
    }
    float p[PL];
    uint32_t key[PL];
#pragma unroll
    for (int q = 0; q < PL; ++q) {
      const int e = lane + 64 * q;
      p[q] = 0.f;
      key[q] = 0;  // padding never wins
      if (e < E) {
        const float pv = round_bf16 ? sigmoid_bf16_of(cur[q]) : sigmoid_f64(to_f32(cur[q]));
        p[q] = pv;
        key[q] = score_key(pv + bq[q]);
      }
    }
    int my_e = 0;  // slot owned by this lane (lane j keeps slot j)
    float my_p = 0.f;
    for (int j = 0; j < k; ++j) {
      uint32_t m = key[0];
#pragma unroll
      for (int q = 1; q < PL; ++q) m = max(m, key[q]);
      m = wave_max_u32(m);
      // the lowest expert whose key is the max: experts l + 64 q, checked in q order
      int be = -1;
#pragma unroll
      for (int q = 0; q < PL; ++q) {
        const uint64_t hit = __ballot(key[q] == m);
        if (be < 0 && hit) be = 64 * q + __builtin_ctzll(hit);
      }
      const int owner = be & 63, oq = be >> 6;  // uniform across the wave
      float pw = p[0];
#pragma unroll
      for (int q = 1; q < PL; ++q) pw = q == oq ? p[q] : pw;
      pw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pw), owner));
      if (lane == owner) {
#pragma unroll
        for (int q = 0; q < PL; ++q) key[q] = q == oq ? 0u : key[q];
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
}

// Reductions over rows of LPR = 16 or 8 lanes by DPP (xor 1, xor 2, mirror within 8 lanes,
// mirror within 16); every lane of a row ends with the row's result.
template <int LPR>
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, true));
  if (LPR == 16) v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, true));
  return v;
}
template <int LPR>
__device__ __forceinline__ uint32_t row_min_u32(uint32_t v) {
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0xB1, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x4E, 0xF, 0xF, false));
  v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x141, 0xF, 0xF, false));
  if (LPR == 16) v = min(v, (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)v, 0x140, 0xF, 0xF, false));
  return v;
}
template <int LPR>
__device__ __forceinline__ float row_sum_f32(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));
  if (LPR == 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, true));
  return v;
}

// bf16 logits, E % 8 == 0, E <= LPR * VPL, k <= LPR: 64 / LPR tokens per wave, one per
// row of LPR lanes. Lane r of a row holds experts VPL r .. VPL r + VPL - 1 (16-byte loads
// of the contiguous logits row); with RB the bf16 probabilities come from kSigmoidBf16.
// Each round takes the row max m of the score keys (DPP within the row), the
// per-candidate hits key == m as wave masks, each lane's lowest hit expert, and the row
// min of those (the lowest expert holding m); the owner lane clears its lowest hit, the
// masks reused for that (a lane's first hit is a scalar mask product). The selected
// probabilities are read back from LDS once at the end. A wave works through its groups
// of rows with the next group's logits loaded while the current one is ranked. Same
// contract and values as route_topk_kernel.
template <int VPL, int LPR, bool RB>
__global__ __launch_bounds__(256) void route_topk_rows_kernel(const uint16_t* __restrict__ logits, int64_t T,
                                                              int E, int k, const float* __restrict__ bias,
                                                              int64_t* __restrict__ out_idx,
                                                              float* __restrict__ out_w,
                                                              float* __restrict__ out_p) {
  constexpr int TPW = 64 / LPR;  // tokens per wave
  __shared__ float ps[4][TPW][LPR * VPL];  // [wave][row][expert]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = lane / LPR, r = lane % LPR;
  const int e0 = r * VPL;
  const bool has = e0 < E;  // E % 8 == 0: each 8-expert chunk of a lane is wholly in [0, E) or out
  float bq[VPL];
#pragma unroll
  for (int q = 0; q < VPL; ++q) bq[q] = e0 + q < E ? bias[e0 + q] : 0.f;
  const int64_t groups = (T + TPW - 1) / TPW;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  // this lane's logits of group g, by buffer loads over the group's rows: lanes past T or E
  // read zeros with no branch, so the wait for the table reads issued before a prefetch
  // can leave the prefetch in flight
  auto load = [&](int64_t gv, uint4* raw) {
    // g is the same in every lane; say so, so that the descriptor stays in scalar registers
    const int64_t g = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(gv >> 32)) << 32) |
                                (uint32_t)__builtin_amdgcn_readfirstlane((int)gv));
    const bool in = g < groups;
    const int64_t rows_left = in ? T - TPW * g : 0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(logits + (in ? TPW * g * (int64_t)E : 0)), (short)0,
        (int)((rows_left < TPW ? rows_left : TPW) * E * 2), 0x00020000);
#pragma unroll
    for (int c = 0; c < VPL / 8; ++c) {
      const uint32_t off = e0 + 8 * c < E ? (uint32_t)(row * E + e0 + 8 * c) * 2u : 0x80000000u;
      raw[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
  };
  uint4 nxt[VPL / 8];
  load((int64_t)blockIdx.x * 4 + wave, nxt);
  for (int64_t g = (int64_t)blockIdx.x * 4 + wave; g < groups; g += nwaves) {
    const int64_t t = g * TPW + row;
    const bool live = t < T && has;
    uint32_t zb[VPL];  // logit bits
#pragma unroll
    for (int c = 0; c < VPL / 8; ++c) {
      const uint32_t w[4] = {nxt[c].x, nxt[c].y, nxt[c].z, nxt[c].w};
#pragma unroll
      for (int u = 0; u < 8; ++u) zb[8 * c + u] = (u & 1) ? w[u >> 1] >> 16 : w[u >> 1] & 0xffffu;
    }
    float p[VPL];
    if constexpr (RB) {
      uint32_t pb[VPL];  // all table reads in flight before the next group's logits are requested
#pragma unroll
      for (int q = 0; q < VPL; ++q) pb[q] = kSigmoidBf16[zb[q]];
      load(g + nwaves, nxt);
#pragma unroll
      for (int q = 0; q < VPL; ++q) p[q] = __uint_as_float(pb[q] << 16);
    } else {
      load(g + nwaves, nxt);
#pragma unroll
      for (int q = 0; q < VPL; ++q) p[q] = sigmoid_f64(__uint_as_float(zb[q] << 16));
    }
    uint32_t key[VPL];
#pragma unroll
    for (int q = 0; q < VPL; ++q) key[q] = live && e0 + q < E ? score_key(p[q] + bq[q]) : 0u;
    if (has) {
#pragma unroll
      for (int q = 0; q < VPL; q += 4)
        *reinterpret_cast<float4*>(&ps[wave][row][e0 + q]) = make_float4(p[q], p[q + 1], p[q + 2], p[q + 3]);
    }
    uint32_t my_e = 0;
    for (int j = 0; j < k; ++j) {
      uint32_t m = key[0];
#pragma unroll
      for (int q = 1; q < VPL; ++q) m = max(m, key[q]);
      m = row_max_u32<LPR>(m);
      uint64_t hit[VPL];
#pragma unroll
      for (int q = 0; q < VPL; ++q) hit[q] = __builtin_amdgcn_ballot_w64(key[q] == m);
      // this lane's lowest expert holding m (none: all ones), then the row's lowest
      uint32_t cand = 0xffffffffu;
#pragma unroll
      for (int q = VPL - 1; q >= 0; --q) cand = __builtin_amdgcn_inverse_ballot_w64(hit[q]) ? (uint32_t)(e0 + q) : cand;
      const uint32_t ew = row_min_u32<LPR>(cand);
      const uint64_t owner = __builtin_amdgcn_ballot_w64(cand == ew);  // one lane per row
      uint64_t seen = 0;
#pragma unroll
      for (int q = 0; q < VPL; ++q) {
        const uint64_t first = hit[q] & owner & ~seen;
        seen |= hit[q];
        key[q] = __builtin_amdgcn_inverse_ballot_w64(first) ? 0u : key[q];
      }
      my_e = r == j ? ew : my_e;
    }
    __builtin_amdgcn_wave_barrier();
    const float my_p = r < k ? ps[wave][row][my_e] : 0.f;
    const float sum = row_sum_f32<LPR>(r < k ? fabsf(my_p) : 0.f);
    const float denom = sum < 1e-12f ? 1e-12f : sum;  // NaN propagates
    if (t < T && r < k) {
      out_idx[t * k + r] = my_e;
      out_w[t * k + r] = my_p / denom;
      if (out_p) out_p[t * k + r] = my_p;
    }
    __builtin_amdgcn_wave_barrier();
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
  if (k <= 16) {
    // the k (expert, grad) pairs read once into scalar registers (k is uniform), then
    // every lane picks its expert's grad: no cross-lane traffic per 64-expert block
    int ek[16];
    float vk[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      ek[j] = j < k ? __builtin_amdgcn_readlane(ej, j) : -1;
      vk[j] = j < k ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dz), j)) : 0.f;
    }
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) v = ek[j] == e ? vk[j] : v;
      if (e < E) row[e] = from_f32<GT>(v);
    }
    return;
  }
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
  // 4 waves per block, 8 blocks per CU at most: the waves loop over the remaining tokens
  const int64_t blocks = cdiv(T, 4) < 2048 ? cdiv(T, 4) : 2048;
  const dim3 grid((unsigned)blocks), block(256);
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
  if (logits_dtype == ZMOE_DTYPE_BF16 && E % 8 == 0 && E <= 256 && k <= 16 && aligned16(logits)) {
    // several tokens per wave, one per row of lanes; a wave ranks ~2 groups of rows
    auto rows = [&](auto vpl, auto lpr, auto rb) {
      constexpr int TPW = 64 / decltype(lpr)::value;
      const int64_t blocks = cdiv(cdiv(T, TPW), 8);
      hipLaunchKernelGGL((route_topk_rows_kernel<decltype(vpl)::value, decltype(lpr)::value, decltype(rb)::value>),
                         dim3((unsigned)(blocks < 1024 ? blocks : 1024)), block, 0, as_stream(stream),
                         (const uint16_t*)logits, T, E, k, expert_biases, topk_idx, topk_weight, topk_prob);
    };
    using I8 = std::integral_constant<int, 8>;
    using I16 = std::integral_constant<int, 16>;
    auto by_rb = [&](auto vpl, auto lpr) {
      if (round_probs_bf16) rows(vpl, lpr, std::true_type{});
      else rows(vpl, lpr, std::false_type{});
    };
    if (E <= 64 && k <= 8) by_rb(I8{}, I8{});         // 8 tokens per wave
    else if (E <= 128 && k <= 8) by_rb(I16{}, I8{});
    else if (E <= 128) by_rb(I8{}, I16{});            // 4 tokens per wave
    else by_rb(I16{}, I16{});
    return check_launch("route_topk");
  }
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
