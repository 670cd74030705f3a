// Newton-Schulz orthogonalisation of a stack of matrices (optimizer/muon.py:6-32),
// the GEMM-heavy core of the MuonMD step on 3-D expert weights (muon.py:399-508,
// called at :449 as zeropower_via_newtonschulz5(update, steps)).
//
// X [E, m, n] bf16 with m <= n (the caller transposes a tall stack, as muon.py:18-19
// does with .mT). Per matrix, in bf16 tensor arithmetic (every product and sum
// rounded to bf16, every GEMM accumulated in fp32 and rounded once):
//   X = X / (||X||_F + 1e-7)
//   repeat steps:  A = X X^T;  B = b A + (c A) A;  X = a X + B X
// The three GEMMs of a step are the grouped rows kernel with one "expert" per
// matrix: A = X X^T reads its right operand as nn.Linear-style rows of X; (cA) A
// and B X read A and X as [K][N]. Their epilogues form cA (a second output of the
// first GEMM) and the b A and a X sums, so each step is three launches and no
// elementwise passes. A and B are symmetric, so their GEMMs run only the tiles on
// or above the diagonal and write each off-diagonal tile's mirror as well.
//
// The Frobenius norm is a deterministic two-pass reduction: fp32 partial sums
// of squares per (matrix, slice), then every slice block sums its matrix's
// partials in a fixed order before scaling.
#include "zmoe_internal.h"

namespace zmoe {

constexpr int kNsThreads = 256;
constexpr int kNsMaxSlices = 64;

__global__ void ns_offsets_kernel(int64_t* off, int E, int64_t m) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < E) off[e] = (int64_t)(e + 1) * m;
}

// partial[e * P + s] = sum of x^2 over slice s of matrix e (chunks of 8 bf16)
__global__ __launch_bounds__(kNsThreads) void ns_sumsq_kernel(const uint16_t* __restrict__ X, int64_t per_chunks,
                                                              int64_t slice_chunks, int P, float* partial) {
  const int s = blockIdx.x, e = blockIdx.y;
  const uint4* x = reinterpret_cast<const uint4*>(X) + (int64_t)e * per_chunks;
  const int64_t c0 = (int64_t)s * slice_chunks;
  const int64_t c1 = c0 + slice_chunks < per_chunks ? c0 + slice_chunks : per_chunks;
  float acc = 0.f;
  for (int64_t c = c0 + threadIdx.x; c < c1; c += kNsThreads) {
    float v[8];
    unpack_chunk(x[c], v, uint16_t{});
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += v[u] * v[u];
  }
  __shared__ float red[kNsThreads / 64];
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < kNsThreads / 64; ++w) t += red[w];
    partial[(int64_t)e * P + s] = t;
  }
}

// Y = bf16(X / bf16(bf16(sqrt(sum x^2)) + 1e-7)) for slice s of matrix e
__global__ __launch_bounds__(kNsThreads) void ns_scale_kernel(const uint16_t* __restrict__ X, uint16_t* Y,
                                                              int64_t per_chunks, int64_t slice_chunks, int P,
                                                              const float* __restrict__ partial) {
  const int s = blockIdx.x, e = blockIdx.y;
  __shared__ float den_s;
  if (threadIdx.x < 64) {
    float t = 0.f;
    for (int i = threadIdx.x; i < P; i += 64) t += partial[(int64_t)e * P + i];
    t = wave_sum(t);
    if (threadIdx.x == 0) {
      const float nrm = to_f32(bf16_bits(sqrtf(t)));
      den_s = to_f32(bf16_bits(nrm + 1e-7f));
    }
  }
  __syncthreads();
  const float den = den_s;
  const uint4* x = reinterpret_cast<const uint4*>(X) + (int64_t)e * per_chunks;
  uint4* y = reinterpret_cast<uint4*>(Y) + (int64_t)e * per_chunks;
  const int64_t c0 = (int64_t)s * slice_chunks;
  const int64_t c1 = c0 + slice_chunks < per_chunks ? c0 + slice_chunks : per_chunks;
  for (int64_t c = c0 + threadIdx.x; c < c1; c += kNsThreads) {
    float v[8];
    unpack_chunk(x[c], v, uint16_t{});
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = v[u] / den;
    y[c] = pack_chunk(v, uint16_t{});
  }
}

struct NsLayout {
  size_t off_offsets, off_partial, off_a, off_p, off_b, off_x, total;
  int P;
  int64_t slice_chunks;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

NsLayout ns_layout(int64_t E, int64_t m, int64_t n) {
  NsLayout L{};
  const int64_t per_chunks = m * n / 8;
  int P = (int)cdiv(per_chunks, (int64_t)kNsThreads * 16);
  P = P < 1 ? 1 : (P > kNsMaxSlices ? kNsMaxSlices : P);
  L.P = P;
  L.slice_chunks = cdiv(per_chunks, P);
  size_t o = 0;
  L.off_offsets = o;
  o += align256((size_t)E * 8);
  L.off_partial = o;
  o += align256((size_t)E * P * 4);
  L.off_a = o;
  o += align256((size_t)(E * m * m) * 2);
  L.off_p = o;
  o += align256((size_t)(E * m * m) * 2);
  L.off_b = o;
  o += align256((size_t)(E * m * m) * 2);
  L.off_x = o;
  o += align256((size_t)(E * m * n) * 2);
  L.total = o;
  return L;
}

// Matrices per pass: the grouped GEMMs address a pass's whole X (and A, B) stack as one
// buffer resource of at most kNsMaxSpan bytes, and take at most 1024 "experts". Larger
// stacks run as consecutive passes of this many matrices over one pass-sized workspace;
// every matrix is independent, so the result does not depend on the split.
constexpr int64_t kNsMaxSpan = 0x7fff0000LL;

int64_t ns_chunk(int64_t E, int64_t m, int64_t n) {
  int64_t c = kNsMaxSpan / (m * n * 2);
  c = c < 1024 ? c : 1024;
  return c < E ? c : E;
}

}  // namespace zmoe

using namespace zmoe;

extern "C" size_t zmoe_newton_schulz5_workspace_bytes(int64_t E, int64_t m, int64_t n) {
  if (E < 1 || m < 1 || n < 1 || m > kNsMaxSpan / 2 / n) return 0;
  return ns_layout(ns_chunk(E, m, n), m, n).total;
}

namespace {

// One pass over Ec matrices at Xuser (workspace laid out for Ec).
int ns_pass(uint16_t* Xuser, int64_t Ec, int64_t m, int64_t n, int steps, float a, float b, float c, char* ws,
            hipStream_t s) {
  const NsLayout L = ns_layout(Ec, m, n);
  int64_t* offsets = reinterpret_cast<int64_t*>(ws + L.off_offsets);
  float* partial = reinterpret_cast<float*>(ws + L.off_partial);
  uint16_t* Abuf = reinterpret_cast<uint16_t*>(ws + L.off_a);
  uint16_t* Pbuf = reinterpret_cast<uint16_t*>(ws + L.off_p);
  uint16_t* Bbuf = reinterpret_cast<uint16_t*>(ws + L.off_b);
  uint16_t* Xtmp = reinterpret_cast<uint16_t*>(ws + L.off_x);

  hipLaunchKernelGGL(ns_offsets_kernel, dim3((unsigned)cdiv(Ec, 256)), dim3(256), 0, s, offsets, (int)Ec, m);
  int rc = check_launch("newton_schulz5 offsets");
  if (rc) return rc;
  // the normalised X goes where the step count makes the last step land in X
  uint16_t* cur = (steps % 2 == 1) ? Xtmp : Xuser;
  uint16_t* nxt = (steps % 2 == 1) ? Xuser : Xtmp;
  const int64_t per_chunks = m * n / 8;
  const dim3 grid((unsigned)L.P, (unsigned)Ec);
  hipLaunchKernelGGL(ns_sumsq_kernel, grid, dim3(kNsThreads), 0, s, Xuser, per_chunks, L.slice_chunks, L.P,
                     partial);
  rc = check_launch("newton_schulz5 norm");
  if (rc) return rc;
  hipLaunchKernelGGL(ns_scale_kernel, grid, dim3(kNsThreads), 0, s, Xuser, cur, per_chunks, L.slice_chunks, L.P,
                     partial);
  rc = check_launch("newton_schulz5 scale");
  if (rc) return rc;

  const int64_t R = Ec * m;
  for (int it = 0; it < steps; ++it) {
    // A = X X^T, and cA as a second output
    NsGemm g1{};
    g1.A = cur; g1.lda = n;
    g1.B = cur; g1.b_estride = m * n; g1.ldb = n; g1.b_kn = false;
    g1.offsets = offsets; g1.R = R; g1.K = (int)n; g1.N = (int)m; g1.E = (int)Ec;
    g1.C = Abuf; g1.ldc = m;
    g1.C2 = Pbuf; g1.ldc2 = m; g1.gamma = c;
    g1.sym_m = (int)m;  // X X^T is symmetric: upper-triangle tiles plus their mirror
    rc = ns_gemm(g1, s);
    if (rc) return rc;
    // B = (cA) A + bA, A read as [K][N] (its columns), so the product does not rely on
    // the rounded A being exactly symmetric
    NsGemm g2{};
    g2.A = Pbuf; g2.lda = m;
    g2.B = Abuf; g2.b_estride = m * m; g2.ldb = m; g2.b_kn = true;
    g2.offsets = offsets; g2.R = R; g2.K = (int)m; g2.N = (int)m; g2.E = (int)Ec;
    g2.C = Bbuf; g2.ldc = m;
    g2.D = Abuf; g2.ldd = m; g2.beta = b;
    g2.sym_m = (int)m;  // (cA) A + bA is symmetric (polynomial in the symmetric A)
    rc = ns_gemm(g2, s);
    if (rc) return rc;
    // X' = B X + aX
    NsGemm g3{};
    g3.A = Bbuf; g3.lda = m;
    g3.B = cur; g3.b_estride = m * n; g3.ldb = n; g3.b_kn = true;
    g3.offsets = offsets; g3.R = R; g3.K = (int)m; g3.N = (int)n; g3.E = (int)Ec;
    g3.C = nxt; g3.ldc = n;
    g3.D = cur; g3.ldd = n; g3.beta = a;
    rc = ns_gemm(g3, s);
    if (rc) return rc;
    uint16_t* t = cur;
    cur = nxt;
    nxt = t;
  }
  return ZMOE_OK;
}

}  // namespace

extern "C" int zmoe_newton_schulz5(void* X, int64_t E, int64_t m, int64_t n, int steps, float a, float b, float c,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  ZMOE_REQUIRE(E >= 1 && m >= 8 && n >= 8 && m <= n && steps >= 0, ZMOE_ERR_SHAPE,
               "newton_schulz5: need E >= 1, 8 <= m <= n, steps >= 0 (E=%lld m=%lld n=%lld)", (long long)E,
               (long long)m, (long long)n);
  ZMOE_REQUIRE(m % 8 == 0 && n % 8 == 0, ZMOE_ERR_ALIGN, "newton_schulz5: m and n must be multiples of 8");
  ZMOE_REQUIRE(m < (1 << 20) && n < (1 << 20) && m * n * 2 <= kNsMaxSpan, ZMOE_ERR_SHAPE,
               "newton_schulz5: one matrix spans more than 2 GiB");
  ZMOE_REQUIRE(X && workspace, ZMOE_ERR_NULL, "newton_schulz5: null pointer");
  ZMOE_REQUIRE(aligned16(X) && (reinterpret_cast<uintptr_t>(workspace) & 255u) == 0, ZMOE_ERR_ALIGN,
               "newton_schulz5: X must be 16-byte and the workspace 256-byte aligned");
  const int64_t chunk = ns_chunk(E, m, n);
  const size_t need = ns_layout(chunk, m, n).total;
  ZMOE_REQUIRE(workspace_bytes >= need, ZMOE_ERR_WORKSPACE, "newton_schulz5: workspace %zu < %zu bytes",
               workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  uint16_t* Xs = static_cast<uint16_t*>(X);
  for (int64_t e0 = 0; e0 < E; e0 += chunk) {
    const int64_t Ec = E - e0 < chunk ? E - e0 : chunk;
    const int rc = ns_pass(Xs + e0 * m * n, Ec, m, n, steps, a, b, c, static_cast<char*>(workspace), s);
    if (rc) return rc;
  }
  return ZMOE_OK;
}
