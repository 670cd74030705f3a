// Grouped expert GEMMs for gfx950 (scattermoe/kernels/ops.py:122-255 and
// :263-438, plus the fused SwiGLU forward/backward of scattermoe/mlp.py:80-86),
// the split-K dense weight grads of the shared expert and gate, and the grouped
// GEMMs of the Newton-Schulz step (optimizer/muon.py:6-32).
//
// Two GEMM shapes, each in a bf16 kernel (the fast path) and an f32 kernel:
//   * rows: C[i, :] = A(i, :) @ B_e for the sorted rows i of expert e (forward and
//     input-grad GEMMs; rows_bf16_kernel / grouped_rows_kernel). Tiles never
//     straddle experts: the M tiles of each expert are laid out back to back, so
//     boundary rows cost at most one partial tile per expert instead of a K loop
//     per expert present in a block.
//   * wgrad: C_e[m, n] = sum_{i in e} DY[i, m] X(i)[n] (weight grads;
//     wgrad_bf16_kernel / grouped_wgrad_kernel), x rows optionally gathered.
//
// bf16 tile machinery (BM x BN = 256 x 256 on 8 waves in a 2x4 grid, two waves per
// SIMD and 128 x 64 outputs per wave; or 128 x 128 on 4 waves in a 2x2 grid):
//   * Operands go HBM -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging) in
//     64-deep stages, double-buffered (a rows tile of at most 64 rows: three stages of its
//     64 rows and the weight block, kloop_small), every wave loading its own share: 128-byte
//     rows with the reduction dimension contiguous (16-byte chunks XOR-swizzled by
//     row so that each 8- or 16-lane group of a fragment read hits distinct banks), or K-major tiles read with
//     ds_read_b64_tr_b16 for operands whose reduction dimension is strided. Each
//     stage has its own scalar buffer descriptor (the k advance and the tail
//     clipping), so issuing a load costs no vector ALU.
//   * v_mfma_f32_16x16x32_bf16 on 8 waves (kloop64_m16; the SwiGLU-backward epilogue,
//     4-wave tiles, the DY-gathered weight grads and the weight grads with the few-rows form
//     inline keep v_mfma_f32_32x32x16_bf16, kloop64), with the B tile as the first operand: each
//     lane ends up holding 4 consecutive output columns of one output row. Every MFMA
//     slot of the K loop is pinned with sched_barrier so loads, fragment reads and the
//     one barrier per stage interleave with the MFMAs.
//   * Epilogue: each wave stages its block in LDS (rounded to the output type, as
//     the reference stores its GEMM outputs) and writes full 128-byte lines to
//     grouped or scattered rows, optionally through SwiGLU, its backward, or the
//     Newton-Schulz terms.
//   * Workgroup -> tile: XCD-aware. Workgroup b runs on XCD b % 8; each XCD takes
//     a contiguous range of the (expert, m-tile, n-tile) sequence so that tiles
//     sharing an expert's weights and rows run on one XCD and share its L2, or,
//     for weight grads and for rows launches under skewed routing, slabs of 32
//     consecutive tiles dealt to the XCDs in turn so that uneven per-tile costs
//     even out (xcd_logical_tile, slab_logical_tile).
// The f32 kernels use the same tiling with VGPR-staged loads, 32-deep stages and
// v_mfma_f32_32x32x2f32 (four per 16-byte fragment).
#include <mutex>
#include <type_traits>
#include <unordered_set>

#include "zmoe_internal.h"

namespace zmoe {

constexpr int kGemmThreads = 256;
constexpr int kRowBytes = 128;
constexpr int kGemmMaxE = 1024;
constexpr int kXcds = 8;

// EPI_STORE_BIAS: EPI_STORE plus a per-expert bias row (a separate instantiation keeps
// the bias loads out of the common kernel's register budget). EPI_NS: the Newton-Schulz
// step outputs (bf16 only): t = bf16(acc); C = bf16(t + bf16(ns_beta * D)) when D
// (p.aux) is given, else t; C2 = bf16(ns_gamma * t) when C2 is given.
enum Epi { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_SWIGLU_BWD = 2, EPI_STORE_BIAS = 3, EPI_NS = 4 };

__device__ __forceinline__ uint32_t lds_off(int row, int chunk) {
  return (uint32_t)(row * kRowBytes + ((chunk ^ (((row >> 1) ^ (row >> 3)) & 7)) << 4));
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int w) {
  return w == 0 ? v.x : (w == 1 ? v.y : (w == 2 ? v.z : v.w));
}

// 8x8 bf16 transpose: in[r] holds columns 0..7 of row r; out[c] holds rows 0..7 of column c.
__device__ __forceinline__ void transpose_block(const uint4 (&in)[8], uint4 (&out)[8]) {
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    const int w = c >> 1;
    out[c].x = __builtin_amdgcn_perm(word_of(in[1], w), word_of(in[0], w), sel);
    out[c].y = __builtin_amdgcn_perm(word_of(in[3], w), word_of(in[2], w), sel);
    out[c].z = __builtin_amdgcn_perm(word_of(in[5], w), word_of(in[4], w), sel);
    out[c].w = __builtin_amdgcn_perm(word_of(in[7], w), word_of(in[6], w), sel);
  }
}
// 4x4 f32 transpose.
__device__ __forceinline__ void transpose_block(const uint4 (&in)[4], uint4 (&out)[4]) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    out[c].x = word_of(in[0], c);
    out[c].y = word_of(in[1], c);
    out[c].z = word_of(in[2], c);
    out[c].w = word_of(in[3], c);
  }
}

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void sts16(char* lds, uint32_t off, const uint4& v) {
  *reinterpret_cast<uint4*>(lds + off) = v;
}
__device__ __forceinline__ uint4 lds16(const char* lds, uint32_t off) {
  return *reinterpret_cast<const uint4*>(lds + off);
}

// ------------------------------------------------------------------ MFMA core
template <typename T> struct Mma;

template <> struct Mma<uint16_t> {
  static constexpr int VEC = 8;
  template <int MI, int NI>
  __device__ __forceinline__ static void step(const char* la, const char* lb, int wm0, int wn0,
                                              f32x16_t (&acc)[MI][NI]) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, g = lane >> 5;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8_t a[MI], b[NI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        a[mi] = __builtin_bit_cast(bf16x8_t, lds16(la, lds_off(wm0 + mi * 32 + r, 2 * s + g)));
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        b[ni] = __builtin_bit_cast(bf16x8_t, lds16(lb, lds_off(wn0 + ni * 32 + r, 2 * s + g)));
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[ni], a[mi], acc[mi][ni], 0, 0, 0);
    }
  }
};

template <> struct Mma<float> {
  static constexpr int VEC = 4;
  template <int MI, int NI>
  __device__ __forceinline__ static void step(const char* la, const char* lb, int wm0, int wn0,
                                              f32x16_t (&acc)[MI][NI]) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, g = lane >> 5;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f32x4_t a[MI], b[NI];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
        a[mi] = __builtin_bit_cast(f32x4_t, lds16(la, lds_off(wm0 + mi * 32 + r, 2 * s + g)));
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        b[ni] = __builtin_bit_cast(f32x4_t, lds16(lb, lds_off(wn0 + ni * 32 + r, 2 * s + g)));
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int ni = 0; ni < NI; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[ni][j], a[mi][j], acc[mi][ni], 0, 0, 0);
    }
  }
};

// ------------------------------------------------------------------ operand loaders
// Rows operand: ROWS rows x 8 chunks, reduction dim contiguous in HBM.
// Thread t owns chunk column t & 7 of rows (t >> 3) + 32 j.
template <typename T, int ROWS>
struct RowsOperand {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int NJ = ROWS / 32;
  const T* ptr[NJ];  // row base + chunk column offset, or null for rows past the tile
  uint4 reg[NJ];

  __device__ __forceinline__ void load(int k0, int K) {
    const int kc = k0 + (threadIdx.x & 7) * VEC;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (ptr[j] != nullptr && kc < K) reg[j] = ldg16(ptr[j] + k0);
      else reg[j] = make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
    const int c = threadIdx.x & 7;
#pragma unroll
    for (int j = 0; j < NJ; ++j) sts16(lds, lds_off((threadIdx.x >> 3) + 32 * j, c), reg[j]);
  }
};

// Transposed operand: a [8*VEC reduction rows] x [COLS] tile whose COLS are
// contiguous in HBM. Block (mb, kg) = VEC reduction rows x VEC columns.
template <typename T, int COLS>
struct TransOperand {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int MB = COLS / VEC;
  static constexpr int NBLK = MB * 8;
  static constexpr int NB = (NBLK + kGemmThreads - 1) / kGemmThreads;
  uint4 reg[NB][VEC];

  __device__ __forceinline__ static int blk(int q) { return (int)threadIdx.x + q * kGemmThreads; }

  // row_ptr(kr) -> pointer to column 0 of reduction row kr (kr relative to the tile), or null
  template <typename RowPtr>
  __device__ __forceinline__ void load(RowPtr row_ptr, int col0, int ncols) {
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int b = blk(q);
      const int mb = b % MB, kg = b / MB;
      const int col = col0 + mb * VEC;
      const bool colok = (NBLK % kGemmThreads == 0 || b < NBLK) && col < ncols;
#pragma unroll
      for (int rr = 0; rr < VEC; ++rr) {
        const T* p = colok ? row_ptr(kg * VEC + rr) : nullptr;
        reg[q][rr] = p != nullptr ? ldg16(p + col) : make_uint4(0, 0, 0, 0);
      }
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int b = blk(q);
      if (NBLK % kGemmThreads != 0 && b >= NBLK) continue;
      const int mb = b % MB, kg = b / MB;
      uint4 t[VEC];
      transpose_block(reg[q], t);
#pragma unroll
      for (int c = 0; c < VEC; ++c) sts16(lds, lds_off(mb * VEC + c, kg), t[c]);
    }
  }
};

// ------------------------------------------------------------------ block scan
template <int NT = kGemmThreads>
__device__ __forceinline__ int block_exclusive_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const int t = tmp[w];
    if (w < wave) base += t;
    tot += t;
  }
  *total = tot;
  return base + x - v;
}

// Logical tile of this workgroup under the XCD-aware mapping, or -1.
__device__ __forceinline__ int xcd_logical_tile(int total) {
  const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
  const int chunk = (total + kXcds - 1) / kXcds;
  const int logical = xcd * chunk + slot;
  return (slot < chunk && logical < total) ? logical : -1;
}

// Logical tile under slabs of kSlab consecutive tiles (the workgroups one XCD holds at
// once) dealt to the XCDs in turn. The weight-grad launches always map this way: a
// weight-grad tile's cost grows with its expert's rows, so xcd_logical_tile's contiguous
// per-XCD ranges (equal tile counts) leave the XCD that holds a popular expert with most
// of the work when routing is skewed: 2.4x the mean at C4's Zipf(1.1) popularity, dW1 +
// dW2 13.0 -> 10.1 ms with slabs. A slab still keeps 32 concurrent tiles of one expert on
// one XCD (same time as the contiguous ranges at C3; slabs of 8 time the same at C4, of 1
// are 3-11% slower at C3). A launch of at most 8 slabs (the dense split-K grads) takes one
// slab of ceil(total / 8) tiles per XCD, i.e. the contiguous ranges, so no XCD sits idle.
// The launches round their grids up to whole slabs on every XCD.
constexpr int kSlab = 32;
// Tile order within one expert, for position `loc` of its ninner x nouter tiles: the
// inner index (the tiles sharing the outer operand block) runs fastest, in serpentine order
// (backwards on odd outer steps, so the tiles either side of a turn share a block too:
// 0.3-0.8% per launch). An expert with at least 2 * kBand inner tiles takes its inner index
// in bands of kBand, the outer index reversed on odd bands, so that the ~32 tiles an XCD
// runs at once span about kBand x 4 tiles instead of one or two outer steps of 16-32:
// a one-expert 262144 x 2048 x 2048 GEMM with one n-tile per column of 32 read X once per
// XCD (8.86 GB from HBM for 1.08 GB of operands; banded 3.23 GB, 2.02 -> 1.84 ms), and
// C4's W1 forward (16 pair-column tiles) read each expert's weights once per two m-tiles
// (banded 4.46 -> 4.30 ms).
constexpr int kBand = 8;
__device__ __forceinline__ void expert_tile_order(int loc, int ninner_all, int nouter, int& inner, int& outer) {
  const int band = ninner_all >= 2 * kBand ? kBand : ninner_all;
  const int b = loc / (band * nouter), lb = loc - b * band * nouter;
  const int ninner = min(band, ninner_all - b * band);
  const int outer0 = lb / ninner, in0 = lb % ninner;
  outer = (b & 1) ? nouter - 1 - outer0 : outer0;
  inner = b * band + ((outer0 & 1) ? ninner - 1 - in0 : in0);
}
__host__ __device__ __forceinline__ int slab_size(int64_t total) {
  const int64_t per_xcd = (total + kXcds - 1) / kXcds;
  return per_xcd < kSlab ? (int)(per_xcd > 0 ? per_xcd : 1) : kSlab;
}
__device__ __forceinline__ int slab_logical_tile(int total, int b = -1) {
  if (b < 0) b = (int)blockIdx.x;
  const int slab = slab_size(total);
  const int xcd = b % kXcds, slot = b / kXcds;
  const int logical = ((slot / slab) * kXcds + xcd) * slab + slot % slab;
  return logical < total ? logical : -1;
}

// ------------------------------------------------------------------ params
struct RowsParams {
  const void* a;
  int64_t lda;
  const int64_t* a_rows;  // gather: A row of sorted row i = a_rows[i] / a_div (null: i)
  int a_div;
  const void* b;
  int64_t b_estride, ldb;
  void* c;
  int64_t ldc;
  const int64_t* c_rows;  // scatter: output row of sorted row i = c_rows[i] (null: i)
  void* c2;               // SwiGLU activation output
  int64_t ldc2;
  const void* aux;        // H for the SwiGLU backward; D for EPI_NS
  int64_t ld_aux;
  float ns_beta, ns_gamma; // EPI_NS scalars
  int ns_sym_m;            // EPI_NS: > 0 when every expert's output is a symmetric m x m matrix:
                           // only tiles on or above the diagonal run, and they also write their mirror
  const void* bias;       // [E, N] or null
  int64_t bias_estride;
  const int64_t* offsets; // inclusive expert ends [E]
  int K, N, E;
  int half;               // SwiGLU pair width f
  int n_tiles;
  int n_major;            // tile order within an expert: n-tiles outer (1) or m-tiles outer (0)
  uint32_t a_bytes;       // addressable bytes from p.a (buffer-resource range)
  uint32_t b_bytes;       // addressable bytes of one expert's weights
  // bf16, per sorted row i (null: none). EPI_SWIGLU: the activation output is
  // row_scale[i] * silu(gate) * h. EPI_SWIGLU_BWD, when A holds unscaled rows:
  // row_scale[i] scales row i of dA after the GEMM, and row_dots[i * dots_ld + c / 64]
  // receives sum_c dA_unscaled * silu(gate) * h over each 64-column block c of row i
  const float* row_scale;
  float* row_dots;
  int dots_ld;
};

struct WgradParams {
  const void* dy;
  int64_t lddy;
  const void* x;
  int64_t ldx;
  const int64_t* x_rows;  // gather: source row of sorted row i = x_rows[i] / x_div (of DY with the DY gather)
  int x_div;
  int x_div_shift;  // log2(x_div) when x_div is a power of two, else -1
  void* dw;  // [E, Ndy, Kx]
  const int64_t* offsets;
  int Ndy, Kx, E;
  int m_tiles, n_tiles;
  uint32_t dy_bytes, x_bytes;  // addressable bytes from p.dy / p.x
  int rows_lo = 0, rows_hi = 0x7fffffff;  // bf16 kernels: only experts with rows_lo <= rows <= rows_hi
  // >= 0: a dense split-K launch over this many rows, "expert" e being split e of E (the
  // ranges of split_end below; offsets unused); < 0: the row ranges come from offsets
  int64_t split_rows = -1;
  // > 0 (the launch with the few-rows form inline): workgroups 0 .. fillers - 1 write the
  // zeros of every empty expert's grad, each a contiguous share; the tiles of empty experts exit
  int fillers = 0;
  // tile order within an expert: n-tiles outer (1, the tiles sharing an X block run
  // together) or m-tiles outer (0, those sharing a DY block)
  int n_major = 0;
};

// Row ranges of the split-K partials as inclusive ends: S near-equal ranges of M rows,
// cut at multiples of 64 rows (whole K-loop stages).
__host__ __device__ __forceinline__ int64_t split_end(int64_t M, int S, int s) {
  const int64_t end = (s + 1 == S) ? M : ((M * (s + 1) / S + 63) / 64) * 64;
  return end < M ? end : M;
}

// Inclusive end of expert (or split) e's rows in a weight-grad launch.
__device__ __forceinline__ int64_t wgrad_rows_end(const WgradParams& p, int e) {
  return p.split_rows >= 0 ? split_end(p.split_rows, p.E, e) : p.offsets[e];
}

struct RowsTile {
  int e, nt, rows, mt;  // mt: m-tile index within the expert (symmetric launches)
  int64_t row0;
};

// Map this workgroup to (expert, m-tile, n-tile) of a rows launch; false if it has no tile.
template <int BM, int NT = kGemmThreads>
__device__ __forceinline__ bool decode_rows_tile(const RowsParams& p, char* smem, RowsTile& t) {
  if (p.ns_sym_m > 0) {
    // m x m outputs, one per expert: the upper-triangle tiles (nt >= mt) in row order
    const int nm = (p.ns_sym_m + BM - 1) / BM;
    const int tri = nm * (nm + 1) / 2;
    const int logical = xcd_logical_tile(p.E * tri);
    if (logical < 0) return false;
    t.e = logical / tri;
    int r = logical % tri, mt = 0;
    while (r >= nm - mt) {
      r -= nm - mt;
      ++mt;
    }
    t.mt = mt;
    t.nt = mt + r;
    t.row0 = (int64_t)t.e * p.ns_sym_m + (int64_t)mt * BM;
    t.rows = min(BM, p.ns_sym_m - mt * BM);
    return true;
  }
  // One pass over the expert ends: each thread counts the m-tiles of its experts, a
  // block scan places them, and the thread whose expert holds this workgroup's m-tile
  // posts (expert, first row, rows) to LDS. The offsets are read once, so the decode
  // costs one global round trip.
  int64_t* found = reinterpret_cast<int64_t*>(smem);  // [0] expert, [1] first row, [2] rows, [3] n-tile
  int* tmp = reinterpret_cast<int*>(smem + 32);
  const int ept = (p.E + NT - 1) / NT;  // <= 4
  const int e0 = threadIdx.x * ept;
  int64_t ebeg[4] = {0, 0, 0, 0}, eend[4] = {0, 0, 0, 0};
  int ntl[4] = {0, 0, 0, 0};
  int local = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = e0 + q;
    if (q < ept && e < p.E) {
      ebeg[q] = e ? p.offsets[e - 1] : 0;
      eend[q] = p.offsets[e];
      const int64_t c = eend[q] > ebeg[q] ? eend[q] - ebeg[q] : 0;
      ntl[q] = (int)((c + BM - 1) / BM);
      local += ntl[q];
    }
  }
  // experts whose rows fit one m-tile, per wave (ballots: no LDS round trips)
  int single = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) single += __builtin_popcountll(__builtin_amdgcn_ballot_w64(ntl[q] == 1));
  int* single_w = tmp + 16;  // per-wave counts; the scan's barrier orders them before the reads
  if ((threadIdx.x & 63) == 0) single_w[threadIdx.x >> 6] = single;
  // expert e owns ntl_e * n_tiles consecutive logical tiles, its m-tiles outer (tiles
  // sharing A rows run together) or its n-tiles outer (tiles sharing B columns do)
  int ttiles;
  int run = block_exclusive_scan<NT>(local * p.n_tiles, tmp, &ttiles);
  int singles = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) singles += single_w[w];
  // Skewed routing, with over a quarter of the experts in a single m-tile: their tiles
  // stream a whole weight block for a few rows (HBM-bound) beside the compute-bound tiles
  // of the popular experts, and slabs give every XCD its share of both (C4: W1 forward 6%,
  // W1 input grad 4% faster). Otherwise each XCD keeps whole experts (1% faster at C3).
  const int logical = 4 * singles > p.E ? slab_logical_tile(ttiles) : xcd_logical_tile(ttiles);
  if (logical < 0) return false;  // uniform per workgroup
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int tiles_e = ntl[q] * p.n_tiles;
    if (logical >= run && logical < run + tiles_e) {  // (ntl[q] is 0 past the last expert)
      int in2, outer;
      expert_tile_order(logical - run, p.n_major ? ntl[q] : p.n_tiles, p.n_major ? p.n_tiles : ntl[q], in2, outer);
      const int mt = p.n_major ? in2 : outer;
      const int64_t r0 = ebeg[q] + (int64_t)mt * BM;
      found[0] = e0 + q;
      found[1] = r0;
      found[2] = min((int64_t)BM, eend[q] - r0);
      found[3] = p.n_major ? outer : in2;
    }
    run += tiles_e;
  }
  __syncthreads();
  t.e = (int)found[0];
  t.row0 = found[1];
  t.rows = (int)found[2];
  t.nt = (int)found[3];
  t.mt = 0;
  __syncthreads();  // the decode area is dead; LDS becomes operand stages
  return true;
}

// ------------------------------------------------------------------ epilogue helpers
template <typename T, int WM, int WN>
struct Stage {
  static constexpr int PITCH = WN * (int)sizeof(T) + 16;  // bytes per staged row
  static constexpr int BYTES = WM * PITCH;                // per wave
};

// Write this wave's accumulators (plus optional bias) into its staging area.
template <typename T, int MI, int NI>
__device__ __forceinline__ void stage_acc(char* st, int pitch, const f32x16_t (&acc)[MI][NI], const T* bias_row,
                                          int col0, int N) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 31, g = lane >> 5;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = mi * 32 + r;
        const int col = ni * 32 + 8 * q + 4 * g;
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          v[u] = acc[mi][ni][4 * q + u];
          if (bias_row != nullptr && col0 + col + u < N) v[u] += to_f32(bias_row[col0 + col + u]);
        }
        char* p = st + row * pitch + col * (int)sizeof(T);
        if constexpr (sizeof(T) == 2) {
          uint2 w;
          w.x = pack_bf16x2(v[0], v[1]);
          w.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<uint2*>(p) = w;
        } else {
          *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        }
        // One 32x32 block at a time: hoisting every accumulator read into VGPRs at
        // once exhausts the register file and spills (scratch traffic counts on
        // vmcnt, which would also drain in-flight operand loads).
        if (q == 3) __builtin_amdgcn_sched_barrier(0);
      }
}

// Stage the accumulators through LDS and write the rows kernel's outputs.
template <typename T, int BM, int BN, int EPI, int MI, int NI>
__device__ __forceinline__ void rows_epilogue(const RowsParams& p, char* smem, const f32x16_t (&acc)[MI][NI],
                                              int e, int64_t row0, int rows, int nt) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int WM = BM / 2, WN = BN / 2;
  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  const int ncol0 = nt * BN;
  using S = Stage<T, WM, WN>;
  char* st = smem + wave * S::BYTES;
  const T* bias_row =
      (EPI == EPI_STORE_BIAS && p.bias) ? reinterpret_cast<const T*>(p.bias) + e * p.bias_estride : nullptr;
  stage_acc<T, MI, NI>(st, S::PITCH, acc, bias_row, ncol0 + wn0, p.N);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  T* C = reinterpret_cast<T*>(p.c);
  if constexpr (EPI == EPI_STORE || EPI == EPI_STORE_BIAS) {
    constexpr int CPR = WN / VEC;  // chunks per staged row
    for (int idx = lane; idx < WM * CPR; idx += 64) {
      const int rr = idx / CPR, cc = idx % CPR;
      const int r = wm0 + rr;
      const int col = ncol0 + wn0 + cc * VEC;
      if (r < rows && col < p.N) {
        const int64_t i = row0 + r;
        const int64_t orow = p.c_rows ? p.c_rows[i] : i;
        *reinterpret_cast<uint4*>(C + orow * p.ldc + col) =
            *reinterpret_cast<const uint4*>(st + rr * S::PITCH + cc * 16);
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    // staged cols: per 64-col pair block pb: [h 32 | g 32] for pair columns jj0 + pb*32 + 0..31
    constexpr int PB = WN / 64;
    constexpr int CPP = 32 / VEC;  // chunks per 32 columns
    T* A2 = reinterpret_cast<T*>(p.c2);
    for (int idx = lane; idx < WM * PB * CPP; idx += 64) {
      const int rr = idx / (PB * CPP);
      const int rem = idx % (PB * CPP);
      const int pb = rem / CPP, cc = rem % CPP;
      const int r = wm0 + rr;
      const int jj = nt * (BN / 2) + (wn0 / 64 + pb) * 32 + cc * VEC;
      if (r < rows && jj < p.half) {
        const int64_t i = row0 + r;
        const int64_t orow = p.c_rows ? p.c_rows[i] : i;
        const uint4 hv = *reinterpret_cast<const uint4*>(st + rr * S::PITCH + (pb * 64 + cc * VEC) * (int)sizeof(T));
        const uint4 gv = *reinterpret_cast<const uint4*>(st + rr * S::PITCH + (pb * 64 + 32 + cc * VEC) * (int)sizeof(T));
        float h[VEC], g[VEC], a[VEC];
        unpack_chunk(hv, h, T{});
        unpack_chunk(gv, g, T{});
#pragma unroll
        for (int q = 0; q < VEC; ++q) a[q] = silu_f(g[q]) * h[q];
        *reinterpret_cast<uint4*>(C + orow * p.ldc + jj) = hv;
        *reinterpret_cast<uint4*>(C + orow * p.ldc + p.half + jj) = gv;
        *reinterpret_cast<uint4*>(A2 + orow * p.ldc2 + jj) = pack_chunk(a, T{});
      }
    }
  } else {  // EPI_SWIGLU_BWD: staged dA for columns ncol0 + wn0 + ...
    constexpr int CPR = WN / VEC;
    const T* Hs = reinterpret_cast<const T*>(p.aux);
    for (int idx = lane; idx < WM * CPR; idx += 64) {
      const int rr = idx / CPR, cc = idx % CPR;
      const int r = wm0 + rr;
      const int col = ncol0 + wn0 + cc * VEC;
      if (r < rows && col < p.N) {
        const int64_t i = row0 + r;
        const int64_t orow = p.c_rows ? p.c_rows[i] : i;
        float da[VEC], h[VEC], g[VEC], dh[VEC], dg[VEC];
        unpack_chunk(*reinterpret_cast<const uint4*>(st + rr * S::PITCH + cc * 16), da, T{});
        unpack_chunk(ldg16(Hs + i * p.ld_aux + col), h, T{});
        unpack_chunk(ldg16(Hs + i * p.ld_aux + p.half + col), g, T{});
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const float s = sigmoid_fast(g[q]);
          dh[q] = da[q] * g[q] * s;
          dg[q] = da[q] * h[q] * s * (1.f + g[q] * (1.f - s));
        }
        *reinterpret_cast<uint4*>(C + orow * p.ldc + col) = pack_chunk(dh, T{});
        *reinterpret_cast<uint4*>(C + orow * p.ldc + p.half + col) = pack_chunk(dg, T{});
      }
    }
  }
}

// ------------------------------------------------------------------ rows kernel
template <typename T, int BM, int BN, bool B_KN, int EPI>
__global__ __launch_bounds__(kGemmThreads) void grouped_rows_kernel(RowsParams p) {
  extern __shared__ __align__(16) char smem[];
  constexpr int VEC = 16 / sizeof(T);
  constexpr int BK = 8 * VEC;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MI = WM / 32, NI = WN / 32;
  static_assert(EPI != EPI_SWIGLU || WN % 64 == 0, "SwiGLU pairs 32-column blocks inside a wave");

  RowsTile tile;
  if (!decode_rows_tile<BM>(p, smem, tile)) return;  // uniform per workgroup
  const int e = tile.e, nt = tile.nt, rows = tile.rows;
  const int64_t row0 = tile.row0;

  constexpr int kStage = (BM + BN) * kRowBytes;
  auto stage_a = [&](int st) { return smem + st * kStage; };
  auto stage_b = [&](int st) { return smem + st * kStage + BM * kRowBytes; };

  const T* A = reinterpret_cast<const T*>(p.a);
  const T* Bw = reinterpret_cast<const T*>(p.b) + (int64_t)e * p.b_estride;

  // ---- A operand (gathered rows)
  RowsOperand<T, BM> opa;
#pragma unroll
  for (int j = 0; j < BM / 32; ++j) {
    const int r = (threadIdx.x >> 3) + 32 * j;
    if (r < rows) {
      const int64_t i = row0 + r;
      const int64_t src = p.a_rows ? p.a_rows[i] / p.a_div : i;
      opa.ptr[j] = A + src * p.lda + (threadIdx.x & 7) * VEC;
    } else {
      opa.ptr[j] = nullptr;
    }
  }

  // ---- B operand (expert weights)
  RowsOperand<T, B_KN ? 32 : BN> opb_rows;
  TransOperand<T, B_KN ? BN : 32> opb_t;
  if constexpr (!B_KN) {
#pragma unroll
    for (int j = 0; j < BN / 32; ++j) {
      const int r = (threadIdx.x >> 3) + 32 * j;
      int n;
      bool ok;
      if constexpr (EPI == EPI_SWIGLU) {
        // B row r -> W1 row: 64-row pair blocks [up 32 | gate 32] of the tile's pair columns
        const int jj = nt * (BN / 2) + (r >> 6) * 32 + (r & 31);
        ok = jj < p.half;
        n = (r & 32) ? p.half + jj : jj;
      } else {
        n = nt * BN + r;
        ok = n < p.N;
      }
      opb_rows.ptr[j] = ok ? Bw + (int64_t)n * p.ldb + (threadIdx.x & 7) * VEC : nullptr;
    }
  }
  const int ncol0 = nt * BN;
  auto b_row_ptr = [&](int k0) {
    return [=](int kr) -> const T* {
      const int kk = k0 + kr;
      return kk < p.K ? Bw + (int64_t)kk * p.ldb : nullptr;
    };
  };

  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  f32x16_t acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[mi][ni][q] = 0.f;

  const int nk = (p.K + BK - 1) / BK;
  // prologue
  opa.load(0, p.K);
  if constexpr (B_KN) opb_t.load(b_row_ptr(0), ncol0, p.N);
  else opb_rows.load(0, p.K);
  opa.store(stage_a(0));
  if constexpr (B_KN) opb_t.store(stage_b(0));
  else opb_rows.store(stage_b(0));
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      const int k1 = (kt + 1) * BK;
      opa.load(k1, p.K);
      if constexpr (B_KN) opb_t.load(b_row_ptr(k1), ncol0, p.N);
      else opb_rows.load(k1, p.K);
    }
    Mma<T>::template step<MI, NI>(stage_a(cur), stage_b(cur), wm0, wn0, acc);
    if (more) {
      opa.store(stage_a(cur ^ 1));
      if constexpr (B_KN) opb_t.store(stage_b(cur ^ 1));
      else opb_rows.store(stage_b(cur ^ 1));
    }
    __syncthreads();
  }

  rows_epilogue<T, BM, BN, EPI>(p, smem, acc, e, row0, rows, nt);
}

template <typename T, int BM, int BN, int MI, int NI>
__device__ __forceinline__ void wgrad_epilogue(const WgradParams& p, char* smem, const f32x16_t (&acc)[MI][NI], int e,
                                               int m0, int n0) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int WM = BM / 2, WN = BN / 2;
  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  using S = Stage<T, WM, WN>;
  char* st = smem + wave * S::BYTES;
  stage_acc<T, MI, NI>(st, S::PITCH, acc, nullptr, 0, 0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  T* DW = reinterpret_cast<T*>(p.dw) + (int64_t)e * p.Ndy * p.Kx;
  constexpr int CPR = WN / VEC;
  for (int idx = lane; idx < WM * CPR; idx += 64) {
    const int rr = idx / CPR, cc = idx % CPR;
    const int m = m0 + wm0 + rr;
    const int n = n0 + wn0 + cc * VEC;
    if (m < p.Ndy && n < p.Kx)
      *reinterpret_cast<uint4*>(DW + (int64_t)m * p.Kx + n) =
          *reinterpret_cast<const uint4*>(st + rr * S::PITCH + cc * 16);
  }
}

// ------------------------------------------------------------------ wgrad kernel
template <typename T, int BM, int BN>
__global__ __launch_bounds__(kGemmThreads) void grouped_wgrad_kernel(WgradParams p) {
  extern __shared__ __align__(16) char smem[];
  constexpr int VEC = 16 / sizeof(T);
  constexpr int BK = 8 * VEC;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int MI = WM / 32, NI = WN / 32;

  const int per_e = p.m_tiles * p.n_tiles;
  const int logical = slab_logical_tile(p.E * per_e);
  if (logical < 0) return;
  const int e = logical / per_e;
  const int rem = logical % per_e;
  const int mt = rem / p.n_tiles, nt = rem % p.n_tiles;
  const int64_t r_begin = e ? p.offsets[e - 1] : 0;
  const int64_t r_end = p.offsets[e];
  const int64_t nrows = r_end > r_begin ? r_end - r_begin : 0;
  const int m0 = mt * BM, n0 = nt * BN;

  constexpr int kStage = (BM + BN) * kRowBytes;
  auto stage_a = [&](int st) { return smem + st * kStage; };
  auto stage_b = [&](int st) { return smem + st * kStage + BM * kRowBytes; };

  const T* DY = reinterpret_cast<const T*>(p.dy);
  const T* X = reinterpret_cast<const T*>(p.x);
  TransOperand<T, BM> opa;
  TransOperand<T, BN> opb;
  auto dy_rows = [&](int64_t k0) {
    return [=](int kr) -> const T* {
      const int64_t rr = k0 + kr;
      return rr < nrows ? DY + (r_begin + rr) * p.lddy : nullptr;
    };
  };
  auto x_rows = [&](int64_t k0) {
    return [=](int kr) -> const T* {
      const int64_t rr = k0 + kr;
      if (rr >= nrows) return nullptr;
      const int64_t i = r_begin + rr;
      const int64_t src = p.x_rows ? p.x_rows[i] / p.x_div : i;
      return X + src * p.ldx;
    };
  };

  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
  f32x16_t acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[mi][ni][q] = 0.f;

  const int nk = (int)((nrows + BK - 1) / BK);
  if (nk > 0) {
    opa.load(dy_rows(0), m0, p.Ndy);
    opb.load(x_rows(0), n0, p.Kx);
    opa.store(stage_a(0));
    opb.store(stage_b(0));
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < nk;
      if (more) {
        const int64_t k1 = (int64_t)(kt + 1) * BK;
        opa.load(dy_rows(k1), m0, p.Ndy);
        opb.load(x_rows(k1), n0, p.Kx);
      }
      Mma<T>::template step<MI, NI>(stage_a(cur), stage_b(cur), wm0, wn0, acc);
      if (more) {
        opa.store(stage_a(cur ^ 1));
        opb.store(stage_b(cur ^ 1));
      }
      __syncthreads();
    }
  }

  wgrad_epilogue<T, BM, BN>(p, smem, acc, e, m0, n0);
}

// Db[e, n] = sum over the expert's rows of DY[i, n] (bias grad, off the GLU path).
template <typename T>
__global__ void bias_grad_kernel(const T* __restrict__ DY, int64_t lddy, const int64_t* __restrict__ off, int N,
                                 int E, T* __restrict__ Db) {
  const int e = blockIdx.y;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N || e >= E) return;
  const int64_t a = e ? off[e - 1] : 0, b = off[e];
  float s = 0.f;
  for (int64_t i = a; i < b; ++i) s += to_f32(DY[i * lddy + n]);
  Db[(int64_t)e * N + n] = from_f32<T>(s);
}


// ==================================================================== bf16 path
// HBM -> LDS with buffer loads that write LDS directly (no staging registers,
// no ds_write; rows past an operand's range read as zero through the buffer
// resource's num_records), reduction-strided operands kept K-major in LDS and
// read with ds_read_b64_tr_b16. The K loop runs over NS LDS stages of KS
// reduction elements each, with NS - 1 stages of HBM loads in flight: the loop is
// bound by load latency unless several tiles are outstanding per CU.
typedef __attribute__((address_space(3))) char lds_char;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef short v8i16_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16;
typedef __attribute__((address_space(3))) uint4 lds_uint4;

constexpr uint32_t kOOB = 0x80000000u;  // any offset >= num_records reads zero



__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void buf_to_lds(__amdgpu_buffer_rsrc_t r, lds_char* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}


// s_waitcnt immediate that waits until at most n vector-memory ops are outstanding.
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Rows-major ("non-transposed") tile: [ROWS][KS bf16], KS*2 bytes per row, 16-byte
// chunks XOR-swizzled by row so MFMA fragment reads are bank-conflict free.
template <int KS>
__device__ __forceinline__ uint32_t nt_off(int row, int chunk) {
  if constexpr (KS == 64) return (uint32_t)(row * 128 + ((chunk ^ ((row & 7) ^ ((row >> 3) & 1))) << 4));
  else return (uint32_t)(row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4));
}
template <int KS>
__device__ __forceinline__ int nt_swz(int row) {
  if constexpr (KS == 64) return (row & 7) ^ ((row >> 3) & 1);
  else return (row >> 2) & 3;
}

// K-major ("transposed") tile: [KS k-rows][COLS], 16-byte chunks XOR (row & 3) * 4 ^
// ((row >> 3) & 1) * 2: the four k-rows one transpose-read touches land in four different
// 64-byte bank groups, and so do the 16-lane groups of a 16 x 16 x 32 fragment read, which
// address k-rows 8 apart (without the second term those hit the same banks).
__device__ __forceinline__ uint32_t t_off(int krow, int col, int row_bytes) {
  return (uint32_t)(krow * row_bytes + ((((col >> 3) ^ ((krow & 3) << 2) ^ (((krow >> 3) & 1) << 1))) << 4) +
                    ((col & 7) << 1));
}

// Fragment reads are inline asm: LLVM's waitcnt pass makes any LDS read it cannot
// disambiguate (the ds_read_tr intrinsic carries no alias info) wait for every
// in-flight LDS-DMA load, which would serialise the stage pipeline. Being asm,
// these reads are invisible to that pass, so the K loops issue their own
// lgkmcnt waits and ties the fragment registers to them with empty asm (data
// dependencies keep every MFMA after the wait that covers its operands).
typedef int v4i32_t __attribute__((ext_vector_type(4)));
typedef int v2i32_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t lds_addr(const lds_char* p) { return (uint32_t)(uintptr_t)p; }

__device__ __forceinline__ v4i32_t asm_ds_read_b128(uint32_t addr) {
  v4i32_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ v2i32_t asm_ds_read_tr16(uint32_t addr) {
  v2i32_t v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
template <int N>
__device__ __forceinline__ void asm_wait_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N < 15 ? N : 15));
}
__device__ __forceinline__ void asm_tie(v4i32_t& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void asm_tie(v2i32_t& v) { asm volatile("" : "+v"(v)); }

// One MFMA operand fragment: lane (r = lane % 32, g = lane / 32) gets k = 16 s + 8 g + 0..7
// of row mn0 + r, as one 16-byte register (non-transposed) or two 8-byte halves.
template <bool TR>
struct Frag {
  v4i32_t w;
  v2i32_t lo, hi;
  static constexpr int kReads = TR ? 2 : 1;
  template <int BMN, int KS>
  __device__ __forceinline__ void read(const lds_char* base, int mn0, int s) {
    const int lane = threadIdx.x & 63;
    if constexpr (!TR) {
      w = asm_ds_read_b128(lds_addr(base) + nt_off<KS>(mn0 + (lane & 31), 2 * s + (lane >> 5)));
    } else {
      // ds_read_b64_tr_b16: in each 16-lane group, lane 4a+b receives element b of the
      // 8-byte rows addressed by lanes a, a+4, a+8, a+12. Lane s16 of group G addresses
      // k-row (16 s + 8 g + 4 q + s16 / 4), columns mn0 + 16 (G & 1) + 4 (s16 % 4) .. +3.
      const int G = lane >> 4, g = lane >> 5, s16 = lane & 15;
      const int krow = 16 * s + 8 * g + (s16 >> 2);
      const int col = mn0 + 16 * (G & 1) + 4 * (s16 & 3);
      lo = asm_ds_read_tr16(lds_addr(base) + t_off(krow, col, BMN * 2));
      hi = asm_ds_read_tr16(lds_addr(base) + t_off(krow + 4, col, BMN * 2));
    }
  }
  // piece h (0 .. kReads-1) of read(): lets callers spread reads between MFMAs
  template <int BMN, int KS>
  __device__ __forceinline__ void read_piece(const lds_char* base, int mn0, int s, int h) {
    const int lane = threadIdx.x & 63;
    if constexpr (!TR) {
      w = asm_ds_read_b128(lds_addr(base) + nt_off<KS>(mn0 + (lane & 31), 2 * s + (lane >> 5)));
    } else {
      const int G = lane >> 4, g = lane >> 5, s16 = lane & 15;
      const int krow = 16 * s + 8 * g + (s16 >> 2) + 4 * h;
      const int col = mn0 + 16 * (G & 1) + 4 * (s16 & 3);
      const v2i32_t v = asm_ds_read_tr16(lds_addr(base) + t_off(krow, col, BMN * 2));
      if (h == 0) lo = v;
      else hi = v;
    }
  }
  __device__ __forceinline__ void tie() {
    if constexpr (!TR) {
      asm_tie(w);
    } else {
      asm_tie(lo);
      asm_tie(hi);
    }
  }
  __device__ __forceinline__ bf16x8_t value() const {
    if constexpr (!TR) return __builtin_bit_cast(bf16x8_t, w);
    else return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3));
  }
};

// Rows-major tile loader: [ROWS][64 bf16] per stage, the reduction dim contiguous in
// HBM. Each wave instruction fills 1 KB of LDS = 8 rows x one 128-byte line; lane i
// takes physical chunk i % 8 of its row, i.e. logical chunk (i % 8) ^ swizzle(row).
// Offsets are relative to the stage's buffer resource (based at k0), so issuing a
// load costs no vector ALU work: the per-stage advance lives in the scalar resource.
// Each of the NS waves loads its own 8 NQ rows.
template <int ROWS, int NS = 4>
struct RowLoad {
  static constexpr int NQ = ROWS / (8 * NS);  // instructions per wave per stage
  static_assert(NQ >= 1, "at least one load per wave");
  uint32_t off[NQ];                           // byte offset of this lane's chunk at k0 = 0, or kOOB
  uint32_t tail[NQ];                          // the same for the final partial stage (chunks past K: kOOB)

  __device__ __forceinline__ static int row_of(int q) {
    return 8 * ((int)(threadIdx.x >> 6) * NQ + q) + (int)((threadIdx.x & 63) >> 3);
  }
  __device__ __forceinline__ static int chunk_of(int q) { return (int)(threadIdx.x & 7) ^ nt_swz<64>(row_of(q)); }
  // row_off: byte offset of the row at k = 0, or kOOB; ktail = K % 64 (0: no partial stage)
  __device__ __forceinline__ void set(int q, uint32_t row_off, int ktail) {
    const int c = chunk_of(q);
    off[q] = row_off == kOOB ? kOOB : row_off + 16u * (uint32_t)c;
    tail[q] = (ktail == 0 || 8 * c < ktail) ? off[q] : kOOB;
  }
  // (a select between the two array elements would be turned back into a dynamically
  // indexed array in scratch memory; the masked XOR keeps both indices constant)
  __device__ __forceinline__ void issue(int q, __amdgpu_buffer_rsrc_t rs, lds_char* stage, int wu, bool last) const {
    const uint32_t m = 0u - (uint32_t)last;
    buf_to_lds(rs, stage + (wu * NQ + q) * 1024, off[q] ^ ((off[q] ^ tail[q]) & m));
  }
};

// K-major tile loader: [64 k-rows][COLS] per stage, COLS contiguous in HBM. Each
// wave instruction fills 1 KB = RPI k-rows; wave w of NS covers k-rows KR w .. KR w + KR - 1.
template <int COLS, int NS = 4>
struct KLoad {
  static constexpr int CPR = COLS / 8;   // chunks per k-row
  static constexpr int NQ = CPR / NS;    // instructions per wave per stage
  static constexpr int RPI = 64 / CPR;   // k-rows per instruction
  static constexpr int KR = 64 / NS;     // k-rows per wave per stage
  static_assert(NQ >= 1 && NQ * RPI == KR, "the waves' k-rows tile the stage");
  uint32_t coff[NQ];  // column byte offset of this lane's chunk, or kOOB past the operand's width
  uint32_t voff[NQ];  // coff + (k-row within the stage) * row pitch, or kOOB

  __device__ __forceinline__ static int krow_of(int q) {
    return (((int)(threadIdx.x >> 6) * NQ + q) * 64 + (int)(threadIdx.x & 63)) / CPR;
  }
  // k-row of this lane within its wave's KR for instruction q: q * RPI + sub()
  __device__ __forceinline__ static int sub() { return (int)(threadIdx.x & 63) / CPR; }
  __device__ __forceinline__ void init(int mn0, int ncols, int64_t pitch_bytes) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int f = ((int)(threadIdx.x >> 6) * NQ + q) * 64 + (int)(threadIdx.x & 63);
      const int kr = f / CPR;
      const int c = (f % CPR) ^ ((kr & 3) << 2) ^ (((kr >> 3) & 1) << 1);
      const int col = mn0 + 8 * c;
      coff[q] = col < ncols ? (uint32_t)col * 2u : kOOB;
      voff[q] = col < ncols ? (uint32_t)((int64_t)kr * pitch_bytes) + coff[q] : kOOB;
    }
  }
  __device__ __forceinline__ void issue(int q, __amdgpu_buffer_rsrc_t rs, lds_char* stage, int wu) const {
    buf_to_lds(rs, stage + (wu * NQ + q) * 1024, voff[q]);
  }
  __device__ __forceinline__ void issue_at(int q, __amdgpu_buffer_rsrc_t rs, lds_char* stage, int wu,
                                           uint32_t v) const {
    buf_to_lds(rs, stage + (wu * NQ + q) * 1024, v);
  }
};

// Buffer resource for the rows [row0 + k0, rows_end) of a row-major operand whose
// rows are `pitch` bytes apart: loads at or past rows_end read zero, and so does
// every load when `on` is false (stages past the end of the loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t stage_rsrc(const char* base, uint32_t span, int64_t first_byte,
                                                           int64_t valid_bytes, bool on) {
  const int64_t room = (int64_t)span - first_byte;
  const int64_t n = valid_bytes < room ? valid_bytes : room;
  return make_rsrc(base + first_byte, (on && n > 0) ? (uint32_t)n : 0u);
}

// The software-pipelined K loop of both bf16 kernels: two LDS stages of 64 reduction
// elements (four 16-deep MFMA steps each). Per stage kt (buffer kt & 1):
//   steps 0..2: each MFMA slot issues the fragment reads of the next step;
//   barrier (after step 2): this wave's loads of stage kt + 1 have landed and every
//     wave has read all of stage kt, so stage kt + 1 is readable and buffer kt & 1
//     is free;
//   step 3: reads step 0 of stage kt + 1, and starts stage kt + 2's loads into
//     buffer kt & 1; the rest of those loads go out during step 0 of stage kt + 1.
// Stage kt + 2's loads thus have steps 1 and 2 of stage kt + 1 to land. Slots are
// pinned with sched_barrier(0); one wave per SIMD keeps the matrix unit fed while
// loads, LDS reads and the barrier are in flight.
// dma(q, buf, kt, on) issues load instruction q (0..LPS-1) of stage kt into buffer
// buf (reading zeros when !on); prefetch(kt) readies the gather indices of stage kt;
// after_prologue_loads() runs once the first loads are in flight.
template <int LPS, int MI, int NI, bool A_T, bool B_T, int BM, int BN, typename Dma, typename Prefetch, typename Hook>
__device__ __forceinline__ void kloop64(int nk, lds_char* lds, int wm0, int wn0, f32x16_t (&acc)[MI][NI], Dma dma,
                                        Prefetch prefetch, Hook after_prologue_loads) {
  constexpr int KS = 64;
  constexpr int kStage = (BM + BN) * KS * 2;
  constexpr int AR = Frag<A_T>::kReads, BR = Frag<B_T>::kReads;
  constexpr int NREAD = MI * AR + NI * BR;        // fragment reads per step
  constexpr int NMMA = MI * NI;                   // MFMAs per step
  constexpr int RPS = (NREAD + NMMA - 1) / NMMA;  // reads per MFMA slot
  constexpr int WIN = 2 * NMMA;                   // load window: step 3 + step 0
  // load j goes to window slot j * WIN / LPS (evenly spread); loads in slots < NMMA
  // belong to step 3 of the previous stage
  constexpr int kEarly = (NMMA * LPS + WIN - 1) / WIN;  // loads j with j * WIN / LPS < NMMA
  Frag<A_T> fa[2][MI];
  Frag<B_T> fb[2][NI];
  auto read_piece = [&](int buf, const lds_char* st, int s, int i) {
    if (i < MI * AR) {
      fa[buf][i / AR].template read_piece<BM, KS>(st, wm0 + (i / AR) * 32, s, i % AR);
    } else {
      const int j = i - MI * AR;
      fb[buf][j / BR].template read_piece<BN, KS>(st + BM * KS * 2, wn0 + (j / BR) * 32, s, j % BR);
    }
  };
  auto tie = [&](int buf) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) fa[buf][mi].tie();
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) fb[buf][ni].tie();
  };
  auto mma = [&](int buf, int i) {
    acc[i / NI][i % NI] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[buf][i % NI].value(), fa[buf][i / NI].value(),
                                                                  acc[i / NI][i % NI], 0, 0, 0);
  };
  // one compute step: MFMAs on fragment buffer `cur`, reads of (rst, rs) into the other
  // buffer, and the loads of window slots [w0, w0 + NMMA) of stage lkt into buffer lbuf
  auto step = [&](int cur, const lds_char* rst, int rs, int w0, int lbuf, int lkt, bool lon) {
    __builtin_amdgcn_sched_barrier(0);
    // a wave in a step that issues operand loads wins issue arbitration over its SIMD
    // partner in an MFMA-only step (0.5-0.8% per launch; the reverse, or raising the
    // priority only around each load, measured no gain or slower)
    if (w0 >= 0) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NMMA; ++i) {
      mma(cur, i);
#pragma unroll
      for (int j = 0; j < LPS; ++j)
        if (w0 >= 0 && j * WIN / LPS == w0 + i) dma(j, lbuf, lkt, lon);
#pragma unroll
      for (int r = 0; r < RPS; ++r)
        if (i * RPS + r < NREAD) read_piece(cur ^ 1, rst, rs, i * RPS + r);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm_wait_lgkm<0>();
    tie(cur ^ 1);
  };
  if (nk <= 0) {
    after_prologue_loads();
    return;
  }
  prefetch(0);
#pragma unroll
  for (int j = 0; j < LPS; ++j) dma(j, 0, 0, true);
  prefetch(1);
#pragma unroll
  for (int j = 0; j < kEarly; ++j) dma(j, 1, 1, nk > 1);
  after_prologue_loads();
  __builtin_amdgcn_s_waitcnt(vm_wait(kEarly));  // stage 0 landed (stage 1's early loads may not have)
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int i = 0; i < NREAD; ++i) read_piece(0, lds, 0, i);
  asm_wait_lgkm<0>();
  tie(0);

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const lds_char* st = lds + buf * kStage;
    const lds_char* nst = lds + (buf ^ 1) * kStage;
    step(0, st, 1, NMMA, buf ^ 1, kt + 1, kt + 1 < nk);  // rest of stage kt + 1's loads
    prefetch(kt + 2);
    step(1, st, 2, -1, 0, 0, false);
    step(0, st, 3, -1, 0, 0, false);
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    asm volatile("s_barrier" ::: "memory");
    step(1, nst, 0, 0, buf, kt + 2, kt + 2 < nk);  // first part of stage kt + 2's loads
  }
  __builtin_amdgcn_s_waitcnt(vm_wait(0));  // loads past the end (zeros) are done before LDS is reused
  __builtin_amdgcn_s_setprio(0);
}

// One 16 x 16 x 32 operand fragment: lane (r = lane % 16, G = lane / 16) gets k = 32 j + 8 G + 0..7
// of row mn0 + r: one 16-byte read of a row-major tile, or two transposing reads of a
// K-major one (lane s16 of group G addresses k-row 32 j + 8 G + 4 q + s16 / 4, columns
// mn0 + 4 (s16 % 4) .. +3; in each 16-lane group lane 4 a + b then receives column
// mn0 + 4 a + b of those four k-rows).
template <bool TR>
struct Frag16 {
  v4i32_t w;
  v2i32_t lo, hi;
  static constexpr int kReads = TR ? 2 : 1;
  template <int BMN, int KS>
  __device__ __forceinline__ void read_piece(const lds_char* base, int mn0, int j, int q) {
    const int lane = threadIdx.x & 63;
    if constexpr (!TR) {
      w = asm_ds_read_b128(lds_addr(base) + nt_off<KS>(mn0 + (lane & 15), 4 * j + (lane >> 4)));
    } else {
      const int G = lane >> 4, s16 = lane & 15;
      const int krow = 32 * j + 8 * G + 4 * q + (s16 >> 2);
      const v2i32_t v = asm_ds_read_tr16(lds_addr(base) + t_off(krow, mn0 + 4 * (s16 & 3), BMN * 2));
      if (q == 0) lo = v;
      else hi = v;
    }
  }
  __device__ __forceinline__ void tie() {
    if constexpr (!TR) {
      asm_tie(w);
    } else {
      asm_tie(lo);
      asm_tie(hi);
    }
  }
  __device__ __forceinline__ bf16x8_t value() const {
    if constexpr (!TR) return __builtin_bit_cast(bf16x8_t, w);
    else return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3));
  }
};

// The K loop of kloop64 on v_mfma_f32_16x16x32_bf16 (same LDS stages, loads, barrier and
// waits). The accumulators are 16 x 16 blocks: acc[mi][ni][2 a + b] holds rows
// 32 mi + 16 a + (lane % 16) and columns 32 ni + 16 b + 4 (lane / 16) + 0..3 of the wave's
// block. A stage's four steps are (32-deep k-step j, half h) = (t / 2, t % 2), half h covering
// the 32-row blocks h MI/2 .. (h + 1) MI/2 - 1: with 8 waves 16 MFMAs per step, as many
// cycles as kloop64's 8. A step reads the next step's A fragments, and in the second half of
// a k-step the next k-step's B fragments too (A held one step, B two). The smaller MFMA
// interleaves better with the loads and fragment reads of the two waves of a SIMD: a probe
// streaming the same loads and LDS reads ran 8-10% more MFMA work per second on it than on
// 32 x 32 x 16, at the same clock.
template <int LPS, int MI, int NI, bool A_T, bool B_T, int BM, int BN, typename Dma, typename Prefetch, typename Hook>
__device__ __forceinline__ void kloop64_m16(int nk, lds_char* lds, int wm0, int wn0, f32x4_t (&acc)[MI][NI][4],
                                            Dma dma, Prefetch prefetch, Hook after_prologue_loads) {
  constexpr int KS = 64;
  constexpr int kStage = (BM + BN) * KS * 2;
  constexpr int HM = MI / 2;              // 32-row blocks per step
  constexpr int NMMA = HM * 2 * NI * 2;   // MFMAs per step
  constexpr int AR = Frag16<A_T>::kReads, BR = Frag16<B_T>::kReads;
  constexpr int NRA = HM * 2 * AR, NRB = NI * 2 * BR;
  constexpr int WIN = 2 * NMMA;
  constexpr int kEarly = (NMMA * LPS + WIN - 1) / WIN;
  static_assert(MI % 2 == 0, "two halves of the 32-row blocks");
  Frag16<A_T> fa[2][HM][2];
  Frag16<B_T> fb[2][NI][2];
  // fragment reads of step t (of the stage in st): read r < NRA is A, else B (t even only)
  auto read = [&](const lds_char* st, int t, int r) {
    const int j = t >> 1, h = t & 1;
    if (r < NRA) {
      const int f = r / AR, q = r % AR, mil = f >> 1, a = f & 1;
      fa[t & 1][mil][a].template read_piece<BM, KS>(st, wm0 + 32 * (h * HM + mil) + 16 * a, j, q);
    } else {
      const int rb = r - NRA, f = rb / BR, q = rb % BR, ni = f >> 1, b = f & 1;
      fb[j & 1][ni][b].template read_piece<BN, KS>(st + BM * KS * 2, wn0 + 32 * ni + 16 * b, j, q);
    }
  };
  auto nread = [](int t) { return (t & 1) ? NRA : NRA + NRB; };
  auto tie = [&](int t) {
#pragma unroll
    for (int i = 0; i < HM; ++i) {
      fa[t & 1][i][0].tie();
      fa[t & 1][i][1].tie();
    }
    if ((t & 1) == 0) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        fb[(t >> 1) & 1][i][0].tie();
        fb[(t >> 1) & 1][i][1].tie();
      }
    }
  };
  auto mma = [&](int t, int i) {
    const int b = i & 1, ni = (i >> 1) % NI, a = (i / (2 * NI)) & 1, mil = i / (4 * NI);
    f32x4_t& c = acc[(t & 1) * HM + mil][ni][2 * a + b];
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[(t >> 1) & 1][ni][b].value(), fa[t & 1][mil][a].value(), c, 0, 0,
                                                0);
  };
  // step t: MFMAs of step t, reads of step (t + 1) % 4 from rst (spread evenly over the
  // step's MFMA slots: 1.5-2% faster per launch at C3 than issued in the first slots), loads
  // of window slots [w0, w0 + NMMA) of stage lkt into buffer lbuf
  auto step = [&](int t, const lds_char* rst, int w0, int lbuf, int lkt, bool lon) {
    const int tn = (t + 1) & 3;
    const int nr = nread(tn);
    __builtin_amdgcn_sched_barrier(0);
    if (w0 >= 0) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NMMA; ++i) {
      mma(t, i);
#pragma unroll
      for (int j = 0; j < LPS; ++j)
        if (w0 >= 0 && j * WIN / LPS == w0 + i) dma(j, lbuf, lkt, lon);
#pragma unroll
      for (int r = 0; r < NRA + NRB; ++r)
        if (r < nr && (r * NMMA) / nr == i) read(rst, tn, r);
      __builtin_amdgcn_sched_barrier(0);
    }
    asm_wait_lgkm<0>();
    tie(tn);
  };
  if (nk <= 0) {
    after_prologue_loads();
    return;
  }
  prefetch(0);
#pragma unroll
  for (int j = 0; j < LPS; ++j) dma(j, 0, 0, true);
  prefetch(1);
#pragma unroll
  for (int j = 0; j < kEarly; ++j) dma(j, 1, 1, nk > 1);
  after_prologue_loads();
  __builtin_amdgcn_s_waitcnt(vm_wait(kEarly));  // stage 0 landed (stage 1's early loads may not have)
  asm volatile("s_barrier" ::: "memory");
#pragma unroll
  for (int r = 0; r < NRA + NRB; ++r) read(lds, 0, r);
  asm_wait_lgkm<0>();
  tie(0);

  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const lds_char* st = lds + buf * kStage;
    const lds_char* nst = lds + (buf ^ 1) * kStage;
    step(0, st, NMMA, buf ^ 1, kt + 1, kt + 1 < nk);  // rest of stage kt + 1's loads
    prefetch(kt + 2);
    step(1, st, -1, 0, 0, false);
    step(2, st, -1, 0, 0, false);
    __builtin_amdgcn_s_waitcnt(vm_wait(0));
    asm volatile("s_barrier" ::: "memory");
    step(3, nst, 0, buf, kt + 2, kt + 2 < nk);  // first part of stage kt + 2's loads
  }
  __builtin_amdgcn_s_waitcnt(vm_wait(0));  // loads past the end (zeros) are done before LDS is reused
  __builtin_amdgcn_s_setprio(0);
}

// The K loop of an 8-wave 256 x BN tile that holds at most kSmallRows rows (an expert's only or
// last m-tile, e.g. the rare experts of a skewed routing): such a tile is bound by its operand
// loads (a few rows against a BN-column block of the weights streamed through the whole
// reduction), not by its MFMAs, and kloop64_m16 gives it one stage of loads in flight. Here only
// the first kSmallRows A rows are loaded (the waves whose RowLoad<256, 8> rows those are), so a
// stage takes (kSmallRows + BN) x 64 x 2 bytes and three of them fit in the kernel's LDS: two
// stages are in flight while one is read (C4: W2 forward 8%, W1 input grad 5% faster; at C3,
// where only last m-tiles are this short, W2 forward and dA 1.5%). Waves 0-3 (the tile's rows
// 0-127) run the MFMAs of rows 0 .. kSmallRows - 1 with the accumulator layout of kloop64_m16;
// waves 4-7 only load. Per stage: wait for this wave's loads of it, barrier (every wave's loads
// are in and every wave is done with the buffer read two stages ago), issue the loads of the
// stage two ahead into that buffer, then read and multiply. dma_a(q, stage, kt, on) and
// dma_b(q, stage, kt, on) issue A / B load q of stage kt into the A / B part of a stage.
constexpr int kSmallRows = 64;
template <int NQA, int NQB, int MI, int NI, bool B_T, int BN, typename DmaA, typename DmaB, typename Hook>
__device__ __forceinline__ void kloop_small(int nk, lds_char* lds, int wm0, int wn0, f32x4_t (&acc)[MI][NI][4],
                                            DmaA dma_a, DmaB dma_b, Hook after_prologue_loads) {
  constexpr int KS = 64;
  constexpr int kA = kSmallRows * KS * 2;
  constexpr int kS = kA + BN * KS * 2;
  constexpr int SM = kSmallRows / 32;              // 32-row blocks with rows
  constexpr int AR = Frag16<false>::kReads, BR = Frag16<B_T>::kReads;
  constexpr int kAWaves = kSmallRows / (8 * NQA);  // RowLoad<256, 8>: wave w loads rows 8 NQA w ..
  static_assert(SM * 32 == kSmallRows && SM <= MI && MI * 32 == 128, "the rows lie in waves 0-3's blocks");
  static_assert(kAWaves * 8 * NQA == kSmallRows, "whole waves load the first kSmallRows rows");
  const int wu = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const bool a_wave = wu < kAWaves;  // wave-uniform
  const bool mma_wave = __builtin_amdgcn_readfirstlane(wm0) == 0;
  auto issue = [&](int buf, int kt, bool on) {
    lds_char* st = lds + buf * kS;
    if (a_wave) {
#pragma unroll
      for (int q = 0; q < NQA; ++q) dma_a(q, st, kt, on);
    }
#pragma unroll
    for (int q = 0; q < NQB; ++q) dma_b(q, st + kA, kt, on);
  };
  if (nk <= 0) {
    after_prologue_loads();
    return;
  }
  issue(0, 0, true);
  issue(1, 1, nk > 1);
  after_prologue_loads();
  int cur = 0;  // buffer of stage kt
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt has landed once at most stage kt + 1's loads are outstanding
    if (a_wave) __builtin_amdgcn_s_waitcnt(vm_wait(NQA + NQB));
    else __builtin_amdgcn_s_waitcnt(vm_wait(NQB));
    asm volatile("s_barrier" ::: "memory");
    issue(cur == 0 ? 2 : cur - 1, kt + 2, kt + 2 < nk);
    if (mma_wave) {
      const lds_char* st = lds + cur * kS;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        Frag16<false> fa[SM][2];
        Frag16<B_T> fb[NI][2];
#pragma unroll
        for (int f = 0; f < 2 * SM; ++f)
#pragma unroll
          for (int q = 0; q < AR; ++q) fa[f >> 1][f & 1].template read_piece<kSmallRows, KS>(st, 16 * f, j, q);
#pragma unroll
        for (int f = 0; f < 2 * NI; ++f)
#pragma unroll
          for (int q = 0; q < BR; ++q)
            fb[f >> 1][f & 1].template read_piece<BN, KS>(st + kA, wn0 + 16 * f, j, q);
        asm_wait_lgkm<0>();
#pragma unroll
        for (int f = 0; f < 2 * SM; ++f) fa[f >> 1][f & 1].tie();
#pragma unroll
        for (int f = 0; f < 2 * NI; ++f) fb[f >> 1][f & 1].tie();
#pragma unroll
        for (int mil = 0; mil < SM; ++mil)
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int ni = 0; ni < NI; ++ni)
#pragma unroll
              for (int b = 0; b < 2; ++b)
                acc[mil][ni][2 * a + b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    fb[ni][b].value(), fa[mil][a].value(), acc[mil][ni][2 * a + b], 0, 0, 0);
      }
    }
    cur = cur == 2 ? 0 : cur + 1;
  }
  __builtin_amdgcn_s_waitcnt(vm_wait(0));  // loads past the end (zeros) are done before LDS is reused
}

// Epilogues: each wave stages its own WM x WN accumulator block in its own LDS area
// (bf16, rows of WN * 2 + 16 bytes) and writes it out row-contiguously, 16 bytes
// per lane, so every store instruction covers whole 128-byte lines. The MFMA layout
// itself would give 8-byte pieces of 32 different rows per store instruction; such
// partial-line writes cost more than the staging. Staging is wave-local: once every
// wave is past the K loop (one barrier) no further workgroup sync is needed.
// In the MFMA layout lane (r = lane % 32, g = lane / 32) holds, for row 32 mi + r,
// the columns 32 ni + 8 q + 4 g + 0..3 in acc[mi][ni][4 q .. 4 q + 3].
template <int WN>
struct WaveStage {
  static constexpr int PITCH = WN * 2 + 16;  // bytes per staged row
  static constexpr int CPR = WN / 8;          // 16-byte chunks per row
};

// GEMM output stores (16 bytes per lane; non-temporal stores measured no faster)
__device__ __forceinline__ void st_out(void* p, const uint4& v) { *reinterpret_cast<uint4*>(p) = v; }

__device__ __forceinline__ uint2 pack4_bf16(const float (&v)[4]) {
  return make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}
__device__ __forceinline__ void unpack4_bf16(uint2 w, float (&v)[4]) {
  v[0] = __uint_as_float(w.x << 16);
  v[1] = __uint_as_float(w.x & 0xffff0000u);
  v[2] = __uint_as_float(w.y << 16);
  v[3] = __uint_as_float(w.y & 0xffff0000u);
}

// rows 32 mi0 .. 32 mi1 - 1 of the wave's block -> staged rows 0 .. 32 (mi1 - mi0) - 1,
// rounded to bf16 (plus the bias row first, if any: one rounding, as an unfused add would not do)
template <int MI, int NI>
__device__ __forceinline__ void wave_stage_bf16(char* st, const f32x16_t (&acc)[MI][NI], int mi0, int mi1,
                                                const uint16_t* bias_cols = nullptr, int bias_ncols = 0) {
  constexpr int PITCH = WaveStage<NI * 32>::PITCH;
  const int lane = threadIdx.x & 63;
  const int r = lane & 31, g = lane >> 5;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    if (mi < mi0 || mi >= mi1) continue;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = 32 * ni + 8 * q + 4 * g;
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = acc[mi][ni][4 * q + u];
        if (bias_cols != nullptr && col < bias_ncols) {  // (columns past N are never stored)
          float bv[4];
          unpack4_bf16(*reinterpret_cast<const uint2*>(bias_cols + col), bv);
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] += bv[u];
        }
        *reinterpret_cast<uint2*>(st + (32 * (mi - mi0) + r) * PITCH + col * 2) = pack4_bf16(v);
      }
  }
}

// The same staging from kloop64_m16's 16 x 16 accumulators (lane (r = lane % 16, g = lane / 16)
// holds, in acc[mi][ni][2 a + b], row 32 mi + 16 a + r, columns 32 ni + 16 b + 4 g + 0..3).
template <int MI, int NI>
__device__ __forceinline__ void wave_stage_bf16(char* st, const f32x4_t (&acc)[MI][NI][4], int mi0, int mi1,
                                                const uint16_t* bias_cols = nullptr, int bias_ncols = 0) {
  constexpr int PITCH = WaveStage<NI * 32>::PITCH;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    if (mi < mi0 || mi >= mi1) continue;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int ab = 0; ab < 4; ++ab) {
        const int a = ab >> 1, b = ab & 1;
        const int col = 32 * ni + 16 * b + 4 * g;
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = acc[mi][ni][ab][u];
        if (bias_cols != nullptr && col < bias_ncols) {
          float bv[4];
          unpack4_bf16(*reinterpret_cast<const uint2*>(bias_cols + col), bv);
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] += bv[u];
        }
        *reinterpret_cast<uint2*>(st + (32 * (mi - mi0) + 16 * a + r) * PITCH + col * 2) = pack4_bf16(v);
      }
  }
}

// The store loops below run in batches of EPI_BATCH chunks per lane: every LDS read
// (staged values, output-row numbers) and global read (H, D) of a batch is issued
// before the first store of the batch, so their latencies overlap instead of adding up
// chunk by chunk.
constexpr int EPI_BATCH = 8;

template <int BM, int BN, int EPI, int MI, int NI, typename AccT>
__device__ __forceinline__ void rows_epilogue_bf16(const RowsParams& p, char* st, const int* row_table,
                                                   const AccT (&acc)[MI][NI], int e, int64_t row0, int rows,
                                                   int nt, int wm0, int wn0, int mt = 0,
                                                   const float* scale_table = nullptr) {
  using S = WaveStage<NI * 32>;
  constexpr int VEC = 8;
  const int lane = threadIdx.x & 63;
  uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
  const int ncol0 = nt * BN + wn0;
  if constexpr (EPI == EPI_SWIGLU) {
    // staged columns per 64: [h 32 | gate 32] for pair columns jj0 + 32 pb + 0..31;
    // A = silu(gate) * h from the bf16-rounded h and gate, as stored in H
    constexpr int PB = NI / 2, CPP = 32 / VEC;  // pair blocks, chunks per 32 columns
    constexpr int ITERS = 16 * MI * PB * CPP / 64;
    constexpr int B = ITERS < EPI_BATCH ? ITERS : EPI_BATCH;
    static_assert(ITERS % B == 0, "batches tile the staged block");
    uint16_t* A2 = reinterpret_cast<uint16_t*>(p.c2);
    const int jj0 = nt * (BN / 2) + (wn0 / 64) * 32;
#pragma unroll
    for (int half = 0; half < 2; ++half) {  // two halves of the rows: 3 outputs per pair need room
      wave_stage_bf16(st, acc, half * MI / 2, (half + 1) * MI / 2, nullptr);
#pragma unroll
      for (int i0 = 0; i0 < ITERS; i0 += B) {
        uint4 hv[B], gv[B];
        int orow[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int idx = lane + 64 * (i0 + u);
          const int rr = idx / (PB * CPP), rem = idx % (PB * CPP);
          const int pb = rem / CPP, cc = rem % CPP;
          hv[u] = *reinterpret_cast<const uint4*>(st + rr * S::PITCH + (pb * 64 + cc * VEC) * 2);
          gv[u] = *reinterpret_cast<const uint4*>(st + rr * S::PITCH + (pb * 64 + 32 + cc * VEC) * 2);
          orow[u] = row_table[wm0 + half * 16 * MI + rr];
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int idx = lane + 64 * (i0 + u);
          const int rr = idx / (PB * CPP), rem = idx % (PB * CPP);
          const int pb = rem / CPP, cc = rem % CPP;
          const int rl = wm0 + half * 16 * MI + rr;
          const int jj = jj0 + pb * 32 + cc * VEC;
          if (rl < rows && jj < p.half) {
            float h[VEC], gt[VEC], a[VEC];
            unpack_chunk(hv[u], h, uint16_t{});
            unpack_chunk(gv[u], gt, uint16_t{});
            const float rs = p.row_scale != nullptr ? scale_table[rl] : 1.f;
#pragma unroll
            for (int q = 0; q < VEC; ++q) a[q] = rs * (silu_f(gt[q]) * h[q]);
            const int64_t o = orow[u];
            st_out(C + o * p.ldc + jj, hv[u]);
            st_out(C + o * p.ldc + p.half + jj, gv[u]);
            st_out(A2 + o * p.ldc2 + jj, pack_chunk(a, uint16_t{}));
          }
        }
      }
    }
    return;
  }
  constexpr int ITERS = 32 * MI * S::CPR / 64;
  constexpr int B = ITERS < EPI_BATCH ? ITERS : EPI_BATCH;
  constexpr int NB = ITERS / B;
  static_assert(ITERS % B == 0, "batches tile the staged block");
  const uint16_t* bias = nullptr;
  if constexpr (EPI == EPI_STORE_BIAS)
    bias = reinterpret_cast<const uint16_t*>(p.bias) + (int64_t)e * p.bias_estride + ncol0;
  wave_stage_bf16(st, acc, 0, MI, bias, p.N - ncol0);
  // chunk (row, column) of item u of batch i
  auto item_rl = [&](int i, int u) { return wm0 + (lane + 64 * (i * B + u)) / S::CPR; };
  auto item_cc = [&](int i, int u) { return (lane + 64 * (i * B + u)) % S::CPR; };
  auto item_ok = [&](int i, int u) { return item_rl(i, u) < rows && ncol0 + item_cc(i, u) * VEC < p.N; };
  // Global operands of the epilogue (H for EPI_SWIGLU_BWD, D for EPI_NS; both in the
  // grouped row order row0 + rl) are read one batch ahead, before the stores of the
  // current batch: a later wait on them then does not also wait for those stores.
  constexpr bool kGlobal = EPI == EPI_SWIGLU_BWD || EPI == EPI_NS;
  const uint16_t* G = reinterpret_cast<const uint16_t*>(p.aux);
  const bool has_g = kGlobal && G != nullptr;
  uint4 g0[2][B], g1[2][B];
  auto load_globals = [&](int i, int buf) {
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (item_ok(i, u)) {
        const uint16_t* r = G + (row0 + item_rl(i, u)) * p.ld_aux + ncol0 + item_cc(i, u) * VEC;
        g0[buf][u] = ldg16(r);
        if constexpr (EPI == EPI_SWIGLU_BWD) g1[buf][u] = ldg16(r + p.half);
      }
    }
  };
  if (has_g) load_globals(0, 0);
  // SwiGLU backward of scaled rows: lanes 8 j .. 8 j + 7 of an item hold the 64 columns of
  // one row (8 chunks of 8), so a row's partial dot product is a sum over 3 lane bits
  const bool dots = EPI == EPI_SWIGLU_BWD && p.row_dots != nullptr;
  static_assert(EPI != EPI_SWIGLU_BWD || S::CPR == 8, "one row per 8 lanes");
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int cur = i & 1;
    uint4 tv[B];
    int orow[B];
    float rsc[B], dot[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      tv[u] = *reinterpret_cast<const uint4*>(st + (item_rl(i, u) - wm0) * S::PITCH + item_cc(i, u) * 16);
      orow[u] = row_table[item_rl(i, u)];
      rsc[u] = 1.f;
      dot[u] = 0.f;
      if constexpr (EPI == EPI_SWIGLU_BWD) {
        if (dots) rsc[u] = scale_table[item_rl(i, u)];
      }
    }
    if (has_g && i + 1 < NB) load_globals(i + 1, cur ^ 1);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      if (!item_ok(i, u)) continue;
      const int col = ncol0 + item_cc(i, u) * VEC;
      const int64_t o = orow[u];
      if constexpr (EPI == EPI_STORE || EPI == EPI_STORE_BIAS) {
        st_out(C + o * p.ldc + col, tv[u]);
      } else if constexpr (EPI == EPI_NS) {
        // out = t + bf16(beta * D) and out2 = bf16(gamma * t) with t = bf16(acc): the rounding
        // points of bf16 tensor arithmetic in muon.py:24-27 (each product and sum rounded)
        uint16_t* C2 = reinterpret_cast<uint16_t*>(p.c2);
        float t[VEC];
        unpack_chunk(tv[u], t, uint16_t{});
        if (C2 != nullptr) {
          float q[VEC];
#pragma unroll
          for (int v = 0; v < VEC; ++v) q[v] = p.ns_gamma * t[v];
          st_out(C2 + o * p.ldc2 + col, pack_chunk(q, uint16_t{}));
        }
        uint4 ov = tv[u];
        if (has_g) {
          float d[VEC], r[VEC];
          unpack_chunk(g0[cur][u], d, uint16_t{});
#pragma unroll
          for (int v = 0; v < VEC; ++v) r[v] = t[v] + to_f32(bf16_bits(p.ns_beta * d[v]));
          ov = pack_chunk(r, uint16_t{});
        }
        st_out(C + o * p.ldc + col, ov);
      } else {  // EPI_SWIGLU_BWD: staged dA (bf16, as the unfused path stores it), H rows in sorted order
        float da[VEC], h[VEC], gt[VEC], dh[VEC], dg[VEC];
        unpack_chunk(tv[u], da, uint16_t{});
        unpack_chunk(g0[cur][u], h, uint16_t{});
        unpack_chunk(g1[cur][u], gt, uint16_t{});
#pragma unroll
        for (int v = 0; v < VEC; ++v) {
          const float sg = sigmoid_fast(gt[v]);
          if (dots) {  // dA = scale * (unscaled dA, bf16); the dot uses the unscaled values
            dot[u] += da[v] * (gt[v] * sg * h[v]);  // A = silu(gate) * h
            da[v] *= rsc[u];
          }
          dh[v] = da[v] * gt[v] * sg;
          dg[v] = da[v] * h[v] * sg * (1.f + gt[v] * (1.f - sg));
        }
        st_out(C + o * p.ldc + col, pack_chunk(dh, uint16_t{}));
        st_out(C + o * p.ldc + p.half + col, pack_chunk(dg, uint16_t{}));
      }
    }
    if constexpr (EPI == EPI_SWIGLU_BWD) {
      if (dots) {
#pragma unroll
        for (int u = 0; u < B; ++u) {
          float s = dot[u];
          s += __shfl_xor(s, 1, 64);
          s += __shfl_xor(s, 2, 64);
          s += __shfl_xor(s, 4, 64);
          if ((lane & 7) == 0 && item_rl(i, u) < rows && ncol0 < p.N)
            p.row_dots[(row0 + item_rl(i, u)) * p.dots_ld + ncol0 / 64] = s;
        }
      }
    }
  }
  if constexpr (EPI == EPI_NS) {
    // Symmetric output (the Gram products of the Newton-Schulz step): a tile above the
    // diagonal also writes its mirror. Output row j of the mirror block is column j of
    // the staged block, read 8 rows at a time with 16-bit LDS reads.
    if (p.ns_sym_m > 0 && nt != mt) {
      constexpr int CPC = 32 * MI / VEC;                 // 16-byte chunks per mirrored row
      constexpr int MITERS = NI * 32 * CPC / 64;
      constexpr int MB = MITERS < EPI_BATCH ? MITERS : EPI_BATCH;
      static_assert(MITERS % MB == 0, "batches tile the mirrored block");
      const uint16_t* D = reinterpret_cast<const uint16_t*>(p.aux);
      uint16_t* C2 = reinterpret_cast<uint16_t*>(p.c2);
      const int64_t ebase = row0 - (int64_t)mt * BM;     // the expert's first row
      const int jcol0 = nt * BN + wn0;                   // the block's first column = first mirrored row
#pragma unroll
      for (int i0 = 0; i0 < MITERS; i0 += MB) {
        uint4 tv[MB], dv[MB];
#pragma unroll
        for (int u = 0; u < MB; ++u) {
          const int idx = lane + 64 * (i0 + u);
          const int c = idx / CPC, rc = idx % CPC;       // staged column, chunk of 8 staged rows
          uint32_t w[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t lo = *reinterpret_cast<const uint16_t*>(st + (rc * VEC + 2 * q) * S::PITCH + c * 2);
            const uint32_t hi = *reinterpret_cast<const uint16_t*>(st + (rc * VEC + 2 * q + 1) * S::PITCH + c * 2);
            w[q] = lo | (hi << 16);
          }
          tv[u] = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if (D != nullptr) {
#pragma unroll
          for (int u = 0; u < MB; ++u) {
            const int idx = lane + 64 * (i0 + u);
            const int c = idx / CPC, rc = idx % CPC;
            if (jcol0 + c < p.N && wm0 + rc * VEC < rows)
              dv[u] = ldg16(D + (ebase + jcol0 + c) * p.ld_aux + mt * BM + wm0 + rc * VEC);
          }
        }
#pragma unroll
        for (int u = 0; u < MB; ++u) {
          const int idx = lane + 64 * (i0 + u);
          const int c = idx / CPC, rc = idx % CPC;
          if (jcol0 + c >= p.N || wm0 + rc * VEC >= rows) continue;
          const int64_t o = ebase + jcol0 + c;
          const int col = mt * BM + wm0 + rc * VEC;
          float t[VEC];
          unpack_chunk(tv[u], t, uint16_t{});
          if (C2 != nullptr) {
            float q[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) q[v] = p.ns_gamma * t[v];
            st_out(C2 + o * p.ldc2 + col, pack_chunk(q, uint16_t{}));
          }
          uint4 ov = tv[u];
          if (D != nullptr) {
            float d[VEC], r[VEC];
            unpack_chunk(dv[u], d, uint16_t{});
#pragma unroll
            for (int v = 0; v < VEC; ++v) r[v] = t[v] + to_f32(bf16_bits(p.ns_beta * d[v]));
            ov = pack_chunk(r, uint16_t{});
          }
          st_out(C + o * p.ldc + col, ov);
        }
      }
    }
  }
}

template <int MI, int NI, typename AccT>
__device__ __forceinline__ void wgrad_epilogue_bf16(const WgradParams& p, char* st, const AccT (&acc)[MI][NI],
                                                    int e, int m0, int n0, int wm0, int wn0) {
  using S = WaveStage<NI * 32>;
  constexpr int ITERS = 32 * MI * S::CPR / 64;
  constexpr int B = ITERS < EPI_BATCH ? ITERS : EPI_BATCH;
  static_assert(ITERS % B == 0, "batches tile the staged block");
  const int lane = threadIdx.x & 63;
  uint16_t* DW = reinterpret_cast<uint16_t*>(p.dw) + (int64_t)e * p.Ndy * p.Kx;
  wave_stage_bf16(st, acc, 0, MI, nullptr);
#pragma unroll
  for (int i0 = 0; i0 < ITERS; i0 += B) {
    uint4 v[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int idx = lane + 64 * (i0 + u);
      v[u] = *reinterpret_cast<const uint4*>(st + (idx / S::CPR) * S::PITCH + (idx % S::CPR) * 16);
    }
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int idx = lane + 64 * (i0 + u);
      const int m = m0 + wm0 + idx / S::CPR, n = n0 + wn0 + (idx % S::CPR) * 8;
      if (m < p.Ndy && n < p.Kx) st_out(DW + (int64_t)m * p.Kx + n, v[u]);
    }
  }
}

// fp32 weight grads (fp32 master weights) through the wave's staging area: 32 rows of the
// wave's block at a time, staged as fp32 rows of WN * 4 + 16 bytes (within the bf16 staging
// area of a block of at least 64 rows), then written row-contiguously, 16 bytes per lane, so
// every store covers whole 128-byte lines (from the MFMA layout directly, a store would be 16
// bytes of each of 32 rows). Wave-local: LDS operations of one wave complete in order.
template <int MI, int NI, typename AccT>
__device__ __forceinline__ void wgrad_epilogue_f32_staged(const WgradParams& p, char* st,
                                                          const AccT (&acc)[MI][NI], int e, int m0, int n0,
                                                          int wm0, int wn0) {
  static_assert(MI >= 2, "the fp32 rows of one 32-row block fit the staging area of two");
  constexpr int WN = NI * 32;
  constexpr int PITCH = WN * 4 + 16;  // bytes per staged fp32 row
  constexpr int CPR = WN / 4;         // 16-byte chunks per row
  constexpr int ITERS = 32 * CPR / 64;
  constexpr int B = ITERS < EPI_BATCH ? ITERS : EPI_BATCH;
  static_assert(ITERS % B == 0, "batches tile the staged rows");
  const int lane = threadIdx.x & 63;
  const int r = lane & 31, g = lane >> 5;
  float* DW = reinterpret_cast<float*>(p.dw) + (int64_t)e * p.Ndy * p.Kx;
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    if constexpr (std::is_same<AccT, f32x16_t>::value) {
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = 32 * ni + 8 * q + 4 * g;
          *reinterpret_cast<float4*>(st + r * PITCH + col * 4) = make_float4(
              acc[mi][ni][4 * q], acc[mi][ni][4 * q + 1], acc[mi][ni][4 * q + 2], acc[mi][ni][4 * q + 3]);
        }
    } else {  // 16 x 16 blocks (kloop64_m16)
      const int r16 = lane & 15, g16 = lane >> 4;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int ab = 0; ab < 4; ++ab) {
          const int col = 32 * ni + 16 * (ab & 1) + 4 * g16;
          *reinterpret_cast<float4*>(st + (16 * (ab >> 1) + r16) * PITCH + col * 4) =
              make_float4(acc[mi][ni][ab][0], acc[mi][ni][ab][1], acc[mi][ni][ab][2], acc[mi][ni][ab][3]);
        }
    }
#pragma unroll
    for (int i0 = 0; i0 < ITERS; i0 += B) {
      uint4 v[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int idx = lane + 64 * (i0 + u);
        v[u] = *reinterpret_cast<const uint4*>(st + (idx / CPR) * PITCH + (idx % CPR) * 16);
      }
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const int idx = lane + 64 * (i0 + u);
        const int m = m0 + wm0 + 32 * mi + idx / CPR, n = n0 + wn0 + (idx % CPR) * 4;
        if (m < p.Ndy && n < p.Kx) st_out(DW + (int64_t)m * p.Kx + n, v[u]);
      }
    }
  }
}

// Wave layout of the bf16 kernels: NW = 4 waves in a 2 x 2 grid, 8 in a 2 x 4 grid or 16
// in a 4 x 4 grid (waves w, w + 4, ... share SIMD w % 4).
template <int BM, int BN, int NW>
struct WaveGrid {
  static_assert(NW == 4 || NW == 8 || NW == 16, "4, 8 or 16 waves");
  static constexpr int GM = NW == 16 ? 4 : 2, GN = NW / GM;
  static constexpr int WM = BM / GM, WN = BN / GN;
  static constexpr int MI = WM / 32, NI = WN / 32;
  __device__ __forceinline__ static int wm0(int wave) { return (wave / GN) * WM; }
  __device__ __forceinline__ static int wn0(int wave) { return (wave % GN) * WN; }
};

// LDS of the bf16 kernels: two operand stages (three short ones in kloop_small), reused by
// the wave staging areas after the K loop, then the rows kernel's output-row table.
template <int BM, int BN, int NW = 4>
constexpr int bf16_stage_bytes() {
  constexpr int loop = 2 * (BM + BN) * 64 * 2;
  constexpr int small = (BM == 256 && NW == 8) ? 3 * (kSmallRows + BN) * 64 * 2 : 0;
  constexpr int epi = NW * WaveGrid<BM, BN, NW>::WM * WaveStage<WaveGrid<BM, BN, NW>::WN>::PITCH;
  constexpr int ops = loop > small ? loop : small;
  return ops > epi ? ops : epi;
}

template <int BM, int BN, bool B_T, int EPI, int NW = 4>
__global__ __launch_bounds__(NW * 64) void rows_bf16_kernel(RowsParams p) {
  extern __shared__ __align__(16) char smem[];
  constexpr int KS = 64;
  using WG = WaveGrid<BM, BN, NW>;
  constexpr int WN = WG::WN;
  constexpr int MI = WG::MI, NI = WG::NI;
  constexpr int kStage = (BM + BN) * KS * 2;
  static_assert(EPI != EPI_SWIGLU || WN % 64 == 0, "SwiGLU pairs 32-column blocks inside a wave");

  RowsTile tile;
  if (!decode_rows_tile<BM, NW * 64>(p, smem, tile)) return;  // uniform per workgroup
  const int e = __builtin_amdgcn_readfirstlane(tile.e);
  const int nt = __builtin_amdgcn_readfirstlane(tile.nt);
  const int rows = tile.rows;
  const int64_t row0 = tile.row0;
  const int wu = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  lds_char* lds = (lds_char*)(smem);  // generic -> LDS address space
  const int ktail = p.K % KS;
  const int nk = (p.K + KS - 1) / KS;

  // Row indices (< 2^31) are read as the low 32-bit words of the int64 entries, all
  // issued before any is used so their latencies overlap.
  using LA = RowLoad<BM, NW>;
  using LBN = RowLoad<B_T ? 8 * NW : BN, NW>;  // (placeholder sizes for the unused loader)
  using LBT = KLoad<B_T ? BN : 8 * NW, NW>;
  LA la;
  int a_src[LA::NQ];
#pragma unroll
  for (int q = 0; q < LA::NQ; ++q) {
    const int r = LA::row_of(q);
    a_src[q] = (int)(row0 + (r < rows ? r : 0));
  }
  if (p.a_rows != nullptr) {
    const int* idx32 = reinterpret_cast<const int*>(p.a_rows);
#pragma unroll
    for (int q = 0; q < LA::NQ; ++q) a_src[q] = idx32[2 * (int64_t)a_src[q]];
#pragma unroll
    for (int q = 0; q < LA::NQ; ++q) a_src[q] /= p.a_div;
  }
#pragma unroll
  for (int q = 0; q < LA::NQ; ++q)
    la.set(q, LA::row_of(q) < rows ? (uint32_t)((int64_t)a_src[q] * p.lda * 2) : kOOB, ktail);
  const int ncol0 = nt * BN;
  LBN lbn;
  LBT lbt;
  if constexpr (!B_T) {
#pragma unroll
    for (int q = 0; q < LBN::NQ; ++q) {
      const int r = LBN::row_of(q);
      int n;
      bool ok;
      if constexpr (EPI == EPI_SWIGLU) {
        const int jj = nt * (BN / 2) + (r >> 6) * 32 + (r & 31);
        ok = jj < p.half;
        n = (r & 32) ? p.half + jj : jj;
      } else {
        n = ncol0 + r;
        ok = n < p.N;
      }
      lbn.set(q, ok ? (uint32_t)((int64_t)n * p.ldb * 2) : kOOB, ktail);
    }
  } else {
    lbt.init(ncol0, p.N, p.ldb * 2);
  }
  const char* a_base = reinterpret_cast<const char*>(p.a);
  const char* b_base = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(p.b) + (int64_t)e * p.b_estride);
  constexpr int NQA = LA::NQ;
  constexpr int LPS = NQA + (B_T ? LBT::NQ : LBN::NQ);  // loads per wave per stage
  auto dma_a = [&](int q, lds_char* sa, int kt, bool on) {
    const int64_t k0 = (int64_t)kt * KS;
    la.issue(q, stage_rsrc(a_base, p.a_bytes, 2 * k0, (int64_t)p.a_bytes, on), sa, wu, kt == nk - 1);
  };
  auto dma_b = [&](int q, lds_char* sb, int kt, bool on) {
    const int64_t k0 = (int64_t)kt * KS;
    if constexpr (!B_T) {
      lbn.issue(q, stage_rsrc(b_base, p.b_bytes, 2 * k0, (int64_t)p.b_bytes, on), sb, wu, kt == nk - 1);
    } else {
      const int64_t pitch = p.ldb * 2;
      lbt.issue(q, stage_rsrc(b_base, p.b_bytes, k0 * pitch, ((int64_t)p.K - k0) * pitch, on), sb, wu);
    }
  };
  auto dma = [&](int q, int buf, int kt, bool on) {
    lds_char* sa = lds + buf * kStage;
    if (q < NQA) dma_a(q, sa, kt, on);
    else dma_b(q - NQA, sa + BM * KS * 2, kt, on);
  };

  const int wave = threadIdx.x >> 6;
  const int wm0 = WG::wm0(wave), wn0 = WG::wn0(wave);
  // 8 waves run the 16 x 16 x 32 K loop (kloop64_m16; the C3 step 2.8% faster than on 32 x 32 x 16
  // MFMAs, the Newton-Schulz pass 2.5%), except with the SwiGLU-backward epilogue, which has no
  // registers left for its extra fragments
  constexpr bool M16 = EPI != EPI_SWIGLU_BWD && NW == 8;
  using Acc = typename std::conditional<M16, f32x4_t[4], f32x16_t>::type;
  Acc acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      if constexpr (M16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[mi][ni][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[mi][ni][q] = 0.f;
      }
    }

  // The tile's output rows go to an LDS table above the operand stages: the index
  // loads are issued before the first operand loads and stored once those are in
  // flight, so their latency hides behind the first stage (row numbers < 2^31).
  // (With 8 waves, the table is written by waves 0-3, which run the loads.)
  static_assert(BM <= 256, "row table written by the first 256 threads");
  int* row_table = reinterpret_cast<int*>(smem + bf16_stage_bytes<BM, BN, NW>());
  float* scale_table = reinterpret_cast<float*>(row_table + BM);
  int orow_v = 0;
  float scale_v = 1.f;
  if (threadIdx.x < BM) {
    const int rl = (int)threadIdx.x;
    const int64_t i = row0 + (rl < rows ? rl : 0);
    orow_v = p.c_rows ? reinterpret_cast<const int*>(p.c_rows)[2 * i] : (int)i;
    if constexpr (EPI == EPI_SWIGLU_BWD || EPI == EPI_SWIGLU) {
      if (p.row_scale != nullptr) scale_v = p.row_scale[i];
    }
  }
  auto hook = [&] {
    if (threadIdx.x < BM) {
      row_table[threadIdx.x] = orow_v;
      if constexpr (EPI == EPI_SWIGLU_BWD || EPI == EPI_SWIGLU) scale_table[threadIdx.x] = scale_v;
    }
  };
  if constexpr (M16) {
    // a tile of at most kSmallRows rows streams its weight block three stages deep
    if (BM == 256 && __builtin_amdgcn_readfirstlane(rows) <= kSmallRows)
      kloop_small<NQA, LPS - NQA, MI, NI, B_T, BN>(nk, lds, wm0, wn0, acc, dma_a, dma_b, hook);
    else
      kloop64_m16<LPS, MI, NI, false, B_T, BM, BN>(nk, lds, wm0, wn0, acc, dma, [](int) {}, hook);
  } else {
    kloop64<LPS, MI, NI, false, B_T, BM, BN>(nk, lds, wm0, wn0, acc, dma, [](int) {}, hook);
  }
  // every wave is done with the operand stages (and has written its row-table entries)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  rows_epilogue_bf16<BM, BN, EPI>(p, smem + wave * 32 * MI * WaveStage<WN>::PITCH, row_table, acc, e, row0, rows,
                                  nt, wm0, wn0, tile.mt, scale_table);
}

// ------------------------------------------------------------------ weight grads of small experts
// DW_e for the experts holding at most kFewRows rows (the long tail of a skewed routing):
// their whole reduction is at most four 16-deep MFMA k-steps, so a tile is write-bound:
// its output against at most 48 KB of operands that the expert's other tiles also read
// (from L2). The expert's rows of DY (BM columns) and X (BN columns) go to LDS as K-major
// tiles, the rows past the expert's end up to the next multiple of 16 zeroed; each wave
// runs MI x NI MFMAs per k-step, and the usual wave-staged epilogue writes full 128-byte
// lines. GATHER / DYG as in wgrad_bf16_kernel. Two forms: wgrad_few_rows_kernel, 128 x 256
// tiles on 4 waves, two workgroups per CU (one's stores in flight while the other loads;
// 6.1 TB/s of dW writes on 250 experts of 2 rows at [4096, 7168], against 3.6 TB/s for the
// 128 x 128 tiles of the K-loop kernel); and inside the 256 x 256 K-loop kernel
// (wgrad_bf16_kernel<..., FEW>), so that one launch covers every expert and the write-bound
// tiles of the rare experts run beside the compute-bound tiles of the popular ones.
constexpr int kFewRows = 64;
constexpr int kFewBM = 128, kFewBN = 256;

// The weight-grad tile of an expert with no rows: exact zeros, written straight to the output
// (no operand loads, LDS or MFMA), 16 bytes per lane so that 8 lanes cover a 128-byte line.
template <int BM, int BN, int NTH, bool OUT_F32>
__device__ __forceinline__ void wgrad_zero_tile(const WgradParams& p, int e, int m0, int n0) {
  constexpr int ES = OUT_F32 ? 4 : 2;        // output element bytes
  constexpr int CPR = BN * ES / 16;          // 16-byte chunks per tile row
  static_assert((BM * CPR) % NTH == 0, "the threads tile the output tile");
  char* DW = reinterpret_cast<char*>(p.dw) + (int64_t)e * p.Ndy * p.Kx * ES;
  const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int it = 0; it < BM * CPR / NTH; ++it) {
    const int idx = (int)threadIdx.x + NTH * it;
    const int m = m0 + idx / CPR, n = n0 + (idx % CPR) * (16 / ES);
    if (m < p.Ndy && n < p.Kx) st_out(DW + ((int64_t)m * p.Kx + n) * ES, z);
  }
}

template <int BM, int BN, int NW, int GATHER, bool DYG, bool OUT_F32>
__device__ __forceinline__ void wgrad_few_rows_tile(const WgradParams& p, char* smem, int e, int64_t r_begin,
                                                    int nrows, int m0, int n0) {
  constexpr int KT = kFewRows;
  constexpr int NTH = NW * 64;
  if (nrows == 0) {
    wgrad_zero_tile<BM, BN, NTH, OUT_F32>(p, e, m0, n0);
    return;
  }
  using WG = WaveGrid<BM, BN, NW>;
  constexpr int MI = WG::MI, NI = WG::NI;
  constexpr int CA = BM / 8, CB = BN / 8;  // 16-byte chunks per k-row of each tile
  constexpr int QA = KT * CA / NTH, QB = KT * CB / NTH;  // chunks per thread
  static_assert(QA * NTH == KT * CA && QB * NTH == KT * CB, "the threads tile the operand tiles");
  const int nks = (nrows + 15) >> 4;  // k-steps (uniform per workgroup)
  const int tid = threadIdx.x;
  const char* dy = reinterpret_cast<const char*>(p.dy);
  const char* x = reinterpret_cast<const char*>(p.x);
  // source row of k-row kr of the gathered operand (kr < nrows)
  auto gathered = [&](int kr) -> int64_t {
    const uint32_t v = reinterpret_cast<const uint32_t*>(p.x_rows)[2 * (r_begin + kr)];  // indices < 2^31
    if constexpr (GATHER == 1) return (int64_t)(v >> p.x_div_shift);
    else return (int64_t)(v / (uint32_t)p.x_div);
  };
  // K-major tiles in LDS: DY^T [KT][BM] then X [KT][BN], 16-byte chunks swizzled as t_off
  // reads them; k-rows up to 16 nks are written (zeros past nrows), the rest never read
  lds_char* lds = (lds_char*)smem;
  char* ta = smem;
  char* tb = smem + KT * BM * 2;
  uint4 va[QA], vb[QB];
#pragma unroll
  for (int q = 0; q < QA; ++q) {
    const int i = tid + NTH * q, kr = i / CA, c = i % CA;
    va[q] = make_uint4(0, 0, 0, 0);
    if (kr < nrows && m0 + 8 * c < p.Ndy) {
      const int64_t row = DYG ? gathered(kr) : r_begin + kr;
      va[q] = ldg16(dy + (row * p.lddy + m0 + 8 * c) * 2);
    }
  }
#pragma unroll
  for (int q = 0; q < QB; ++q) {
    const int i = tid + NTH * q, kr = i / CB, c = i % CB;
    vb[q] = make_uint4(0, 0, 0, 0);
    if (kr < nrows && n0 + 8 * c < p.Kx) {
      const int64_t row = (GATHER != 0 && !DYG) ? gathered(kr) : r_begin + kr;
      vb[q] = ldg16(x + (row * p.ldx + n0 + 8 * c) * 2);
    }
  }
#pragma unroll
  for (int q = 0; q < QA; ++q) {
    const int i = tid + NTH * q, kr = i / CA, c = i % CA;
    if (kr < 16 * nks) *reinterpret_cast<uint4*>(ta + t_off(kr, 8 * c, BM * 2)) = va[q];
  }
#pragma unroll
  for (int q = 0; q < QB; ++q) {
    const int i = tid + NTH * q, kr = i / CB, c = i % CB;
    if (kr < 16 * nks) *reinterpret_cast<uint4*>(tb + t_off(kr, 8 * c, BN * 2)) = vb[q];
  }
  __syncthreads();
  const int wave = tid >> 6;
  const int wm0 = WG::wm0(wave), wn0 = WG::wn0(wave);
  f32x16_t acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[mi][ni][q] = 0.f;
  for (int s = 0; s < nks; ++s) {
    Frag<true> fa[MI], fb[NI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) fa[mi].template read<BM, KT>(lds, wm0 + 32 * mi, s);
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) fb[ni].template read<BN, KT>(lds + KT * BM * 2, wn0 + 32 * ni, s);
    asm_wait_lgkm<0>();
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) fa[mi].tie();
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) fb[ni].tie();
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ni].value(), fa[mi].value(), acc[mi][ni], 0, 0, 0);
  }
  __syncthreads();  // every wave has read the operand tiles; LDS becomes the staging areas
  char* st = smem + wave * 32 * MI * WaveStage<WG::WN>::PITCH;
  if constexpr (OUT_F32)
    wgrad_epilogue_f32_staged(p, st, acc, e, m0, n0, wm0, wn0);
  else
    wgrad_epilogue_bf16(p, st, acc, e, m0, n0, wm0, wn0);
}

// Zero filler f of p.fillers: the grads of the experts with no rows, concatenated in expert
// order, are cut into equal contiguous shares of 16-byte units; this workgroup writes share f.
// One workgroup stores ~150 GB/s and 32 reach 4.6 TB/s (a fill probe on MI355X), so a few
// long-lived fillers write the zeros beside the K-loop tiles on the other CUs, where one
// 128 KB zero tile per workgroup took every CU in turn for each empty expert.
template <int NTH, bool OUT_F32>
__device__ __forceinline__ void wgrad_zero_fill(const WgradParams& p, char* smem, int f) {
  constexpr int ES = OUT_F32 ? 4 : 2;
  int* empty = reinterpret_cast<int*>(smem);  // [E] ranks -> expert ids
  int* tmp = empty + kGemmMaxE;
  const int ept = (p.E + NTH - 1) / NTH;  // experts per thread (E <= 1024, NTH = 512: <= 2)
  int flags = 0, cnt = 0;
  for (int q = 0; q < ept; ++q) {
    const int e = (int)threadIdx.x * ept + q;
    if (e < p.E) {
      const int64_t b = e ? p.offsets[e - 1] : 0;
      if (p.offsets[e] <= b) {
        flags |= 1 << q;
        ++cnt;
      }
    }
  }
  int n_empty;
  int rank = block_exclusive_scan<NTH>(cnt, tmp, &n_empty);
  for (int q = 0; q < ept; ++q)
    if (flags & (1 << q)) empty[rank++] = (int)threadIdx.x * ept + q;
  __syncthreads();
  if (n_empty == 0) return;
  const int64_t units_e = (int64_t)p.Ndy * p.Kx * ES / 16;  // 16-byte units per expert grad
  const int64_t total = units_e * n_empty;
  const int64_t u0 = total * f / p.fillers, u1 = total * (f + 1) / p.fillers;
  uint4* dw = reinterpret_cast<uint4*>(p.dw);
  const uint4 z = make_uint4(0, 0, 0, 0);
  for (int64_t u = u0; u < u1;) {
    const int k = (int)(u / units_e);
    const int64_t in = u - (int64_t)k * units_e;
    const int64_t run = min(units_e - in, u1 - u);
    uint4* dst = dw + (int64_t)empty[k] * units_e + in;
    for (int64_t i = threadIdx.x; i < run; i += NTH) dst[i] = z;
    u += run;
  }
}

// GATHER: 0 = x rows in sorted order; 1 = gathered, row = index >> shift; 2 = gathered,
// row = index / x_div. Both gathered forms keep the K loop free of branches. DYG: the
// gather applies to the DY rows instead (x rows then in sorted order).
template <int BM, int BN, int GATHER, bool OUT_F32 = false, int NW = 4, bool DYG = false, bool FEW = false>
__global__ __launch_bounds__(NW * 64) void wgrad_bf16_kernel(WgradParams p) {
  static_assert(!DYG || GATHER != 0, "a DY gather needs a gather mode");
  extern __shared__ __align__(16) char smem[];
  constexpr int KS = 64;
  using WG = WaveGrid<BM, BN, NW>;
  constexpr int WN = WG::WN;
  constexpr int MI = WG::MI, NI = WG::NI;
  constexpr int kStage = (BM + BN) * KS * 2;

  const int per_e = p.m_tiles * p.n_tiles;
  if constexpr (FEW) {
    if ((int)blockIdx.x < p.fillers) {
      wgrad_zero_fill<NW * 64, OUT_F32>(p, smem, (int)blockIdx.x);
      return;
    }
  }
  const int logical = slab_logical_tile(p.E * per_e, (int)blockIdx.x - (FEW ? p.fillers : 0));
  if (logical < 0) return;
  const int e = logical / per_e;
  const int rem = logical % per_e;
  int w_inner, w_outer;
  expert_tile_order(rem, p.n_major ? p.m_tiles : p.n_tiles, p.n_major ? p.n_tiles : p.m_tiles, w_inner, w_outer);
  const int mt = p.n_major ? w_inner : w_outer;
  const int nt = p.n_major ? w_outer : w_inner;
  const int64_t r_begin = e ? wgrad_rows_end(p, e - 1) : 0;
  const int64_t r_end = wgrad_rows_end(p, e);
  const int nrows = r_end > r_begin ? (int)(r_end - r_begin) : 0;
  if (nrows < p.rows_lo || nrows > p.rows_hi) return;  // the other launch of a split covers this expert
  const int m0 = mt * BM, n0 = nt * BN;
  if (nrows == 0) {
    if (!FEW || p.fillers == 0) wgrad_zero_tile<BM, BN, NW * 64, OUT_F32>(p, e, m0, n0);
    return;
  }
  if constexpr (FEW) {  // an expert of at most kFewRows rows: the write-bound form, no K loop
    if (nrows <= kFewRows) {
      wgrad_few_rows_tile<BM, BN, NW, GATHER, DYG, OUT_F32>(p, smem, e, r_begin, nrows, m0, n0);
      return;
    }
  }
  const int wu = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  lds_char* lds = (lds_char*)(smem);  // generic -> LDS address space
  const int nk = (nrows + KS - 1) / KS;

  using LA = KLoad<BM, NW>;
  using LB = KLoad<BN, NW>;
  constexpr int KR = LB::KR;  // k-rows (gathered x rows) per wave per stage
  LA la;
  LB lb;
  la.init(m0, p.Ndy, p.lddy * 2);
  lb.init(n0, p.Kx, p.ldx * 2);
  constexpr int LPS = LA::NQ + LB::NQ;
  const char* dy_base = reinterpret_cast<const char*>(p.dy);
  const char* x_base = reinterpret_cast<const char*>(p.x);

  // Gathered x rows: the wave's KR k-rows of a stage come as byte offsets in scalar
  // registers. Their indices are fetched one stage ahead with one vector load per wave
  // (lanes 0..KR-1, the low 32-bit words of the int64 entries) and moved to scalar
  // registers with v_readlane when the stage's loads are set up. A vector load counts
  // on vmcnt, which the K loop only waits on at its barrier; scalar loads would count on
  // lgkmcnt and stall every fragment-read wait until they returned. Rows past the
  // expert's end get kOOBRow, which stays out of range after adding any column offset.
  constexpr uint32_t kOOBRow = 0x7ffffff0u;
  const uint32_t* xr32 = reinterpret_cast<const uint32_t*>(p.x_rows);
  uint32_t src_off[KR];
  uint32_t pend = 0;  // this lane's index word for the next stage (lanes 0..KR-1 hold the wave's k-rows)
  const int64_t ldx2 = p.ldx * 2;
  const int64_t ldg2 = DYG ? p.lddy * 2 : ldx2;  // row pitch of the gathered operand
  auto issue_idx = [&](int kt) -> uint32_t {
    const int pos = kt * KS + KR * wu + (int)(threadIdx.x & (KR - 1));
    return xr32[2 * (r_begin + (pos < nrows ? pos : nrows - 1))];
  };
  // stage kt's indices (in pend) -> src_off, and the next stage's load issued; stages at or
  // past nk get kOOBRow everywhere and re-read the last valid index (no branch in the loop)
  auto fetch_src = [&](int kt) {
    const int base = kt * KS + KR * wu;
    uint32_t v[KR];  // gather indices are below 2^31 (R < 2^31)
#pragma unroll
    for (int j = 0; j < KR; ++j) v[j] = (uint32_t)__builtin_amdgcn_readlane((int)pend, j);
    pend = issue_idx(kt + 1);
    if constexpr (GATHER == 1) {
#pragma unroll
      for (int j = 0; j < KR; ++j) v[j] >>= p.x_div_shift;
    } else {
#pragma unroll
      for (int j = 0; j < KR; ++j) v[j] /= (uint32_t)p.x_div;
    }
    // row byte offsets fit in 32 bits: the gathered operand spans less than 2 GiB
#pragma unroll
    for (int j = 0; j < KR; ++j) src_off[j] = base + j < nrows ? v[j] * (uint32_t)ldg2 : kOOBRow;
  };
  // the gathered row offset of this lane's k-row for instruction qq of loader L: k-row
  // qq * RPI + sub() of the wave's KR; qq is a compile-time constant here (unrolled), so
  // the pick indexes the array with constants only (a select between array elements is
  // turned back into a dynamically indexed array, i.e. scratch memory; the masked XOR
  // keeps every index constant)
  auto pick = [&](auto* loader_tag, int qq) -> uint32_t {
    using L = typename std::remove_pointer<decltype(loader_tag)>::type;
    static_assert(L::RPI == 2 || L::RPI == 4, "two or four k-rows per load instruction");
    const int sub = L::sub();
    const uint32_t m1 = 0u - (uint32_t)(sub & 1);
    const uint32_t s0 = src_off[qq * L::RPI], s1 = src_off[qq * L::RPI + 1];
    uint32_t v = s0 ^ ((s0 ^ s1) & m1);
    if constexpr (L::RPI == 4) {
      const uint32_t s2 = src_off[qq * L::RPI + 2], s3 = src_off[qq * L::RPI + 3];
      const uint32_t hi = s2 ^ ((s2 ^ s3) & m1);
      v = v ^ ((v ^ hi) & (0u - (uint32_t)((sub >> 1) & 1)));
    }
    return v;
  };
  auto dma = [&](int q, int buf, int kt, bool on) {
    lds_char* sa = lds + buf * kStage;
    lds_char* sb = sa + BM * KS * 2;
    const int64_t k0 = (int64_t)kt * KS;
    if (q < LA::NQ) {
      if constexpr (DYG) {
        // kOOBRow + coff and v + kOOB both stay below 2^32 and at or above 2^31 - 16
        la.issue_at(q, make_rsrc(dy_base, on ? p.dy_bytes : 0u), sa, wu, pick((LA*)nullptr, q) + la.coff[q]);
      } else {
        const int64_t pitch = p.lddy * 2;
        la.issue(q, stage_rsrc(dy_base, p.dy_bytes, (r_begin + k0) * pitch, ((int64_t)nrows - k0) * pitch, on),
                 sa, wu);
      }
    } else if constexpr (GATHER != 0 && !DYG) {
      const int qq = q - LA::NQ;
      lb.issue_at(qq, make_rsrc(x_base, on ? p.x_bytes : 0u), sb, wu, pick((LB*)nullptr, qq) + lb.coff[qq]);
    } else {
      const int64_t pitch = ldx2;
      lb.issue(q - LA::NQ, stage_rsrc(x_base, p.x_bytes, (r_begin + k0) * pitch, ((int64_t)nrows - k0) * pitch, on),
               sb, wu);
    }
  };

  const int wave = threadIdx.x >> 6;
  const int wm0 = WG::wm0(wave), wn0 = WG::wn0(wave);
  // 8 waves run the 16 x 16 x 32 K loop, except with the DY gather (dW2), which measured 1-3%
  // slower on it at C3 and C4, and in the launch with the few-rows form inline (dW1 under
  // skewed routing: 2-4% slower at C4)
  constexpr bool M16 = NW == 8 && !DYG && !FEW;
  using Acc = typename std::conditional<M16, f32x4_t[4], f32x16_t>::type;
  Acc acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      if constexpr (M16) {
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[mi][ni][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[mi][ni][q] = 0.f;
      }
    }

  if constexpr (GATHER != 0) {
    if (nk > 0) pend = issue_idx(0);
  }
  auto prefetch = [&](int kt) {
    if constexpr (GATHER != 0) fetch_src(kt);
  };
  if constexpr (M16)
    kloop64_m16<LPS, MI, NI, true, true, BM, BN>(nk, lds, wm0, wn0, acc, dma, prefetch, [] {});
  else
    kloop64<LPS, MI, NI, true, true, BM, BN>(nk, lds, wm0, wn0, acc, dma, prefetch, [] {});
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // every wave is done with the stages
  char* st = smem + wave * 32 * MI * WaveStage<WN>::PITCH;
  if constexpr (OUT_F32)
    wgrad_epilogue_f32_staged(p, st, acc, e, m0, n0, wm0, wn0);
  else
    wgrad_epilogue_bf16(p, st, acc, e, m0, n0, wm0, wn0);
}

template <int GATHER, bool DYG, bool OUT_F32 = false>
__global__ __launch_bounds__(256, 2) void wgrad_few_rows_kernel(WgradParams p) {
  extern __shared__ __align__(16) char smem[];
  const int per_e = p.m_tiles * p.n_tiles;
  const int logical = slab_logical_tile(p.E * per_e);
  if (logical < 0) return;
  const int e = logical / per_e;
  const int rem = logical % per_e;
  const int mt = rem / p.n_tiles, nt = rem % p.n_tiles;
  const int64_t r_begin = e ? wgrad_rows_end(p, e - 1) : 0;
  const int64_t r_end = wgrad_rows_end(p, e);
  const int nrows = r_end > r_begin ? (int)(r_end - r_begin) : 0;
  if (nrows < p.rows_lo || nrows > p.rows_hi) return;  // another launch covers this expert
  wgrad_few_rows_tile<kFewBM, kFewBN, 4, GATHER, DYG, OUT_F32>(p, smem, e, r_begin, nrows, mt * kFewBM,
                                                               nt * kFewBN);
}

constexpr int few_rows_lds_bytes() {
  constexpr int operands = kFewRows * (kFewBM + kFewBN) * 2;
  constexpr int staging = 4 * WaveGrid<kFewBM, kFewBN, 4>::WM * WaveStage<WaveGrid<kFewBM, kFewBN, 4>::WN>::PITCH;
  return operands > staging ? operands : staging;
}

// ------------------------------------------------------------------ dense split-K weight grads
// The row range of an unsplit dense weight grad as a one-entry offsets array (for the
// grouped entry point it runs through).
__global__ void split_offsets_kernel(int64_t* __restrict__ off, int64_t M, int S) {
  const int s = threadIdx.x;
  if (s < S) off[s] = split_end(M, S, s);
}

// out[i] = sum over s of part[s][i] (fp32), rounded once to the output type.
template <typename T>
__global__ __launch_bounds__(256) void reduce_splits_kernel(const float* __restrict__ part, int S, int64_t n,
                                                            T* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  float4 a = *reinterpret_cast<const float4*>(part + i);
  for (int s2 = 1; s2 < S; ++s2) {
    const float4 b = *reinterpret_cast<const float4*>(part + (int64_t)s2 * n + i);
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
  }
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint2*>(out + i) = make_uint2(pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w));
  } else {
    *reinterpret_cast<float4*>(out + i) = a;
  }
}

// ------------------------------------------------------------------ host side
template <typename T, int BM, int BN>
constexpr int rows_lds_bytes() {
  constexpr int main_loop = 2 * (BM + BN) * kRowBytes;
  constexpr int staging = 4 * Stage<T, BM / 2, BN / 2>::BYTES;
  constexpr int decode = (kGemmMaxE + 4 + 8) * 4;
  constexpr int m = main_loop > staging ? main_loop : staging;
  return m > decode ? m : decode;
}

// bf16 kernels: two 64-deep operand stages (+ the rows kernel's output-row table);
// the epilogue works from registers.
template <int BM, int BN, int NW = 4>
constexpr int bf16_lds_bytes() {
  constexpr int main_loop = bf16_stage_bytes<BM, BN, NW>() + BM * 8;  // stages / staging + row and scale tables
  constexpr int decode = (kGemmMaxE + 4 + 16) * 4;
  return main_loop > decode ? main_loop : decode;
}

// One attribute call per kernel (keyed by the kernel's address: instantiations share a
// function type), under a lock, since callers may launch from several host threads.
template <typename K>
int prepare(K kernel, int lds_bytes) {
  static std::mutex mu;
  static std::unordered_set<const void*> done;
  const void* key = reinterpret_cast<const void*>(kernel);
  std::lock_guard<std::mutex> lock(mu);
  if (done.count(key)) return ZMOE_OK;
  hipError_t e = hipFuncSetAttribute(key, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes);
  if (e != hipSuccess) return set_error(ZMOE_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
  done.insert(key);
  return ZMOE_OK;
}

template <typename K>
int launch_rows_kernel(K kern, int lds, int BM, const RowsParams& p, int64_t R, hipStream_t s,
                       int threads = kGemmThreads) {
  int rc = prepare(kern, lds);
  if (rc) return rc;
  const int64_t mt_bound = cdiv(R, BM) + (R < p.E ? R : p.E);
  int64_t total = mt_bound * p.n_tiles;
  total = cdiv(total, (int64_t)kXcds * kSlab) * kXcds * kSlab;  // covers either mapping (decode_rows_tile)
  ZMOE_REQUIRE(total < (int64_t)0x7fffffff, ZMOE_ERR_SHAPE, "grouped gemm: too many tiles");
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(threads), lds, s, p);
  return check_launch("grouped rows kernel");
}

template <int BM, int BN, bool B_KN, int EPI>
int launch_rows_f32(const RowsParams& p, int64_t R, hipStream_t s) {
  return launch_rows_kernel(grouped_rows_kernel<float, BM, BN, B_KN, EPI>, rows_lds_bytes<float, BM, BN>(), BM, p,
                            R, s);
}

// 256 x 256 tiles run with 8 waves (two per SIMD: while one wave is held issuing its
// LDS-DMA loads, the other issues MFMAs), 128 x 128 tiles with 4. (16 waves measured
// slower: 64 x 64 per wave doubles the fragment reads per MFMA and leaves 128 registers
// per wave.)
constexpr int kBigWaves = 8;

template <int BM, int BN, bool B_KN, int EPI>
int launch_rows_bf16(const RowsParams& p, int64_t R, hipStream_t s) {
  constexpr int NW = BM == 256 ? kBigWaves : 4;
  return launch_rows_kernel(rows_bf16_kernel<BM, BN, B_KN, EPI, NW>, bf16_lds_bytes<BM, BN, NW>(), BM, p, R, s,
                            NW * 64);
}

template <typename K>
int launch_wgrad_kernel(K kern, int lds, int BM, int BN, WgradParams p, hipStream_t s, int threads = kGemmThreads) {
  int rc = prepare(kern, lds);
  if (rc) return rc;
  p.m_tiles = (int)cdiv(p.Ndy, BM);
  p.n_tiles = (int)cdiv(p.Kx, BN);
  // n-tiles outer (tiles sharing a gathered X block together) pays only while an XCD's 32
  // resident tiles span most of X's column blocks: dW1 at C3 (6 x 8 tiles per expert) 2%
  // faster, at C4 (16 x 28) 8% slower than m-tiles outer, which then keeps the gathered
  // rows' column blocks together in time
  if (p.m_tiles * p.n_tiles > 64) p.n_major = 0;
  int64_t total = (int64_t)p.E * p.m_tiles * p.n_tiles;
  const int slab = slab_size(total);
  total = cdiv(total, (int64_t)kXcds * slab) * kXcds * slab;  // whole slabs on every XCD (slab_logical_tile)
  total += p.fillers;  // a multiple of kXcds: the tiles keep their XCDs
  ZMOE_REQUIRE(total < (int64_t)0x7fffffff, ZMOE_ERR_SHAPE, "group_bwd_w: too many tiles");
  hipLaunchKernelGGL(kern, dim3((unsigned)total), dim3(threads), lds, s, p);
  return check_launch("grouped wgrad kernel");
}

template <int GATHER, bool OUT_F32, bool DYG = false, bool FEW = false>
int launch_wgrad_big(const WgradParams& p, hipStream_t s) {
  constexpr int NW = kBigWaves;
  return launch_wgrad_kernel(wgrad_bf16_kernel<256, 256, GATHER, OUT_F32, NW, DYG, FEW>,
                             bf16_lds_bytes<256, 256, NW>(), 256, 256, p, s, NW * 64);
}

// Large tiles when the average expert holds enough rows to fill them.
inline bool use_big_tiles(int64_t R, int E, int64_t N) { return R >= (int64_t)E * 256 && N >= 256; }

// Weight grads under a skewed routing (fewer than 1024 rows per expert on average): the
// experts holding at most kFewRows rows take the write-bound few-rows form. With X's rows
// gathered (dW1) it runs inside the 256 x 256 K-loop launch: one launch over every expert,
// each workgroup picking its form from its expert's row count (C4: dW1 6.27 -> 6.08 ms).
// With DY's rows gathered (dW2) it is a launch of its own (wgrad_few_rows_kernel, 128 x 256
// tiles, two workgroups per CU) before the K-loop launch, each launch covering every
// expert's tiles and the workgroups of the other launch's experts exiting at once: the
// inline form measured 10% slower there (3.13 -> 3.45 ms at C4).
// Zero fillers of the launch with the few-rows form inline (wgrad_zero_fill): C4's dW1
// 6.12-6.15 -> 6.02-6.03 ms with 32 (16: 6.28, the fill outlasts the tiles; 64: 6.05).
// A multiple of kXcds, so that every tile keeps its XCD.
constexpr int kZeroFillers = 32;
inline int wgrad_small_rows(int64_t R, int E) { return R < (int64_t)E * 1024 ? kFewRows : 0; }

// ==================================================================== small-M streaming path
// Forward rows GEMMs when the experts hold few rows (the small-batch regime, e.g. a
// decode step): the weights are then the only large operand and the GEMM is bound by
// streaming them from HBM. Each wave owns 32 weight rows (16 SwiGLU pairs: their h and
// gate rows) and streams them from HBM straight into MFMA operand registers (no LDS, no
// barriers), kStreamDepth 64-deep stages ahead, multiplying them with up to 32 of the
// expert's rows per pass, which come from L2. v_mfma_f32_32x32x16_bf16 takes the weight
// fragment as its first operand, so lane (r, g) ends up with 4 consecutive output
// columns (weight rows 8 q + 4 g .. + 3) of expert row r.
// Measured at d = 2048, E = 128, k = 8 (W1 with SwiGLU + W2): 219 vs 237 us for the tiled
// kernels at T = 32, even at T = 128, slower from T = 256 on; depths 2, 3 and 4 time the same.
constexpr int kStreamDepth = 2;
constexpr int kStreamRowsPerExpert = 8;  // dispatch bound on R / E

template <int EPI>
__global__ __launch_bounds__(256) void stream_rows_kernel(RowsParams p, int wtiles_per_e) {
  const int lane = (int)(threadIdx.x & 63);
  const int wpe = (wtiles_per_e + 3) / 4;  // workgroups per expert
  const int e = (int)blockIdx.x / wpe;
  const int wt = ((int)blockIdx.x % wpe) * 4 + (int)(threadIdx.x >> 6);
  if (e >= p.E || wt >= wtiles_per_e) return;  // (waves are independent: no barriers)
  const int64_t e_begin = e ? p.offsets[e - 1] : 0;
  const int64_t count = p.offsets[e] - e_begin;
  if (count <= 0) return;
  const int r = lane & 31, g = lane >> 5;
  int n;
  bool nok;
  if constexpr (EPI == EPI_SWIGLU) {
    const int jj = wt * 16 + (r & 15);
    nok = jj < p.half;
    n = (r & 16) ? p.half + jj : jj;
  } else {
    n = wt * 32 + r;
    nok = n < p.N;
  }
  const char* b_base = reinterpret_cast<const char*>(reinterpret_cast<const uint16_t*>(p.b) + (int64_t)e * p.b_estride);
  const __amdgpu_buffer_rsrc_t brs = make_rsrc(b_base, p.b_bytes);
  const __amdgpu_buffer_rsrc_t ars = make_rsrc(p.a, p.a_bytes);
  // offsets of this lane's 16 bytes at k = 0 (kOOB: reads zero); + 128 per 64-deep stage, + 32 per step
  const uint32_t boff = nok ? (uint32_t)((int64_t)n * p.ldb * 2) + 16u * (uint32_t)g : kOOB;
  const int nkc = p.K / 64;
  uint16_t* C = reinterpret_cast<uint16_t*>(p.c);
  for (int64_t mb = 0; mb < count; mb += 32) {
    uint32_t aoff = kOOB;
    if (mb + r < count) {
      int64_t src = e_begin + mb + r;
      if (p.a_rows != nullptr) src = reinterpret_cast<const int*>(p.a_rows)[2 * src] / p.a_div;
      aoff = (uint32_t)(src * p.lda * 2) + 16u * (uint32_t)g;
    }
    f32x16_t acc;
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.f;
    v4i32_t wf[kStreamDepth][4], xf[kStreamDepth][4];
    auto load = [&](int buf, int kc) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t ko = (uint32_t)kc * 128u + 32u * (uint32_t)s;
        wf[buf][s] = __builtin_bit_cast(v4i32_t, __builtin_amdgcn_raw_buffer_load_b128(brs, boff + ko, 0, 0));
        xf[buf][s] = __builtin_bit_cast(v4i32_t, __builtin_amdgcn_raw_buffer_load_b128(ars, aoff + ko, 0, 0));
      }
    };
#pragma unroll
    for (int u = 0; u < kStreamDepth; ++u)
      if (u < nkc) load(u, u);
    for (int kc = 0; kc < nkc; kc += kStreamDepth) {
#pragma unroll
      for (int u = 0; u < kStreamDepth; ++u) {
        if (kc + u < nkc) {
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, wf[u][s]),
                                                          __builtin_bit_cast(bf16x8_t, xf[u][s]), acc, 0, 0, 0);
          if (kc + u + kStreamDepth < nkc) load(u, kc + u + kStreamDepth);
        }
      }
    }
    if (mb + r >= count) continue;
    const int64_t i = e_begin + mb + r;  // sorted row
    const int64_t o = p.c_rows ? reinterpret_cast<const int*>(p.c_rows)[2 * i] : i;
    if constexpr (EPI == EPI_SWIGLU) {
      // acc[4 q + u]: h of pair wt 16 + 8 q + 4 g + u for q = 0, 1; its gate at q + 2
      uint16_t* A2 = reinterpret_cast<uint16_t*>(p.c2);
      const float rs = p.row_scale != nullptr ? p.row_scale[i] : 1.f;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int pr = wt * 16 + 8 * q + 4 * g;
        if (pr >= p.half) continue;
        float h[4], gt[4], a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          h[u] = to_f32(bf16_bits(acc[4 * q + u]));
          gt[u] = to_f32(bf16_bits(acc[4 * (q + 2) + u]));
          a[u] = rs * (silu_f(gt[u]) * h[u]);
        }
        *reinterpret_cast<uint2*>(C + o * p.ldc + pr) = pack4_bf16(h);
        *reinterpret_cast<uint2*>(C + o * p.ldc + p.half + pr) = pack4_bf16(gt);
        *reinterpret_cast<uint2*>(A2 + o * p.ldc2 + pr) = pack4_bf16(a);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c0 = wt * 32 + 8 * q + 4 * g;
        if (c0 >= p.N) continue;
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = acc[4 * q + u];
        *reinterpret_cast<uint2*>(C + o * p.ldc + c0) = pack4_bf16(v);
      }
    }
  }
}

template <int EPI>
int launch_stream_rows(const RowsParams& p, hipStream_t s) {
  const int wtiles = EPI == EPI_SWIGLU ? (int)cdiv(p.half, 16) : (int)cdiv(p.N, 32);
  const int64_t blocks = (int64_t)p.E * cdiv(wtiles, 4);
  ZMOE_REQUIRE(blocks < (int64_t)0x7fffffff, ZMOE_ERR_SHAPE, "grouped gemm: too many tiles");
  hipLaunchKernelGGL(stream_rows_kernel<EPI>, dim3((unsigned)blocks), dim3(256), 0, s, p, wtiles);
  return check_launch("grouped rows streaming kernel");
}

template <bool B_KN, int EPI>
int dispatch_rows(int dtype, RowsParams p, int64_t R, int bn_for_tiles_div, hipStream_t s) {
  // n_tiles: along N (or along pair columns for SwiGLU, BN/2 pairs per tile)
  if (dtype == ZMOE_DTYPE_BF16) {
    if constexpr (!B_KN && (EPI == EPI_STORE || EPI == EPI_SWIGLU)) {
      // few rows per expert: stream the weights (the K loop takes whole 64-deep stages)
      if (R <= (int64_t)kStreamRowsPerExpert * p.E && p.K % 64 == 0) return launch_stream_rows<EPI>(p, s);
    }
    // tile order within an expert: the tiles that share the gathered operand run
    // together. With A rows gathered (W1 forward, dA) the m-tiles are outer; with A
    // contiguous the n-tiles are, so the tiles sharing B columns run together (measured
    // at C3: W2 forward 3%, W1 input grad 2% faster; n-major W1 forward 1% slower)
    p.n_major = p.a_rows == nullptr ? 1 : 0;
    if (use_big_tiles(R, p.E, p.N)) {
      p.n_tiles = (int)cdiv(bn_for_tiles_div, EPI == EPI_SWIGLU ? 128 : 256);
      return launch_rows_bf16<256, 256, B_KN, EPI>(p, R, s);
    }
    p.n_tiles = (int)cdiv(bn_for_tiles_div, EPI == EPI_SWIGLU ? 64 : 128);
    return launch_rows_bf16<128, 128, B_KN, EPI>(p, R, s);
  }
  p.n_tiles = (int)cdiv(bn_for_tiles_div, EPI == EPI_SWIGLU ? 64 : 128);
  return launch_rows_f32<128, 128, B_KN, EPI>(p, R, s);
}

int ns_gemm(const NsGemm& g, hipStream_t s) {
  ZMOE_REQUIRE(g.E >= 1 && g.E <= kGemmMaxE && g.K >= 8 && g.N >= 8 && g.K % 8 == 0 && g.N % 8 == 0 &&
                   g.R >= 0 && g.R < 0x7fffffffLL,
               ZMOE_ERR_SHAPE, "ns_gemm: bad sizes");
  if (g.R == 0) return ZMOE_OK;
  RowsParams p{};
  p.a = g.A;
  p.lda = g.lda;
  p.b = g.B;
  p.b_estride = g.b_estride;
  p.ldb = g.ldb;
  p.c = g.C;
  p.ldc = g.ldc;
  p.c2 = g.C2;
  p.ldc2 = g.ldc2;
  p.aux = g.D;
  p.ld_aux = g.ldd;
  p.ns_beta = g.beta;
  p.ns_gamma = g.gamma;
  p.ns_sym_m = g.sym_m;
  p.offsets = g.offsets;
  p.K = g.K;
  p.N = g.N;
  p.E = g.E;
  const int64_t a_span = ((g.R - 1) * g.lda + g.K) * 2;
  const int64_t b_span = g.b_kn ? ((int64_t)(g.K - 1) * g.ldb + g.N) * 2 : ((int64_t)(g.N - 1) * g.ldb + g.K) * 2;
  ZMOE_REQUIRE(a_span <= 0x7fff0000LL && b_span <= 0x7fff0000LL, ZMOE_ERR_SHAPE, "ns_gemm: operand spans 2 GiB");
  p.a_bytes = (uint32_t)a_span;
  p.b_bytes = (uint32_t)b_span;
  if (use_big_tiles(g.R, g.E, g.N)) {
    p.n_tiles = (int)cdiv(g.N, 256);
    return g.b_kn ? launch_rows_bf16<256, 256, true, EPI_NS>(p, g.R, s)
                  : launch_rows_bf16<256, 256, false, EPI_NS>(p, g.R, s);
  }
  p.n_tiles = (int)cdiv(g.N, 128);
  return g.b_kn ? launch_rows_bf16<128, 128, true, EPI_NS>(p, g.R, s)
                : launch_rows_bf16<128, 128, false, EPI_NS>(p, g.R, s);
}

}  // namespace zmoe

using namespace zmoe;

namespace {

int vec_elems(int dtype) { return dtype == ZMOE_DTYPE_BF16 ? 8 : 4; }

// Bytes addressable from a matrix base: (rows - 1) * ld + cols elements.
int64_t span_bytes(int64_t rows, int64_t ld, int64_t cols, int dtype) {
  return rows <= 0 ? 0 : ((rows - 1) * ld + cols) * dtype_size(dtype);
}
// Buffer-resource ranges: every valid offset stays below this, and the out-of-range
// markers (kOOB = 2^31, gathered-row marker 2^31 - 16, plus column offsets) stay above it.
constexpr int64_t kMaxSpan = 0x7fff0000LL;
// Row counts and row indices travel as 32-bit values inside the kernels.
constexpr int64_t kMaxRows = 0x7fffffffLL;
bool ok_rows(int dtype, const void* ptr, int64_t ld) {
  return aligned16(ptr) && (ld % vec_elems(dtype)) == 0;
}

}  // namespace

extern "C" int zmoe_scatter2scatter(const void* X, int64_t x_stride_m, const void* W, int64_t w_stride_e,
                                    int64_t w_stride_k, int64_t w_stride_n, const void* b, int64_t b_stride_e,
                                    const int64_t* sorted_expert_idxs, const int64_t* sorted_scattered_idxs,
                                    const int64_t* expert_offsets, int64_t M, int64_t K, int64_t N, int E, int k,
                                    int x_grouped, int y_grouped, int dtype, void* Y, int64_t y_stride_m,
                                    void* stream) {
  (void)sorted_expert_idxs;  // rows are assigned to experts through expert_offsets
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "scatter2scatter: dtype %d", dtype);
  ZMOE_REQUIRE(M >= 0 && K >= 1 && N >= 1 && E >= 1 && E <= kGemmMaxE && k >= 1, ZMOE_ERR_SHAPE,
               "scatter2scatter: bad sizes (M=%lld K=%lld N=%lld E=%d k=%d)", (long long)M, (long long)K,
               (long long)N, E, k);
  ZMOE_REQUIRE(K < (1 << 30) && N < (1 << 30), ZMOE_ERR_SHAPE, "scatter2scatter: K/N too large");
  ZMOE_REQUIRE(M < kMaxRows && M * k < kMaxRows, ZMOE_ERR_SHAPE, "scatter2scatter: M*k must be below 2^31");
  const int64_t R = x_grouped ? M : M * k;
  if (R == 0) return ZMOE_OK;
  ZMOE_REQUIRE(X && W && Y && expert_offsets, ZMOE_ERR_NULL, "scatter2scatter: null pointer");
  ZMOE_REQUIRE((x_grouped && y_grouped) || sorted_scattered_idxs, ZMOE_ERR_NULL,
               "scatter2scatter: sorted_scattered_idxs required unless x_grouped and y_grouped");
  const int v = vec_elems(dtype);
  ZMOE_REQUIRE(K % v == 0 && N % v == 0 && ok_rows(dtype, X, x_stride_m) && ok_rows(dtype, Y, y_stride_m) &&
                   aligned16(W) && w_stride_e % v == 0,
               ZMOE_ERR_ALIGN, "scatter2scatter: K, N and strides must be multiples of %d elements", v);
  RowsParams p{};
  p.a = X;
  p.lda = x_stride_m;
  p.a_rows = x_grouped ? nullptr : sorted_scattered_idxs;
  p.a_div = k;
  p.b = W;
  p.b_estride = w_stride_e;
  p.c = Y;
  p.ldc = y_stride_m;
  p.c_rows = y_grouped ? nullptr : sorted_scattered_idxs;
  p.bias = b;
  p.bias_estride = b_stride_e;
  p.offsets = expert_offsets;
  p.K = (int)K;
  p.N = (int)N;
  p.E = E;
  const int64_t a_span = span_bytes(M, x_stride_m, K, dtype);
  ZMOE_REQUIRE(a_span <= kMaxSpan, ZMOE_ERR_SHAPE, "scatter2scatter: X spans more than 2 GiB");
  p.a_bytes = (uint32_t)a_span;
  hipStream_t s = as_stream(stream);
  if (w_stride_k == 1) {  // W[e] stored [N][K]
    ZMOE_REQUIRE(w_stride_n % v == 0, ZMOE_ERR_ALIGN, "scatter2scatter: weight row stride");
    p.ldb = w_stride_n;
    const int64_t b_span = span_bytes(N, w_stride_n, K, dtype);
    ZMOE_REQUIRE(b_span <= kMaxSpan, ZMOE_ERR_SHAPE, "scatter2scatter: one expert's W spans more than 2 GiB");
    p.b_bytes = (uint32_t)b_span;
    return b ? dispatch_rows<false, EPI_STORE_BIAS>(dtype, p, R, (int)N, s)
             : dispatch_rows<false, EPI_STORE>(dtype, p, R, (int)N, s);
  }
  ZMOE_REQUIRE(w_stride_n == 1, ZMOE_ERR_SHAPE, "scatter2scatter: W needs unit stride along K or N");
  ZMOE_REQUIRE(w_stride_k % v == 0, ZMOE_ERR_ALIGN, "scatter2scatter: weight row stride");
  p.ldb = w_stride_k;
  const int64_t b_span = span_bytes(K, w_stride_k, N, dtype);
  ZMOE_REQUIRE(b_span <= kMaxSpan, ZMOE_ERR_SHAPE, "scatter2scatter: one expert's W spans more than 2 GiB");
  p.b_bytes = (uint32_t)b_span;
  return b ? dispatch_rows<true, EPI_STORE_BIAS>(dtype, p, R, (int)N, s)
           : dispatch_rows<true, EPI_STORE>(dtype, p, R, (int)N, s);
}

namespace {
int glu_w1_forward_impl(const void* X, int64_t x_stride_m, const void* W1, const int64_t* sorted_scattered_idxs,
                        const int64_t* expert_offsets, int64_t T, int64_t d, int64_t f, int E, int k, int dtype,
                        const float* row_scale, void* H, void* A, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "glu_w1_forward: dtype %d", dtype);
  ZMOE_REQUIRE(T >= 0 && d >= 1 && f >= 1 && E >= 1 && E <= kGemmMaxE && k >= 1, ZMOE_ERR_SHAPE,
               "glu_w1_forward: bad sizes");
  ZMOE_REQUIRE(d < (1 << 30) && f < (1 << 29), ZMOE_ERR_SHAPE, "glu_w1_forward: d/f too large");
  ZMOE_REQUIRE(T < kMaxRows && T * k < kMaxRows, ZMOE_ERR_SHAPE, "glu_w1_forward: T*k must be below 2^31");
  const int64_t R = T * k;
  if (R == 0) return ZMOE_OK;
  ZMOE_REQUIRE(X && W1 && H && A && sorted_scattered_idxs && expert_offsets, ZMOE_ERR_NULL,
               "glu_w1_forward: null pointer");
  const int v = vec_elems(dtype);
  ZMOE_REQUIRE(d % v == 0 && f % v == 0 && ok_rows(dtype, X, x_stride_m) && aligned16(W1) && aligned16(H) &&
                   aligned16(A),
               ZMOE_ERR_ALIGN, "glu_w1_forward: d and f must be multiples of %d elements", v);
  RowsParams p{};
  p.a = X;
  p.lda = x_stride_m;
  p.a_rows = sorted_scattered_idxs;
  p.a_div = k;
  p.b = W1;
  p.b_estride = 2 * f * d;
  p.ldb = d;
  p.c = H;
  p.ldc = 2 * f;
  p.c2 = A;
  p.ldc2 = f;
  p.offsets = expert_offsets;
  p.K = (int)d;
  p.N = (int)(2 * f);
  p.E = E;
  p.half = (int)f;
  const int64_t a_span = span_bytes(T, x_stride_m, d, dtype), b_span = span_bytes(2 * f, d, d, dtype);
  ZMOE_REQUIRE(a_span <= kMaxSpan && b_span <= kMaxSpan, ZMOE_ERR_SHAPE,
               "glu_w1_forward: X or one expert's W1 spans more than 2 GiB");
  p.a_bytes = (uint32_t)a_span;
  p.b_bytes = (uint32_t)b_span;
  p.row_scale = row_scale;
  return dispatch_rows<false, EPI_SWIGLU>(dtype, p, R, (int)f, as_stream(stream));
}
}  // namespace

extern "C" int zmoe_glu_w1_forward(const void* X, int64_t x_stride_m, const void* W1,
                                   const int64_t* sorted_expert_idxs, const int64_t* sorted_scattered_idxs,
                                   const int64_t* expert_offsets, int64_t T, int64_t d, int64_t f, int E, int k,
                                   int dtype, void* H, void* A, void* stream) {
  (void)sorted_expert_idxs;
  return glu_w1_forward_impl(X, x_stride_m, W1, sorted_scattered_idxs, expert_offsets, T, d, f, E, k, dtype, nullptr,
                             H, A, stream);
}

extern "C" int zmoe_glu_w1_forward_scaled(const void* X, int64_t x_stride_m, const void* W1,
                                          const int64_t* sorted_expert_idxs, const int64_t* sorted_scattered_idxs,
                                          const int64_t* expert_offsets, int64_t T, int64_t d, int64_t f, int E,
                                          int k, int dtype, const float* row_scale, void* H, void* A,
                                          void* stream) {
  (void)sorted_expert_idxs;
  ZMOE_REQUIRE(dtype == ZMOE_DTYPE_BF16, ZMOE_ERR_DTYPE, "glu_w1_forward_scaled: bf16 only (dtype %d)", dtype);
  ZMOE_REQUIRE(T <= 0 || k <= 0 || row_scale != nullptr, ZMOE_ERR_NULL, "glu_w1_forward_scaled: null row_scale");
  return glu_w1_forward_impl(X, x_stride_m, W1, sorted_scattered_idxs, expert_offsets, T, d, f, E, k, dtype,
                             row_scale, H, A, stream);
}

extern "C" int zmoe_glu_w2_backward_dh(const void* dYg, const void* W2, const void* H,
                                       const int64_t* sorted_expert_idxs, const int64_t* expert_offsets, int64_t R,
                                       int64_t d, int64_t f, int E, int dtype, void* dH, void* stream) {
  (void)sorted_expert_idxs;
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "glu_w2_backward_dh: dtype %d", dtype);
  ZMOE_REQUIRE(R >= 0 && d >= 1 && f >= 1 && E >= 1 && E <= kGemmMaxE, ZMOE_ERR_SHAPE,
               "glu_w2_backward_dh: bad sizes");
  ZMOE_REQUIRE(d < (1 << 30) && f < (1 << 29), ZMOE_ERR_SHAPE, "glu_w2_backward_dh: d/f too large");
  ZMOE_REQUIRE(R < kMaxRows, ZMOE_ERR_SHAPE, "glu_w2_backward_dh: R must be below 2^31");
  if (R == 0) return ZMOE_OK;
  ZMOE_REQUIRE(dYg && W2 && H && dH && expert_offsets, ZMOE_ERR_NULL, "glu_w2_backward_dh: null pointer");
  const int v = vec_elems(dtype);
  ZMOE_REQUIRE(d % v == 0 && f % v == 0 && aligned16(dYg) && aligned16(W2) && aligned16(H) && aligned16(dH),
               ZMOE_ERR_ALIGN, "glu_w2_backward_dh: d and f must be multiples of %d elements", v);
  RowsParams p{};
  p.a = dYg;
  p.lda = d;
  p.a_rows = nullptr;
  p.a_div = 1;
  p.b = W2;  // logical B[kk in d][n in f] = W2[e][kk][n]
  p.b_estride = d * f;
  p.ldb = f;
  p.c = dH;
  p.ldc = 2 * f;
  p.aux = H;
  p.ld_aux = 2 * f;
  p.offsets = expert_offsets;
  p.K = (int)d;
  p.N = (int)f;
  p.E = E;
  p.half = (int)f;
  const int64_t a_span = span_bytes(R, d, d, dtype), b_span = span_bytes(d, f, f, dtype);
  ZMOE_REQUIRE(a_span <= kMaxSpan && b_span <= kMaxSpan, ZMOE_ERR_SHAPE,
               "glu_w2_backward_dh: dYg or one expert's W2 spans more than 2 GiB");
  p.a_bytes = (uint32_t)a_span;
  p.b_bytes = (uint32_t)b_span;
  return dispatch_rows<true, EPI_SWIGLU_BWD>(dtype, p, R, (int)f, as_stream(stream));
}

namespace zmoe {
// gates [R] in slot order -> sorted order (the row scales of the dA GEMM)
__global__ __launch_bounds__(256) void gather_gates_kernel(const float* __restrict__ gates,
                                                           const int64_t* __restrict__ ss, int64_t R,
                                                           float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < R) out[i] = gates[ss[i]];
}
// d_gates[ss[i]] = sum of row i's partial dot products, in column-block order
__global__ __launch_bounds__(256) void gate_dots_kernel(const float* __restrict__ dots, int P,
                                                        const int64_t* __restrict__ ss, int64_t R,
                                                        float* __restrict__ d_gates) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= R) return;
  float s = 0.f;
  for (int q = 0; q < P; ++q) s += dots[i * P + q];
  d_gates[ss[i]] = s;
}
}  // namespace zmoe

extern "C" size_t zmoe_glu_w2_backward_dh_gates_workspace_bytes(int64_t R, int64_t f) {
  if (R < 0 || f < 1) return 0;
  return (size_t)align_up(R * 4, 256) + (size_t)align_up(R * cdiv(f, 64) * 4, 256);
}

extern "C" int zmoe_glu_w2_backward_dh_gates(const void* dout, int64_t T, int k, const void* W2, const void* H,
                                             const int64_t* sorted_expert_idxs,
                                             const int64_t* sorted_scattered_idxs, const int64_t* expert_offsets,
                                             const float* gates, int64_t d, int64_t f, int E, int dtype, void* dH,
                                             float* d_gates, void* workspace, size_t workspace_bytes,
                                             void* stream) {
  (void)sorted_expert_idxs;
  ZMOE_REQUIRE(dtype == ZMOE_DTYPE_BF16, ZMOE_ERR_DTYPE, "glu_w2_backward_dh_gates: bf16 only (dtype %d)", dtype);
  ZMOE_REQUIRE(T >= 0 && T < kMaxRows && k >= 1 && d >= 1 && f >= 1 && E >= 1 && E <= kGemmMaxE, ZMOE_ERR_SHAPE,
               "glu_w2_backward_dh_gates: bad sizes");
  ZMOE_REQUIRE(d < (1 << 30) && f < (1 << 29), ZMOE_ERR_SHAPE, "glu_w2_backward_dh_gates: d/f too large");
  const int64_t R = T * k;
  ZMOE_REQUIRE(R < kMaxRows, ZMOE_ERR_SHAPE, "glu_w2_backward_dh_gates: T * k must be below 2^31");
  if (R == 0) return ZMOE_OK;
  ZMOE_REQUIRE(dout && W2 && H && dH && sorted_scattered_idxs && expert_offsets && gates && d_gates && workspace,
               ZMOE_ERR_NULL, "glu_w2_backward_dh_gates: null pointer");
  ZMOE_REQUIRE(workspace_bytes >= zmoe_glu_w2_backward_dh_gates_workspace_bytes(R, f), ZMOE_ERR_WORKSPACE,
               "glu_w2_backward_dh_gates: workspace too small");
  const int v = vec_elems(dtype);
  ZMOE_REQUIRE(d % v == 0 && f % v == 0 && aligned16(dout) && aligned16(W2) && aligned16(H) && aligned16(dH) &&
                   aligned16(workspace),
               ZMOE_ERR_ALIGN, "glu_w2_backward_dh_gates: d and f must be multiples of %d elements", v);
  float* scale = reinterpret_cast<float*>(workspace);
  float* dots = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + align_up(R * 4, 256));
  const int P = (int)cdiv(f, 64);
  RowsParams p{};
  p.a = dout;  // sorted row i reads token ss[i] / k
  p.lda = d;
  p.a_rows = sorted_scattered_idxs;
  p.a_div = k;
  p.b = W2;
  p.b_estride = d * f;
  p.ldb = f;
  p.c = dH;
  p.ldc = 2 * f;
  p.aux = H;
  p.ld_aux = 2 * f;
  p.offsets = expert_offsets;
  p.K = (int)d;
  p.N = (int)f;
  p.E = E;
  p.half = (int)f;
  p.row_scale = scale;
  p.row_dots = dots;
  p.dots_ld = P;
  const int64_t a_span = span_bytes(T, d, d, dtype), b_span = span_bytes(d, f, f, dtype);
  ZMOE_REQUIRE(a_span <= kMaxSpan && b_span <= kMaxSpan, ZMOE_ERR_SHAPE,
               "glu_w2_backward_dh_gates: dout or one expert's W2 spans more than 2 GiB");
  p.a_bytes = (uint32_t)a_span;
  p.b_bytes = (uint32_t)b_span;
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)cdiv(R, 256)), block(256);
  hipLaunchKernelGGL(gather_gates_kernel, grid, block, 0, s, gates, sorted_scattered_idxs, R, scale);
  int rc = check_launch("glu_w2_backward_dh_gates: gather");
  if (rc) return rc;
  rc = dispatch_rows<true, EPI_SWIGLU_BWD>(dtype, p, R, (int)f, s);
  if (rc) return rc;
  hipLaunchKernelGGL(gate_dots_kernel, grid, block, 0, s, dots, P, sorted_scattered_idxs, R, d_gates);
  return check_launch("glu_w2_backward_dh_gates: gate sums");
}

namespace {
// bf16 weight grads: 256 x 256 tiles when the experts are large enough, 128 x 128 otherwise,
// and the small experts split off under a skewed routing. DYG: the gather is on DY's rows.
template <bool DYG, bool OUT_F32 = false>
int group_bwd_w_bf16(WgradParams p, int64_t M, int E, int64_t N, int64_t K, hipStream_t s) {
  const bool big = use_big_tiles(M, E, N) && K >= 256;
  const int gather = p.x_rows ? (p.x_div_shift >= 0 ? 1 : 2) : 0;
  if (DYG && gather == 0) return zmoe::set_error(ZMOE_ERR_NULL, "group_bwd_w: the DY gather needs indices");
  auto small_tiles = [&](const WgradParams& q) -> int {
    if (gather == 1)
      return launch_wgrad_kernel(wgrad_bf16_kernel<128, 128, 1, OUT_F32, 4, DYG>, bf16_lds_bytes<128, 128>(), 128,
                                 128, q, s);
    if (gather == 2)
      return launch_wgrad_kernel(wgrad_bf16_kernel<128, 128, 2, OUT_F32, 4, DYG>, bf16_lds_bytes<128, 128>(), 128,
                                 128, q, s);
    if constexpr (!DYG)
      return launch_wgrad_kernel(wgrad_bf16_kernel<128, 128, 0, OUT_F32>, bf16_lds_bytes<128, 128>(), 128, 128, q, s);
    return (int)ZMOE_ERR_NULL;  // not reached (checked above)
  };
  auto few_rows_tiles = [&](const WgradParams& q) -> int {
    if (gather == 1)
      return launch_wgrad_kernel(wgrad_few_rows_kernel<1, DYG, OUT_F32>, few_rows_lds_bytes(), kFewBM, kFewBN, q, s,
                                 256);
    if (gather == 2)
      return launch_wgrad_kernel(wgrad_few_rows_kernel<2, DYG, OUT_F32>, few_rows_lds_bytes(), kFewBM, kFewBN, q, s,
                                 256);
    if constexpr (!DYG)
      return launch_wgrad_kernel(wgrad_few_rows_kernel<0, false, OUT_F32>, few_rows_lds_bytes(), kFewBM, kFewBN, q,
                                 s, 256);
    return (int)ZMOE_ERR_NULL;  // not reached (checked above)
  };
  const int split = big ? wgrad_small_rows(M, E) : 0;
  if constexpr (!DYG) {
    if (split > 0) {  // one launch: each workgroup picks its form; the first ones fill the empty experts' zeros
      p.fillers = kZeroFillers;
      if (gather == 1) return launch_wgrad_big<1, OUT_F32, false, true>(p, s);
      if (gather == 2) return launch_wgrad_big<2, OUT_F32, false, true>(p, s);
      return launch_wgrad_big<0, OUT_F32, false, true>(p, s);
    }
  }
  int rc = 0;
  if (split > 0) {  // experts of at most `split` rows on the write-bound kernel, the rest below
    WgradParams q = p;
    q.rows_hi = split;
    rc = few_rows_tiles(q);
    p.rows_lo = split + 1;
  }
  if (rc) return rc;
  if (!big) return small_tiles(p);
  if (gather == 1) return launch_wgrad_big<1, OUT_F32, DYG>(p, s);
  if (gather == 2) return launch_wgrad_big<2, OUT_F32, DYG>(p, s);
  if constexpr (!DYG) return launch_wgrad_big<0, OUT_F32>(p, s);
  return (int)ZMOE_ERR_NULL;  // not reached
}

// bf16 operands, bf16 or fp32 output (fp32 straight from the accumulators: the grads of
// fp32 master weights under bf16 autocast)
template <bool DYG>
int group_bwd_w_bf16_out(WgradParams p, int64_t M, int E, int64_t N, int64_t K, int out_dtype, hipStream_t s) {
  return out_dtype == ZMOE_DTYPE_F32 ? group_bwd_w_bf16<DYG, true>(p, M, E, N, K, s)
                                     : group_bwd_w_bf16<DYG, false>(p, M, E, N, K, s);
}
}  // namespace

extern "C" int zmoe_group_bwd_w_gather_dy(const void* DY, int64_t dy_stride_m, const int64_t* dy_gather_idxs,
                                          int dy_gather_div, const void* X, int64_t x_stride_m,
                                          const int64_t* expert_offsets, int64_t M, int64_t N, int64_t K, int E,
                                          int dtype, int out_dtype, void* DWt, void* stream) {
  ZMOE_REQUIRE(dtype == ZMOE_DTYPE_BF16, ZMOE_ERR_DTYPE, "group_bwd_w_gather_dy: bf16 only (dtype %d)", dtype);
  ZMOE_REQUIRE(out_dtype == ZMOE_DTYPE_BF16 || out_dtype == ZMOE_DTYPE_F32, ZMOE_ERR_DTYPE,
               "group_bwd_w_gather_dy: out_dtype %d", out_dtype);
  ZMOE_REQUIRE(M >= 0 && N >= 1 && K >= 1 && E >= 1 && E <= kGemmMaxE && dy_gather_div >= 1, ZMOE_ERR_SHAPE,
               "group_bwd_w_gather_dy: bad sizes");
  ZMOE_REQUIRE(N < (1 << 30) && K < (1 << 30), ZMOE_ERR_SHAPE, "group_bwd_w_gather_dy: N/K too large");
  ZMOE_REQUIRE(M < kMaxRows, ZMOE_ERR_SHAPE, "group_bwd_w_gather_dy: M must be below 2^31");
  ZMOE_REQUIRE(DWt && expert_offsets, ZMOE_ERR_NULL, "group_bwd_w_gather_dy: null pointer");
  ZMOE_REQUIRE(M == 0 || (DY && X && dy_gather_idxs), ZMOE_ERR_NULL, "group_bwd_w_gather_dy: null operand");
  const int v = vec_elems(dtype);
  ZMOE_REQUIRE(N % v == 0 && K % v == 0 && aligned16(DWt) && (M == 0 || (ok_rows(dtype, DY, dy_stride_m) &&
                                                                          ok_rows(dtype, X, x_stride_m))),
               ZMOE_ERR_ALIGN, "group_bwd_w_gather_dy: N, K and strides must be multiples of %d elements", v);
  WgradParams p{};
  p.dy = DY;
  p.lddy = dy_stride_m;
  p.x = X;
  p.ldx = x_stride_m;
  p.x_rows = dy_gather_idxs;
  p.x_div = dy_gather_div;
  p.x_div_shift = (dy_gather_div & (dy_gather_div - 1)) == 0 ? __builtin_ctz(dy_gather_div) : -1;
  p.dw = DWt;
  p.offsets = expert_offsets;
  p.Ndy = (int)N;
  p.Kx = (int)K;
  p.E = E;
  const int64_t dy_span = span_bytes(cdiv(M, dy_gather_div), dy_stride_m, N, dtype);
  const int64_t x_span = span_bytes(M, x_stride_m, K, dtype);
  ZMOE_REQUIRE(dy_span <= kMaxSpan && x_span <= kMaxSpan, ZMOE_ERR_SHAPE,
               "group_bwd_w_gather_dy: DY or X spans more than 2 GiB");
  p.dy_bytes = (uint32_t)dy_span;
  p.x_bytes = (uint32_t)x_span;
  if (M == 0) p.x_rows = nullptr;  // no rows: every expert's tiles write zeros (no gather)
  return M == 0 ? group_bwd_w_bf16_out<false>(p, M, E, N, K, out_dtype, as_stream(stream))
                : group_bwd_w_bf16_out<true>(p, M, E, N, K, out_dtype, as_stream(stream));
}

extern "C" int zmoe_group_bwd_w(const void* DY, int64_t dy_stride_m, const void* X, int64_t x_stride_m,
                                const int64_t* x_gather_idxs, int x_gather_div, const int64_t* expert_offsets,
                                int64_t M, int64_t N, int64_t K, int E, int dtype, int out_dtype, void* DWt,
                                void* Db, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "group_bwd_w: dtype %d", dtype);
  ZMOE_REQUIRE(out_dtype == dtype || (dtype == ZMOE_DTYPE_BF16 && out_dtype == ZMOE_DTYPE_F32), ZMOE_ERR_DTYPE,
               "group_bwd_w: out_dtype %d with operands of dtype %d (fp32 output of bf16 operands, or the "
               "operands' dtype)", out_dtype, dtype);
  ZMOE_REQUIRE(Db == nullptr || out_dtype == dtype, ZMOE_ERR_DTYPE, "group_bwd_w: the bias grad is in DY's dtype");
  ZMOE_REQUIRE(M >= 0 && N >= 1 && K >= 1 && E >= 1 && E <= kGemmMaxE && x_gather_div >= 1, ZMOE_ERR_SHAPE,
               "group_bwd_w: bad sizes");
  ZMOE_REQUIRE(N < (1 << 30) && K < (1 << 30), ZMOE_ERR_SHAPE, "group_bwd_w: N/K too large");
  ZMOE_REQUIRE(M < kMaxRows, ZMOE_ERR_SHAPE, "group_bwd_w: M must be below 2^31");
  ZMOE_REQUIRE(DWt && expert_offsets, ZMOE_ERR_NULL, "group_bwd_w: null pointer");
  ZMOE_REQUIRE(M == 0 || (DY && X), ZMOE_ERR_NULL, "group_bwd_w: null operand");
  const int v = vec_elems(dtype);
  ZMOE_REQUIRE(N % v == 0 && K % v == 0 && aligned16(DWt) && (M == 0 || (ok_rows(dtype, DY, dy_stride_m) &&
                                                                          ok_rows(dtype, X, x_stride_m))),
               ZMOE_ERR_ALIGN, "group_bwd_w: N, K and strides must be multiples of %d elements", v);
  WgradParams p{};
  p.dy = DY;
  p.lddy = dy_stride_m;
  p.x = X;
  p.ldx = x_stride_m;
  p.x_rows = x_gather_idxs;
  p.x_div = x_gather_div;
  p.x_div_shift = (x_gather_div > 0 && (x_gather_div & (x_gather_div - 1)) == 0) ? __builtin_ctz(x_gather_div) : -1;
  // the tiles sharing a gathered X block run together when an expert's tiles are few (see
  // launch_wgrad_kernel); with DY gathered instead, m-tiles outer
  p.n_major = x_gather_idxs != nullptr ? 1 : 0;
  p.dw = DWt;
  p.offsets = expert_offsets;
  p.Ndy = (int)N;
  p.Kx = (int)K;
  p.E = E;
  const int64_t x_rows_n = x_gather_idxs ? cdiv(M, x_gather_div) : M;
  const int64_t dy_span = span_bytes(M, dy_stride_m, N, dtype), x_span = span_bytes(x_rows_n, x_stride_m, K, dtype);
  ZMOE_REQUIRE(dy_span <= kMaxSpan && x_span <= kMaxSpan, ZMOE_ERR_SHAPE, "group_bwd_w: DY or X spans more than 2 GiB");
  p.dy_bytes = (uint32_t)dy_span;
  p.x_bytes = (uint32_t)x_span;
  hipStream_t s = as_stream(stream);
  int rc;
  if (dtype == ZMOE_DTYPE_BF16) {
    rc = group_bwd_w_bf16_out<false>(p, M, E, N, K, out_dtype, s);
  } else {
    rc = launch_wgrad_kernel(grouped_wgrad_kernel<float, 128, 128>, rows_lds_bytes<float, 128, 128>(), 128, 128, p,
                             s);
  }
  if (rc || Db == nullptr) return rc;
  const dim3 grid((unsigned)cdiv(N, 256), (unsigned)E), block(256);
  if (dtype == ZMOE_DTYPE_BF16)
    hipLaunchKernelGGL(bias_grad_kernel<uint16_t>, grid, block, 0, s, (const uint16_t*)DY, dy_stride_m,
                       expert_offsets, (int)N, E, (uint16_t*)Db);
  else
    hipLaunchKernelGGL(bias_grad_kernel<float>, grid, block, 0, s, (const float*)DY, dy_stride_m, expert_offsets,
                       (int)N, E, (float*)Db);
  return check_launch("bias_grad_kernel");
}

// Workspace: a 512-byte header (the one-entry row range of an unsplit launch; the split
// launches compute their ranges in the kernel; the header keeps the partials 256-byte
// aligned) + S fp32 partials of [N, K].
constexpr int kDenseMaxSplits = 64;
constexpr size_t kDenseHeaderBytes = kDenseMaxSplits * sizeof(int64_t);

extern "C" size_t zmoe_dense_wgrad_workspace_bytes(int64_t N, int64_t K, int splits) {
  if (N < 1 || K < 1 || splits < 1) return kDenseHeaderBytes;
  if (N >= (1 << 30) || K >= (1 << 30) || splits > kDenseMaxSplits) return 0;  // sizes dense_wgrad rejects
  return kDenseHeaderBytes + (size_t)splits * (size_t)N * (size_t)K * 4u;
}

extern "C" int zmoe_dense_wgrad(const void* DY, int64_t dy_stride_m, const void* X, int64_t x_stride_m, int64_t M,
                                int64_t N, int64_t K, int dtype, int out_dtype, int splits, void* DW,
                                void* workspace, size_t workspace_bytes, void* stream) {
  ZMOE_REQUIRE(dtype_ok(dtype), ZMOE_ERR_DTYPE, "dense_wgrad: dtype %d", dtype);
  ZMOE_REQUIRE(out_dtype == dtype || (dtype == ZMOE_DTYPE_BF16 && out_dtype == ZMOE_DTYPE_F32), ZMOE_ERR_DTYPE,
               "dense_wgrad: out_dtype %d with operands of dtype %d", out_dtype, dtype);
  ZMOE_REQUIRE(M >= 0 && N >= 1 && K >= 1 && splits >= 1 && splits <= kDenseMaxSplits, ZMOE_ERR_SHAPE,
               "dense_wgrad: bad sizes (M=%lld N=%lld K=%lld splits=%d)", (long long)M, (long long)N, (long long)K,
               splits);
  ZMOE_REQUIRE(N < (1 << 30) && K < (1 << 30) && M < kMaxRows, ZMOE_ERR_SHAPE, "dense_wgrad: sizes too large");
  ZMOE_REQUIRE(DW && workspace, ZMOE_ERR_NULL, "dense_wgrad: null pointer");
  ZMOE_REQUIRE(M == 0 || (DY && X), ZMOE_ERR_NULL, "dense_wgrad: null operand");
  const int S = dtype == ZMOE_DTYPE_BF16 ? splits : 1;  // fp32 runs unsplit (direct fp32 output)
  ZMOE_REQUIRE(workspace_bytes >= zmoe_dense_wgrad_workspace_bytes(N, K, S > 1 ? S : 0), ZMOE_ERR_WORKSPACE,
               "dense_wgrad: workspace of %zu bytes is too small", workspace_bytes);
  const int v = vec_elems(dtype);
  ZMOE_REQUIRE(N % v == 0 && K % v == 0 && aligned16(DW) && aligned16(workspace) &&
                   (M == 0 || (ok_rows(dtype, DY, dy_stride_m) && ok_rows(dtype, X, x_stride_m))),
               ZMOE_ERR_ALIGN, "dense_wgrad: N, K and strides must be multiples of %d elements", v);
  hipStream_t s = as_stream(stream);
  int rc = ZMOE_OK;
  if (S == 1) {
    int64_t* off = reinterpret_cast<int64_t*>(workspace);
    hipLaunchKernelGGL(split_offsets_kernel, dim3(1), dim3(64), 0, s, off, M, S);
    rc = check_launch("split_offsets_kernel");
    if (rc) return rc;
    return zmoe_group_bwd_w(DY, dy_stride_m, X, x_stride_m, nullptr, 1, off, M, N, K, 1, dtype, out_dtype, DW,
                            nullptr, stream);
  }
  WgradParams p{};
  p.dy = DY;
  p.lddy = dy_stride_m;
  p.x = X;
  p.ldx = x_stride_m;
  p.x_rows = nullptr;
  p.x_div = 1;
  p.x_div_shift = 0;
  p.dw = reinterpret_cast<char*>(workspace) + kDenseHeaderBytes;
  p.offsets = nullptr;
  p.split_rows = M;  // the split ranges are computed in the kernel
  p.Ndy = (int)N;
  p.Kx = (int)K;
  p.E = S;
  const int64_t dy_span = span_bytes(M, dy_stride_m, N, dtype), x_span = span_bytes(M, x_stride_m, K, dtype);
  ZMOE_REQUIRE(dy_span <= kMaxSpan && x_span <= kMaxSpan, ZMOE_ERR_SHAPE, "dense_wgrad: DY or X spans more than 2 GiB");
  p.dy_bytes = (uint32_t)dy_span;
  p.x_bytes = (uint32_t)x_span;
  if (use_big_tiles(M, S, N) && K >= 256)
    rc = launch_wgrad_big<0, true>(p, s);
  else
    rc = launch_wgrad_kernel(wgrad_bf16_kernel<128, 128, 0, true>, bf16_lds_bytes<128, 128>(), 128, 128, p, s);
  if (rc) return rc;
  const int64_t n = N * K;  // multiple of 8
  if (out_dtype == ZMOE_DTYPE_F32)
    hipLaunchKernelGGL(reduce_splits_kernel<float>, dim3((unsigned)cdiv(n / 4, 256)), dim3(256), 0, s,
                       reinterpret_cast<const float*>(p.dw), S, n, reinterpret_cast<float*>(DW));
  else
    hipLaunchKernelGGL(reduce_splits_kernel<uint16_t>, dim3((unsigned)cdiv(n / 4, 256)), dim3(256), 0, s,
                       reinterpret_cast<const float*>(p.dw), S, n, reinterpret_cast<uint16_t*>(DW));
  return check_launch("reduce_splits_kernel");
}
