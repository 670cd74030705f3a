// Expert counting and the stable expert sort (scattermoe/parallel_experts.py:6-28).
//
// flatten_sort_count is an LDS counting sort over R = T*k slots:
//   1. tile histograms: each 256-thread block counts kSortTile slots into LDS
//      (E+1 buckets; bucket E collects out-of-range ids) and writes them into a
//      bucket-major table, table[e * ntiles + tile];
//   2+3. for at most 256 tiles and 65536 counts (every C1-C5 shape), the counts are
//      written as 16-bit values and one scatter launch follows, in which each block
//      sums the table's bucket rows itself (all tiles, and the tiles before its own),
//      scans the totals and ranks its tile as in 3 below; otherwise:
//   2. one block turns the table into per-tile bucket bases: one wave per bucket
//      reads the bucket's contiguous row of tile counts (16-byte loads), the row
//      totals are scanned over the buckets in LDS, then each wave prefix-scans its
//      rows in place; it also writes the inclusive expert_offsets and the flag;
//   3. each block re-reads its tile in order, 256 slots per round; a wave finds
//      lanes holding the same expert with a ballot per id bit, ranks itself
//      among them, and adds the counts of the earlier waves, so equal experts
//      keep slot order (stable).
// Out-of-range ids land after every valid slot (bucket E) with their original
// value, so every output stays a permutation; the scan raises a flag.
#include <mutex>

#include "zmoe_internal.h"

namespace zmoe {

constexpr int kSortTile = 1024;
constexpr int kSortThreads = 256;
constexpr int kSortMaxE = 1024;
constexpr size_t kSortHeader = 256;  // flag + padding at the start of the workspace
constexpr int kScanThreads = 1024;

__device__ __forceinline__ int bucket_of(int64_t v, int E) { return (v >= 0 && v < E) ? (int)v : E; }

template <typename CT>
__global__ __launch_bounds__(kSortThreads) void sort_hist_kernel(const int64_t* __restrict__ idx, int64_t R,
                                                                 int E, int ntiles, CT* __restrict__ table) {
  __shared__ int32_t h[kSortMaxE + 1];
  for (int e = threadIdx.x; e <= E; e += kSortThreads) h[e] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
#pragma unroll
  for (int i = 0; i < kSortTile / kSortThreads; ++i) {
    const int64_t s = base + i * kSortThreads + threadIdx.x;
    if (s < R) atomicAdd(&h[bucket_of(idx[s], E)], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += kSortThreads) table[(int64_t)e * ntiles + blockIdx.x] = (CT)h[e];
}

// Sum (mode 0) or exclusive prefix plus `start` written back in place (mode 1) of one
// bucket's row of ntiles counts, by one wave. Lanes take 4 consecutive tiles per step
// (one 16-byte load when the row is 16-byte aligned, ntiles % 4 == 0).
__device__ __forceinline__ int64_t scan_row(int32_t* __restrict__ row, int ntiles, int lane, bool vec,
                                            int64_t start, bool write) {
  int64_t run = start;
  for (int c0 = 0; c0 < ntiles; c0 += 256) {
    const int i0 = c0 + lane * 4;
    int32_t v[4] = {0, 0, 0, 0};
    if (vec && i0 + 3 < ntiles) {
      const int4 q = *reinterpret_cast<const int4*>(row + i0);
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = i0 + u < ntiles ? row[i0 + u] : 0;
    }
    const int32_t mine = v[0] + v[1] + v[2] + v[3];
    // inclusive wave scan of the lane sums
    int32_t inc = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t t = __shfl_up(inc, o, 64);
      if (lane >= o) inc += t;
    }
    if (write) {
      int64_t pos = run + (inc - mine);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (i0 + u < ntiles) row[i0 + u] = (int32_t)pos;
        pos += v[u];
      }
    }
    run += __shfl(inc, 63, 64);
  }
  return run;
}

// Rows of at most 256 tiles (R <= 262144 slots), kScanRows buckets per wave: every row a
// wave owns is loaded at once and kept in registers between the totals and the write-back.
constexpr int kScanRows = 17;  // E + 1 <= 272 buckets (C3: 129, C4: 257)

__device__ __forceinline__ int32_t wave_incl_scan(int32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

__global__ __launch_bounds__(kScanThreads) void sort_scan_kernel(int32_t* __restrict__ table, int ntiles, int E,
                                                                 int64_t* __restrict__ offsets,
                                                                 int32_t* __restrict__ flag) {
  __shared__ int64_t tot[kSortMaxE + 1];
  __shared__ int64_t start[kSortMaxE + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = kScanThreads / 64;
  const bool vec = (ntiles & 3) == 0;
  const bool fast = vec && ntiles <= 256 && E + 1 <= nwaves * kScanRows;
  int4 row[kScanRows];
  int32_t inc[kScanRows];
  if (fast) {  // one batch of loads per wave, rows kept for the write-back
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
      const int e = wave + r * nwaves;
      row[r] = make_int4(0, 0, 0, 0);
      if (e <= E && lane * 4 < ntiles) row[r] = *reinterpret_cast<const int4*>(table + (int64_t)e * ntiles + lane * 4);
    }
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) inc[r] = wave_incl_scan(row[r].x + row[r].y + row[r].z + row[r].w, lane);
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
      const int e = wave + r * nwaves;
      if (e <= E && lane == 63) tot[e] = inc[r];
    }
  } else {
    for (int e = wave; e <= E; e += nwaves) {
      const int64_t t = scan_row(table + (int64_t)e * ntiles, ntiles, lane, vec, 0, false);
      if (lane == 0) tot[e] = t;
    }
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of the E+1 bucket totals, 64 buckets per step
    int64_t run = 0;
    for (int e0 = 0; e0 <= E; e0 += 64) {
      const int e = e0 + lane;
      const int64_t mine = e <= E ? tot[e] : 0;
      int64_t inc = mine;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int64_t u = __shfl_up(inc, o, 64);
        if (lane >= o) inc += u;
      }
      if (e <= E) {
        start[e] = run + inc - mine;
        if (e < E) offsets[e] = run + inc;
        if (e == E) flag[0] = mine > 0 ? 1 : 0;
      }
      run += __shfl(inc, 63, 64);
    }
  }
  __syncthreads();
  if (fast) {
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
      const int e = wave + r * nwaves;
      if (e <= E && lane * 4 < ntiles) {
        const int32_t b = (int32_t)start[e] + inc[r] - (row[r].x + row[r].y + row[r].z + row[r].w);
        *reinterpret_cast<int4*>(table + (int64_t)e * ntiles + lane * 4) =
            make_int4(b, b + row[r].x, b + row[r].x + row[r].y, b + row[r].x + row[r].y + row[r].z);
      }
    }
    return;
  }
  for (int e = wave; e <= E; e += nwaves)
    scan_row(table + (int64_t)e * ntiles, ntiles, lane, vec, start[e], true);
}

// Each wave owns kSortTile / 4 consecutive slots of the block's tile. Pass 1: the wave
// counts its slots per bucket (peer groups by ballots over the id bits, the group leader
// adds the group size). After one barrier every wave's base for bucket e is the tile's
// base plus the counts of the waves before it. Pass 2 re-ranks the slots 64 at a time in
// slot order, with no further block barrier: stable within the wave, and the waves'
// ranges follow slot order.
constexpr int kWaveSlots = kSortTile / (kSortThreads / 64);

__device__ __forceinline__ uint64_t peer_mask(int key, int nbits) {
  uint64_t peers = ~0ull;
  for (int b = 0; b < nbits + 1; ++b) {
    const bool bit = (key >> b) & 1;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(
    const int64_t* __restrict__ idx, int64_t R, int E, int ntiles, const int32_t* __restrict__ table,
    int64_t* __restrict__ sorted_expert, int64_t* __restrict__ sorted_slot, int32_t* __restrict__ inverse) {
  __shared__ int32_t wcount[kSortThreads / 64][kSortMaxE + 1];  // pass 1: per-wave bucket counts
  __shared__ int32_t wpos[kSortThreads / 64][kSortMaxE + 1];    // pass 2: per-wave running positions
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int e = threadIdx.x; e <= E; e += kSortThreads)
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) wcount[w][e] = 0;
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E need nbits bits
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t s0 = (int64_t)blockIdx.x * kSortTile + (int64_t)wave * kWaveSlots;
  int64_t v[kWaveSlots / 64];
  int key[kWaveSlots / 64];
#pragma unroll
  for (int r = 0; r < kWaveSlots / 64; ++r) {
    const int64_t s = s0 + r * 64 + lane;
    v[r] = s < R ? idx[s] : 0;
    key[r] = s < R ? bucket_of(v[r], E) : E + 1;  // lanes past R use an id no live lane has
  }
  uint64_t peers[kWaveSlots / 64];  // lanes of this wave holding the same bucket, kept for pass 2
#pragma unroll
  for (int r = 0; r < kWaveSlots / 64; ++r) {
    peers[r] = peer_mask(key[r], nbits);
    if (key[r] <= E && __popcll(peers[r] & lt_mask) == 0) wcount[wave][key[r]] += __popcll(peers[r]);
  }
  __syncthreads();
  // this wave's running position per bucket: tile base + counts of the earlier waves
  for (int e = lane; e <= E; e += 64) {
    int32_t base = table[(int64_t)e * ntiles + blockIdx.x];
    for (int w = 0; w < wave; ++w) base += wcount[w][e];
    wpos[wave][e] = base;  // only this wave touches its row from here on
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int r = 0; r < kWaveSlots / 64; ++r) {
    const int64_t s = s0 + r * 64 + lane;
    const int rank = __popcll(peers[r] & lt_mask);
    const bool live = key[r] <= E;
    int pos = 0;
    if (live) pos = wpos[wave][key[r]] + rank;
    __builtin_amdgcn_wave_barrier();
    if (live && rank == 0) wpos[wave][key[r]] += __popcll(peers[r]);
    __builtin_amdgcn_wave_barrier();
    if (live) {
      sorted_expert[pos] = v[r];
      sorted_slot[pos] = s;
      if (inverse) inverse[s] = pos;
    }
  }
}

// Two-launch form of the sort for at most kFusedMaxTiles tiles and kFusedMaxTable counts
// (every C1-C5 shape): the scatter blocks derive the bucket bases themselves, so the one-block scan
// launch between histogram and scatter goes away. Block b reads the whole tile table of
// 16-bit counts (L2-resident after the histogram launch; 16 lanes per bucket row,
// 16-byte loads), sums each bucket over all tiles and over the tiles before b, scans the
// bucket totals, and ranks its tile as sort_scatter_kernel does, with eight waves of
// 128 slots.
constexpr int kFusedThreads = 512;
constexpr int kFusedWaves = kFusedThreads / 64;
constexpr int kFusedWaveSlots = kSortTile / kFusedWaves;
constexpr int64_t kFusedMaxTable = 1 << 16;
constexpr int kFusedMaxTiles = 256;  // R <= 262144 slots: one 16-byte piece of a bucket row per lane

// Inclusive prefix sum over the wave by DPP: shifts within rows of 16 lanes, then each
// row's last lane broadcast into the rows after it.
__device__ __forceinline__ int32_t wave_incl_scan_dpp(int32_t v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return v;
}

// Sum over a row of 16 lanes by DPP; every lane of the row ends with it.
__device__ __forceinline__ int32_t row16_sum_i32(int32_t v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);   // quad_perm 1,0,3,2
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);   // quad_perm 2,3,0,1
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, true);  // row_half_mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, true);  // row_mirror
  return v;
}

__global__ __launch_bounds__(kFusedThreads) void sort_scatter_scan_kernel(
    const int64_t* __restrict__ idx, int64_t R, int E, int ntiles, const uint16_t* __restrict__ table,
    int64_t* __restrict__ offsets, int32_t* __restrict__ flag, int64_t* __restrict__ sorted_expert,
    int64_t* __restrict__ sorted_slot, int32_t* __restrict__ inverse) {
  // pass 1: per-wave bucket counts, turned in place into each wave's running positions
  __shared__ int32_t wcount[kFusedWaves][kSortMaxE + 1];
  __shared__ int32_t tot[kSortMaxE + 1];                  // bucket totals over every tile
  __shared__ int32_t base[kSortMaxE + 1];                 // counts before this tile, then its bucket bases
  __shared__ int32_t part[kFusedWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.x;
  for (int e = threadIdx.x; e <= E; e += kFusedThreads)
#pragma unroll
    for (int w = 0; w < kFusedWaves; ++w) wcount[w][e] = 0;
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E need nbits bits
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t s0 = (int64_t)b * kSortTile + (int64_t)wave * kFusedWaveSlots;
  int64_t v[kFusedWaveSlots / 64];
  int key[kFusedWaveSlots / 64];
#pragma unroll
  for (int r = 0; r < kFusedWaveSlots / 64; ++r) {
    const int64_t s = s0 + r * 64 + lane;
    v[r] = s < R ? idx[s] : 0;
    key[r] = s < R ? bucket_of(v[r], E) : E + 1;  // lanes past R use an id no live lane has
  }
  // bucket rows of the tile table (16-bit counts, bucket-major): each bucket's sum over all
  // tiles and over the tiles before this one. A 16-lane group reads one row at a time, lane
  // l tiles 16 l .. 16 l + 15 (ntiles <= 256; two 16-byte loads when rows are 16-byte
  // aligned); a wave issues the loads of all its rows (kRowPasses per batch) before
  // reducing any, by packed 16-bit adds and then DPP within the group. Rows go to the 32
  // groups rotated by the block index, so that the blocks sharing an L2 read different
  // rows at any one time.
  {
    constexpr int kRowPasses = 5;  // E + 1 <= 160 buckets in one batch (C3: 129)
    const int grp = wave * 4 + (lane >> 4), gl = lane & 15;
    const int t0 = gl * 16;
    const bool vec = (ntiles & 7) == 0;
    // the tiles before this one: all of lanes < gb, the first pb of lane gb (same for every row)
    const int gb = b >> 4, pb = b & 15;
    uint32_t pmask[8];  // 16-bit halves of lane gb's words that hold earlier tiles
#pragma unroll
    for (int j = 0; j < 8; ++j) pmask[j] = 2 * j + 1 < pb ? 0xffffffffu : (2 * j < pb ? 0x0000ffffu : 0u);
    for (int r0 = 0; r0 <= E; r0 += 32 * kRowPasses) {
      uint32_t w[kRowPasses][8];
      int ev[kRowPasses];
#pragma unroll
      for (int u = 0; u < kRowPasses; ++u) {
        const int e = r0 + u * 32 + ((grp + b) & 31);
        ev[u] = e;
#pragma unroll
        for (int j = 0; j < 8; ++j) w[u][j] = 0;
        if (e <= E && t0 < ntiles) {
          const uint16_t* row = table + (int64_t)e * ntiles + t0;
          if (vec) {
            const uint4 lo = *reinterpret_cast<const uint4*>(row);
            w[u][0] = lo.x; w[u][1] = lo.y; w[u][2] = lo.z; w[u][3] = lo.w;
            if (t0 + 8 < ntiles) {
              const uint4 hi = *reinterpret_cast<const uint4*>(row + 8);
              w[u][4] = hi.x; w[u][5] = hi.y; w[u][6] = hi.z; w[u][7] = hi.w;
            }
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const uint32_t a0 = t0 + 2 * j < ntiles ? row[2 * j] : 0u;
              const uint32_t a1 = t0 + 2 * j + 1 < ntiles ? row[2 * j + 1] : 0u;
              w[u][j] = a0 | (a1 << 16);
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kRowPasses; ++u) {
        // packed sums: each half adds at most 8 counts of <= 1024, so no carry crosses halves
        uint32_t sa = 0, sp = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          sa += w[u][j];
          sp += w[u][j] & pmask[j];
        }
        const int32_t all = (int32_t)((sa & 0xffffu) + (sa >> 16));
        const int32_t part = (int32_t)((sp & 0xffffu) + (sp >> 16));
        int32_t bef = gl < gb ? all : (gl == gb ? part : 0);
        const int32_t ta = row16_sum_i32(all), tb = row16_sum_i32(bef);
        if (gl == 0 && ev[u] <= E) {
          tot[ev[u]] = ta;
          base[ev[u]] = tb;
        }
      }
    }
  }
  __syncthreads();  // wcount zeroed; tot and base complete
  uint64_t peers[kFusedWaveSlots / 64];  // lanes of this wave holding the same bucket, kept for pass 2
#pragma unroll
  for (int r = 0; r < kFusedWaveSlots / 64; ++r) {
    peers[r] = peer_mask(key[r], nbits);
    if (key[r] <= E && __popcll(peers[r] & lt_mask) == 0) wcount[wave][key[r]] += __popcll(peers[r]);
  }
  // exclusive scan of the bucket totals: thread t owns buckets t * per .. t * per + per - 1
  const int per = (E + 1 + kFusedThreads - 1) / kFusedThreads;  // <= 3
  const int eb = (int)threadIdx.x * per;
  int32_t mine = 0;
  for (int u = 0; u < per; ++u)
    if (eb + u <= E) mine += tot[eb + u];
  const int32_t inc = wave_incl_scan_dpp(mine);
  if (lane == 63) part[wave] = inc;
  __syncthreads();  // pass-1 counts and the wave totals of the scan are in LDS
  int32_t run = inc - mine;
  for (int w = 0; w < wave; ++w) run += part[w];
  for (int u = 0; u < per; ++u) {
    const int e = eb + u;
    if (e <= E) {
      const int32_t t = tot[e];
      // wave w's first position in bucket e: bucket start + counts of the earlier tiles +
      // counts of the earlier waves of this tile
      int32_t pos = run + base[e];
#pragma unroll
      for (int w = 0; w < kFusedWaves; ++w) {
        const int32_t c = wcount[w][e];
        wcount[w][e] = pos;
        pos += c;
      }
      if (b == 0) {
        if (e < E) offsets[e] = (int64_t)run + t;
        else flag[0] = t > 0 ? 1 : 0;
      }
      run += t;
    }
  }
  __syncthreads();  // every wave's running positions are in LDS
  int32_t* wpos_row = wcount[wave];  // only this wave touches its row from here on
#pragma unroll
  for (int r = 0; r < kFusedWaveSlots / 64; ++r) {
    const int64_t s = s0 + r * 64 + lane;
    const int rank = __popcll(peers[r] & lt_mask);
    const bool live = key[r] <= E;
    int pos = 0;
    if (live) pos = wpos_row[key[r]] + rank;
    __builtin_amdgcn_wave_barrier();
    if (live && rank == 0) wpos_row[key[r]] += __popcll(peers[r]);
    __builtin_amdgcn_wave_barrier();
    if (live) {
      sorted_expert[pos] = v[r];
      sorted_slot[pos] = s;
      if (inverse) inverse[s] = pos;
    }
  }
}

__global__ void zero_i64_kernel(int64_t* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(kSortThreads) void bincount_kernel(const int64_t* __restrict__ idx, int64_t R, int E,
                                                                unsigned long long* __restrict__ counts) {
  __shared__ int32_t h[kSortMaxE];
  for (int e = threadIdx.x; e < E; e += kSortThreads) h[e] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  for (int i = threadIdx.x; i < kSortTile; i += kSortThreads) {
    const int64_t s = base + i;
    if (s < R) {
      const int64_t v = idx[s];
      if (v >= 0 && v < E) atomicAdd(&h[v], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kSortThreads)
    if (h[e]) atomicAdd(&counts[e], (unsigned long long)h[e]);
}

// offsets[e] = #{i : sorted[i] <= e} by binary search over the sorted list.
__global__ void offsets_from_sorted_kernel(const int64_t* __restrict__ sorted, int64_t R, int E,
                                           int64_t* __restrict__ offsets) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  int64_t lo = 0, hi = R;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (sorted[mid] <= e) lo = mid + 1;
    else hi = mid;
  }
  offsets[e] = lo;
}

}  // namespace zmoe

using namespace zmoe;

extern "C" size_t zmoe_sort_workspace_bytes(int64_t R, int E) {
  if (E < 1 || E > kSortMaxE || R >= (int64_t)0x7fffffff) return 0;  // sizes the sort rejects
  const int64_t ntiles = cdiv(R > 0 ? R : 1, kSortTile);
  return kSortHeader + (size_t)ntiles * (size_t)(E + 1) * sizeof(int32_t);
}

extern "C" const int32_t* zmoe_sort_error_flag(const void* workspace) {
  return reinterpret_cast<const int32_t*>(workspace);
}

namespace {

int sort_shape_checks(int64_t R, int E, int64_t* expert_offsets, const char* name) {
  ZMOE_REQUIRE(E >= 1 && E <= kSortMaxE, ZMOE_ERR_SHAPE, "%s: need 1 <= E <= %d (E=%d)", name, kSortMaxE, E);
  ZMOE_REQUIRE(R >= 0 && R < (int64_t)0x7fffffff, ZMOE_ERR_SHAPE, "%s: R=%lld out of range", name, (long long)R);
  ZMOE_REQUIRE(expert_offsets, ZMOE_ERR_NULL, "%s: null expert_offsets", name);
  return ZMOE_OK;
}

int sort_pointer_checks(const int64_t* expert_idxs, int64_t R, int64_t* sorted_expert_idxs,
                        int64_t* sorted_scattered_idxs, const char* name) {
  ZMOE_REQUIRE(R == 0 || (expert_idxs && sorted_expert_idxs && sorted_scattered_idxs), ZMOE_ERR_NULL,
               "%s: null pointer", name);
  return ZMOE_OK;
}

// The launches over a workspace laid out as [flag | header padding | tile table]: the
// tile histograms, then the scatter that derives the bucket bases itself, or (for empty
// inputs and larger tables) the one-block scan and the scatter.
// Every byte they read is written earlier in the same call, so nothing needs clearing.
int sort_launch(const int64_t* expert_idxs, int64_t R, int E, int64_t* sorted_expert_idxs,
                int64_t* sorted_scattered_idxs, int64_t* expert_offsets, int32_t* inverse, int32_t* flag,
                int32_t* table, hipStream_t s, const char* name) {
  const int ntiles = (int)cdiv(R, kSortTile);
  if (ntiles > 0 && ntiles <= kFusedMaxTiles && (int64_t)(E + 1) * ntiles <= kFusedMaxTable) {
    // tile counts (<= kSortTile) as 16-bit values
    uint16_t* table16 = reinterpret_cast<uint16_t*>(table);
    hipLaunchKernelGGL(sort_hist_kernel<uint16_t>, dim3(ntiles), dim3(kSortThreads), 0, s, expert_idxs, R, E, ntiles,
                       table16);
    hipLaunchKernelGGL(sort_scatter_scan_kernel, dim3(ntiles), dim3(kFusedThreads), 0, s, expert_idxs, R, E,
                       ntiles, table16, expert_offsets, flag, sorted_expert_idxs, sorted_scattered_idxs, inverse);
    return check_launch(name);
  }
  if (ntiles > 0)
    hipLaunchKernelGGL(sort_hist_kernel<int32_t>, dim3(ntiles), dim3(kSortThreads), 0, s, expert_idxs, R, E, ntiles,
                       table);
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, table, ntiles, E, expert_offsets, flag);
  if (ntiles > 0)
    hipLaunchKernelGGL(sort_scatter_kernel, dim3(ntiles), dim3(kSortThreads), 0, s, expert_idxs, R, E, ntiles,
                       table, sorted_expert_idxs, sorted_scattered_idxs, inverse);
  return check_launch(name);
}

}  // namespace

extern "C" int zmoe_flatten_sort_count(const int64_t* expert_idxs, int64_t R, int E, int64_t* sorted_expert_idxs,
                                       int64_t* sorted_scattered_idxs, int64_t* expert_offsets, int32_t* inverse,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  int rc = sort_shape_checks(R, E, expert_offsets, "flatten_sort_count");
  if (rc) return rc;
  ZMOE_REQUIRE(workspace, ZMOE_ERR_NULL, "flatten_sort_count: null workspace");
  ZMOE_REQUIRE(workspace_bytes >= zmoe_sort_workspace_bytes(R, E), ZMOE_ERR_WORKSPACE,
               "flatten_sort_count: workspace %zu < %zu bytes", workspace_bytes, zmoe_sort_workspace_bytes(R, E));
  rc = sort_pointer_checks(expert_idxs, R, sorted_expert_idxs, sorted_scattered_idxs, "flatten_sort_count");
  if (rc) return rc;
  int32_t* flag = reinterpret_cast<int32_t*>(workspace);
  int32_t* tile_hist = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) + kSortHeader);
  return sort_launch(expert_idxs, R, E, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets, inverse, flag,
                     tile_hist, as_stream(stream), "flatten_sort_count");
}

// ------------------------------------------------------------------ no-allocation variant
// The sort's workspace as a file-scope device array, for callers that cannot allocate.
// Every GPU the library runs on holds one copy, at its own address, until the process
// ends. In host code the array's name is not a device address: kernels get the pointer
// that hipGetSymbolAddress returns for the current device (looked up once per device).
constexpr size_t kSortScratchBytes = ZMOE_SORT_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kSortScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  ZMOE_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxDevices, ZMOE_ERR_HIP,
               "flatten_sort_count_noalloc: hipGetDevice failed (%s, device %d)", hipGetErrorString(e), dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    ZMOE_REQUIRE(e == hipSuccess && ptr != nullptr, ZMOE_ERR_HIP,
                 "flatten_sort_count_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                 hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ZMOE_OK;
}

}  // namespace

extern "C" int zmoe_flatten_sort_count_noalloc(const int64_t* expert_idxs, int64_t R, int E,
                                               int64_t* sorted_expert_idxs, int64_t* sorted_scattered_idxs,
                                               int64_t* expert_offsets, int32_t* inverse, int32_t* error_flag,
                                               void* stream) {
  int rc = sort_shape_checks(R, E, expert_offsets, "flatten_sort_count_noalloc");
  if (rc) return rc;
  const size_t need = zmoe_sort_workspace_bytes(R, E);
  ZMOE_REQUIRE(need <= kSortScratchBytes, ZMOE_ERR_WORKSPACE,
               "flatten_sort_count_noalloc: R=%lld slots over E=%d experts need %zu bytes of scratch, above its "
               "%zu-byte maximum (ceil(R / %d) * (E + 1) * 4 + %zu); use zmoe_flatten_sort_count with a workspace",
               (long long)R, E, need, kSortScratchBytes, kSortTile, kSortHeader);
  rc = sort_pointer_checks(expert_idxs, R, sorted_expert_idxs, sorted_scattered_idxs, "flatten_sort_count_noalloc");
  if (rc) return rc;
  void* base = nullptr;
  rc = scratch_for_current_device(&base);
  if (rc) return rc;
  int32_t* flag = error_flag ? error_flag : reinterpret_cast<int32_t*>(base);
  int32_t* tile_hist = reinterpret_cast<int32_t*>(static_cast<char*>(base) + kSortHeader);
  return sort_launch(expert_idxs, R, E, sorted_expert_idxs, sorted_scattered_idxs, expert_offsets, inverse, flag,
                     tile_hist, as_stream(stream), "flatten_sort_count_noalloc");
}

extern "C" int zmoe_bincount(const int64_t* expert_idxs, int64_t R, int E, int64_t* counts, void* stream) {
  ZMOE_REQUIRE(E >= 1 && E <= kSortMaxE, ZMOE_ERR_SHAPE, "bincount: need 1 <= E <= %d", kSortMaxE);
  ZMOE_REQUIRE(R >= 0, ZMOE_ERR_SHAPE, "bincount: R < 0");
  ZMOE_REQUIRE(counts && (R == 0 || expert_idxs), ZMOE_ERR_NULL, "bincount: null pointer");
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(zero_i64_kernel, dim3((unsigned)cdiv(E, 256)), dim3(256), 0, s, counts, E);
  const int ntiles = (int)cdiv(R, kSortTile);
  if (ntiles > 0)
    hipLaunchKernelGGL(bincount_kernel, dim3(ntiles), dim3(kSortThreads), 0, s, expert_idxs, R, E,
                       reinterpret_cast<unsigned long long*>(counts));
  return check_launch("bincount");
}

extern "C" int zmoe_offsets_from_sorted(const int64_t* sorted_expert_idxs, int64_t R, int E,
                                        int64_t* expert_offsets, void* stream) {
  ZMOE_REQUIRE(E >= 1 && R >= 0, ZMOE_ERR_SHAPE, "offsets_from_sorted: bad sizes");
  ZMOE_REQUIRE(expert_offsets && (R == 0 || sorted_expert_idxs), ZMOE_ERR_NULL, "offsets_from_sorted: null pointer");
  hipLaunchKernelGGL(offsets_from_sorted_kernel, dim3((unsigned)cdiv(E, 256)), dim3(256), 0, as_stream(stream),
                     sorted_expert_idxs, R, E, expert_offsets);
  return check_launch("offsets_from_sorted");
}
