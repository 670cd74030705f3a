// Expert counting and the stable expert sort (scattermoe/parallel_experts.py:6-28).
//
// flatten_sort_count is a three-launch LDS counting sort over R = T*k slots:
//   1. tile histograms: each 256-thread block counts kSortTile slots into LDS
//      (E+1 buckets; bucket E collects out-of-range ids);
//   2. one block turns the [tiles x buckets] table into per-tile bucket bases
//      (column prefix over tiles, then an exclusive scan over buckets) and
//      writes the inclusive expert_offsets;
//   3. each block re-reads its tile in order, 256 slots per round; a wave finds
//      lanes holding the same expert with a ballot per id bit, ranks itself
//      among them, and adds the counts of the earlier waves, so equal experts
//      keep slot order (stable).
// Out-of-range ids land after every valid slot (bucket E) with their original
// value, so every output stays a permutation; the scan raises a flag.
#include <mutex>

#include "zmoe_internal.h"

namespace zmoe {

constexpr int kSortTile = 2048;
constexpr int kSortThreads = 256;
constexpr int kSortMaxE = 1024;
constexpr size_t kSortHeader = 256;  // flag + padding at the start of the workspace

__device__ __forceinline__ int bucket_of(int64_t v, int E) { return (v >= 0 && v < E) ? (int)v : E; }

__global__ __launch_bounds__(kSortThreads) void sort_hist_kernel(const int64_t* __restrict__ idx, int64_t R,
                                                                 int E, int32_t* __restrict__ tile_hist) {
  __shared__ int32_t h[kSortMaxE + 1];
  for (int e = threadIdx.x; e <= E; e += kSortThreads) h[e] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kSortTile;
  for (int i = threadIdx.x; i < kSortTile; i += kSortThreads) {
    const int64_t s = base + i;
    if (s < R) atomicAdd(&h[bucket_of(idx[s], E)], 1);
  }
  __syncthreads();
  int32_t* out = tile_hist + (int64_t)blockIdx.x * (E + 1);
  for (int e = threadIdx.x; e <= E; e += kSortThreads) out[e] = h[e];
}

// Single block of 1024 threads; buckets are strided over the threads. A bucket's column
// is walked kScanBatch tiles at a time, all of a batch's loads issued before any is used
// (one memory round trip per batch instead of per tile).
constexpr int kScanBatch = 16;
__global__ __launch_bounds__(1024) void sort_scan_kernel(int32_t* __restrict__ tile_hist, int ntiles, int E,
                                                         int64_t* __restrict__ offsets,
                                                         int32_t* __restrict__ flag) {
  __shared__ int64_t tot[kSortMaxE + 1];
  __shared__ int64_t start[kSortMaxE + 1];
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    int64_t total = 0;
    for (int b0 = 0; b0 < ntiles; b0 += kScanBatch) {
      int32_t c[kScanBatch];
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j)
        c[j] = b0 + j < ntiles ? tile_hist[(int64_t)(b0 + j) * (E + 1) + e] : 0;
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j) total += c[j];
    }
    tot[e] = total;
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // E+1 <= 1025 buckets: a serial scan is cheap next to the column sums
    int64_t run = 0;
    for (int q = 0; q <= E; ++q) {
      start[q] = run;
      run += tot[q];
    }
    flag[0] = tot[E] > 0 ? 1 : 0;
  }
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    if (e < E) offsets[e] = start[e] + tot[e];
    int64_t run = start[e];
    for (int b0 = 0; b0 < ntiles; b0 += kScanBatch) {
      int32_t c[kScanBatch];
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j)
        c[j] = b0 + j < ntiles ? tile_hist[(int64_t)(b0 + j) * (E + 1) + e] : 0;
#pragma unroll
      for (int j = 0; j < kScanBatch; ++j) {
        if (b0 + j < ntiles) tile_hist[(int64_t)(b0 + j) * (E + 1) + e] = (int32_t)run;
        run += c[j];
      }
    }
  }
}

__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(
    const int64_t* __restrict__ idx, int64_t R, int E, const int32_t* __restrict__ tile_base,
    int64_t* __restrict__ sorted_expert, int64_t* __restrict__ sorted_slot, int32_t* __restrict__ inverse) {
  __shared__ int32_t base[kSortMaxE + 1];
  __shared__ int32_t wcount[kSortThreads / 64][kSortMaxE + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int32_t* tb = tile_base + (int64_t)blockIdx.x * (E + 1);
  for (int e = threadIdx.x; e <= E; e += kSortThreads) {
    base[e] = tb[e];
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) wcount[w][e] = 0;
  }
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) <= E) ++nbits;  // ids 0..E need nbits bits
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t tile0 = (int64_t)blockIdx.x * kSortTile;
  for (int r = 0; r < kSortTile; r += kSortThreads) {
    const int64_t s = tile0 + r + threadIdx.x;
    const bool live = s < R;
    int64_t v = 0;
    int key = E + 1;  // lanes past R use an id no live lane has
    if (live) {
      v = idx[s];
      key = bucket_of(v, E);
    }
    uint64_t peers = ~0ull;
    for (int b = 0; b < nbits + 1; ++b) {
      const bool bit = (key >> b) & 1;
      const uint64_t m = __ballot(bit);
      peers &= bit ? m : ~m;
    }
    const int rank = __popcll(peers & lt_mask);
    const int cnt = __popcll(peers);
    const bool leader = rank == 0;
    if (live && leader) wcount[wave][key] = cnt;
    __syncthreads();
    if (live) {
      int pos = base[key] + rank;
      for (int w = 0; w < wave; ++w) pos += wcount[w][key];
      sorted_expert[pos] = v;
      sorted_slot[pos] = s;
      if (inverse) inverse[s] = pos;
    }
    __syncthreads();
    if (live && leader) {
      atomicAdd(&base[key], cnt);
      wcount[wave][key] = 0;
    }
    __syncthreads();
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

// The three launches over a workspace laid out as [flag | header padding | tile table];
// every byte they read is written earlier in the same call, so nothing needs clearing.
int sort_launch(const int64_t* expert_idxs, int64_t R, int E, int64_t* sorted_expert_idxs,
                int64_t* sorted_scattered_idxs, int64_t* expert_offsets, int32_t* inverse, int32_t* flag,
                int32_t* tile_hist, hipStream_t s, const char* name) {
  const int ntiles = (int)cdiv(R, kSortTile);
  if (ntiles > 0)
    hipLaunchKernelGGL(sort_hist_kernel, dim3(ntiles), dim3(kSortThreads), 0, s, expert_idxs, R, E, tile_hist);
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(1024), 0, s, tile_hist, ntiles, E, expert_offsets, flag);
  if (ntiles > 0)
    hipLaunchKernelGGL(sort_scatter_kernel, dim3(ntiles), dim3(kSortThreads), 0, s, expert_idxs, R, E, tile_hist,
                       sorted_expert_idxs, sorted_scattered_idxs, inverse);
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
