// Token->expert permute: a stable counting sort of the flattened (token, k) pairs
// by expert, on the device (the reference sorts on the host with std::stable_sort,
// Native/QwenNative/engine.mm:2104-2126, or calls mlx-lm _gather_sort,
// qwen4_exp.py:865-868).
//
//   count   : one wave per chunk of 1024 pairs counts its experts in LDS
//   scan    : one workgroup turns the per-chunk counts into per-chunk bases,
//             per-expert offsets, and the (expert, first row) tile list
//   scatter : one wave per chunk walks its pairs in order, 64 at a time; lanes
//             with the same expert find each other with ballots, so every pair's
//             row is base + its rank among earlier same-expert pairs: stable.
//
// Invalid expert ids (< 0 or >= E) are left out of every list; their inverse is -1.
#include "wm_common.h"

namespace wm {

constexpr int PERMUTE_CHUNK = 1024;
constexpr int PERMUTE_MAX_EXPERTS = 1024;

__global__ void __launch_bounds__(64) permute_count_kernel(const int32_t* __restrict__ idx, int64_t pairs, int experts,
                                                          int32_t* __restrict__ chunk_counts) {
  __shared__ int32_t counts[PERMUTE_MAX_EXPERTS];
  int lane = threadIdx.x;
  int64_t chunk = blockIdx.x;
  for (int e = lane; e < experts; e += 64) counts[e] = 0;
  __syncthreads();
  int64_t begin = chunk * PERMUTE_CHUNK, end = min<int64_t>(pairs, begin + PERMUTE_CHUNK);
  for (int64_t p = begin + lane; p < end; p += 64) {
    int e = idx[p];
    if (e >= 0 && e < experts) atomicAdd(&counts[e], 1);
  }
  __syncthreads();
  for (int e = lane; e < experts; e += 64) chunk_counts[chunk * experts + e] = counts[e];
}

// One workgroup of 1024 threads. chunk_counts[c][e] becomes the first row of
// chunk c's pairs of expert e.
__global__ void __launch_bounds__(1024) permute_scan_kernel(int32_t* __restrict__ chunk_counts, int64_t chunks,
                                                           int experts, int tile_rows, int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ tiles,
                                                           int32_t* __restrict__ tile_count) {
  __shared__ int32_t total[PERMUTE_MAX_EXPERTS];
  __shared__ int32_t ntiles[PERMUTE_MAX_EXPERTS];
  __shared__ int32_t scan_a[PERMUTE_MAX_EXPERTS];
  __shared__ int32_t scan_b[PERMUTE_MAX_EXPERTS];
  int e = threadIdx.x;
  int32_t running = 0;
  if (e < experts) {
    for (int64_t c = 0; c < chunks; ++c) {
      int32_t n = chunk_counts[c * experts + e];
      chunk_counts[c * experts + e] = running;
      running += n;
    }
  }
  total[e] = e < experts ? running : 0;
  ntiles[e] = e < experts ? (running + tile_rows - 1) / tile_rows : 0;
  __syncthreads();
  // Inclusive Hillis-Steele scans of total and ntiles over 1024 entries.
  int32_t* a = scan_a;
  int32_t* b = scan_b;
  a[e] = total[e];
  __syncthreads();
  for (int offset = 1; offset < PERMUTE_MAX_EXPERTS; offset <<= 1) {
    b[e] = a[e] + (e >= offset ? a[e - offset] : 0);
    __syncthreads();
    int32_t* t = a; a = b; b = t;
  }
  int32_t row_base = a[e] - total[e];
  __syncthreads();
  a[e] = ntiles[e];
  __syncthreads();
  for (int offset = 1; offset < PERMUTE_MAX_EXPERTS; offset <<= 1) {
    b[e] = a[e] + (e >= offset ? a[e - offset] : 0);
    __syncthreads();
    int32_t* t = a; a = b; b = t;
  }
  int32_t tile_base = a[e] - ntiles[e];
  if (e < experts) {
    offsets[e] = row_base;
    if (e == experts - 1) {
      offsets[experts] = row_base + total[e];
      tile_count[0] = tile_base + ntiles[e];
    }
    for (int j = 0; j < ntiles[e]; ++j) {
      tiles[2 * (tile_base + j)] = e;
      tiles[2 * (tile_base + j) + 1] = row_base + j * tile_rows;
    }
    for (int64_t c = 0; c < chunks; ++c) chunk_counts[c * experts + e] += row_base;
  }
}

__global__ void __launch_bounds__(64) permute_scatter_kernel(const int32_t* __restrict__ idx, int64_t pairs,
                                                            int experts, const int32_t* __restrict__ chunk_base,
                                                            int32_t* __restrict__ order,
                                                            int32_t* __restrict__ inverse) {
  __shared__ int32_t base[PERMUTE_MAX_EXPERTS];
  int lane = threadIdx.x;
  int64_t chunk = blockIdx.x;
  for (int e = lane; e < experts; e += 64) base[e] = chunk_base[chunk * experts + e];
  __syncthreads();
  int bits = 32 - __clz(experts);  // enough bits to tell experts (and the sentinel `experts`) apart
  int64_t begin = chunk * PERMUTE_CHUNK, end = min<int64_t>(pairs, begin + PERMUTE_CHUNK);
  for (int64_t p0 = begin; p0 < end; p0 += 64) {
    int64_t p = p0 + lane;
    bool in_range = p < end;
    int e = in_range ? idx[p] : -1;
    bool valid = in_range && e >= 0 && e < experts;
    uint32_t key = valid ? (uint32_t)e : (uint32_t)experts;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < bits; ++bit) {
      uint64_t set = __ballot((key >> bit) & 1u);
      peers &= ((key >> bit) & 1u) ? set : ~set;
    }
    uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int rank = __popcll(peers & below);
    int32_t row = valid ? base[e] + rank : -1;
    // Every lane has read base[] above; the last lane of each expert advances it.
    bool last = valid && (peers >> lane) == 1ull;
    __builtin_amdgcn_wave_barrier();
    if (last) base[e] = row + 1;
    __builtin_amdgcn_wave_barrier();
    if (valid) order[row] = (int32_t)p;
    if (in_range) inverse[p] = row;
  }
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT size_t wm_permute_workspace_size(int64_t pairs, int32_t experts) {
  int64_t chunks = (pairs + PERMUTE_CHUNK - 1) / PERMUTE_CHUNK;
  return (size_t)(chunks > 0 ? chunks : 1) * (size_t)(experts > 0 ? experts : 1) * sizeof(int32_t);
}

WM_EXPORT int wm_permute(const int32_t* indices, int64_t pairs, int32_t experts, int32_t tile_rows, int32_t* order,
                         int32_t* inverse, int32_t* offsets, int32_t* tiles, int32_t* tile_count, void* workspace,
                         size_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (pairs < 0 || pairs > (int64_t)0x7fffffff) fail("wm_permute: pairs must be in 0..2^31-1");
    if (experts < 1 || experts > PERMUTE_MAX_EXPERTS) fail("wm_permute: experts must be in 1..1024");
    if (tile_rows < 1) fail("wm_permute: tile_rows must be positive");
    if (workspace_bytes < wm_permute_workspace_size(pairs, experts)) fail("wm_permute: workspace too small");
    if (!offsets || !tile_count || !workspace || (pairs > 0 && (!indices || !order || !inverse || !tiles)))
      fail("wm_permute: null pointer");
    int64_t chunks = (pairs + PERMUTE_CHUNK - 1) / PERMUTE_CHUNK;
    int32_t* counts = (int32_t*)workspace;
    hipStream_t s = as_stream(stream);
    if (chunks > 0) {
      hipLaunchKernelGGL(permute_count_kernel, dim3((unsigned)chunks), dim3(64), 0, s, indices, pairs, experts, counts);
      check_launch("permute_count");
    }
    hipLaunchKernelGGL(permute_scan_kernel, dim3(1), dim3(1024), 0, s, counts, chunks, experts, tile_rows, offsets,
                       tiles, tile_count);
    check_launch("permute_scan");
    if (chunks > 0) {
      hipLaunchKernelGGL(permute_scatter_kernel, dim3((unsigned)chunks), dim3(64), 0, s, indices, pairs, experts,
                         counts, order, inverse);
      check_launch("permute_scatter");
    }
  });
}

}  // extern "C"
