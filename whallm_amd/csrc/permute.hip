// Token->expert permute: a stable counting sort of the flattened (token, k) pairs
// by expert, on the device (the reference sorts on the host with std::stable_sort,
// Native/QwenNative/engine.mm:2104-2126, or calls mlx-lm _gather_sort,
// qwen4_exp.py:865-868).
//
//   count   : one wave per chunk of 256 pairs counts its experts in LDS
//   colscan : a workgroup per 64 experts turns each expert's column of chunk counts into
//             exclusive prefixes over the chunks (16 segments of chunks per expert, in
//             parallel), and writes each expert's total
//   offsets : one workgroup scans the expert totals into offsets[E + 1] and the
//             (expert, first row) tile list
//   scatter : one wave per chunk walks its pairs in order, 64 at a time; lanes with the
//             same expert find each other with ballots, so every pair's row is base + its
//             rank among earlier same-expert pairs: stable.
//
// Invalid expert ids (< 0 or >= E) are left out of every list; their inverse is -1.
#include "wm_common.h"

namespace wm {

constexpr int PERMUTE_CHUNK = 256;
constexpr int PERMUTE_MAX_EXPERTS = 1024;
constexpr int SCAN_EXPERTS = 64;  // experts per colscan workgroup (one per lane)
constexpr int SCAN_SEGS = 16;     // chunk segments per expert (one per wave)

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

// Workgroup b: experts 64 b + lane; wave w: chunks [chunks w / 16, chunks (w + 1) / 16).
// chunk_counts[c][e] becomes the number of expert-e pairs in chunks before c; totals[e]
// the expert's pairs.
__global__ void __launch_bounds__(1024) permute_colscan_kernel(int32_t* __restrict__ chunk_counts, int64_t chunks,
                                                              int experts, int32_t* __restrict__ totals) {
  __shared__ int32_t part[SCAN_SEGS][SCAN_EXPERTS];
  const int lane = threadIdx.x % 64, s = threadIdx.x / 64;
  const int e = blockIdx.x * SCAN_EXPERTS + lane;
  const bool live = e < experts;
  const int64_t c0 = chunks * s / SCAN_SEGS, c1 = chunks * (s + 1) / SCAN_SEGS;
  constexpr int BATCH = 8;
  int32_t sum = 0;
  if (live) {
    for (int64_t c = c0; c < c1; c += BATCH) {
      int32_t v[BATCH];
#pragma unroll
      for (int q = 0; q < BATCH; ++q) v[q] = c + q < c1 ? chunk_counts[(c + q) * experts + e] : 0;
#pragma unroll
      for (int q = 0; q < BATCH; ++q) sum += v[q];
    }
  }
  part[s][lane] = sum;
  __syncthreads();
  int32_t before = 0, total = 0;
#pragma unroll
  for (int q = 0; q < SCAN_SEGS; ++q) {
    const int32_t v = part[q][lane];
    before += q < s ? v : 0;
    total += v;
  }
  if (live) {
    int32_t running = before;
    for (int64_t c = c0; c < c1; c += BATCH) {
      int32_t v[BATCH];
#pragma unroll
      for (int q = 0; q < BATCH; ++q) v[q] = c + q < c1 ? chunk_counts[(c + q) * experts + e] : 0;
#pragma unroll
      for (int q = 0; q < BATCH; ++q)
        if (c + q < c1) {
          chunk_counts[(c + q) * experts + e] = running;
          running += v[q];
        }
    }
    if (s == 0) totals[e] = total;
  }
}

// Inclusive prefix sum over the 1024 threads of the block (wave shuffles, then the 16
// wave totals). Every thread of the block must call it.
__device__ __forceinline__ int32_t block_inclusive_scan(int32_t v, int32_t* wave_total) {
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  if (lane == 63) wave_total[wave] = v;
  __syncthreads();
  int32_t before = 0;
  for (int w = 0; w < wave; ++w) before += wave_total[w];
  __syncthreads();  // wave_total is reused by the next call
  return v + before;
}

// One workgroup of 1024 threads, thread e = expert e: offsets[e] (exclusive scan of the
// totals), offsets[E], the tile count, and expert e's tiles (expert, first row) at its
// place in the list.
__global__ void __launch_bounds__(1024) permute_offsets_kernel(const int32_t* __restrict__ totals, int experts,
                                                              int tile_rows, int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ tiles,
                                                              int32_t* __restrict__ tile_count) {
  __shared__ int32_t wave_total[16];
  __shared__ int32_t tile_start[PERMUTE_MAX_EXPERTS + 1];
  __shared__ int32_t row_start[PERMUTE_MAX_EXPERTS];
  const int e = threadIdx.x;
  const int32_t mine = e < experts ? totals[e] : 0;
  const int32_t my_tiles = (mine + tile_rows - 1) / tile_rows;
  const int32_t rows_incl = block_inclusive_scan(mine, wave_total);
  const int32_t tiles_incl = block_inclusive_scan(my_tiles, wave_total);
  if (e < experts) {
    const int32_t row0 = rows_incl - mine, tile0 = tiles_incl - my_tiles;
    offsets[e] = row0;
    tile_start[e] = tile0;
    row_start[e] = row0;
    if (e == experts - 1) {
      offsets[experts] = rows_incl;
      tile_count[0] = tiles_incl;
      tile_start[experts] = tiles_incl;
    }
  }
  __syncthreads();
  // The whole block writes the tile list (a hot expert owns hundreds of tiles). Tile t belongs
  // to the last expert whose first tile is <= t: experts without tiles share their start with
  // the next expert that has some, and come before it.
  const int32_t n_tiles = tile_start[experts];
  for (int32_t t = e; t < n_tiles; t += (int32_t)blockDim.x) {
    int lo = 0, hi = experts - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tile_start[mid] <= t) lo = mid; else hi = mid - 1;
    }
    tiles[2 * t] = lo;
    tiles[2 * t + 1] = row_start[lo] + (t - tile_start[lo]) * tile_rows;
  }
}

__global__ void __launch_bounds__(64) permute_scatter_kernel(const int32_t* __restrict__ idx, int64_t pairs,
                                                            int experts, const int32_t* __restrict__ chunk_base,
                                                            const int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ order,
                                                            int32_t* __restrict__ inverse) {
  __shared__ int32_t base[PERMUTE_MAX_EXPERTS];
  const int lane = threadIdx.x;
  const int64_t chunk = blockIdx.x;
  for (int e = lane; e < experts; e += 64) base[e] = chunk_base[chunk * experts + e] + offsets[e];
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
  const size_t e = (size_t)(experts > 0 ? experts : 1);
  return ((size_t)(chunks > 0 ? chunks : 1) * e + e) * sizeof(int32_t);  // chunk counts, then totals
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
    int32_t* totals = counts + (size_t)(chunks > 0 ? chunks : 1) * experts;
    hipStream_t s = as_stream(stream);
    if (chunks > 0) {
      hipLaunchKernelGGL(permute_count_kernel, dim3((unsigned)chunks), dim3(64), 0, s, indices, pairs, experts, counts);
      check_launch("permute_count");
    }
    hipLaunchKernelGGL(permute_colscan_kernel, dim3((unsigned)((experts + SCAN_EXPERTS - 1) / SCAN_EXPERTS)),
                       dim3(64 * SCAN_SEGS), 0, s, counts, chunks, experts, totals);
    check_launch("permute_colscan");
    hipLaunchKernelGGL(permute_offsets_kernel, dim3(1), dim3(1024), 0, s, totals, experts, tile_rows, offsets, tiles,
                       tile_count);
    check_launch("permute_offsets");
    if (chunks > 0) {
      hipLaunchKernelGGL(permute_scatter_kernel, dim3((unsigned)chunks), dim3(64), 0, s, indices, pairs, experts, counts,
                         offsets, order, inverse);
      check_launch("permute_scatter");
    }
  });
}

}  // extern "C"
