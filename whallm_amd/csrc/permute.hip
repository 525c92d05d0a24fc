// Token->expert permute: a stable counting sort of the flattened (token, k) pairs
// by expert, on the device (the reference sorts on the host with std::stable_sort,
// Native/QwenNative/engine.mm:2104-2126, or calls mlx-lm _gather_sort,
// qwen4_exp.py:865-868).
//
//   count   : one wave per chunk of 256 pairs counts its experts in LDS
//   colscan : a workgroup per 64 experts turns each expert's column of chunk counts into
//             exclusive prefixes over the chunks (16 segments of chunks per expert, in
//             parallel), and writes each expert's total
//   scatter : one wave per chunk computes the experts' offsets (an exclusive scan of the
//             totals), walks its pairs in order, 64 at a time; lanes with the same expert
//             find each other with ballots, so every pair's row is base + its rank among
//             earlier same-expert pairs: stable. Wave 0 also writes the offsets and the
//             (expert, first row) tile list.
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

// Exclusive scan of n values (n <= 64 * 16) held lane-major by one wave: lane l owns
// entries [l * per, (l + 1) * per). Writes the exclusive prefixes to out[] (LDS) and
// returns the total in every lane.
template <typename Value>
__device__ __forceinline__ int32_t wave_exclusive_scan(int n, int lane, Value value, int32_t* out) {
  const int per = (n + 63) / 64;
  int32_t mine = 0;
  for (int q = 0; q < per; ++q) {
    const int i = lane * per + q;
    if (i < n) mine += value(i);
  }
  int32_t incl = mine;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  int32_t run = incl - mine;
  for (int q = 0; q < per; ++q) {
    const int i = lane * per + q;
    if (i < n) {
      out[i] = run;
      run += value(i);
    }
  }
  return __shfl(incl, 63, 64);
}

__global__ void __launch_bounds__(64) permute_scatter_kernel(const int32_t* __restrict__ idx, int64_t pairs,
                                                            int experts, const int32_t* __restrict__ chunk_base,
                                                            const int32_t* __restrict__ totals, int tile_rows,
                                                            int32_t* __restrict__ order, int32_t* __restrict__ inverse,
                                                            int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ tiles,
                                                            int32_t* __restrict__ tile_count) {
  __shared__ int32_t base[PERMUTE_MAX_EXPERTS];
  __shared__ int32_t first_tile[PERMUTE_MAX_EXPERTS];
  const int lane = threadIdx.x;
  const int64_t chunk = blockIdx.x;
  const int32_t rows = wave_exclusive_scan(experts, lane, [&](int e) { return totals[e]; }, base);
  __syncthreads();
  if (chunk == 0) {
    // offsets and the tile list: expert e's tiles are first_tile[e] .. + ceil(total / tile_rows)
    const int32_t n_tiles = wave_exclusive_scan(
        experts, lane, [&](int e) { return (totals[e] + tile_rows - 1) / tile_rows; }, first_tile);
    __syncthreads();
    for (int e = lane; e < experts; e += 64) {
      offsets[e] = base[e];
      const int32_t n = (totals[e] + tile_rows - 1) / tile_rows;
      for (int32_t q = 0; q < n; ++q) {
        tiles[2 * (first_tile[e] + q)] = e;
        tiles[2 * (first_tile[e] + q) + 1] = base[e] + q * tile_rows;
      }
    }
    if (lane == 0) {
      offsets[experts] = rows;
      tile_count[0] = n_tiles;
    }
  }
  for (int e = lane; e < experts; e += 64) base[e] += chunk_base[chunk * experts + e];
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
    // with no pairs one scatter wave still writes the (empty) offsets and tile count
    hipLaunchKernelGGL(permute_scatter_kernel, dim3((unsigned)(chunks > 0 ? chunks : 1)), dim3(64), 0, s, indices,
                       pairs, experts, counts, totals, tile_rows, order, inverse, offsets, tiles, tile_count);
    check_launch("permute_scatter");
  });
}

}  // extern "C"
