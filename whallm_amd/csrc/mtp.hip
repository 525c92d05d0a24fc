// MTP acceptance: verify n draft tokens against n + 1 target rows over the vocabulary.
//
// Greedy (temperature 0; Sampler.verify, runtime/deepseek_v4_ssd/native_qwen.py:395-400;
// dspark._verify, dspark.py:862-873): accept drafts while each equals the argmax of
// its target row (ties to the lower index, a NaN beats every number as in np.argmax);
// the next token is the argmax of the first mismatching row, or of row n.
// Rejection (native_qwen.py:401-408; dspark.py:875-898): accept draft i while
// u_i <= min(1, exp(t_i[tok] - d_i[tok])); at the first rejection sample from the
// residual max(exp(t_i) - exp(d_i), 0) (from exp(t_i - max t_i) when it sums to 0);
// with every draft accepted sample row n's target. Sampling is inverse-CDF with the
// caller's uniform u_n: the first index whose running sum exceeds u_n * total
// (numpy Generator.choice, searchsorted side='right'). A draft id outside the
// vocabulary counts as rejected.
//
// Rows are at most a few x 129,280 fp32: the kernels are latency-bound, so they
// split a row over chunk blocks and finish in one single-block kernel.
#include <cmath>

#include "wm_common.h"

namespace wm {

constexpr int MTP_THREADS = 256;
constexpr int MTP_CHUNK = 4096;       // vocabulary entries per block of a row pass
constexpr int MTP_MAX_ROWS = 16;      // drafts + 1
constexpr int MTP_MAX_CHUNKS = 1024;  // vocabulary up to 4 M entries

struct MtpArg {
  float v;
  int i;
};

// Larger value wins; a NaN beats every number; equal values (or two NaNs) -> lower index.
__device__ __forceinline__ MtpArg mtp_better(MtpArg a, MtpArg b) {
  const bool an = isnan(a.v), bn = isnan(b.v);
  if (an || bn) {
    if (an && bn) return a.i <= b.i ? a : b;
    return an ? a : b;
  }
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}

__device__ MtpArg mtp_block_argmax(MtpArg m) {
  __shared__ MtpArg part[MTP_THREADS / 64];
  for (int off = 32; off > 0; off >>= 1) {
    MtpArg o;
    o.v = __shfl_xor(m.v, off, 64);
    o.i = __shfl_xor(m.i, off, 64);
    m = mtp_better(m, o);
  }
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  if (lane == 0) part[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < MTP_THREADS / 64; ++w) m = mtp_better(m, part[w]);
    part[0] = m;
  }
  __syncthreads();
  m = part[0];
  __syncthreads();
  return m;
}

__device__ float mtp_block_sum(float v) {
  __shared__ float part[MTP_THREADS / 64];
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  if (lane == 0) part[wave] = v;
  __syncthreads();
  float s = 0.0f;
  for (int w = 0; w < MTP_THREADS / 64; ++w) s += part[w];
  __syncthreads();
  return s;
}

// ---- greedy: per (chunk, row) argmax, then one block decides
__global__ void __launch_bounds__(MTP_THREADS) mtp_argmax_chunks_kernel(const float* __restrict__ logits, int vocab,
                                                                       int chunks, MtpArg* __restrict__ parts) {
  const int c = blockIdx.x, row = blockIdx.y;
  const float* r = logits + (size_t)row * vocab;
  const int lo = c * MTP_CHUNK, hi = min(vocab, lo + MTP_CHUNK);
  MtpArg m = {-INFINITY, 0x7fffffff};
  for (int i = lo + threadIdx.x; i < hi; i += MTP_THREADS) m = mtp_better(m, MtpArg{r[i], i});
  m = mtp_block_argmax(m);
  if (threadIdx.x == 0) parts[(size_t)row * chunks + c] = m;
}

__global__ void __launch_bounds__(MTP_THREADS) mtp_greedy_decide_kernel(const MtpArg* __restrict__ parts, int chunks,
                                                                       const int32_t* __restrict__ drafts, int n,
                                                                       int32_t* __restrict__ out) {
  __shared__ int best[MTP_MAX_ROWS];
  for (int row = 0; row <= n; ++row) {
    MtpArg m = {-INFINITY, 0x7fffffff};
    for (int c = threadIdx.x; c < chunks; c += MTP_THREADS) m = mtp_better(m, parts[(size_t)row * chunks + c]);
    m = mtp_block_argmax(m);
    if (threadIdx.x == 0) best[row] = m.i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int accepted = 0;
    while (accepted < n && drafts[accepted] == best[accepted]) ++accepted;
    out[0] = accepted;
    out[1] = best[accepted];
  }
}

// ---- rejection
// meta: [0] row to sample from, [1] 1 = residual of that row (else its target)
__global__ void __launch_bounds__(64) mtp_reject_decide_kernel(const float* __restrict__ target, const float* __restrict__ draft,
                                                              const int32_t* __restrict__ drafts, int n, int vocab,
                                                              const float* __restrict__ uniforms, int32_t* __restrict__ meta,
                                                              int32_t* __restrict__ out) {
  if (threadIdx.x != 0) return;
  int row = n, residual = 0;
  for (int i = 0; i < n; ++i) {
    const int tok = drafts[i];
    // a draft id outside the vocabulary is rejected (it has no probability to test)
    const bool valid = tok >= 0 && tok < vocab;
    const float accept = valid ? fminf(1.0f, expf(target[(size_t)i * vocab + tok] - draft[(size_t)i * vocab + tok]))
                               : -1.0f;
    if (uniforms[i] > accept) {
      row = i;
      residual = 1;
      break;
    }
  }
  meta[0] = row;
  meta[1] = residual;
  out[0] = row;  // accepted drafts
}

// per chunk of the chosen row: residual sum, target max and sum of exp(t - max)
struct MtpChunk {
  float residual, tmax, tsum;
};

__global__ void __launch_bounds__(MTP_THREADS) mtp_reject_chunks_kernel(const float* __restrict__ target,
                                                                       const float* __restrict__ draft, int vocab,
                                                                       const int32_t* __restrict__ meta,
                                                                       MtpChunk* __restrict__ parts) {
  const int c = blockIdx.x;
  const int row = meta[0];
  const bool residual = meta[1] != 0;
  const float* t = target + (size_t)row * vocab;
  const float* d = draft + (size_t)row * vocab;
  const int lo = c * MTP_CHUNK, hi = min(vocab, lo + MTP_CHUNK);
  float rsum = 0.0f, tmax = -INFINITY;
  for (int i = lo + threadIdx.x; i < hi; i += MTP_THREADS) {
    tmax = fmaxf(tmax, t[i]);
    if (residual) rsum += fmaxf(expf(t[i]) - expf(d[i]), 0.0f);
  }
  __shared__ float mx[MTP_THREADS / 64];
  for (int off = 32; off > 0; off >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, off, 64));
  if (threadIdx.x % 64 == 0) mx[threadIdx.x / 64] = tmax;
  __syncthreads();
  tmax = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
  __syncthreads();
  float tsum = 0.0f;
  if (tmax > -INFINITY)  // a chunk of -inf log-probabilities carries no weight
    for (int i = lo + threadIdx.x; i < hi; i += MTP_THREADS) tsum += expf(t[i] - tmax);
  rsum = mtp_block_sum(rsum);
  tsum = mtp_block_sum(tsum);
  if (threadIdx.x == 0) parts[c] = MtpChunk{rsum, tmax, tsum};
}

// Inverse CDF: pick the chunk whose running total first exceeds u * total (one
// thread over the chunk totals), then the element inside it (block scans of
// MTP_THREADS entries). If rounding leaves the goal at or past the total, the
// last index with positive weight is taken.
__global__ void __launch_bounds__(MTP_THREADS) mtp_reject_sample_kernel(const float* __restrict__ target,
                                                                       const float* __restrict__ draft, int vocab,
                                                                       int chunks, const MtpChunk* __restrict__ parts,
                                                                       const int32_t* __restrict__ meta,
                                                                       const float* __restrict__ uniforms, int n,
                                                                       int32_t* __restrict__ out) {
  __shared__ int s_chunk, s_mode, s_first, s_last;
  __shared__ float s_before, s_goal, s_gmax;
  __shared__ float scan[MTP_THREADS];
  const int row = meta[0];
  const float* t = target + (size_t)row * vocab;
  const float* d = draft + (size_t)row * vocab;
  if (threadIdx.x == 0) {
    float rtotal = 0.0f, gmax = -INFINITY;
    for (int c = 0; c < chunks; ++c) {
      rtotal += parts[c].residual;
      gmax = fmaxf(gmax, parts[c].tmax);
    }
    const int mode = (meta[1] != 0 && rtotal > 0.0f) ? 1 : 0;  // 1 residual, 0 target
    float total = 0.0f;
    for (int c = 0; c < chunks; ++c) total += mode ? parts[c].residual : (parts[c].tsum > 0.0f ? parts[c].tsum * expf(parts[c].tmax - gmax) : 0.0f);
    const float goal = uniforms[n] * total;
    float before = 0.0f;
    int chosen = -1, last = 0;
    for (int c = 0; c < chunks; ++c) {
      const float w = mode ? parts[c].residual : (parts[c].tsum > 0.0f ? parts[c].tsum * expf(parts[c].tmax - gmax) : 0.0f);
      if (w > 0.0f) last = c;
      if (chosen < 0 && w > 0.0f && before + w > goal) chosen = c;
      if (chosen < 0) before += w;
    }
    if (chosen < 0) {  // goal at or past the total: the last chunk with weight
      chosen = last;
      before = 0.0f;
      for (int c = 0; c < last; ++c) before += mode ? parts[c].residual : (parts[c].tsum > 0.0f ? parts[c].tsum * expf(parts[c].tmax - gmax) : 0.0f);
    }
    s_chunk = chosen;
    s_before = before;
    s_goal = goal;
    s_gmax = gmax;
    s_mode = mode;
    s_first = 0x7fffffff;
    s_last = -1;
  }
  __syncthreads();
  const int lo = s_chunk * MTP_CHUNK, hi = min(vocab, lo + MTP_CHUNK);
  float running = s_before;
  for (int base = lo; base < hi; base += MTP_THREADS) {
    const int i = base + threadIdx.x;
    float w = 0.0f;
    if (i < hi) w = s_mode ? fmaxf(expf(t[i]) - expf(d[i]), 0.0f) : expf(t[i] - s_gmax);
    scan[threadIdx.x] = w;
    __syncthreads();
    for (int off = 1; off < MTP_THREADS; off <<= 1) {  // inclusive scan
      const float add = (int)threadIdx.x >= off ? scan[threadIdx.x - off] : 0.0f;
      __syncthreads();
      scan[threadIdx.x] += add;
      __syncthreads();
    }
    if (w > 0.0f) {
      atomicMax(&s_last, i);
      if (running + scan[threadIdx.x] > s_goal) atomicMin(&s_first, i);
    }
    running += scan[MTP_THREADS - 1];
    __syncthreads();
    if (s_first != 0x7fffffff) break;  // block-uniform: read after the barrier
  }
  if (threadIdx.x == 0) out[1] = s_first != 0x7fffffff ? s_first : (s_last >= 0 ? s_last : lo);
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT size_t wm_mtp_workspace_size(int32_t drafts, int32_t vocab) {
  if (drafts < 0 || vocab < 1) return 0;
  const size_t chunks = ((size_t)vocab + MTP_CHUNK - 1) / MTP_CHUNK;
  return 256 + (size_t)(drafts + 1) * chunks * sizeof(MtpArg) + chunks * sizeof(MtpChunk);
}

WM_EXPORT int wm_mtp_verify_greedy(const float* target_logits, const int32_t* drafts, int32_t n_drafts, int32_t vocab,
                                   int32_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (n_drafts < 0 || n_drafts + 1 > MTP_MAX_ROWS) fail("wm_mtp_verify_greedy: drafts must be in 0..15");
    if (vocab < 1 || (vocab + MTP_CHUNK - 1) / MTP_CHUNK > MTP_MAX_CHUNKS)
      fail("wm_mtp_verify_greedy: vocab must be in 1..4194304");
    if (!target_logits || !out || !workspace || (n_drafts > 0 && !drafts)) fail("wm_mtp_verify_greedy: null pointer");
    if (workspace_bytes < wm_mtp_workspace_size(n_drafts, vocab) || (uintptr_t)workspace % 16)
      fail("wm_mtp_verify_greedy: workspace too small or misaligned");
    const int chunks = (vocab + MTP_CHUNK - 1) / MTP_CHUNK;
    MtpArg* parts = reinterpret_cast<MtpArg*>((char*)workspace + 256);
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(mtp_argmax_chunks_kernel, dim3(chunks, n_drafts + 1), dim3(MTP_THREADS), 0, s, target_logits,
                       vocab, chunks, parts);
    check_launch("mtp_argmax_chunks");
    hipLaunchKernelGGL(mtp_greedy_decide_kernel, dim3(1), dim3(MTP_THREADS), 0, s, parts, chunks, drafts, n_drafts, out);
    check_launch("mtp_greedy_decide");
  });
}

WM_EXPORT int wm_mtp_verify_rejection(const float* target_logp, const float* draft_logp, const int32_t* drafts,
                                      int32_t n_drafts, int32_t vocab, const float* uniforms, int32_t* out,
                                      void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (n_drafts < 0 || n_drafts + 1 > MTP_MAX_ROWS) fail("wm_mtp_verify_rejection: drafts must be in 0..15");
    if (vocab < 1 || (vocab + MTP_CHUNK - 1) / MTP_CHUNK > MTP_MAX_CHUNKS)
      fail("wm_mtp_verify_rejection: vocab must be in 1..4194304");
    if (!target_logp || !uniforms || !out || !workspace || (n_drafts > 0 && (!drafts || !draft_logp)))
      fail("wm_mtp_verify_rejection: null pointer");
    if (workspace_bytes < wm_mtp_workspace_size(n_drafts, vocab) || (uintptr_t)workspace % 16)
      fail("wm_mtp_verify_rejection: workspace too small or misaligned");
    const int chunks = (vocab + MTP_CHUNK - 1) / MTP_CHUNK;
    int32_t* meta = reinterpret_cast<int32_t*>(workspace);
    MtpChunk* parts = reinterpret_cast<MtpChunk*>((char*)workspace + 256 + (size_t)(n_drafts + 1) * chunks * sizeof(MtpArg));
    // With no drafts the draft pointer is never read (the row sampled is the target's).
    const float* dl = draft_logp ? draft_logp : target_logp;
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(mtp_reject_decide_kernel, dim3(1), dim3(64), 0, s, target_logp, dl, drafts, n_drafts, vocab,
                       uniforms, meta, out);
    check_launch("mtp_reject_decide");
    hipLaunchKernelGGL(mtp_reject_chunks_kernel, dim3(chunks), dim3(MTP_THREADS), 0, s, target_logp, dl, vocab, meta,
                       parts);
    check_launch("mtp_reject_chunks");
    hipLaunchKernelGGL(mtp_reject_sample_kernel, dim3(1), dim3(MTP_THREADS), 0, s, target_logp, dl, vocab, chunks,
                       parts, meta, uniforms, n_drafts, out);
    check_launch("mtp_reject_sample");
  });
}

}  // extern "C"
