// Message words between workgroups of one launch: a 64-bit word carries a value and an epoch,
// written and read with agent-scope relaxed atomics, so a reader polls the data itself and
// needs no flag, no grid barrier and no L2-wide fence (on MI355X an agent-scope release or
// acquire writes back or invalidates the XCD's whole L2). Every launch advances its epochs,
// so words left by an earlier launch never match.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace wm {

constexpr uint32_t MSG_SPIN_LIMIT = 1u << 20;  // poll rounds before a wait gives up
constexpr uint32_t MSG_STALLED = 1;            // status value a wait that ran out raises

__device__ __forceinline__ void ll_put(uint64_t* p, uint32_t bits, uint32_t epoch) {
  __hip_atomic_store(p, ((uint64_t)epoch << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Reads base[index(m)] for m < N (index(m) < 0: no word) with all N loads in flight,
// re-polls only the words whose top EBITS bits do not equal `epoch` (mod 2^EBITS)
// yet, then hands each word to store(m, word). Bounded: after MSG_SPIN_LIMIT rounds it
// raises the status word to MSG_STALLED; it also stops (ok = false) once another
// workgroup has raised the status word.
template <int N, int EBITS = 32, typename Index, typename Store>
__device__ __forceinline__ void ll_gather_at(const uint64_t* base, Index index, uint32_t epoch, uint32_t* status,
                                             bool& ok, Store store, uint32_t* rounds = nullptr) {
  const uint32_t want = EBITS == 32 ? epoch : (epoch & ((1u << EBITS) - 1));
  auto tag = [](uint64_t v) { return (uint32_t)(v >> (64 - EBITS)); };
  uint64_t v[N];
#pragma unroll
  for (int m = 0; m < N; ++m) {
    const int i = index(m);
    v[m] = i >= 0 ? __hip_atomic_load(&base[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                  : (uint64_t)want << (64 - EBITS);
  }
  uint32_t spins = 0;
  while (ok) {
    bool ready = true;
#pragma unroll
    for (int m = 0; m < N; ++m) ready &= tag(v[m]) == want;
    if (ready) break;
    if (++spins > MSG_SPIN_LIMIT) {
      __hip_atomic_store(status, MSG_STALLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = false;
      break;
    }
    if ((spins & 255) == 0 && __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
      ok = false;
      break;
    }
    // no sleep between rounds: each round already waits for its loads to return (a 64- or
    // 128-clock pause there measured the same or up to 3% slower)
#pragma unroll
    for (int m = 0; m < N; ++m) {
      const int i = index(m);
      if (i >= 0 && tag(v[m]) != want)
        v[m] = __hip_atomic_load(&base[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
#pragma unroll
  for (int m = 0; m < N; ++m)
    if (index(m) >= 0) store(m, v[m]);
  if (rounds) *rounds = spins;
}

// ll_gather_at over base[first + m * stride] (indices below limit); store(index, word).
template <int N, int EBITS = 32, typename Store>
__device__ __forceinline__ void ll_gather(const uint64_t* base, int first, int stride, int limit, uint32_t epoch,
                                          uint32_t* status, bool& ok, Store store, uint32_t* rounds = nullptr) {
  ll_gather_at<N, EBITS>(
      base, [&](int m) { const int i = first + m * stride; return i < limit ? i : -1; }, epoch, status, ok,
      [&](int m, uint64_t v) { store(first + m * stride, v); }, rounds);
}

// Workgroup barrier over LDS only: this wave's LDS operations complete (lgkmcnt 0),
// then the hardware barrier. __syncthreads() would also wait for this wave's global
// stores, and since the vector memory counter drains in order, for every weight load
// still in flight; message words need no such wait (their epochs order them).
__device__ __forceinline__ void ds_barrier() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited for
  __builtin_amdgcn_s_barrier();
  __asm__ __volatile__("" ::: "memory");
}

// Values that travel two to a message word as 24-bit floats (sign, exponent, 15 mantissa
// bits, rounded to nearest even) under a 16-bit epoch: bits 0-23 the first value, 24-47
// the second, 48-63 the epoch.
__device__ __forceinline__ uint32_t f32_to_f24(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u + 0x7fu + ((u >> 8) & 1u)) >> 8;
}
__device__ __forceinline__ float f24_to_f32(uint32_t b) { return __uint_as_float(b << 8); }
__device__ __forceinline__ uint64_t f24_pair_word(float a, float b, uint32_t epoch) {
  return ((uint64_t)(epoch & 0xffffu) << 48) | ((uint64_t)f32_to_f24(b) << 24) | f32_to_f24(a);
}

}  // namespace wm
