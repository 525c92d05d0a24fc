// One decode layer of the MXFP4 MoE in one launch: the step a decoder layer takes between
// its attention blocks (DecoderLayer.feed_forward -> SparseMoE, qwen4_exp.py:1146 and
// :1036-1051; the native engine's expert step with its pre-norm, router GEMV and shared
// gate, Native/QwenNative/engine.mm:2073-2236), for one token:
//
//   x = bf16(rmsnorm(r) * w_norm);  logits = x . Wr^T;  (idx, w) = softmax top-k;
//   y = sum_k w_k FFN_k(x) + sigmoid(x . g) FFN_shared(x);  r' = r + bf16(y).
//
// The per-layer path launches norm_router, route, gate_up and down (four dependent kernels,
// ~31 us a layer at C2); here 256 workgroups of 4 waves, all resident, run the whole layer
// with two grid-wide exchanges, both in message words (messages.h: value and epoch in one
// 64-bit word, agent-scope relaxed atomics, no L2-wide fences):
//   1. every workgroup normalises r into LDS (x, bf16) and computes its share of the router
//      logits (one wave per expert row, rows loaded before the norm) and publishes them
//      (fp32 | 32-bit epoch); in every workgroup wave 0 gathers all E logits into LDS and all
//      four waves route them redundantly (the wave top-k of route_device.h: same selections as
//      wm_route_softmax_topk on the same logits), each into its own copy of the entries, so no
//      workgroup barrier stands between the top-k and a wave's weight loads;
//   2. gate_up: the (entry, intermediate index) pairs of the K routed experts and the shared one
//      are spread evenly over the 1024 waves, an even number to a wave; each wave streams its
//      gate and up rows (64 lanes x 16 bytes a row chunk), dots them with x held in registers
//      and publishes act two values to a word (24-bit floats | 16-bit epoch);
//   3. down: workgroup b owns output rows [H/256 b, H/256 (b + 1)); its waves split the layer's
//      entries. Each workgroup stores the epoch into its own flag word (256 bytes apart, so no
//      two workgroups write one line: shared counters serialise their atomics) once its waves
//      have issued their act stores; one wave polls the 256 flags (four words a lane a round)
//      and only then do the waves gather their entries' act words into LDS, so no wave polls
//      act words while others still stream weights. The down rows are loaded into registers
//      after the flag store (waves 1-3) or after the flag polls (wave 0): issued earlier, they
//      share the CU's memory queue with the gate_up rows, the flag store and the polls, and
//      the vector memory counter drains in order. Then y = sum_k w_k act_k . Wd_k[o] +
//      gate act_s . Wd_s[o] in fp32 (lanes, then waves).
//
// Exchanges use per-call epochs kept in the state buffer (each workgroup's own word), so the
// same launch can be replayed from a graph; every wait is bounded and raises the status word.
#include <cmath>
#include <string>

#include "messages.h"
#include "moe_internal.h"
#include "route_device.h"
#include "wm_common.h"

// Phase timestamps of the profiling build (phase_trace_lds.h; nothing in the library): slot
// epoch % 128, points 0 start, 1 x in LDS, 2 logits published, 3 logits in LDS (every wave),
// 4 routed (the wave's entries in LDS), 5 gate_up computed and published, 6 act gathered,
// 7 done; 8 top-k done, 10 act flags complete, 11 flag stored and (waves 1-3) down rows
// issued, 12 gate_up rows issued, 13 first pair computed.
#ifndef WM_DS_TRACE
#define WM_DS_TRACE(layer, point)
#endif
#ifndef WM_DS_TRACE_FLUSH
#define WM_DS_TRACE_FLUSH(layer)
#endif

namespace wm {
namespace dl {

constexpr int WGS = 256;                 // workgroups (all resident: 256 threads, ~170 VGPRs)
constexpr int WAVES = 4;
constexpr int THREADS = 64 * WAVES;
constexpr int MAX_ENTRIES = 12;          // routed (k <= 11) + shared
constexpr int MAX_EXPERTS = 1024;        // router rows: 4 per workgroup
constexpr uint32_t ST_STALLED = MSG_STALLED, ST_NO_ROUTE = 4;

// State buffer (zero-filled once by the caller): logit words, act words, per-workgroup
// epochs and the status word.
struct Layout {
  size_t logits, act, flags, epoch, status, total;
};
__host__ __device__ inline Layout layout(int experts, int inter) {
  Layout d;
  size_t at = 0;
  d.logits = at;  at += (size_t)MAX_EXPERTS * 8;
  d.act = at;     at += (size_t)MAX_ENTRIES * (inter / 2) * 8;
  d.flags = at;   at += (size_t)WGS * 256;
  d.epoch = at;   at += (size_t)WGS * 4;
  d.status = at;  at += 256;
  d.total = at;
  (void)experts;
  return d;
}

struct Params {
  const float* r;            // [H] fp32 residual
  float* r_out;              // [H] r + bf16(y) (may alias r), nullable
  const uint16_t* norm_w;    // [H] bf16 RMSNorm weight, nullable (no weight)
  float eps;
  const uint16_t* router;    // [E, H] bf16
  const uint16_t* gate_vec;  // [H] bf16 shared-expert gate, nullable (ungated shared expert)
  wm_mxfp4_experts routed;
  wm_mxfp4_experts shared;
  int has_shared;
  int experts, k, norm_topk;
  uint16_t* y;               // [H] bf16 MoE output, nullable
  uint16_t* x_out;           // [H] bf16 normalised input, nullable
  float* logits_out;         // [E] fp32, nullable
  int32_t* idx_out;          // [k] int32, nullable
  float* w_out;              // [k] fp32, nullable
  uint8_t* state;
};

// The fields of an expert table the kernel reads, staged in LDS once per launch, and the
// regions of each entry of the call: per-entry selections then read LDS, never the kernel
// arguments through a lane-dependent address (a vector load of the argument segment whose
// latency each later weight load would wait for).
struct TableDesc {
  const uint8_t* gate_up;
  const uint8_t* gate_up_scales;
  const uint8_t* down;
  const uint8_t* down_scales;
  int64_t gate_up_stride, gate_up_scales_stride, down_stride, down_scales_stride;
  const int32_t* slots;
  int up_first;
  float limit;
};
__device__ __forceinline__ void stage_table(TableDesc& d, const wm_mxfp4_experts& t) {
  d.gate_up = (const uint8_t*)t.gate_up;
  d.gate_up_scales = (const uint8_t*)t.gate_up_scales;
  d.down = (const uint8_t*)t.down;
  d.down_scales = (const uint8_t*)t.down_scales;
  d.gate_up_stride = t.gate_up_stride;
  d.gate_up_scales_stride = t.gate_up_scales_stride;
  d.down_stride = t.down_stride;
  d.down_scales_stride = t.down_scales_stride;
  d.slots = t.slots;
  d.up_first = t.up_first;
  d.limit = t.swiglu_limit;
}
struct EntryRegions {
  const uint8_t* gate_up;
  const uint8_t* gate_up_scales;
  const uint8_t* down;
  const uint8_t* down_scales;
  int up_first;
  float limit;
};

// Workgroup b's act flag (its word, 256 bytes from the next): the call's epoch, stored once
// per call on every path.
__device__ __forceinline__ void mark_done(uint32_t* flags, int b, uint32_t epoch) {
  __hip_atomic_store(&flags[b * 64], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Row chunks of 1 KB (64 lanes x 16 bytes): a gate_up row of H / 2 bytes spans CH chunks; the
// lanes past the row's end in the last chunk load nothing.
template <int H>
struct GateUpShape {
  static constexpr int CH = (H / 2 + 1023) / 1024;
};

// The down rows' lane split (as the per-layer decode kernel's): LPR lanes per row, GPL groups
// of 32 values per lane, lanes past the row's last group idle.
template <int I>
struct DownShape {
  static constexpr int G = I / 32;
  static constexpr int LPR = G >= 64 ? 64 : (G > 16 ? (G % 16 == 0 ? 16 : 4) : (G > 8 ? 16 : (G > 4 ? 8 : 4)));
  static constexpr int GPL = (G + LPR - 1) / LPR;
  static constexpr int NS = 64 / LPR;  // rows a wave reads at once
};

template <int H, int I, int PMAX>
__global__ void __launch_bounds__(THREADS) moe_layer_kernel(Params p) {
  static_assert(H % WGS == 0 && I % 32 == 0, "fused decode layer shape");
  static_assert(PMAX % 2 == 0, "act pairs: an even number of (entry, index) pairs a wave");
  constexpr int CH = GateUpShape<H>::CH;
  using DS = DownShape<I>;
  constexpr int RPB = H / WGS;                          // output rows of a workgroup
  constexpr int STEPS = (RPB + DS::NS - 1) / DS::NS;    // down row loads per entry
  constexpr int EPW = (MAX_ENTRIES + WAVES - 1) / WAVES;  // down entries per wave

  __shared__ __attribute__((aligned(16))) uint32_t xs[H / 2];  // x as bf16 pairs
  __shared__ float red[2 * WAVES];
  // every wave routes the same logits and keeps its own copy of the entries
  __shared__ float rw_w[WAVES][MAX_ENTRIES];
  __shared__ int rres_w[WAVES][MAX_ENTRIES];  // entry resident (its slot map entry, if any, >= 0)
  __shared__ __attribute__((aligned(16))) float lg[MAX_EXPERTS];
  __shared__ float part[WAVES][RPB];
  // gathered act rows, value v of a row at 4 (G q + g) + c for v = 32 g + 4 q + c (G = I / 32):
  // the down lanes reading four values of groups g, g + 1, ... hit consecutive 16 bytes
  __shared__ __attribute__((aligned(16))) float acts[MAX_ENTRIES][I];
  __shared__ TopkScratch topk[WAVES];
  __shared__ TableDesc tdesc[2];  // 0 routed, 1 shared
  __shared__ EntryRegions ent_w[WAVES][MAX_ENTRIES];
  __shared__ uint32_t epoch_s;
  __shared__ int fail_s;

  const int b = blockIdx.x, tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const Layout L = layout(p.experts, I);
  uint64_t* logit_words = reinterpret_cast<uint64_t*>(p.state + L.logits);
  uint64_t* act_words = reinterpret_cast<uint64_t*>(p.state + L.act);
  uint32_t* flags = reinterpret_cast<uint32_t*>(p.state + L.flags);  // one per 256 bytes
  uint32_t* epochs = reinterpret_cast<uint32_t*>(p.state + L.epoch);
  uint32_t* status = reinterpret_cast<uint32_t*>(p.state + L.status);
  const int E = p.experts, K = p.k;
  const int NE = K + (p.has_shared ? 1 : 0);

  // ---- router rows (before the norm: they do not depend on x) and the epoch
  const int e_row = b + WGS * wave;  // this wave's router row, if any
  uint4 rrow[H / 512];                // H bf16 = H / 512 chunks of 1 KB (64 lanes x 16 bytes)
  const bool has_row = e_row < E;
  if (has_row) {
#pragma unroll
    for (int c = 0; c < H / 512; ++c)
      rrow[c] = gload16(p.router + (int64_t)e_row * H + 512 * c + 8 * lane);
  }
  uint4 grow[H / 512];  // the shared gate vector, on the last wave
  const bool gate_wave = wave == WAVES - 1 && p.gate_vec != nullptr;
  if (gate_wave) {
#pragma unroll
    for (int c = 0; c < H / 512; ++c) grow[c] = gload16(p.gate_vec + 512 * c + 8 * lane);
  }
  if (tid == 0) {
    epoch_s = epochs[b] + 1;
    fail_s = 0;
    stage_table(tdesc[0], p.routed);
    stage_table(tdesc[1], p.shared);
  }
  // this workgroup's residual rows, for the residual add at the end
  const float r_rows = tid < RPB ? p.r[RPB * b + tid] : 0.0f;
  WM_DS_TRACE((epochs[b] + 1) & 127, 0);

  // ---- x = bf16(rmsnorm(r) * w) (wm_norm_router's arithmetic): each thread H / 256 values
  static_assert(H % 512 == 0, "router rows of whole 1 KB chunks, an even share of r per thread");
  constexpr int VPT = H / THREADS;
  float rv[VPT];
#pragma unroll
  for (int q = 0; q < VPT; q += 2) {
    const float2 v = *reinterpret_cast<const float2*>(p.r + VPT * tid + q);
    rv[q] = v.x;
    rv[q + 1] = v.y;
  }
  float ss = 0.0f;
#pragma unroll
  for (int q = 0; q < VPT; ++q) ss += rv[q] * rv[q];
  ss = segment_sum<64>(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float inv = rsqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + p.eps);
  const uint32_t epoch = epoch_s;
#pragma unroll
  for (int q = 0; q < VPT; q += 2) {
    float a = rv[q] * inv, c = rv[q + 1] * inv;
    if (p.norm_w) {
      const uint32_t wpair = *reinterpret_cast<const uint32_t*>(p.norm_w + VPT * tid + q);
      a *= bf16_bits_to_f32(wpair & 0xffffu);
      c *= bf16_bits_to_f32(wpair >> 16);
    }
    xs[(VPT * tid + q) / 2] = (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(c) << 16);
  }
  __syncthreads();
  WM_DS_TRACE(epoch & 127, 1);
  if (b == 0 && p.x_out)
    for (int i = tid; i < H / 2; i += THREADS) reinterpret_cast<uint32_t*>(p.x_out)[i] = xs[i];

  // ---- router logits of this workgroup's rows, published; the shared gate
  if (has_row) {
    float a = 0.0f;
#pragma unroll
    for (int c = 0; c < H / 512; ++c) {
      const uint4 wq = rrow[c];
      const uint4 xq = *reinterpret_cast<const uint4*>(&xs[(512 * c + 8 * lane) / 2]);
      a = dot2_bf16(bits_to_bf16x2(wq.x), bits_to_bf16x2(xq.x), a);
      a = dot2_bf16(bits_to_bf16x2(wq.y), bits_to_bf16x2(xq.y), a);
      a = dot2_bf16(bits_to_bf16x2(wq.z), bits_to_bf16x2(xq.z), a);
      a = dot2_bf16(bits_to_bf16x2(wq.w), bits_to_bf16x2(xq.w), a);
    }
    a = segment_sum<64>(a);
    if (lane == 0) {
      ll_put(&logit_words[e_row], __float_as_uint(a), epoch);
      if (p.logits_out) p.logits_out[e_row] = a;
    }
  }
  float gate = 1.0f;
  if (gate_wave) {
    float a = 0.0f;
#pragma unroll
    for (int c = 0; c < H / 512; ++c) {
      const uint4 wq = grow[c];
      const uint4 xq = *reinterpret_cast<const uint4*>(&xs[(512 * c + 8 * lane) / 2]);
      a = dot2_bf16(bits_to_bf16x2(wq.x), bits_to_bf16x2(xq.x), a);
      a = dot2_bf16(bits_to_bf16x2(wq.y), bits_to_bf16x2(xq.y), a);
      a = dot2_bf16(bits_to_bf16x2(wq.z), bits_to_bf16x2(xq.z), a);
      a = dot2_bf16(bits_to_bf16x2(wq.w), bits_to_bf16x2(xq.w), a);
    }
    a = segment_sum<64>(a);
    gate = 1.0f / (1.0f + __expf(-a));
  }
  if (gate_wave && lane == 0) red[4] = gate;
  WM_DS_TRACE(epoch & 127, 2);

  // ---- wave 0 gathers every logit (bounded polls) into LDS; every wave routes them (the same
  // selections: one function of the same values) and sets up its own copy of the entries, so
  // no barrier separates the top-k from the weight loads
  constexpr int PER = MAX_EXPERTS / 64;
  if (wave == 0) {
    bool ok = true;
    float lv[PER];  // logit of expert lane + 64 m in lv[m]
    ll_gather_at<PER>(
        logit_words, [&](int m) { return lane + 64 * m < E ? lane + 64 * m : -1; }, epoch, status, ok,
        [&](int m, uint64_t v) { lv[m] = __uint_as_float((uint32_t)v); });
    ok = __all(ok);
    if (!ok && lane == 0) fail_s = 1;
#pragma unroll
    for (int m = 0; m < PER; ++m) lg[lane + 64 * m] = lv[m];
  }
  ds_barrier();
  WM_DS_TRACE(epoch & 127, 3);
  if (fail_s) {  // every workgroup gathers the same words, so all leave here
    if (tid == 0) {
      mark_done(flags, b, epoch);
      epochs[b] = epoch;
    }
    return;
  }
  float* rw = rw_w[wave];
  int* rres = rres_w[wave];
  EntryRegions* ent = ent_w[wave];
  {
    int sel = 0;
    float w = 0.0f, full;
    if (E <= 512) {
      float v8[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) v8[m] = lg[lane + 64 * m];
      wave_route_softmax_vals<8>(v8, E, K, p.norm_topk != 0, lane, topk[wave], sel, w, false, full);
    } else {
      float lv[PER];
#pragma unroll
      for (int m = 0; m < PER; ++m) lv[m] = lg[lane + 64 * m];
      wave_route_softmax_vals<PER>(lv, E, K, p.norm_topk != 0, lane, topk[wave], sel, w, false, full);
    }
    WM_DS_TRACE(epoch & 127, 8);
    // a selection outside [0, E) (fewer than k selectable logits, e.g. NaN) ends the call
    if (__any(lane < K && (sel < 0 || sel >= E))) {  // the same in every wave and workgroup
      if (tid == 0) {
        __hip_atomic_store(status, ST_NO_ROUTE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mark_done(flags, b, epoch);
        epochs[b] = epoch;
      }
      return;
    }
    if (wave == 0 && b == 0 && lane < K) {
      if (p.idx_out) p.idx_out[lane] = sel;
      if (p.w_out) p.w_out[lane] = w;
    }
    if (lane < NE) {  // the entries' regions and residency (a non-resident expert contributes nothing)
      const int e = lane < K ? sel : -1;  // -1: the shared expert
      const TableDesc& t = tdesc[e < 0 ? 1 : 0];
      int64_t slot = e < 0 ? 0 : e;
      bool resident = true;
      if (t.slots) {
        const int32_t s = gload<int32_t>(t.slots + slot);
        resident = s >= 0;
        slot = s < 0 ? 0 : s;  // not resident: slot 0 keeps every address inside the pool
      }
      rres[lane] = resident;
      rw[lane] = e < 0 ? (p.gate_vec ? red[4] : 1.0f) : w;
      EntryRegions r;
      r.gate_up = t.gate_up + slot * t.gate_up_stride;
      r.gate_up_scales = t.gate_up_scales + slot * t.gate_up_scales_stride;
      r.down = t.down + slot * t.down_stride;
      r.down_scales = t.down_scales + slot * t.down_scales_stride;
      r.up_first = t.up_first;
      r.limit = t.limit;
      ent[lane] = r;
    }
    wave_lds_sync();
  }
  WM_DS_TRACE(epoch & 127, 4);

  // down rows of this wave's entries (wave, wave + 4, ...) for the workgroup's rows, loaded
  // into registers after the act publish (issue_down)
  const int o0 = RPB * b;
  const int slot = lane / DS::LPR, gl = lane % DS::LPR;
  uint4 dq[EPW][STEPS][DS::GPL];
  uint32_t ds_[EPW][STEPS][DS::GPL];
  // ---- gate_up: this wave's (entry, intermediate index) pairs
  {
    const int gw = b * WAVES + wave, nwaves = WGS * WAVES;
    const int total = NE * I;  // even: I is
    const int per = 2 * ((total + 2 * nwaves - 1) / (2 * nwaves));
    const int n0 = gw * per;
    uint32_t xr[CH][16];  // x values [1024 c + 32 lane, +32) of a row chunk (H / 2 bytes a row)
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool in = 1024 * c + 16 * lane < H / 2;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = in ? *reinterpret_cast<const uint4*>(&xs[(2048 * c + 32 * lane) / 2 + 4 * q])
                           : make_uint4(0, 0, 0, 0);
        xr[c][4 * q] = v.x; xr[c][4 * q + 1] = v.y; xr[c][4 * q + 2] = v.z; xr[c][4 * q + 3] = v.w;
      }
    }
    uint4 wq[PMAX][2][CH];
    uint32_t sq[PMAX][2][CH];
    float actv[PMAX];
    // every load issued (dead pairs read entry 0's row 0, lanes past a row's end its first
    // chunk); the values are masked where they are used
#pragma unroll
    for (int u = 0; u < PMAX; ++u) {
      const int n = n0 + u;
      const bool live = u < per && n < total;
      const int entry = live ? n / I : 0, i = live ? n % I : 0;
      const EntryRegions& r = ent[entry];
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // h 0: gate row, 1: up row
        const int row = (h ^ r.up_first) ? I + i : i;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int off = 1024 * c + 16 * lane;
          const int offc = off < H / 2 ? off : 0;
          wq[u][h][c] = gload16(r.gate_up + (int64_t)row * (H / 2) + offc);
          sq[u][h][c] = gload<uint8_t>(r.gate_up_scales + (int64_t)row * (H / 32) + offc / 16);
        }
      }
    }
    WM_DS_TRACE(epoch & 127, 12);
#pragma unroll
    for (int u = 0; u < PMAX; ++u) {
      if (u == 1) WM_DS_TRACE(epoch & 127, 13);
      const int n = n0 + u;
      const bool live = u < per && n < total;  // wave-uniform
      const int entry = live ? n / I : 0, i = live ? n % I : 0;
      float g2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const uint32_t words[4] = {wq[u][h][c].x, wq[u][h][c].y, wq[u][h][c].z, wq[u][h][c].w};
          // lanes past the row's end: scale 0 (a 255 byte would be inf, inf x 0 NaN)
          const float sc = 1024 * c + 16 * lane < H / 2 ? e8m0_scale_operand(sq[u][h][c]) : 0.0f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            wm_bf16x2 wv[4];
            fp4x8_to_bf16(words[j], sc, wv);
#pragma unroll
            for (int m = 0; m < 4; ++m) a = dot2_bf16(wv[m], bits_to_bf16x2(xr[c][4 * j + m]), a);
          }
        }
        g2[h] = segment_sum<64>(a);
      }
      const float limit = ent[entry].limit;
      float g = g2[0], u2 = g2[1];  // wave-uniform (segment_sum gives every lane the sum)
      if (limit > 0.0f) {
        g = fminf(g, limit);
        u2 = fminf(fmaxf(u2, -limit), limit);
      }
      actv[u] = live && rres[entry] ? silu(g) * u2 : 0.0f;
    }
    // lane q publishes the word of pairs n0 + 2q and n0 + 2q + 1 (same entry: I is even)
#pragma unroll
    for (int q = 0; q < PMAX / 2; ++q) {
      const int n = n0 + 2 * q;
      if (lane == q && 2 * q < per && n < total)
        __hip_atomic_store(&act_words[n / 2], f24_pair_word(actv[2 * q], actv[2 * q + 1], epoch), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  WM_DS_TRACE(epoch & 127, 5);
  // Every down load is issued (lanes and entries past the end read entry 0's first row, in
  // bounds) so none waits for another; their values are masked where they are used.
  auto issue_down = [&]() {
#pragma unroll
    for (int j = 0; j < EPW; ++j) {
      const int entry = wave + WAVES * j;
      const EntryRegions& r = ent[entry < NE ? entry : 0];
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        const int row = st * DS::NS + slot;
        const int o = o0 + (row < RPB ? row : 0);
#pragma unroll
        for (int gp = 0; gp < DS::GPL; ++gp) {
          const int g = gl + gp * DS::LPR;
          const int gc = g < DS::G ? g : 0;
          dq[j][st][gp] = gload16(r.down + (int64_t)o * (I / 2) + 16 * gc);
          ds_[j][st][gp] = gload<uint8_t>(r.down_scales + (int64_t)o * DS::G + gc);
        }
      }
    }
  };
  // ---- wait for every workgroup's act words: once its four waves have issued their act
  // stores, the workgroup stores the epoch into its flag (without waiting for the stores'
  // acknowledgements: the gather below checks every word's epoch and re-polls a late one);
  // wave 0 polls the 256 flags, four a lane (with a pause between rounds), instead of every
  // wave polling its act words while others still stream weights
  ds_barrier();
  if (tid == 0) mark_done(flags, b, epoch);
  if (wave != 0) issue_down();  // after the flag store, which would queue behind them
  WM_DS_TRACE(epoch & 127, 11);
  if (wave == 0) {
    static_assert(WGS == 4 * 64, "four flags a lane");
    bool ok = true;
    auto behind = [&]() {
      uint32_t f[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        f[j] = __hip_atomic_load(&flags[(lane + 64 * j) * 64], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bool late = false;
#pragma unroll
      for (int j = 0; j < 4; ++j) late |= (int32_t)(f[j] - epoch) < 0;
      return late;
    };
    uint32_t spins = 0;
    while (behind()) {
      if (++spins > MSG_SPIN_LIMIT) {
        __hip_atomic_store(status, ST_STALLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = false;
        break;
      }
      if ((spins & 63) == 0 && __hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (!__all(ok) && lane == 0) fail_s = 1;
  }
  if (wave == 0) issue_down();  // after the polls, which would wait for these loads
  ds_barrier();
  WM_DS_TRACE(epoch & 127, 10);
  if (fail_s) {
    if (tid == 0) epochs[b] = epoch;
    return;
  }
  // ---- gather the act rows of this wave's down entries (wave, wave + 4, ...) into LDS (every
  // word still checked against the epoch: the flags order nothing)
  {
    constexpr int WPE = I / 2;             // act words an entry
    constexpr int NPL = (WPE + 63) / 64;   // words a lane gathers per entry
    bool ok = true;
    ll_gather_at<EPW * NPL, 16>(
        act_words,
        [&](int m) {
          const int entry = wave + WAVES * (m / NPL), w = (m % NPL) * 64 + lane;
          return entry < NE && w < WPE ? entry * WPE + w : -1;
        },
        epoch, status, ok,
        [&](int m, uint64_t v) {
          const int entry = wave + WAVES * (m / NPL), w = (m % NPL) * 64 + lane;
          const int v0 = 2 * w, at = 4 * (DS::G * ((v0 % 32) / 4) + v0 / 32) + v0 % 4;
          *reinterpret_cast<float2*>(&acts[entry][at]) =
              make_float2(f24_to_f32((uint32_t)v & 0xffffffu), f24_to_f32((uint32_t)(v >> 24) & 0xffffffu));
        });
    if (!ok) fail_s = 1;
  }
  __syncthreads();
  WM_DS_TRACE(epoch & 127, 6);
  if (fail_s) {
    if (tid == 0) epochs[b] = epoch;
    return;
  }

  // ---- down: y[o] = sum over the wave's entries of w act . Wd[o]
  float acc[STEPS];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) acc[st] = 0.0f;
#pragma unroll
  for (int j = 0; j < EPW; ++j) {
    const int entry = wave + WAVES * j;
    const bool live = entry < NE && rres[entry < NE ? entry : 0];  // wave-uniform
    const float w = live ? rw[entry] : 0.0f;
    const float* arow = acts[live ? entry : 0];
#pragma unroll
    for (int gp = 0; gp < DS::GPL; ++gp) {
      const int g = gl + gp * DS::LPR;
      float av[32];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float4 v = live && g < DS::G ? *reinterpret_cast<const float4*>(arow + 4 * (DS::G * q + g))
                                            : make_float4(0, 0, 0, 0);
        av[4 * q] = v.x; av[4 * q + 1] = v.y; av[4 * q + 2] = v.z; av[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        // rows past the block, groups past the row and dead entries: scale 0
        const bool valid = live && st * DS::NS + slot < RPB && g < DS::G;
        const float scale = valid ? e8m0_scale_operand(ds_[j][st][gp]) : 0.0f;
        const uint32_t words[4] = {dq[j][st][gp].x, dq[j][st][gp].y, dq[j][st][gp].z, dq[j][st][gp].w};
        float s = 0.0f;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) {
            wm_f32x2 wf;
            switch (bb) {
              case 0: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[jj], scale, 0); break;
              case 1: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[jj], scale, 1); break;
              case 2: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[jj], scale, 2); break;
              default: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[jj], scale, 3); break;
            }
            s = fmaf(wf[0], av[8 * jj + 2 * bb], s);
            s = fmaf(wf[1], av[8 * jj + 2 * bb + 1], s);
          }
        }
        acc[st] = fmaf(w, s, acc[st]);
      }
    }
  }
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const float v = segment_sum<DS::LPR>(acc[st]);
    const int row = st * DS::NS + slot;
    if (gl == 0 && row < RPB) part[wave][row] = v;
  }
  __syncthreads();
  if (tid < RPB) {
    const int o = o0 + tid;
    const float v = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
    const uint16_t yb = f32_to_bf16_bits(v);
    if (p.y) p.y[o] = yb;
    if (p.r_out) p.r_out[o] = r_rows + bf16_bits_to_f32(yb);
  }
  WM_DS_TRACE(epoch & 127, 7);
  WM_DS_TRACE_FLUSH(epoch & 127);
  if (tid == 0) epochs[b] = epoch;
}

}  // namespace dl

// Shapes with a fused instantiation (hidden, intermediate).
#define WM_DL_SHAPES(X) X(1024, 512) X(2048, 512)

bool moe_layer_fused_supports(int hidden, int inter, int k) {
  if (k < 1 || k > dl::MAX_ENTRIES - 1) return false;
#define WM_DL_TRY(HH, II) if (hidden == HH && inter == II) return true;
  WM_DL_SHAPES(WM_DL_TRY)
#undef WM_DL_TRY
  return false;
}

size_t moe_layer_state_size(int experts, int inter) { return dl::layout(experts, inter).total; }

void moe_layer_fused(const dl::Params& p, int hidden, int inter, hipStream_t s) {
#define WM_DL_RUN(HH, II)                                                                                     \
  if (hidden == HH && inter == II) {                                                                           \
    constexpr int PMAX = 2 * ((dl::MAX_ENTRIES * II + 2 * dl::WGS * dl::WAVES - 1) / (2 * dl::WGS * dl::WAVES)); \
    hipLaunchKernelGGL((dl::moe_layer_kernel<HH, II, PMAX>), dim3(dl::WGS), dim3(dl::THREADS), 0, s, p);       \
    check_launch("moe_layer_kernel");                                                                          \
    return;                                                                                                    \
  }
  WM_DL_SHAPES(WM_DL_RUN)
#undef WM_DL_RUN
  fail("moe layer: no fused instantiation for this shape");
}

// r_out = r + bf16(y) for the unfused path.
__global__ void __launch_bounds__(256) residual_add_kernel(const float* __restrict__ r, const uint16_t* __restrict__ y,
                                                           int n, float* __restrict__ r_out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) r_out[i] = r[i] + bf16_bits_to_f32(y[i]);
}

// The unfused path's buffers, after the fused path's state in the same caller buffer.
struct Scratch {
  size_t x, logits, idx, w, y, act, total;
};
static Scratch scratch_layout(int experts, int hidden, int inter, int k, size_t base) {
  auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
  Scratch sc;
  size_t at = al(base);
  sc.x = at;      at += al((size_t)hidden * 2);
  sc.logits = at; at += al((size_t)experts * 4);
  sc.idx = at;    at += al((size_t)k * 4);
  sc.w = at;      at += al((size_t)k * 4);
  sc.y = at;      at += al((size_t)hidden * 2);
  sc.act = at;    at += al((size_t)(k + 1) * inter * 4);
  sc.total = at;
  return sc;
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT size_t wm_moe_layer_decode_state_size(int32_t experts, int32_t hidden, int32_t inter, int32_t k) {
  if (experts < 1 || hidden < 1 || inter < 1 || k < 1) return 0;
  return scratch_layout(experts, hidden, inter, k, dl::layout(experts, inter).total).total;
}

WM_EXPORT size_t wm_moe_layer_decode_status_offset(int32_t experts, int32_t inter) {
  return dl::layout(experts, inter).status;
}

WM_EXPORT int wm_moe_layer_decode(const float* residual, float* residual_out, const void* norm_weight, float eps,
                                  const void* router, const void* shared_gate, int32_t experts, int32_t k,
                                  int32_t norm_topk_prob, const wm_mxfp4_experts* routed,
                                  const wm_mxfp4_experts* shared, void* y, void* x_out, float* logits_out,
                                  int32_t* indices_out, float* weights_out, void* state, size_t state_bytes,
                                  void* stream) {
  return guarded([&] {
    if (!residual || !router || !routed || !state) fail("wm_moe_layer_decode: null pointer");
    validate_experts(routed, "routed experts", false);
    if (shared) {
      validate_experts(shared, "shared expert", true);
      if (shared->hidden != routed->hidden || shared->inter != routed->inter)
        fail("wm_moe_layer_decode: the shared expert's shape differs from the routed experts'");
    }
    if (routed->tiled || (shared && shared->tiled))
      fail("wm_moe_layer_decode: the decode layer reads tables in the row layout");
    const int H = routed->hidden, I = routed->inter;
    if (experts != routed->experts) fail("wm_moe_layer_decode: experts differs from the table's");
    if (experts < 1 || experts > dl::MAX_EXPERTS) fail("wm_moe_layer_decode: experts must be in 1..1024");
    if (k < 1 || k > 32 || k > experts) fail("wm_moe_layer_decode: k must be in 1..min(32, experts)");
    if (state_bytes < wm_moe_layer_decode_state_size(experts, H, I, k)) fail("wm_moe_layer_decode: state too small");
    for (const void* q : {(const void*)residual, (const void*)residual_out, norm_weight, router, shared_gate,
                          (const void*)y, (const void*)x_out})
      if ((uintptr_t)q % 16) fail("wm_moe_layer_decode: vectors and the router must be 16-byte aligned");
    if (!decode_mxfp4_supports(H, I)) fail("wm_moe_layer_decode: hidden and intermediate above 16384");
    hipStream_t s = as_stream(stream);
    if (moe_layer_fused_supports(H, I, k)) {
      dl::Params p;
      p.r = residual;
      p.r_out = residual_out;
      p.norm_w = (const uint16_t*)norm_weight;
      p.eps = eps;
      p.router = (const uint16_t*)router;
      p.gate_vec = (const uint16_t*)shared_gate;
      p.routed = *routed;
      p.shared = shared ? *shared : *routed;
      p.has_shared = shared ? 1 : 0;
      p.experts = experts;
      p.k = k;
      p.norm_topk = norm_topk_prob;
      p.y = (uint16_t*)y;
      p.x_out = (uint16_t*)x_out;
      p.logits_out = logits_out;
      p.idx_out = indices_out;
      p.w_out = weights_out;
      p.state = (uint8_t*)state;
      moe_layer_fused(p, H, I, s);
      return;
    }
    // unfused: norm + router, routing, the decode GEMV kernels, the residual add
    const Scratch sc = scratch_layout(experts, H, I, k, dl::layout(experts, I).total);
    uint8_t* base = (uint8_t*)state;
    uint16_t* xb = x_out ? (uint16_t*)x_out : (uint16_t*)(base + sc.x);
    float* lg = logits_out ? logits_out : (float*)(base + sc.logits);
    int32_t* ib = indices_out ? indices_out : (int32_t*)(base + sc.idx);
    float* wb = weights_out ? weights_out : (float*)(base + sc.w);
    uint16_t* yb = y ? (uint16_t*)y : (uint16_t*)(base + sc.y);
    if (wm_norm_router(residual, nullptr, norm_weight, 1, H, eps, router, experts, nullptr, nullptr, 0, xb, nullptr, lg,
                       nullptr, stream) != 0)
      fail(std::string("wm_moe_layer_decode: ") + wm_last_error());
    if (wm_route_softmax_topk(lg, 1, experts, k, norm_topk_prob, ib, wb, nullptr, stream) != 0)
      fail(std::string("wm_moe_layer_decode: ") + wm_last_error());
    decode_mxfp4(xb, 1, ib, wb, k, *routed, shared, (const uint16_t*)shared_gate, yb, true, (float*)(base + sc.act), s);
    if (residual_out) {
      hipLaunchKernelGGL(residual_add_kernel, dim3((H + 255) / 256), dim3(256), 0, s, residual, yb, H, residual_out);
      check_launch("residual_add");
    }
  });
}

}  // extern "C"
