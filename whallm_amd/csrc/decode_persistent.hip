// Persistent decode: one launch carries one token through every MoE layer.
//
// The per-layer kernel chain (decode.hip, stack.hip) is latency-bound at one token:
// each kernel boundary and each dependent HBM round trip costs microseconds while
// a layer's 18 MB of weights streams in ~2.3 us. Here 256 workgroups (8 XCDs x 32,
// the hardware XCC of block b is b % 8) stay resident and exchange small messages:
//
//   A  (per XCD x): act[k][i] = silu(x . Wg_k[i]) * (x . Wu_k[i]) for i in the XCD's
//      64-wide slice [64x, 64x+64) of every selected expert k (10 routed + shared).
//      A tile is 8 gate rows + the 8 matching up rows; one wave reduces it over the
//      full hidden width with 16 scaled MFMAs (v_mfma_scale_f32_16x16x128_f8f6f4):
//      the weights enter as stored (E2M1 codes, one E8M0 scale per 32 = one MFMA
//      lane's block), x enters as two E4M3 terms (hi + lo, each with its own E8M0
//      scale) which together reproduce every bf16 x exactly when |x| >= 2^-13 max|x|.
//   B  (per XCD x, rows 64j..64j+63 per workgroup j): split-K partial of the down
//      projection over the slice, weighted by the routing weight:
//      p_x[o] = sum_k w_k act_k[slice] . Wd_k[o][slice], again on scaled MFMAs, with
//      w_k act_k split into three E4M3 terms (12 significant bits) under a per-32
//      scale; the down weights are repacked slice-major so each row-slice is 32
//      contiguous bytes.
//   R  r[o] += bf16(sum_x p_x[o]) (fixed x order, so every XCD gets the same r),
//      then the XCD gathers the full r and its rmsnorm statistics for the next layer.
//
// Each exchange has low fan-in (act: within the XCD; partials: the 8 workgroups
// sharing a row block; r: within the XCD). Messages are 64-bit words carrying the
// value and an epoch, written and read with agent-scope relaxed atomics, so a
// reader polls the data itself: no flags, no grid barriers, no L2-wide fences. A
// gather costs about the words each polling wave reads per lane, so act values and
// partials travel two to a word and the act and r gathers are spread over the waves.
// Weight loads run a phase ahead: the A tile of layer l+1 is in flight from the end
// of phase A(l), the down rows of layer l+1 from the end of layer l's phase B.
//
// Replaces, for the decode case, the per-layer host loop of the native engine
// (Native/QwenNative/engine.mm:1567-1588 -> experts() :2073-2236) and its host
// top-k (:2086-2100); routing runs in the launch prologue from the given logits.
#include <cmath>
#include <mutex>

#include "messages.h"
#include "moe_internal.h"
#include "route_device.h"

namespace wm {

constexpr int DS_H = 2048;            // hidden
constexpr int DS_I = 512;             // expert intermediate
constexpr int DS_X = 8;               // XCDs
constexpr int DS_J = 32;              // workgroups per XCD
constexpr int DS_WGS = DS_X * DS_J;   // 256
constexpr int DS_SLICE = DS_I / DS_X; // 64 intermediate columns per XCD
constexpr int DS_ROWS = DS_H / DS_J;  // 64 output rows per workgroup
constexpr int DS_NE_MAX = 12;         // routed + shared experts per layer
constexpr int DS_KB = DS_H / 128;     // K-steps of a phase-A tile (128 per MFMA)
constexpr uint32_t DS_SPIN_LIMIT = MSG_SPIN_LIMIT;
// Status word values (0 = healthy): a message wait ran out, the caller's cancel word was
// set, a selected expert is not resident (its slot map entry is negative).
constexpr uint32_t DS_STALLED = 1, DS_CANCELLED = 2, DS_NOT_RESIDENT = 3, DS_NO_ROUTE = 4;
static_assert(DS_STALLED == MSG_STALLED, "the message waits raise DS_STALLED");
constexpr int DS_MAX_LAYERS = 128;    // layer descriptors kept in LDS
constexpr int DS_CW = 3;                      // compute waves (prefetch weights and compute)
constexpr int DS_THREADS = (DS_CW + 1) * 64;  // + one message wave (polls and publishes)
constexpr int DS_FMT_FP8 = 0, DS_FMT_FP4 = 4;  // MFMA operand formats (E4M3, E2M1)
constexpr int DS_RW = (DS_ROWS + 2) / 3;      // words carrying one workgroup's 64 r rows as bf16 triples

typedef int ds_v8i __attribute__((ext_vector_type(8)));
typedef float ds_v4f __attribute__((ext_vector_type(4)));

struct DSLayout {
  size_t route, act, part, r, epoch, status, total;
};

__host__ __device__ inline DSLayout ds_layout(int layers) {
  DSLayout d;
  size_t at = 0;
  d.route = at;  at += (size_t)DS_X * layers * 32 * 8;  // per XCD: 2 K <= 32 words a layer
  d.act = at;    at += (size_t)2 * DS_X * DS_NE_MAX * DS_SLICE * 8;
  d.part = at;   at += (size_t)2 * DS_X * DS_H * 8;
  d.r = at;      at += (size_t)2 * DS_X * DS_J * DS_RW * 8;
  d.epoch = at;  at += (size_t)DS_WGS * 4;
  d.status = at; at += 256;
  d.total = at;
  return d;
}

// Store of a message word read only by workgroups of the writer's own XCD. With
// LOCAL, a workgroup-scope store: it is written through the CU's L1 into the XCD's
// L2, where the readers' agent-scope loads find it, and goes no further (measured
// on MI355X; the launcher enables LOCAL only after checking that block b runs on
// XCC b % 8). Without LOCAL, an agent-scope store.
template <bool LOCAL>
__device__ __forceinline__ void ll_put_xcd(uint64_t* p, uint64_t word) {
  if constexpr (LOCAL) __hip_atomic_store(p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else __hip_atomic_store(p, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Phase timestamps and notes for the profiling build of whallm_amd.phase_trace (both expand
// to nothing in the library). Points of the compute waves: 0 S0, 1 S0b, 3 phase A done
// (the wave's act gathered), 5 shared gate ready, 4 next A tile issued, 6 phase B done; of
// the message wave: 8 S0, 2 gate published, 11 S2, 4 partial published, 12 partials
// gathered, 6 r published, 13 r gathered; notes: 15 / 7 = re-poll rounds of the partial and
// r gathers.
#ifndef WM_DS_TRACE
#define WM_DS_TRACE(layer, point)
#endif
#ifndef WM_DS_NOTE
#define WM_DS_NOTE(layer, point, value)
#endif

// bf16 rounding on the gfx950 conversion v_cvt_pk_bf16_f32 (round to nearest even, as
// f32_to_bf16_bits; a NaN stays a NaN). Branch-free, where the integer form costs an
// exec-mask branch per value: these roundings sit on the per-layer critical path.
typedef __bf16 ds_bf16x2 __attribute__((ext_vector_type(2)));
typedef float ds_f2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t ds_bf16_pair(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((ds_f2){a, b}, ds_bf16x2));
}
__device__ __forceinline__ uint16_t ds_bf16_bits(float v) { return (uint16_t)ds_bf16_pair(v, 0.0f); }
__device__ __forceinline__ float bf16_round_f(float v) { return __uint_as_float(ds_bf16_pair(v, 0.0f) << 16); }

// ---- E4M3 term splitting -------------------------------------------------------
// E8M0 exponent s that puts amax / 2^(s-127) in [128, 256) (E4M3's largest finite is
// 448); at least 1 so the scale stays a normal number. amax 0 gives 1.
__device__ __forceinline__ int e4m3_term_exponent(float amax) {
  int be = (int)((__float_as_uint(amax) >> 23) & 0xff);
  return be - 7 > 1 ? be - 7 : 1;
}
// 2^(e-127) for a biased exponent e in 1..254.
__device__ __forceinline__ float pow2_biased(int e) { return __uint_as_float((uint32_t)e << 23); }
// Two f32 -> E4M3 (round to nearest even) into bytes 0..1 of a word.
__device__ __forceinline__ uint32_t e4m3_pair(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
}
template <int SEL>
__device__ __forceinline__ float e4m3_byte(uint32_t w) { return __builtin_amdgcn_cvt_f32_fp8((int)w, SEL); }

// Workgroup state shared by the two roles.
struct DSShared {
  __attribute__((aligned(16))) float r[DS_H];
  // x as E4M3 terms in MFMA B-operand order: [term hi/lo][K-step][lane group][32 bytes]
  __attribute__((aligned(16))) uint8_t xb[2][DS_KB][4][32];
  __attribute__((aligned(16))) float act[DS_NE_MAX][DS_SLICE];
  // phase-B operand staging per compute wave and K-step: [term][lane group][32 bytes]
  __attribute__((aligned(16))) uint8_t bstage[DS_CW][2][3][4][32];
  __attribute__((aligned(16))) float tile_out[DS_CW][16];
  __attribute__((aligned(16))) float partb[DS_CW][3][DS_ROWS];
  uint16_t rpack[3 * DS_RW];  // bf16 of this workgroup's r rows (+ zero pad) for packing
  int slot[DS_MAX_LAYERS][16];
  float w[DS_MAX_LAYERS][16];
  wm_decode_layer desc[DS_MAX_LAYERS];
  float gate;   // sigmoid(x . g) of the current layer
  float eps;
  float ssw[4];  // each wave's share of sum r^2 of the next layer's r
  float mxw[4];  // and of max |r|
  int r_go;      // layers whose r rows this workgroup has published (the compute waves' r polls wait for it)
  int gate_l;    // layers whose shared gate is in sh.gate (the wave with the shared expert waits for it)
  int failures;
  TopkScratch topk;  // the prologue's routing (the message wave)
};

// Per-launch constants of one workgroup.
struct DSCtx {
  int L, K, NE, x, j, lane, wave;
  uint32_t base;
  uint64_t *route_ll, *act_ll, *part_ll, *r_ll;
  uint32_t* status;
  const int32_t* cancel;  // nullable: a word the host sets to stop the launch
  float* trace;           // nullable: [L][H] fp32 residual after each layer
};

// x = bf16(r * inv) as two E4M3 terms: hi = e4m3(x / 2^(s-127)), lo = e4m3((x / 2^(s-127)
// - hi) * 16) under scale 2^(s-131). Thread t handles x[8t .. 8t+7]; x[n] with
// n = 128 kb + 64 h + 16 g + e sits at byte 16 h + e of xb[term][kb][g], the order in
// which the MFMA's B lanes of group g pair with the A lanes (block 4 kb + a, a = 0..3).
__device__ __forceinline__ void ds_build_x(DSShared& sh, int tid, float inv, float xmax) {
  const int s_hi = e4m3_term_exponent(xmax);
  const float f = pow2_biased(254 - s_hi);
  const int n0 = tid * 8;
  const float4 ra = *reinterpret_cast<const float4*>(&sh.r[n0]);
  const float4 rb = *reinterpret_cast<const float4*>(&sh.r[n0 + 4]);
  const float rv[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
  uint32_t hw[2], lw[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const uint32_t x01 = ds_bf16_pair(rv[4 * p] * inv, rv[4 * p + 1] * inv);
    const uint32_t x23 = ds_bf16_pair(rv[4 * p + 2] * inv, rv[4 * p + 3] * inv);
    const float h[4] = {__uint_as_float(x01 << 16) * f, __uint_as_float(x01 & 0xffff0000u) * f,
                        __uint_as_float(x23 << 16) * f, __uint_as_float(x23 & 0xffff0000u) * f};
    uint32_t w01 = e4m3_pair(h[0], h[1]), w23 = e4m3_pair(h[2], h[3]);
    float l0 = (h[0] - e4m3_byte<0>(w01)) * 16.0f, l1 = (h[1] - e4m3_byte<1>(w01)) * 16.0f;
    float l2 = (h[2] - e4m3_byte<0>(w23)) * 16.0f, l3 = (h[3] - e4m3_byte<1>(w23)) * 16.0f;
    hw[p] = (w01 & 0xffffu) | (w23 << 16);
    lw[p] = (e4m3_pair(l0, l1) & 0xffffu) | (e4m3_pair(l2, l3) << 16);
  }
  const int kb = n0 >> 7, h = (n0 >> 6) & 1, g = (n0 >> 4) & 3, e = n0 & 15;
  const int off = (kb * 4 + g) * 32 + 16 * h + e;
  *reinterpret_cast<uint2*>(&sh.xb[0][0][0][0] + off) = make_uint2(hw[0], hw[1]);
  *reinterpret_cast<uint2*>(&sh.xb[1][0][0][0] + off) = make_uint2(lw[0], lw[1]);
}

// A wave's share of the rmsnorm statistics of r (lane 0 writes; combined after the next barrier).
__device__ __forceinline__ void ds_norm_part(DSShared& sh, float ss, float mx, int lane, int wave) {
  ss = segment_sum<64>(ss);
  mx = segment_max<64>(mx);
  if (lane == 0) {
    sh.ssw[wave] = ss;
    sh.mxw[wave] = mx;
  }
}

// 1 / rms(r) and max |bf16(r * inv)| from the four shares, in a fixed order, so every wave
// of every workgroup gets the same values.
__device__ __forceinline__ void ds_norm(const DSShared& sh, float& inv, float& xmax) {
  const float ss = (sh.ssw[0] + sh.ssw[1]) + (sh.ssw[2] + sh.ssw[3]);
  const float mx = fmaxf(fmaxf(sh.mxw[0], sh.mxw[1]), fmaxf(sh.mxw[2], sh.mxw[3]));
  inv = rsqrtf(ss / (float)DS_H + sh.eps);
  xmax = bf16_round_f(mx * inv);
}

// Wave `wave`'s quarter of the XCD's r words (bf16 triples under a 16-bit epoch) into
// sh.r, and its share of the statistics. Every wave gathers a quarter, so each polls
// 3 words a lane instead of one wave polling 11.
constexpr int DS_R_SHARE = DS_J * DS_RW / 4;
static_assert(DS_J * DS_RW % 4 == 0, "r words split over four waves");
__device__ __forceinline__ void ds_gather_r_share(DSShared& sh, const DSCtx& c, const uint64_t* r_buf, uint32_t e_r,
                                                  int wave, bool& ok, uint32_t* rounds) {
  float ss = 0.0f, mx = 0.0f;
  ll_gather<(DS_R_SHARE + 63) / 64, 16>(r_buf + wave * DS_R_SHARE, c.lane, 64, DS_R_SHARE, e_r, c.status, ok,
                                        [&](int i, uint64_t v) {
    const int w = wave * DS_R_SHARE + i;
    const int jj = w / DS_RW, t = 3 * (w % DS_RW);
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      if (t + u < DS_ROWS) {
        const float rv = bf16_bits_to_f32((uint32_t)(v >> (16 * u)) & 0xffffu);
        sh.r[jj * DS_ROWS + t + u] = rv;
        ss += rv * rv;
        mx = fmaxf(mx, fabsf(rv));
      }
    }
  }, rounds);
  ds_norm_part(sh, ss, mx, c.lane, wave);
  if (!ok) sh.failures = 1;
}

// The act words of the experts compute wave `wave`'s phase B reads (4 wave .. 4 wave + 3,
// 32 words each) into sh.act; no other wave reads them, so no barrier is needed.
__device__ __forceinline__ void ds_gather_act_own(DSShared& sh, const DSCtx& c, const uint64_t* act_buf,
                                                  uint32_t e_act, int wave, bool& ok) {
  const int first = wave * 4 * (DS_SLICE / 2), n = min(4 * (DS_SLICE / 2), c.NE * (DS_SLICE / 2) - first);
  ll_gather<2, 16>(act_buf + first, c.lane, 64, n, e_act, c.status, ok, [&](int i, uint64_t v) {
    const int w = first + i;
    const int e = w / (DS_SLICE / 2), cc = 2 * (w % (DS_SLICE / 2));
    sh.act[e][cc] = f24_to_f32((uint32_t)v & 0xffffffu);
    sh.act[e][cc + 1] = f24_to_f32((uint32_t)(v >> 24) & 0xffffffu);
  });
}

// The two roles run separate loops (so their registers do not overlap) and meet at
// the same three barriers per layer:
//   S0: r_l and its statistics' shares in LDS -> every wave builds a quarter of x
//   S0b: x terms in LDS -> compute waves: phase A (one tile each), publish act, gather
//                          the act of the four experts their phase B reads, prefetch
//                          the A tile of l+1, phase B partials into LDS (the wave with
//                          the shared expert first waits for the gate's LDS flag)
//                          message wave: shared gate, its flag
//   S2: partials   -> (every wave leaves here if a message wait ran out)
//                     compute waves: prefetch B(l+1), wait for the message wave's r
//                     publish (LDS counter), gather a quarter of the XCD's r
//                     message wave: publish the row block's partial, gather the 8
//                     XCDs' partials, r += bf16(sum), publish r, gather its quarter
// One wave per SIMD.
template <bool LOCAL, bool DOWN_ROWS>
__device__ __forceinline__ void ds_compute_role(DSShared& sh, const DSCtx& c) {
  const int lane = c.lane, wave = c.wave, x = c.x, j = c.j, K = c.K, NE = c.NE;
  const int tiles = 8 * NE;                     // phase-A tiles of the XCD
  const int col = lane & 15, grp = lane >> 4;   // MFMA lane: row / column and K group

  auto expert_base = [&](int l, int k, const uint8_t*& gu, const uint8_t*& gus, const uint8_t*& dn,
                         const uint8_t*& dns) {
    const wm_decode_layer& D = sh.desc[l];
    if (k < K) {
      int64_t slot = sh.slot[l][k];
      gu = (const uint8_t*)D.gate_up + slot * D.gate_up_stride;
      gus = (const uint8_t*)D.gate_up_scales + slot * D.gate_up_scales_stride;
      dn = (const uint8_t*)D.down + slot * D.down_stride;
      dns = (const uint8_t*)D.down_scales + slot * D.down_scales_stride;
    } else {
      gu = (const uint8_t*)D.shared_gate_up;
      gus = (const uint8_t*)D.shared_gate_up_scales;
      dn = (const uint8_t*)D.shared_down;
      dns = (const uint8_t*)D.shared_down_scales;
    }
  };

  // Phase-A tile t of this wave: expert t / 8, slice rows 8 (t % 8) .. +7 (gate, then up).
  // Lanes beyond the XCD's tiles re-read a valid tile (a cache hit) so every load is
  // unconditional; a branch among in-flight loads would make the compiler wait for all.
  int t_mine = j + DS_J * wave;
  const bool tile_valid = t_mine < tiles;
  if (!tile_valid) t_mine = t_mine % tiles;
  const int tk = t_mine >> 3, tq = t_mine & 7;
  const int arow = col < 8 ? DS_SLICE * x + 8 * tq + col : DS_I + DS_SLICE * x + 8 * tq + (col - 8);
  uint4 aw[DS_KB];
  uint4 as4[4];
  auto issue_a = [&](int l) {
    const uint8_t *gu, *gus, *dn, *dns;
    expert_base(l, tk, gu, gus, dn, dns);
    // scales first: the first MFMA needs them with the first weight load
    const uint8_t* sp = gus + (size_t)arow * (DS_H / 32);
#pragma unroll
    for (int m = 0; m < 4; ++m) as4[m] = gload16(sp + 16 * m);
    const uint8_t* rp = gu + (size_t)arow * (DS_H / 2) + 16 * grp;
#pragma unroll
    for (int kb = 0; kb < DS_KB; ++kb) aw[kb] = gload16(rp + 64 * kb);
  };

  // Phase-B K-steps 2 wave + i (i = 0, 1): experts 2 kb and 2 kb + 1 of the slice.
  // Lane (row r, group a) reads half a % 2 of expert 2 kb + a / 2's row-slice for each
  // of the four 16-row tiles; missing experts re-read the step's first expert.
  // Slice-major down (DOWN_ROWS false): row o's slice x is 32 bytes at (x H + o) 32 and its
  // two scale bytes at (x H + o) 2, so a dword holds rows o and o ^ 1. The reference row
  // layout (DOWN_ROWS true, e.g. blobs of the slot cache): the slice is 32 bytes at
  // o I/2 + 32 x and its scale bytes at o I/32 + 2 x, so a dword holds slices x and x ^ 1.
  uint4 bw[2][4];
  uint32_t bs[2][4];
  const int bshift = 8 * (2 * (DOWN_ROWS ? (x & 1) : (col & 1)) + (grp & 1));  // byte of the scale word
  auto issue_b = [&](int l) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kb = 2 * wave + i;
      int e = 2 * kb + (grp >> 1);
      if (e >= NE) e = 2 * kb < NE ? 2 * kb : 0;
      const uint8_t *gu, *gus, *dn, *dns;
      expert_base(l, e, gu, gus, dn, dns);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        const size_t o = (size_t)j * DS_ROWS + 16 * rt + col;
        if constexpr (DOWN_ROWS) {
          bw[i][rt] = gload16(dn + o * (DS_I / 2) + x * (DS_SLICE / 2) + 16 * (grp & 1));
          bs[i][rt] = gload<uint32_t>(dns + o * (DS_I / 32) + ((x * (DS_SLICE / 32)) & ~3));
        } else {
          const size_t row = (size_t)x * DS_H + o;
          bw[i][rt] = gload16(dn + row * (DS_SLICE / 2) + 16 * (grp & 1));
          bs[i][rt] = gload<uint32_t>(dns + ((row * (DS_SLICE / 32)) & ~(size_t)3));
        }
      }
    }
  };

  bool ok = true;
  issue_a(0);
  issue_b(0);
  for (int l = 0; l < c.L; ++l) {
    const uint32_t e_act = c.base + 2 + 3 * l;
    uint64_t* act_buf = c.act_ll + ((size_t)(l & 1) * DS_X + x) * DS_NE_MAX * DS_SLICE;
    ds_barrier();  // S0: r_l and its statistics' shares in LDS
    WM_DS_TRACE(l, 0);
    float inv, xmax;
    ds_norm(sh, inv, xmax);
    ds_build_x(sh, c.wave * 64 + lane, inv, xmax);
    ds_barrier();  // S0b: x terms in LDS
    WM_DS_TRACE(l, 1);
    // ---- phase A: one 16-row tile over the hidden width
    {
      const int s_hi = e4m3_term_exponent(xmax);
      // lanes of columns >= 2 feed unused outputs; a scale below 2^-127 only arises for
      // x below 2^-113, so clamping it changes nothing measurable
      const int sb = (col & 1) ? (s_hi > 4 ? s_hi - 4 : 0) : s_hi;
      const uint8_t* xp = &sh.xb[col & 1][0][grp][0];
      // B operands come from LDS three K-steps ahead of their MFMA, so LDS latency
      // overlaps the MFMA chain instead of adding to every step
      constexpr int PF = 3;
      uint4 blo[PF], bhi[PF];
#pragma unroll
      for (int q = 0; q < PF; ++q) {
        blo[q] = *reinterpret_cast<const uint4*>(xp + q * 128);
        bhi[q] = *reinterpret_cast<const uint4*>(xp + q * 128 + 16);
      }
      ds_v4f acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < DS_KB; ++kb) {
        const uint4 lo = blo[kb % PF], hi = bhi[kb % PF];
        if (kb + PF < DS_KB) {
          blo[kb % PF] = *reinterpret_cast<const uint4*>(xp + (kb + PF) * 128);
          bhi[kb % PF] = *reinterpret_cast<const uint4*>(xp + (kb + PF) * 128 + 16);
        }
        const ds_v8i bv = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        const ds_v8i av = {(int)aw[kb].x, (int)aw[kb].y, (int)aw[kb].z, (int)aw[kb].w, 0, 0, 0, 0};
        const uint32_t sw = kb % 4 == 0 ? as4[kb / 4].x : kb % 4 == 1 ? as4[kb / 4].y : kb % 4 == 2 ? as4[kb / 4].z : as4[kb / 4].w;
        const int sa = (int)((sw >> (8 * grp)) & 0xffu);
        if (kb & 1)
          acc1 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc1, DS_FMT_FP4, DS_FMT_FP8, 0, sa, 0, sb);
        else
          acc0 = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc0, DS_FMT_FP4, DS_FMT_FP8, 0, sa, 0, sb);
        __builtin_amdgcn_sched_barrier(0);  // keep the read-ahead where it is written
      }
      // column 0 holds the hi term's dot products, column 1 the lo term's
      float d[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc0[i] + acc1[i];
        d[i] = v + dpp_f<0xB1>(v);
      }
      if (col == 0) *reinterpret_cast<float4*>(&sh.tile_out[wave][4 * grp]) = make_float4(d[0], d[1], d[2], d[3]);
      {
        const float g = sh.tile_out[wave][lane & 7], u = sh.tile_out[wave][8 + (lane & 7)];
        const float a = silu(g) * u;
        const float a_next = dpp_f<0xB1>(a);  // the odd lane's value
        if (tile_valid && lane < 8 && !(lane & 1))
          ll_put_xcd<LOCAL>(&act_buf[tk * (DS_SLICE / 2) + 4 * tq + lane / 2],
                            ((uint64_t)(e_act & 0xffffu) << 48) | ((uint64_t)f32_to_f24(a_next) << 24) | f32_to_f24(a));
      }
    }
    ds_gather_act_own(sh, c, act_buf, e_act, wave, ok);
    if (!ok) sh.failures = 1;
    WM_DS_TRACE(l, 3);
    if (4 * wave <= K && K < 4 * wave + 4) {  // this wave's K-steps include the shared expert
      uint32_t spins = 0;
      while (__hip_atomic_load(&sh.gate_l, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <= l) {
        if (++spins > DS_SPIN_LIMIT) {
          __hip_atomic_store(c.status, DS_STALLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = false;
          sh.failures = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    WM_DS_TRACE(l, 5);
    // The A tile of l + 1 is issued after this wave's act gather, not before: issued
    // earlier, its loads sit in the CU's memory queue ahead of the act polls and delay them
    // by their whole transfer (measured: the act gather ended 1.5 us later per layer)
    issue_a(l + 1 < c.L ? l + 1 : l);
    WM_DS_TRACE(l, 4);
    // ---- phase B: split-K partials of rows 64 j .. 64 j + 63 over this wave's K-steps
    {
      ds_v4f accb[4];
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) accb[rt] = ds_v4f{0.f, 0.f, 0.f, 0.f};
      // both K-steps' B operands are staged first, so one LDS write-read round trip serves
      // all eight MFMAs
      int sbs[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int kb = 2 * wave + i;
        sbs[i] = 0;
        if (2 * kb < NE) {
          // B operand: w_e act_e as three E4M3 terms. A B lane's scale covers the same
          // 32-value K block as the A lanes of its group (block a = expert 2 kb + a / 2,
          // columns 32 (a % 2) ..), which the register layout spreads over two B lane
          // groups: element t of block a sits in group 2 (a % 2) + t / 16 at byte
          // 16 (a / 2) + t % 16. Row a of this wave splits block a, two values a lane.
          const int t2 = 2 * (lane & 15);
          const int e = 2 * kb + (grp >> 1);
          const int cc = 32 * (grp & 1) + t2;
          const float we = e < K ? sh.w[l][e] : (e < NE ? sh.gate : 0.0f);
          float2 av = *reinterpret_cast<const float2*>(&sh.act[e][cc]);
          const float v0 = e < NE ? av.x * we : 0.0f, v1 = e < NE ? av.y * we : 0.0f;
          const float gmax = segment_max<16>(fmaxf(fabsf(v0), fabsf(v1)));
          const int s = e4m3_term_exponent(gmax);
          const float f = pow2_biased(254 - s);
          const float h0 = v0 * f, h1 = v1 * f;
          const uint32_t c0 = e4m3_pair(h0, h1);
          const float m0 = (h0 - e4m3_byte<0>(c0)) * 16.0f, m1 = (h1 - e4m3_byte<1>(c0)) * 16.0f;
          const uint32_t c1 = e4m3_pair(m0, m1);
          const float n0 = (m0 - e4m3_byte<0>(c1)) * 16.0f, n1 = (m1 - e4m3_byte<1>(c1)) * 16.0f;
          const uint32_t c2 = e4m3_pair(n0, n1);
          uint8_t* st = &sh.bstage[wave][i][0][0][0];
          const int at = (2 * (grp & 1) + (t2 >> 4)) * 32 + 16 * (grp >> 1) + (t2 & 15);
          *reinterpret_cast<uint16_t*>(st + 0 * 128 + at) = (uint16_t)c0;
          *reinterpret_cast<uint16_t*>(st + 1 * 128 + at) = (uint16_t)c1;
          *reinterpret_cast<uint16_t*>(st + 2 * 128 + at) = (uint16_t)c2;
          sbs[i] = s;
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int kb = 2 * wave + i;
        if (2 * kb < NE) {
          const uint8_t* st = &sh.bstage[wave][i][0][0][0];
          const int term = col < 3 ? col : 0;  // columns >= 3 feed unused outputs
          const uint4 blo = *reinterpret_cast<const uint4*>(st + term * 128 + grp * 32);
          const uint4 bhi = *reinterpret_cast<const uint4*>(st + term * 128 + grp * 32 + 16);
          const ds_v8i bv = {(int)blo.x, (int)blo.y, (int)blo.z, (int)blo.w,
                             (int)bhi.x, (int)bhi.y, (int)bhi.z, (int)bhi.w};
          const int s = sbs[i];
          const int sb = s > 4 * term ? s - 4 * term : 0;
#pragma unroll
          for (int rt = 0; rt < 4; ++rt) {
            const ds_v8i aop = {(int)bw[i][rt].x, (int)bw[i][rt].y, (int)bw[i][rt].z, (int)bw[i][rt].w, 0, 0, 0, 0};
            accb[rt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aop, bv, accb[rt], DS_FMT_FP4, DS_FMT_FP8, 0,
                                                                        (int)((bs[i][rt] >> bshift) & 0xffu), 0, sb);
          }
        }
      }
      // rows 4 g .. 4 g + 3 of each tile, column = term; the message wave adds the terms
      if (col < 3) {
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
          *reinterpret_cast<float4*>(&sh.partb[wave][col][16 * rt + 4 * grp]) =
              make_float4(accb[rt][0], accb[rt][1], accb[rt][2], accb[rt][3]);
      }
    }
    WM_DS_TRACE(l, 6);
    ds_barrier();  // S2: partials in LDS
    if (sh.failures != 0) break;  // a message wait ran out (every wave leaves here)
    issue_b(l + 1 < c.L ? l + 1 : l);
    // ---- this wave's quarter of r_{l+1}, once this workgroup's message wave has published
    // its rows (so these polls do not queue beside its partial gather)
    {
      uint32_t spins = 0;
      while (__hip_atomic_load(&sh.r_go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <= l) {
        if (++spins > DS_SPIN_LIMIT) {
          __hip_atomic_store(c.status, DS_STALLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      const uint64_t* r_buf = c.r_ll + ((size_t)(l & 1) * DS_X + x) * DS_J * DS_RW;
      ds_gather_r_share(sh, c, r_buf, c.base + 4 + 3 * l, wave, ok, nullptr);
    }
  }
}

template <bool LOCAL>
__device__ __forceinline__ void ds_message_role(DSShared& sh, const DSCtx& c, float& r_own) {
  const int lane = c.lane, x = c.x, j = c.j;
  bool ok = true;
  for (int l = 0; l < c.L; ++l) {
    const int par = l & 1;
    const uint32_t e_part = c.base + 3 + 3 * l, e_r = c.base + 4 + 3 * l;
    uint64_t* part_buf = c.part_ll + (size_t)par * DS_X * DS_H;
    uint64_t* r_buf = c.r_ll + ((size_t)par * DS_X + x) * DS_J * DS_RW;
    // the cancel word is read at the top of the layer and looked at after the shared gate,
    // whose loads are issued after it (loads complete in order), so the read adds no wait of
    // its own
    int32_t cancel_word = 0;
    if (c.cancel && lane == 0) cancel_word = __hip_atomic_load(c.cancel, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const uint8_t* sg = (const uint8_t*)sh.desc[l].shared_gate;
    uint4 gw[4] = {};
    if (sg) {
#pragma unroll
      for (int m = 0; m < 4; ++m) gw[m] = gload16(sg + (lane + 64 * m) * 16);
    }
    ds_barrier();  // S0
    WM_DS_TRACE(l, 8);
    float inv, xmax;
    ds_norm(sh, inv, xmax);
    ds_build_x(sh, DS_CW * 64 + lane, inv, xmax);
    ds_barrier();  // S0b
    // ---- shared-expert gate sigmoid(x . g); lane: x[8 (lane + 64 m) .. + 7]
    {
      float gv = 1.0f;
      if (sg) {
        float a = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int n = 8 * (lane + 64 * m);
          const float4 ra = *reinterpret_cast<const float4*>(&sh.r[n]);
          const float4 rb = *reinterpret_cast<const float4*>(&sh.r[n + 4]);
          const float rv[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
          const uint32_t g4[4] = {gw[m].x, gw[m].y, gw[m].z, gw[m].w};
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const uint32_t xv = ds_bf16_pair(rv[2 * h] * inv, rv[2 * h + 1] * inv);
            a = dot2_bf16(bits_to_bf16x2(xv), bits_to_bf16x2(g4[h]), a);
          }
        }
        a = segment_sum<64>(a);
        gv = 1.0f / (1.0f + __expf(-a));
      }
      if (lane == 0) {
        sh.gate = gv;
        __hip_atomic_store(&sh.gate_l, l + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    uint32_t rounds = 0;
    WM_DS_TRACE(l, 2);
    if (__builtin_amdgcn_readfirstlane(cancel_word) != 0) {
      // leave after this layer's phase B; the others see the status word in their next wait
      if (lane == 0) __hip_atomic_store(c.status, DS_CANCELLED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = false;
    }
    if (!ok) sh.failures = 1;
    ds_barrier();  // S2
    if (sh.failures != 0) break;
    WM_DS_TRACE(l, 11);
    // ---- row block partial -> the 8 XCDs; sum them (x order); r += bf16(sum); gather r_{l+1}
    float p = 0.0f;
#pragma unroll
    for (int w = 0; w < DS_CW; ++w)
      p += (sh.partb[w][0][lane] + sh.partb[w][1][lane]) + sh.partb[w][2][lane];
    WM_DS_TRACE(l, 4);
    float y;
    {  // two rows a word as 24-bit floats under a 16-bit epoch
      const float p_next = dpp_f<0xB1>(p);
      if (!(lane & 1))
        __hip_atomic_store(&part_buf[(size_t)x * (DS_H / 2) + j * (DS_ROWS / 2) + lane / 2],
                           ((uint64_t)(e_part & 0xffffu) << 48) | ((uint64_t)f32_to_f24(p_next) << 24) | f32_to_f24(p),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // lanes 0-31 gather row pair `lane` from XCDs 0-3, lanes 32-63 from XCDs 4-7
      float s0 = 0.0f, s1 = 0.0f;
      const uint64_t* src = part_buf + (size_t)(4 * (lane >> 5)) * (DS_H / 2) + j * (DS_ROWS / 2) + (lane & 31);
      ll_gather<DS_X / 2, 16>(src, 0, DS_H / 2, (DS_X / 2) * (DS_H / 2), e_part, c.status, ok, [&](int, uint64_t v) {
        s0 += f24_to_f32((uint32_t)v & 0xffffffu);
        s1 += f24_to_f32((uint32_t)(v >> 24) & 0xffffffu);
      }, &rounds);
      // (XCDs 0-3) + (XCDs 4-7) in both halves, then row 64 j + lane from pair lane / 2
      const auto q0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(s0), __float_as_uint(s0), false, false);
      const auto q1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(s1), __float_as_uint(s1), false, false);
      const float o0 = __uint_as_float(lane < 32 ? q0[1] : q0[0]), o1 = __uint_as_float(lane < 32 ? q1[1] : q1[0]);
      const float y0 = lane < 32 ? s0 + o0 : o0 + s0, y1 = lane < 32 ? s1 + o1 : o1 + s1;
      const int from = (lane >> 1) * 4;
      const float a0 = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(y0)));
      const float a1 = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(y1)));
      y = (lane & 1) ? a1 : a0;
    }
    WM_DS_NOTE(l, 15, rounds);
    WM_DS_TRACE(l, 12);
    r_own += bf16_round_f(y);
    if (c.trace && x == 0) c.trace[(size_t)l * DS_H + j * DS_ROWS + lane] = r_own;
    // publish the row block as bf16 triples under a 16-bit epoch (the hidden state that
    // feeds the next rmsnorm is bf16, as in the reference's bf16 residual stream; the
    // owner keeps accumulating r in fp32)
    sh.rpack[lane] = ds_bf16_bits(r_own);
    if (lane < 3 * DS_RW - DS_ROWS) sh.rpack[DS_ROWS + lane] = 0;
    if (lane < DS_RW) {
      const uint64_t word = ((uint64_t)(e_r & 0xffffu) << 48) | ((uint64_t)sh.rpack[3 * lane + 2] << 32) |
                            ((uint64_t)sh.rpack[3 * lane + 1] << 16) | sh.rpack[3 * lane];
      ll_put_xcd<LOCAL>(&r_buf[j * DS_RW + lane], word);
    }
    WM_DS_TRACE(l, 6);
    __hip_atomic_store(&sh.r_go, l + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    ds_gather_r_share(sh, c, r_buf, e_r, DS_CW, ok, &rounds);
    WM_DS_NOTE(l, 7, rounds);
    WM_DS_TRACE(l, 13);
  }
}

template <int PER_LANE, bool LOCAL, bool DOWN_ROWS>
__global__ void __launch_bounds__(DS_THREADS, 1) decode_persistent_kernel(
    const float* __restrict__ logits, int L, int E, int K, int norm_topk, const wm_decode_layer* layers,
    float* __restrict__ residual, float eps, uint16_t* __restrict__ x_out, uint8_t* state,
    const int32_t* cancel, float* trace) {
  __shared__ DSShared sh;
  const int b = blockIdx.x, tid = threadIdx.x;
  const DSLayout lay = ds_layout(L);
  DSCtx c;
  c.L = L;
  c.K = K;
  c.NE = K + 1;
  c.x = b % DS_X;
  c.j = b / DS_X;
  c.lane = tid % 64;
  c.wave = tid / 64;
  c.route_ll = (uint64_t*)(state + lay.route);
  c.act_ll = (uint64_t*)(state + lay.act);
  c.part_ll = (uint64_t*)(state + lay.part);
  c.r_ll = (uint64_t*)(state + lay.r);
  c.status = (uint32_t*)(state + lay.status);
  c.cancel = cancel;
  c.trace = trace;
  uint32_t* wg_epoch = (uint32_t*)(state + lay.epoch);
  c.base = wg_epoch[b];
  const uint32_t e_route = c.base + 1;
  const bool msg = c.wave == DS_CW;
  bool ok = true;

  // ---- prologue. Its memory round trips overlap: the message wave of workgroup b < L
  // routes layer b while every wave copies the descriptors and r_0 and the epoch arrives.
  static_assert(DS_MAX_LAYERS <= DS_WGS, "a workgroup routes one layer at most");
  int sel = 0;
  float w = 0.0f, full;
  if (msg && b < L)
    wave_route_softmax<PER_LANE>(logits + (size_t)b * E, E, K, norm_topk != 0, c.lane, sh.topk, sel, w, false, full);
  for (int i = tid; i < L * (int)(sizeof(wm_decode_layer) / 8); i += DS_THREADS)
    reinterpret_cast<uint64_t*>(sh.desc)[i] = reinterpret_cast<const uint64_t*>(layers)[i];
  for (int i = tid; i < DS_H; i += DS_THREADS) sh.r[i] = residual[i];
  float r_own = msg ? residual[c.j * DS_ROWS + c.lane] : 0.0f;  // the message wave owns rows 64j + lane
  if (tid == 0) sh.failures = 0;
  if (tid == 0) sh.eps = eps;
  if (tid == 0) sh.r_go = 0;
  if (tid == 0) sh.gate_l = 0;
  if (tid < 4) sh.ssw[tid] = sh.mxw[tid] = 0.0f;  // the prologue's r_0 statistics are the message wave's share
  __syncthreads();  // failures is cleared before any wave can raise it; every wave holds its epoch
  // Every launch advances the epochs by the same amount, whether it completes or not, so
  // words left by a launch that ended early never match a later launch's epochs.
  if (tid == 0) wg_epoch[b] = c.base + 3 * (uint32_t)L + 5;
  // Routes travel as 2 K words per layer (K ids, then K weights), written once per XCD, so
  // an XCD's 32 workgroups poll lines of their own instead of all 256 polling the same ones.
  const int rw = 2 * K;
  if (msg && b < L && c.lane < K) {
#pragma unroll
    for (int xc = 0; xc < DS_X; ++xc) {
      uint64_t* dst = c.route_ll + ((size_t)xc * L + b) * rw;
      ll_put(&dst[c.lane], (uint32_t)sel, e_route);
      ll_put(&dst[K + c.lane], __float_as_uint(w), e_route);
    }
  }
  {  // every wave gathers a quarter of the route words
    const uint64_t* src = c.route_ll + (size_t)c.x * L * rw;
    const int quarter = (L * rw + 3) / 4, end = min((c.wave + 1) * quarter, L * rw);
    for (int s = c.wave * quarter; s < end; s += 64 * 4)
      ll_gather<4>(src, s + c.lane, 64, end, e_route, c.status, ok, [&](int i, uint64_t word) {
        const uint32_t v = (uint32_t)word;
        const int l = i / rw, k = i - l * rw;
        if (k < K) sh.slot[l][k] = (int)v;
        else sh.w[l][k - K] = __uint_as_float(v);
      });
  }
  if (!ok) sh.failures = 1;
  ds_barrier();
  if (sh.failures != 0) return;
  // Expert ids -> slots once, so the prefetch loops read only LDS. Before any address is
  // formed, a selection outside [0, E) (a logits row with fewer than K selectable values,
  // e.g. all NaN, gives the top-k's sentinel id) raises failure bit 2, and a negative map
  // entry (an expert that is not resident) bit 1; either ends the launch before any layer
  // runs: every workgroup reads the same routes and map and leaves here, and the status
  // word tells the caller (4 no valid route, 3 not resident).
  for (int i = tid; i < L * 16; i += DS_THREADS) {
    int l = i / 16, k = i % 16;
    const int32_t* slots = sh.desc[l].slots;
    if (k < K) {
      const int e = sh.slot[l][k];
      if (e < 0 || e >= E) {
        __hip_atomic_fetch_or(&sh.failures, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        sh.slot[l][k] = 0;
      } else if (slots) {
        const int32_t v = gload<int32_t>(slots + e);
        if (v < 0) __hip_atomic_fetch_or(&sh.failures, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        sh.slot[l][k] = max(0, v);
      }
    }
  }
  ds_barrier();
  if (sh.failures != 0) {
    if (tid == 0)
      __hip_atomic_store(c.status, (sh.failures & 2) ? DS_NO_ROUTE : DS_NOT_RESIDENT, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (msg) {  // rmsnorm statistics of r_0 (every LDS read issued before the first use)
    float ss = 0.0f, mx = 0.0f;
    static_assert(DS_H % 256 == 0, "each lane reads whole float4 chunks of r");
    float4 v[DS_H / 256];
#pragma unroll
    for (int q = 0; q < DS_H / 256; ++q) v[q] = *reinterpret_cast<const float4*>(&sh.r[4 * (c.lane + 64 * q)]);
#pragma unroll
    for (int q = 0; q < DS_H / 256; ++q) {
      ss += v[q].x * v[q].x + v[q].y * v[q].y + v[q].z * v[q].z + v[q].w * v[q].w;
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[q].x), fabsf(v[q].y)), fmaxf(fabsf(v[q].z), fabsf(v[q].w))));
    }
    ds_norm_part(sh, ss, mx, c.lane, DS_CW);
  }
  // No barrier here: the compute waves issue layer 0's weight loads while the message wave
  // computes the statistics, which the first S0 barrier publishes.

  if (msg) ds_message_role<LOCAL>(sh, c, r_own);
  else ds_compute_role<LOCAL, DOWN_ROWS>(sh, c);
  ds_barrier();  // every wave's share of r_L's statistics
  if (sh.failures != 0) return;

  // ---- outputs (XCD 0's message waves): r_L and rmsnorm(r_L)
  if (msg && c.x == 0) {
    float inv, xmax;
    ds_norm(sh, inv, xmax);
    residual[c.j * DS_ROWS + c.lane] = r_own;
    if (x_out) x_out[c.j * DS_ROWS + c.lane] = f32_to_bf16_bits(r_own * inv);
  }
}

// Repack of down regions into the slice-major layout: one thread per (expert, slice, row).
__global__ void __launch_bounds__(256) repack_down_kernel(const uint8_t* __restrict__ src,
                                                          const uint8_t* __restrict__ src_scales, int64_t src_stride,
                                                          int64_t src_scales_stride, int experts, int H, int I,
                                                          uint8_t* __restrict__ dst, uint8_t* __restrict__ dst_scales) {
  int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t total = (int64_t)experts * DS_X * H;
  if (n >= total) return;
  int o = (int)(n % H);
  int s = (int)((n / H) % DS_X);
  int e = (int)(n / ((int64_t)H * DS_X));
  const int row_bytes = I / 2, slice_bytes = I / 16;             // packed bytes per row / per slice-row
  const int row_scales = I / 32, slice_scales = I / 256;
  const uint8_t* sp = src + e * src_stride + (int64_t)o * row_bytes + s * slice_bytes;
  uint8_t* dp = dst + (int64_t)e * H * row_bytes + ((int64_t)s * H + o) * slice_bytes;
  for (int q = 0; q < slice_bytes / 16; ++q) reinterpret_cast<uint4*>(dp)[q] = reinterpret_cast<const uint4*>(sp)[q];
  const uint8_t* ss = src_scales + e * src_scales_stride + (int64_t)o * row_scales + s * slice_scales;
  uint8_t* ds = dst_scales + (int64_t)e * H * row_scales + ((int64_t)s * H + o) * slice_scales;
  for (int q = 0; q < slice_scales; ++q) ds[q] = ss[q];
}

// XCC of each block of a DS_WGS-block launch (the hardware register, low 4 bits).
__global__ void __launch_bounds__(64) xcc_map_kernel(uint32_t* out) {
  if (threadIdx.x == 0) {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    out[blockIdx.x] = v & 0xfu;
  }
}

// Whether block b of a DS_WGS-block launch runs on XCC b % DS_X on the current
// device, checked once per device with a probe launch on `s`. Only then are the
// messages that stay within one XCD written with XCD-local stores. The probe
// allocates and synchronises, so it is not run while `s` is being captured into a
// graph: such a launch uses device-scope stores (call wm_decode_xcd_local before
// capturing to decide once).
static bool xcd_local_ok(hipStream_t s) {
  static std::mutex mu;
  static int known[64];  // 0 unknown, 1 yes, 2 no
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  std::lock_guard<std::mutex> lock(mu);
  if (known[dev] == 0) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone) return false;
    bool ok = false;
    uint32_t* d = nullptr;
    if (hipMalloc(&d, DS_WGS * sizeof(uint32_t)) == hipSuccess) {
      uint32_t h[DS_WGS] = {};
      hipLaunchKernelGGL(xcc_map_kernel, dim3(DS_WGS), dim3(64), 0, s, d);
      if (hipGetLastError() == hipSuccess &&
          hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, s) == hipSuccess &&
          hipStreamSynchronize(s) == hipSuccess) {
        ok = true;
        for (int b = 0; b < DS_WGS; ++b) ok &= h[b] == (uint32_t)(b % DS_X);
      }
      (void)hipFree(d);
    }
    known[dev] = ok ? 1 : 2;
  }
  return known[dev] == 1;
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT int wm_decode_xcd_local(void* stream) {
  int r = 0;
  int rc = guarded([&] { r = xcd_local_ok(as_stream(stream)) ? 1 : 0; });
  return rc != 0 ? -1 : r;
}

WM_EXPORT int wm_repack_down_slices(const void* src, const void* src_scales, int64_t src_stride,
                                    int64_t src_scales_stride, int32_t experts, int32_t hidden, int32_t inter, void* dst,
                                    void* dst_scales, void* stream) {
  return guarded([&] {
    if (experts < 0 || hidden < 1 || inter % 256) fail("wm_repack_down_slices: inter must be a multiple of 256");
    if (experts == 0) return;
    if (!src || !src_scales || !dst || !dst_scales) fail("wm_repack_down_slices: null pointer");
    if (((uintptr_t)src | (uintptr_t)dst | (uintptr_t)src_stride) % 16)
      fail("wm_repack_down_slices: weight regions must be 16-byte aligned");
    int64_t total = (int64_t)experts * DS_X * hidden;
    hipLaunchKernelGGL(repack_down_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, as_stream(stream),
                       (const uint8_t*)src, (const uint8_t*)src_scales, src_stride, src_scales_stride, experts, hidden,
                       inter, (uint8_t*)dst, (uint8_t*)dst_scales);
    check_launch("repack_down");
  });
}

WM_EXPORT size_t wm_decode_state_size(int32_t layers, int32_t experts) {
  (void)experts;
  return layers > 0 ? ds_layout(layers).total : 0;
}

WM_EXPORT size_t wm_decode_status_offset(int32_t layers, int32_t experts) {
  (void)experts;
  return layers > 0 ? ds_layout(layers).status : 0;
}

WM_EXPORT int wm_moe_decode_persistent_mxfp4(const float* logits, int32_t layers, int32_t experts, int32_t k,
                                             int32_t hidden, int32_t inter, const wm_decode_layer* layers_dev,
                                             float* residual, float eps, void* x_out, void* state, size_t state_bytes,
                                             int32_t down_row_layout, const int32_t* cancel, float* residual_trace,
                                             void* stream) {
  return guarded([&] {
    if (hidden != DS_H || inter != DS_I)
      fail("wm_moe_decode_persistent_mxfp4: supports hidden 2048 and intermediate 512");
    if (layers < 1 || layers > DS_MAX_LAYERS) fail("wm_moe_decode_persistent_mxfp4: layers must be in 1..128");
    if (k < 1 || k + 1 > DS_NE_MAX || k > experts) fail("wm_moe_decode_persistent_mxfp4: k must be in 1..11");
    if (experts < 1 || experts > 1024) fail("wm_moe_decode_persistent_mxfp4: experts must be in 1..1024");
    if (!logits || !layers_dev || !residual || !state) fail("wm_moe_decode_persistent_mxfp4: null pointer");
    if (state_bytes < ds_layout(layers).total || (uintptr_t)state % 8)
      fail("wm_moe_decode_persistent_mxfp4: state buffer too small or misaligned");
    hipStream_t s = as_stream(stream);
    const int per_lane = (experts + 63) / 64;
    const bool local = xcd_local_ok(s);
#define WM_DP(P, LOC, ROWS) hipLaunchKernelGGL((decode_persistent_kernel<P, LOC, ROWS>), dim3(DS_WGS), dim3(DS_THREADS), 0, \
                                               s, logits, layers, experts, k, 1, layers_dev, residual, eps, \
                                               (uint16_t*)x_out, (uint8_t*)state, cancel, residual_trace)
#define WM_DP_ROWS(P, LOC) if (down_row_layout) WM_DP(P, LOC, true); else WM_DP(P, LOC, false)
    if (per_lane <= 8) {
      if (local) { WM_DP_ROWS(8, true); } else { WM_DP_ROWS(8, false); }
    } else {
      if (local) { WM_DP_ROWS(16, true); } else { WM_DP_ROWS(16, false); }
    }
#undef WM_DP_ROWS
#undef WM_DP
    check_launch("decode_persistent");
  });
}

}  // extern "C"
