// The step before the MoE in one launch: the residual add and RMSNorm that produce the
// expert input, with the router GEMV and the shared expert's gate GEMV fused into the
// norm's epilogue:
//   v = r + y (y optional),  x = bf16(v * rsqrt(mean(v^2) + eps) * w_norm)  (w_norm optional),
//   logits[t, e] = x[t] . W_router[e],  shared_logit[t] = x[t] . g.
// The reference runs these as separate dispatches (the norm, then linear(router),
// linear(shared_gate): Native/QwenNative/engine.mm:2074-2079, with the norm in the
// hyper-connection mix before it); fused, the expert input is built once per block in
// LDS and never re-read from HBM for the GEMVs, and routing (wm_route_softmax_topk /
// wm_route_scored) follows on the device with no host step.
//
// Grid (row blocks, token blocks). A block owns TB tokens and RB consecutive output rows
// (router rows, then the gate row as row E). Every block recomputes the norm of its TB
// tokens (r and y are L2-resident after the first block of a token group) and keeps x as
// a [TB][H] bf16 tile in LDS (TB up to 16, within 96 KB); row block 0 also writes x and
// r + y to HBM. Each wave takes rows wave, wave + 4, ...: a lane streams 16-byte chunks
// of the weight row once and
// applies each to the TB tokens' x chunks (V_DOT2_F32_BF16), then one wave reduction
// per token.
#include <algorithm>
#include <cmath>

#include "moe_internal.h"

namespace wm {

typedef __bf16 nr_bf16x8 __attribute__((ext_vector_type(8)));
typedef float nr_f32x4 __attribute__((ext_vector_type(4)));

// Statistics of v = r + y for tokens t0 .. t0 + nt, then the x tile [TB][stride] (uint4 =
// 8 bf16; tokens past nt are zero). The writer block also stores x and v to HBM. Ends with
// a block barrier.
template <int TB>
__device__ __forceinline__ void build_x_tile(const float* __restrict__ r, const uint16_t* __restrict__ y,
                                             const uint16_t* __restrict__ nw, int t0, int nt, int hidden, float eps,
                                             bool writer, uint16_t* __restrict__ x_out, float* __restrict__ r_out,
                                             uint4* tile, int stride, float* inv_s,
                                             const uint16_t* __restrict__ xin = nullptr) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int chunks = hidden / 8;
  if (xin) {  // a plain linear: the tile is the given bf16 rows
    for (int t = 0; t < TB; ++t)
      for (int c = threadIdx.x; c < chunks; c += 256)
        tile[t * stride + c] = t < nt ? ((const uint4*)(xin + (int64_t)(t0 + t) * hidden))[c] : make_uint4(0, 0, 0, 0);
    __syncthreads();
    return;
  }
  constexpr int QU = 8;  // float4 loads in flight per lane
  const int quads = hidden / 4;
  for (int t = wave; t < nt; t += 4) {
    const float4* rr = (const float4*)(r + (int64_t)(t0 + t) * hidden);
    const uint2* yy = y ? (const uint2*)(y + (int64_t)(t0 + t) * hidden) : nullptr;
    float ss = 0.0f;
    for (int q0 = lane; q0 < quads; q0 += 64 * QU) {
      float4 v[QU];
      uint2 b[QU];
#pragma unroll
      for (int j = 0; j < QU; ++j) {
        const int q = q0 + 64 * j;
        v[j] = q < quads ? rr[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        b[j] = (yy && q < quads) ? yy[q] : make_uint2(0, 0);
      }
#pragma unroll
      for (int j = 0; j < QU; ++j) {
        float4 u = v[j];
        u.x += bf16_bits_to_f32(b[j].x & 0xffffu);
        u.y += bf16_bits_to_f32(b[j].x >> 16);
        u.z += bf16_bits_to_f32(b[j].y & 0xffffu);
        u.w += bf16_bits_to_f32(b[j].y >> 16);
        ss += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w;
      }
    }
    ss = segment_sum<64>(ss);
    if (lane == 0) inv_s[t] = rsqrtf(ss / (float)hidden + eps);
  }
  __syncthreads();
  // the tile, TU tokens at a time so their loads are in flight together
  constexpr int TU = TB < 4 ? TB : 4;
  for (int tb0 = 0; tb0 < TB; tb0 += TU) {
    for (int c = threadIdx.x; c < chunks; c += 256) {
      float4 ra[TU], rb[TU];
      uint4 yb[TU];
#pragma unroll
      for (int u = 0; u < TU; ++u) {
        const int t = tb0 + u;
        if (t < nt) {
          const float4* rr = (const float4*)(r + (int64_t)(t0 + t) * hidden) + 2 * c;
          ra[u] = rr[0];
          rb[u] = rr[1];
          yb[u] = y ? ((const uint4*)(y + (int64_t)(t0 + t) * hidden))[c] : make_uint4(0, 0, 0, 0);
        }
      }
      uint32_t nwv[4] = {0, 0, 0, 0};
      if (nw) {
        uint4 n4 = ((const uint4*)nw)[c];
        nwv[0] = n4.x, nwv[1] = n4.y, nwv[2] = n4.z, nwv[3] = n4.w;
      }
#pragma unroll
      for (int u = 0; u < TU; ++u) {
        const int t = tb0 + u;
        uint4* xt = tile + t * stride;
        if (t >= nt) {
          xt[c] = make_uint4(0, 0, 0, 0);
          continue;
        }
        const float inv = inv_s[t];
        float v[8] = {ra[u].x, ra[u].y, ra[u].z, ra[u].w, rb[u].x, rb[u].y, rb[u].z, rb[u].w};
        const uint32_t w4[4] = {yb[u].x, yb[u].y, yb[u].z, yb[u].w};
        uint32_t packed[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (y) {
            v[2 * j] += bf16_bits_to_f32(w4[j] & 0xffffu);
            v[2 * j + 1] += bf16_bits_to_f32(w4[j] >> 16);
          }
          float lo = v[2 * j] * inv, hi = v[2 * j + 1] * inv;
          if (nw) {
            lo *= bf16_bits_to_f32(nwv[j] & 0xffffu);
            hi *= bf16_bits_to_f32(nwv[j] >> 16);
          }
          packed[j] = (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
        }
        const uint4 xv = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        xt[c] = xv;
        if (writer) {
          const int64_t row = (int64_t)(t0 + t) * hidden;
          ((uint4*)(x_out + row))[c] = xv;
          if (r_out) {
            float4* ro = (float4*)(r_out + row) + 2 * c;
            ro[0] = make_float4(v[0], v[1], v[2], v[3]);
            ro[1] = make_float4(v[4], v[5], v[6], v[7]);
          }
        }
      }
    }
  }
  __syncthreads();
}

// Output row e: a router row, or the shared gate as row `experts`.
__device__ __forceinline__ const uint4* weight_row(const uint16_t* router, const uint16_t* gate, int experts,
                                                   int hidden, int e) {
  return (const uint4*)(e < experts ? router + (int64_t)e * hidden : gate);
}

__device__ __forceinline__ void store_row(float* logits, float* shared_logit, int experts, int t, int e, float v) {
  if (e < experts) logits[(int64_t)t * experts + e] = v;
  else shared_logit[t] = v;
}

// Few tokens (decode): a block owns rows_per_block rows (4: one per wave), and each wave
// loads its row's first NR_PREFETCH chunks per lane before the norm, so the weight stream
// overlaps the statistics and the tile.
constexpr int NR_PREFETCH = 8;

template <int TB>
__global__ void __launch_bounds__(256) norm_router_kernel(
    const float* __restrict__ r, const uint16_t* __restrict__ y, const uint16_t* __restrict__ nw, int tokens,
    int hidden, float eps, const uint16_t* __restrict__ router, int experts, const uint16_t* __restrict__ gate,
    int rows_per_block, uint16_t* __restrict__ x_out, float* __restrict__ r_out, float* __restrict__ logits,
    float* __restrict__ shared_logit) {
  extern __shared__ uint4 x_tile[];  // [TB][hidden / 8]
  __shared__ float inv_s[TB];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int t0 = blockIdx.y * TB;
  const int nt = min(TB, tokens - t0);
  const int chunks = hidden / 8;
  const int rows = experts + (gate ? 1 : 0);
  const int first = blockIdx.x * rows_per_block;
  const int last = min(rows, first + rows_per_block);
  const int e0 = first + wave;

  uint4 pre[NR_PREFETCH];
  if (e0 < last) {
    const uint4* w = weight_row(router, gate, experts, hidden, e0);
#pragma unroll
    for (int j = 0; j < NR_PREFETCH; ++j)
      if (lane + 64 * j < chunks) pre[j] = w[lane + 64 * j];
  }
  build_x_tile<TB>(r, y, nw, t0, nt, hidden, eps, blockIdx.x == 0, x_out, r_out, x_tile, chunks, inv_s);

  for (int e = e0; e < last; e += 4) {
    const uint4* w = weight_row(router, gate, experts, hidden, e);
    float acc[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) acc[t] = 0.0f;
    auto apply = [&](uint4 wv, int c) {
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        uint4 xv = x_tile[t * chunks + c];
        float a = acc[t];
        a = dot2_bf16(bits_to_bf16x2(wv.x), bits_to_bf16x2(xv.x), a);
        a = dot2_bf16(bits_to_bf16x2(wv.y), bits_to_bf16x2(xv.y), a);
        a = dot2_bf16(bits_to_bf16x2(wv.z), bits_to_bf16x2(xv.z), a);
        a = dot2_bf16(bits_to_bf16x2(wv.w), bits_to_bf16x2(xv.w), a);
        acc[t] = a;
      }
    };
#pragma unroll
    for (int j = 0; j < NR_PREFETCH; ++j) {
      const int c = lane + 64 * j;
      if (c < chunks) apply(e == e0 ? pre[j] : w[c], c);
    }
    for (int c = lane + 64 * NR_PREFETCH; c < chunks; c += 64) apply(w[c], c);
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      float s = segment_sum<64>(acc[t]);
      if (lane == t && t < nt) store_row(logits, shared_logit, experts, t0 + t, e, s);
    }
  }
}

// Many tokens (prefill): the router GEMM on MFMA. A block owns TB tokens (8 or 16 columns
// of V_MFMA_F32_16X16X32_BF16; columns past TB are zero) and every output row; the x tile
// rows are padded by 16 bytes so the 16 tokens' reads fall on distinct banks. Wave w
// takes 16-row groups w, w + 4, ... four at a time: per 32-wide K step, four weight
// fragments (16 bytes per lane, loaded four steps ahead) against one x fragment.
// Operands: lane l holds row / token l % 16 and K chunk (l / 16) of each 32-wide step (the
// same lane-to-K map for both, so the K order inside a step cancels); the result holds
// token l % 16 for rows 4 (l / 16) .. +3 of the group. With `packed` (wm_repack_router)
// each fragment is one contiguous 1 KB read instead of 16 rows x 64 bytes.

// The packed router: [groups][hidden / 32][64 lanes] uint4, lane l of group g and step s
// holding row 16 g + l % 16 (router rows, then the gate row, then zeros; one spare zero
// group follows when the gate is packed), 8 values from column 32 s + 8 (l / 16).
__global__ void __launch_bounds__(256) repack_router_kernel(const uint4* __restrict__ router,
                                                            const uint4* __restrict__ gate, int experts, int hidden,
                                                            int64_t total, uint4* __restrict__ packed) {
  const int steps = hidden / 32, chunks = hidden / 8;
  for (int64_t o = blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
    const int lane = (int)(o % 64);
    const int64_t gs = o / 64;
    const int st = (int)(gs % steps), g = (int)(gs / steps);
    const int row = 16 * g + lane % 16, chunk = 4 * st + lane / 16;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < experts) v = router[(int64_t)row * chunks + chunk];
    else if (row == experts && gate) v = gate[chunk];
    packed[o] = v;
  }
}
template <int TB>
__global__ void __launch_bounds__(256) norm_router_mfma_kernel(
    const float* __restrict__ r, const uint16_t* __restrict__ y, const uint16_t* __restrict__ nw, int tokens,
    int hidden, float eps, const uint16_t* __restrict__ router, int experts, const uint16_t* __restrict__ gate,
    const uint4* __restrict__ packed, uint16_t* __restrict__ x_out, float* __restrict__ r_out,
    float* __restrict__ logits, float* __restrict__ shared_logit, const uint16_t* __restrict__ xin) {
  extern __shared__ uint4 x_tile[];  // [TB][hidden / 8 + 1]
  __shared__ float inv_s[TB];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int t0 = blockIdx.x * TB;
  const int nt = min(TB, tokens - t0);
  const int chunks = hidden / 8, stride = chunks + 1, steps = hidden / 32;
  build_x_tile<TB>(r, y, nw, t0, nt, hidden, eps, xin == nullptr, x_out, r_out, x_tile, stride, inv_s, xin);

  const int rows = experts + (gate ? 1 : 0);
  const int groups = (rows + 15) / 16;
  const int n = lane % 16, kq = lane / 16;
  constexpr int NCOL = TB > 16 ? TB / 16 : 1;  // 16-token column blocks
  const uint4* xb[NCOL];
  bool has_col[NCOL];
#pragma unroll
  for (int cb = 0; cb < NCOL; ++cb) {
    has_col[cb] = 16 * cb + n < TB;
    xb[cb] = x_tile + (has_col[cb] ? 16 * cb + n : 0) * stride + kq;
  }
  for (int g0 = wave; g0 < groups; g0 += 16) {
    const uint4* wp[4];
    const int wstep = packed ? 64 : 4;  // uint4s from one K step's fragment to the next
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = (g0 + 4 * j) * 16 + n;
      if (packed)  // fragment-major: group g's step-s fragment is 64 consecutive uint4, one per lane
        wp[j] = packed + (int64_t)min(g0 + 4 * j, groups - 1) * steps * 64 + lane;
      else
        wp[j] = weight_row(router, gate, experts, hidden, e < rows ? e : 0) + kq;
    }
    // four K steps of fragments in flight: set u holds step s + u
    constexpr int PD = 4;
    nr_f32x4 acc[4][NCOL];
    uint4 a[PD][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int cb = 0; cb < NCOL; ++cb) acc[j][cb] = nr_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < PD; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (g0 + 4 * j < groups) a[u][j] = wp[j][wstep * (u < steps ? u : 0)];
    for (int s = 0; s < steps; s += PD) {
#pragma unroll
      for (int u = 0; u < PD; ++u) {
        if (s + u < steps) {
          uint4 bv[NCOL];
#pragma unroll
          for (int cb = 0; cb < NCOL; ++cb) bv[cb] = has_col[cb] ? xb[cb][4 * (s + u)] : make_uint4(0, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (g0 + 4 * j >= groups) break;  // wave-uniform: a last batch with fewer groups
#pragma unroll
            for (int cb = 0; cb < NCOL; ++cb)
              acc[j][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(nr_bf16x8, a[u][j]),
                                                                   __builtin_bit_cast(nr_bf16x8, bv[cb]), acc[j][cb],
                                                                   0, 0, 0);
            if (s + u + PD < steps) a[u][j] = wp[j][wstep * (s + u + PD)];
          }
        }
      }
    }
#pragma unroll
    for (int cb = 0; cb < NCOL; ++cb) {
      const int t = 16 * cb + n;
      if (t >= nt) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = (g0 + 4 * j) * 16 + 4 * kq + i;
          if (e < rows) store_row(logits, shared_logit, experts, t0 + t, e, acc[j][cb][i]);
        }
    }
  }
}

// The MFMA path's token block: 32 tokens (two column blocks per weight fragment) or 16 when
// the padded x tile fits 150 KB of LDS, else 8; 0 (the dot-product path) below 16 tokens or
// when hidden is not a multiple of 32.
static int mfma_token_block(int tokens, int hidden) {
  if (tokens < 16 || hidden % 32) return 0;
  if (tokens >= 32 && (size_t)32 * (hidden / 8 + 1) * 16 + 128 <= 150 * 1024) return 32;
  for (int tb : {16, 8})
    if ((size_t)tb * (hidden / 8 + 1) * 16 + 64 <= 150 * 1024) return tb;
  return 0;
}

// The dot-product path's token block: the largest whose x tile (plus the 64-byte
// statistics array) fits 96 KB of LDS, no larger than the tokens.
static int pick_token_block(int tokens, int hidden) {
  const int fit = (96 * 1024 - 64) / (hidden * 2);
  for (int tb : {16, 8, 4, 2}) if (tb <= fit && tokens >= tb) return tb;
  return 1;
}

// logits = x . w^T on the router GEMM's MFMA path (a tile of x as given, no norm), for
// wm_linear_bf16 at 64+ tokens. False when the shape does not suit it (the caller then uses
// the one-wave-per-output kernel).
// Whether linear_bf16_mfma takes x [tokens, hidden] (its x tile must fit the LDS).
bool linear_bf16_mfma_fits(int tokens, int hidden) { return tokens >= 64 && mfma_token_block(tokens, hidden) > 0; }

bool linear_bf16_mfma(const void* x, const void* w, int tokens, int hidden, int outputs, float* out, hipStream_t s) {
  const int tb = tokens >= 64 ? mfma_token_block(tokens, hidden) : 0;
  if (!tb || ((uintptr_t)x % 16) || ((uintptr_t)w % 16)) return false;
  const int blocks = (tokens + tb - 1) / tb;
  const size_t lds = (size_t)tb * (hidden / 8 + 1) * 16;
#define WM_LIN(TB) hipLaunchKernelGGL(norm_router_mfma_kernel<TB>, dim3(blocks), dim3(256), lds, s, nullptr, nullptr, \
                                      nullptr, tokens, hidden, 0.0f, (const uint16_t*)w, outputs, nullptr, nullptr, \
                                      nullptr, nullptr, out, nullptr, (const uint16_t*)x)
  if (tb == 32) WM_LIN(32);
  else if (tb == 16) WM_LIN(16);
  else WM_LIN(8);
#undef WM_LIN
  check_launch("linear_bf16 (MFMA)");
  return true;
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT size_t wm_router_packed_bytes(int32_t experts, int32_t hidden, int32_t has_gate) {
  if (experts < 1 || hidden < 32 || hidden % 32) return 0;
  // one spare zero group when the gate row is packed, so the size alone tells whether it is
  const int g = has_gate ? 1 : 0;
  return (size_t)((experts + g + 15) / 16 + g) * 16 * hidden * 2;
}

WM_EXPORT int wm_repack_router(const void* router, const void* shared_gate, int32_t experts, int32_t hidden,
                               void* packed, void* stream) {
  return guarded([&] {
    if (experts < 1 || hidden < 32 || hidden % 32) fail("wm_repack_router: hidden must be a multiple of 32");
    if (!router || !packed) fail("wm_repack_router: null pointer");
    for (const void* p : {router, shared_gate, (const void*)packed})
      if (p && ((uintptr_t)p % 16)) fail("wm_repack_router: tensors must be 16-byte aligned");
    const int64_t total = (int64_t)wm_router_packed_bytes(experts, hidden, shared_gate != nullptr) / 16;
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(repack_router_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), (const uint4*)router,
                       (const uint4*)shared_gate, experts, hidden, total, (uint4*)packed);
    check_launch("repack_router");
  });
}

WM_EXPORT int wm_norm_router(const float* residual, const void* y, const void* norm_weight, int32_t tokens,
                             int32_t hidden, float eps, const void* router, int32_t experts, const void* shared_gate,
                             const void* router_packed, size_t router_packed_bytes, void* x,
                             float* residual_out, float* logits, float* shared_logit, void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_norm_router: negative token count");
    if (hidden < 8 || hidden % 8 || hidden * 2 > 64 * 1024) fail("wm_norm_router: hidden must be a multiple of 8 up to 32768");
    if (experts < 1) fail("wm_norm_router: experts must be at least 1");
    if ((shared_gate == nullptr) != (shared_logit == nullptr))
      fail("wm_norm_router: shared_gate and shared_logit go together");
    if (tokens == 0) return;
    if (!residual || !router || !x || !logits) fail("wm_norm_router: null pointer");
    // Row block 0 writes x and v while other blocks still read residual and y.
    auto overlap = [](const void* p, size_t pn, const void* q, size_t qn) {
      const char *a = (const char*)p, *b = (const char*)q;
      return p && q && a < b + qn && b < a + pn;
    };
    const size_t n4 = (size_t)tokens * hidden * sizeof(float), n2 = (size_t)tokens * hidden * 2;
    if (overlap(residual_out, n4, residual, n4) || overlap(residual_out, n4, y, n2))
      fail("wm_norm_router: residual_out must not overlap residual or y (other blocks still read them)");
    if (overlap(x, n2, residual, n4) || overlap(x, n2, y, n2))
      fail("wm_norm_router: x must not overlap residual or y (other blocks still read them)");
    if (router_packed && (hidden % 32 || router_packed_bytes != wm_router_packed_bytes(experts, hidden, shared_gate != nullptr)))
      fail("wm_norm_router: the packed router does not match experts, hidden and the shared gate (wm_router_packed_bytes)");
    for (const void* p : {(const void*)residual, y, norm_weight, router, shared_gate, router_packed, (const void*)x,
                          (const void*)residual_out})
      if (p && ((uintptr_t)p % 16)) fail("wm_norm_router: tensors must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    const int rows = experts + (shared_gate ? 1 : 0);
    const int mfma_tb = mfma_token_block(tokens, hidden);
    if (mfma_tb) {
      const int blocks = (tokens + mfma_tb - 1) / mfma_tb;
      const size_t lds = (size_t)mfma_tb * (hidden / 8 + 1) * 16;
#define WM_NRM(TB) hipLaunchKernelGGL(norm_router_mfma_kernel<TB>, dim3(blocks), dim3(256), lds, s, residual, \
                                      (const uint16_t*)y, (const uint16_t*)norm_weight, tokens, hidden, eps, \
                                      (const uint16_t*)router, experts, (const uint16_t*)shared_gate, \
                                      (const uint4*)router_packed, (uint16_t*)x, residual_out, logits, shared_logit, \
                                      nullptr)
      if (mfma_tb == 32) WM_NRM(32);
      else if (mfma_tb == 16) WM_NRM(16);
      else WM_NRM(8);
#undef WM_NRM
      check_launch("norm_router_mfma");
      return;
    }
    const int tb = pick_token_block(tokens, hidden);
    // The rows spread over many blocks (4 per block, one per wave), as few tokens leave
    // the weight stream as the only work.
    const int token_blocks = (tokens + tb - 1) / tb;
    if (token_blocks > 65535) fail("wm_norm_router: too many tokens for one call");
    const int rows_per_block = 4;
    dim3 grid((rows + rows_per_block - 1) / rows_per_block, token_blocks);
    const size_t lds = (size_t)tb * hidden * 2;
#define WM_NR(TB) hipLaunchKernelGGL(norm_router_kernel<TB>, grid, dim3(256), lds, s, residual, (const uint16_t*)y, \
                                     (const uint16_t*)norm_weight, tokens, hidden, eps, (const uint16_t*)router, experts, \
                                     (const uint16_t*)shared_gate, rows_per_block, (uint16_t*)x, residual_out, logits, \
                                     shared_logit)
    switch (tb) {
      case 16: WM_NR(16); break;
      case 8: WM_NR(8); break;
      case 4: WM_NR(4); break;
      case 2: WM_NR(2); break;
      default: WM_NR(1); break;
    }
#undef WM_NR
    check_launch("norm_router");
  });
}

}  // extern "C"
