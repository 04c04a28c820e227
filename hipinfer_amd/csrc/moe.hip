// Mixture-of-Experts router and experts on gfx950 (the reference's hi_moe_router,
// hi_moe_work_bytes, hi_moe_experts; src/api.cu:849-911, kernels src/kernels.cuh:2044-2276,
// numerics docs/moe-design.md:186-201).
//
// Rounding follows the reference: router logits rounded to fp16; top-k by value with NaN above
// numbers and ties to the lower expert index; weights = softmax over the k (norm_topk) or over
// all E, rounded to fp16 when the model rounds them; each expert's SwiGLU as silu_mul; each
// expert's down projection rounded to fp16, times its weight (rounded again for fp16 weights),
// summed over the k in fp32 in slot order, rounded once, scaled (rounded) when scale != 1, and
// added to the residual with one fp16 add.
//
// Two expert paths, as the reference:
//  * GEMV (decode, few rows): one wave per (pair, unit) streams the selected experts' gate/up
//    rows; one wave per (token, hidden column) does the k down-projection dot products and the
//    weighted combine in slot order. Each wave issues all the loads of a round together (a round
//    covers a whole row at the usual sizes), so a kernel costs about one memory round trip.
//    Fixed launch shape, the expert choice stays on the device.
//  * grouped (prefill): a counting sort of the M*k (token, slot) pairs by expert, which also
//    writes each expert's row-tile prefix; a gather; two grouped MFMA GEMM launches (gate/up with
//    the SwiGLU epilogue, then down) in which every block finds its expert from the prefix; and
//    the combine. Unlike the reference (which copies the per-expert counts to the host and
//    launches one GEMM per expert, api.cu:901-909) nothing returns to the host, so the grouped
//    path is graph-capturable too.
// Expert ids outside [0, E) are never dereferenced: such a slot contributes nothing.
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "gemm.h"
#include "hi_internal.h"

namespace {

constexpr int kMoeNormTopk = 1, kMoeFp16Weights = 2;

// v beats (best, bi): NaN above numbers; equal values (and NaN vs NaN) go to the lower index
// (reference argmax_better, kernels.cuh:1886-1890).
__device__ __forceinline__ bool argmax_better(float v, int i, float best, int bi) {
  const bool vn = v != v, bn = best != best;
  return (vn != bn) ? vn : ((vn | (v == best)) ? i < bi : v > best);  // selects, no branches
}

// ------------------------------------------------------------------ router
// The router's three steps, shared by the router kernel and the fused decode kernel so that both
// produce the same bits:
//  * logits: the block's waves take experts two at a time, each loading the row's chunks and both
//    expert rows together (CH chunks of 8 halves per lane per round), so a row costs about one
//    memory round trip; every expert's dot product runs in the same order whatever the number of
//    waves; rounded to fp16 (the router linear's output dtype);
//  * top k by rank: argmax_better is a strict total order on (logit, index), so the expert that
//    exactly j others beat is the j-th pick of the sequential argmax; every expert's rank is
//    counted in parallel (rank_key turns the order into an unsigned compare, one ballot counts 64
//    rivals);
//  * weights: softmax over the k (norm_topk) or over all E, rounded to fp16 when the model rounds.
constexpr int kRouterWaves = 16;
template <int CH>
__device__ __forceinline__ void router_logits(const f16* __restrict__ xr, const f16* __restrict__ Wr, int E, int H,
                                              int nwaves, int wave, int lane, float* logit) {
  const int H8 = H / 8;
  for (int e0 = wave; e0 < E; e0 += 2 * nwaves) {
    const int e1 = e0 + nwaves;
    const f16* w0 = Wr + (int64_t)e0 * H;
    const f16* w1 = Wr + (int64_t)min(e1, E - 1) * H;
    float a0 = 0.f, a1 = 0.f;
    for (int g = 0; g < H8; g += 64 * CH) {
      u32x4 xv[CH], v0[CH], v1[CH];
#pragma unroll
      for (int j = 0; j < CH; j++) {
        const int c = g + j * 64 + lane;
        const int cc = c < H8 ? c : 0;  // past the row: a valid chunk, zeroed below
        xv[j] = *reinterpret_cast<const u32x4*>(xr + 8 * cc);
        v0[j] = *reinterpret_cast<const u32x4*>(w0 + 8 * cc);
        v1[j] = *reinterpret_cast<const u32x4*>(w1 + 8 * cc);
      }
#pragma unroll
      for (int j = 0; j < CH; j++) {
        const bool ok = g + j * 64 + lane < H8;
#pragma unroll
        for (int p = 0; p < 4; p++) {
          const f16x2 x2 = as_h2(ok ? xv[j][p] : 0u);
          a0 = dot2(as_h2(v0[j][p]), x2, a0);
          a1 = dot2(as_h2(v1[j][p]), x2, a1);
        }
      }
    }
    a0 = wave_sum(a0);
    a1 = wave_sum(a1);
    if (lane == 0) {
      logit[e0] = (float)(f16)a0;  // the router linear is rounded to fp16
      if (e1 < E) logit[e1] = (float)(f16)a1;
    }
  }
}

// Sort key of (logit v, expert i) in argmax_better's order: NaN above every number, -0 equal to +0,
// numbers by value (sign-magnitude bits mapped to an increasing unsigned), equal values to the lower
// index (the low word falls as i rises). Expert o beats expert e exactly when key(o) > key(e).
__device__ __forceinline__ uint64_t rank_key(float v, int i) {
  uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  if (v != v) u = 0xFFFFFFFFu;
  return ((uint64_t)u << 32) | (0xFFFFFFFFu - (uint32_t)i);
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l), hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}

// Every wave of the block calls this with all 64 lanes: lane l holds the keys of experts l, l + 64,
// ...; wave w ranks experts w, w + nwaves, ... with one ballot per 64 candidates.
__device__ __forceinline__ void router_topk(const float* logit, int E, int k, int nwaves, int wave, int lane,
                                            float* selv, int* seli) {
  constexpr int C = kMoeMaxE / 64;
  uint64_t key[C];
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int o = c * 64 + lane;
    key[c] = o < E ? rank_key(logit[o], o) : 0ull;  // 0 beats nothing
  }
  for (int e = wave; e < E; e += nwaves) {
    const int ce = e >> 6, le = e & 63;
    uint64_t ke = 0;
#pragma unroll
    for (int c = 0; c < C; c++)
      if (c == ce) ke = readlane_u64(key[c], le);
    int r = 0;
#pragma unroll
    for (int c = 0; c < C; c++)
      if (c * 64 < E) r += __popcll(__ballot(key[c] > ke));
    if (r < k && lane == 0) {
      seli[r] = e;
      selv[r] = logit[e];
    }
  }
}

// One wave: the k weights of token t into idx_out / w_out (descending by logit).
__device__ __forceinline__ void router_weights(const float* logit, const float* selv, const int* seli, int E, int k,
                                               int flags, int lane, int t, int* __restrict__ idx_out,
                                               float* __restrict__ w_out) {
  const float mx = selv[0];
  const float ej = lane < k ? expf(selv[lane] - mx) : 0.f;  // lane j: slot j's exponential
  float denom = 0.f;
  if (flags & kMoeNormTopk) {
    for (int j = 0; j < k; j++) denom += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ej), j));  // slot order
  } else {
    float sum = 0.f;
    for (int e = lane; e < E; e += 64) sum += expf(logit[e] - mx);
    denom = wave_sum(sum);
  }
  if (lane < k) {
    float wj = ej / denom;
    if (flags & kMoeFp16Weights) wj = (float)(f16)wj;
    idx_out[(int64_t)t * k + lane] = seli[lane];
    w_out[(int64_t)t * k + lane] = wj;
  }
}

// One block of 16 waves per token row.
template <int CH>
__global__ void __launch_bounds__(kRouterWaves * 64) moe_router_kernel(const f16* __restrict__ xn, int64_t ldx,
                                                                      const f16* __restrict__ Wr, int E, int H, int k,
                                                                      int flags, int* __restrict__ idx_out,
                                                                      float* __restrict__ w_out) {
  __shared__ float logit[kMoeMaxE];
  __shared__ float selv[kMoeMaxK];
  __shared__ int seli[kMoeMaxK];
  const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  router_logits<CH>(xn + t * ldx, Wr, E, H, kRouterWaves, wave, lane, logit);
  __syncthreads();
  router_topk(logit, E, k, kRouterWaves, wave, lane, selv, seli);
  __syncthreads();
  if (wave == 0) router_weights(logit, selv, seli, E, k, flags, lane, t, idx_out, w_out);
}

// Chunks of 8 halves per lane per load round for a row of n halves: one round covers the row up to
// n = 64 * 8 * 4.
inline int chunks_for(int n) { return n <= 512 ? 1 : n <= 1024 ? 2 : 4; }

// ------------------------------------------------------------------ GEMV expert path
// Gate/up + SwiGLU: one wave per (token-slot pair p, output unit o); unit o of expert e reads rows
// (o/16)*32 + o%16 and that + 16 of wgu[e] [2I, H]. A round issues both rows' and the activation's
// chunks together (CH per lane), so a unit of H <= 64 * 8 * CH costs one round trip.
constexpr int kMoeWaves = 8;
template <int CH>
__global__ void __launch_bounds__(kMoeWaves * 64) moe_gemv_gu_kernel(const f16* __restrict__ xn, int64_t ldx,
                                                                     const f16* __restrict__ wgu,
                                                                     const int* __restrict__ idx, int n, int k, int E,
                                                                     int H, int I, f16* __restrict__ act) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * kMoeWaves + (threadIdx.x >> 6);
  if (w >= (int64_t)n * I) return;
  const int p = (int)(w / I), o = (int)(w - (int64_t)p * I);
  const int e = idx[p];
  if (e < 0 || e >= E) {  // no expert: this slot's activation is zero
    if (lane == 0) act[(int64_t)p * I + o] = (f16)0.f;
    return;
  }
  const int r0 = (o >> 4) * 32 + (o & 15);
  const f16* g = wgu + ((int64_t)e * 2 * I + r0) * H;
  const f16* u = g + 16 * (int64_t)H;
  const f16* xr = xn + (int64_t)(p / k) * ldx;
  const int H8 = H / 8;
  float ag = 0.f, au = 0.f;
  for (int b = 0; b < H8; b += 64 * CH) {
    u32x4 xv[CH], gv[CH], uv[CH];
#pragma unroll
    for (int j = 0; j < CH; j++) {
      const int c = b + j * 64 + lane, cc = c < H8 ? c : 0;
      xv[j] = *reinterpret_cast<const u32x4*>(xr + 8 * cc);
      gv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g + 8 * cc));
      uv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(u + 8 * cc));
    }
#pragma unroll
    for (int j = 0; j < CH; j++) {
      const bool ok = b + j * 64 + lane < H8;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const f16x2 x2 = as_h2(ok ? xv[j][q] : 0u);
        ag = dot2(as_h2(gv[j][q]), x2, ag);
        au = dot2(as_h2(uv[j][q]), x2, au);
      }
    }
  }
  ag = wave_sum(ag);
  au = wave_sum(au);
  if (lane == 0) act[(int64_t)p * I + o] = silu_mul(ag, au);
}

// Router + gate/up + SwiGLU in one launch (the GEMV path of hi_moe_route_experts): a block of 16
// waves serves one token-slot pair p = t*k + j and 16 consecutive units (I % 16 == 0), so it first
// computes token t's logits and top k with the router's own steps and wave count (the same bits as
// moe_router_kernel, in one memory round trip for E <= 32; every block reads the router weights,
// E*H*2 bytes, mostly from L2), then streams slot j's expert rows as moe_gemv_gu_kernel does. The
// block of pair t*k and unit 0 also writes the token's idx / w, which the down projection reads.
constexpr int kFusedWaves = kRouterWaves;
template <int CH>
__global__ void __launch_bounds__(kFusedWaves * 64) moe_route_gu_kernel(const f16* __restrict__ xn, int64_t ldx,
                                                                      const f16* __restrict__ Wr,
                                                                      const f16* __restrict__ wgu, int n, int k, int E,
                                                                      int H, int I, int flags, int* __restrict__ idx_out,
                                                                      float* __restrict__ w_out, f16* __restrict__ act) {
  __shared__ float logit[kMoeMaxE];
  __shared__ float selv[kMoeMaxK];
  __shared__ int seli[kMoeMaxK];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t w0 = (int64_t)blockIdx.x * kFusedWaves;
  const int p = (int)(w0 / I), t = p / k, j = p - t * k;
  const f16* xr = xn + (int64_t)t * ldx;
  router_logits<CH>(xr, Wr, E, H, kFusedWaves, wave, lane, logit);
  __syncthreads();
  router_topk(logit, E, k, kFusedWaves, wave, lane, selv, seli);
  __syncthreads();
  if (j == 0 && w0 == (int64_t)p * I && wave == 0) router_weights(logit, selv, seli, E, k, flags, lane, t, idx_out, w_out);
  const int64_t w = w0 + wave;
  if (w >= (int64_t)n * I) return;
  const int o = (int)(w - (int64_t)p * I);
  const int e = seli[j];
  const int r0 = (o >> 4) * 32 + (o & 15);
  const f16* g = wgu + ((int64_t)e * 2 * I + r0) * H;
  const f16* u = g + 16 * (int64_t)H;
  const int H8 = H / 8;
  float ag = 0.f, au = 0.f;
  for (int b = 0; b < H8; b += 64 * CH) {
    u32x4 xv[CH], gv[CH], uv[CH];
#pragma unroll
    for (int q = 0; q < CH; q++) {
      const int c = b + q * 64 + lane, cc = c < H8 ? c : 0;
      xv[q] = *reinterpret_cast<const u32x4*>(xr + 8 * cc);
      gv[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g + 8 * cc));
      uv[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(u + 8 * cc));
    }
#pragma unroll
    for (int q = 0; q < CH; q++) {
      const bool ok = b + q * 64 + lane < H8;
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const f16x2 x2 = as_h2(ok ? xv[q][h] : 0u);
        ag = dot2(as_h2(gv[q][h]), x2, ag);
        au = dot2(as_h2(uv[q][h]), x2, au);
      }
    }
  }
  ag = wave_sum(ag);
  au = wave_sum(au);
  if (lane == 0) act[(int64_t)p * I + o] = silu_mul(ag, au);
}

// Down projection + weighted combine + residual: one wave per (token b, hidden column h). All k
// (expert row, activation row) chunk pairs of a round are loaded together; the k dot products are
// then reduced one by one and combined in slot order. KM >= k bounds the per-wave registers.
template <int KM>
__global__ void __launch_bounds__(kMoeWaves * 64) moe_gemv_down_kernel(const f16* __restrict__ act,
                                                                       const f16* __restrict__ wdown,
                                                                       const int* __restrict__ idx,
                                                                       const float* __restrict__ wts, int M, int k,
                                                                       int E, int H, int I, int flags, float scale,
                                                                       f16* x, int64_t ldx) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * kMoeWaves + (threadIdx.x >> 6);
  if (w >= (int64_t)M * H) return;
  const int b = (int)(w / H), h = (int)(w - (int64_t)b * H);
  int ex[KM];
#pragma unroll
  for (int j = 0; j < KM; j++) ex[j] = j < k ? idx[(int64_t)b * k + j] : -1;
  float acc[KM];
#pragma unroll
  for (int j = 0; j < KM; j++) acc[j] = 0.f;
  const int I8 = I / 8;
  for (int c0 = 0; c0 < I8; c0 += 64) {
    const int c = c0 + lane, cc = c < I8 ? c : 0;
    u32x4 wv[KM], av[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) {
      if (j < k) {
        const int e = (ex[j] >= 0 && ex[j] < E) ? ex[j] : 0;  // an id outside [0, E) is dropped below
        wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wdown + ((int64_t)e * H + h) * I + 8 * cc));
        av[j] = *reinterpret_cast<const u32x4*>(act + ((int64_t)b * k + j) * I + 8 * cc);
      }
    }
#pragma unroll
    for (int j = 0; j < KM; j++) {
      if (j < k) {
#pragma unroll
        for (int q = 0; q < 4; q++) acc[j] = dot2(as_h2(wv[j][q]), as_h2(c < I8 ? av[j][q] : 0u), acc[j]);
      }
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < KM; j++) {
    if (j < k && ex[j] >= 0 && ex[j] < E) {  // uniform over the wave
      float c = (float)(f16)wave_sum(acc[j]) * wts[(int64_t)b * k + j];
      asm volatile("" : "+v"(c));  // the fp32 product is what gets rounded to fp16
      sum += (flags & kMoeFp16Weights) ? (float)(f16)c : c;
    }
  }
  if (lane == 0) {
    f16 o = (f16)sum;
    if (scale != 1.f) {
      float t = (float)o * scale;
      asm volatile("" : "+v"(t));  // fp32 product, then fp16 (two roundings)
      o = (f16)t;
    }
    f16* dst = x + (int64_t)b * ldx + h;
    *dst = *dst + o;
  }
}

// ------------------------------------------------------------------ grouped path
// Counting sort of the n (token, slot) pairs by expert, by one block of kSortThreads: off[E+1] the
// exclusive prefix of the per-expert counts, tiles[E+1] the same of their row tiles of kGrpBM, perm[q] the pair at sorted position q. Pairs
// whose expert id lies outside [0, E) are left out. The two prefixes are one wave's scan (four
// experts a lane); a thread's ids of a pass are requested together. The order within an expert
// follows the LDS atomics: every GEMM row is computed on its own, so it changes no result.
constexpr int kSortThreads = 1024;
__global__ void __launch_bounds__(kSortThreads) moe_sort_kernel(const int* __restrict__ idx, int n, int E,
                                                                int* __restrict__ off, int* __restrict__ tiles,
                                                                int* __restrict__ perm) {
  __shared__ int cnt[kMoeMaxE], cur[kMoeMaxE];
  const int tid = threadIdx.x;
  constexpr int P = 4;  // ids a thread requests together
  for (int e = tid; e < E; e += kSortThreads) cnt[e] = 0;
  __syncthreads();
  int ev0[P];  // the ids of the last (for n <= P * kSortThreads: the only) round
  for (int p0 = 0; p0 < n; p0 += P * kSortThreads) {
#pragma unroll
    for (int j = 0; j < P; j++) {
      const int p = p0 + j * kSortThreads + tid;
      ev0[j] = p < n ? idx[p] : -1;
    }
#pragma unroll
    for (int j = 0; j < P; j++)
      if (ev0[j] >= 0 && ev0[j] < E) atomicAdd(&cnt[ev0[j]], 1);
  }
  __syncthreads();
  if (tid < 64) {
    static_assert(kMoeMaxE <= 4 * 64, "four experts a lane");
    int c[4], tl[4], cs = 0, ts = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int e = 4 * tid + j;
      c[j] = e < E ? cnt[e] : 0;
      tl[j] = (c[j] + kGrpBM - 1) / kGrpBM;
      cs += c[j];
      ts += tl[j];
    }
    int ic = cs, it = ts;  // inclusive scan over the lanes
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int oc = __shfl_up(ic, d, 64), ot = __shfl_up(it, d, 64);
      if (tid >= d) {
        ic += oc;
        it += ot;
      }
    }
    int ec = ic - cs, et = it - ts;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int e = 4 * tid + j;
      if (e < E) {
        off[e] = ec;
        cur[e] = ec;
        tiles[e] = et;
      }
      ec += c[j];
      et += tl[j];
    }
    if (tid == 63) {
      off[E] = ic;
      tiles[E] = it;
    }
  }
  __syncthreads();
  for (int p0 = 0; p0 < n; p0 += P * kSortThreads) {
    int ev[P];
    if (n <= P * kSortThreads) {  // one round: the ids of the first pass are still in registers
#pragma unroll
      for (int j = 0; j < P; j++) ev[j] = ev0[j];
    } else {
#pragma unroll
      for (int j = 0; j < P; j++) {
        const int p = p0 + j * kSortThreads + tid;
        ev[j] = p < n ? idx[p] : -1;
      }
    }
#pragma unroll
    for (int j = 0; j < P; j++)
      if (ev[j] >= 0 && ev[j] < E) perm[atomicAdd(&cur[ev[j]], 1)] = p0 + j * kSortThreads + tid;
  }
}

// x[t] += scale * fp16(sum_j w_tj * y[t*k + j]) with the GEMV path's roundings, the slots in order
// (y in pair order, as the grouped down GEMM scatters it; a slot whose expert id lies outside
// [0, E) has no row and contributes nothing). One block per token, 8 columns per thread; a
// thread's k rows are requested together.
template <int KM>
__global__ void __launch_bounds__(128) moe_combine_kernel(const f16* __restrict__ y, const int* __restrict__ idx,
                                                          const float* __restrict__ wts, int k, int E, int H,
                                                          int flags, float scale, f16* x, int64_t ldx) {
  const int t = blockIdx.x;
  f16* xr = x + (int64_t)t * ldx;
  bool ok[KM];
  float wj[KM];
#pragma unroll
  for (int j = 0; j < KM; j++) {
    const int e = j < k ? idx[(int64_t)t * k + j] : -1;
    ok[j] = e >= 0 && e < E;
    wj[j] = j < k ? wts[(int64_t)t * k + j] : 0.f;
  }
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) {
    // every slot's row is requested at once, a skipped slot's too (its bytes lie inside y and are
    // never used), so the loads do not wait for the ids
    f16x8 v[KM];
#pragma unroll
    for (int j = 0; j < KM; j++)
      v[j] = j < k ? *reinterpret_cast<const f16x8*>(y + ((int64_t)t * k + j) * H + 8 * i) : f16x8{};
    f16x8 xv = *reinterpret_cast<const f16x8*>(xr + 8 * i);
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KM; j++) {
      if (!ok[j]) continue;  // uniform over the block
#pragma unroll
      for (int u = 0; u < 8; u++) {
        float c = (float)v[j][u] * wj[j];
        asm volatile("" : "+v"(c));  // the fp32 product is what gets rounded to fp16
        s[u] += (flags & kMoeFp16Weights) ? (float)(f16)c : c;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      f16 o = (f16)s[u];
      if (scale != 1.f) {
        float tt = (float)o * scale;
        asm volatile("" : "+v"(tt));  // fp32 product, then fp16 (two roundings)
        o = (f16)tt;
      }
      xv[u] = xv[u] + o;
    }
    *reinterpret_cast<f16x8*>(xr + 8 * i) = xv;
  }
}

// One grouped MFMA GEMM launch over the experts (gemm_kernel in grouped mode, tile kGrpBM x kGrpBN):
// sorted rows [off[e], off[e+1]) of expert e times W + e * wstride_bytes. gather: A row q is
// A row perm[q] / k (A has a_rows rows); scatter: C row q goes to C row perm[q].
template <int EPI>
int grouped_gemm(const f16* A, int lda, int a_rows, const f16* W, int64_t wstride_bytes, f16* C, int ldc, int N, int K,
                 const int* off, const int* tiles, const int* perm, int k, bool gather, bool scatter, int E,
                 int max_row_tiles, hipStream_t s) {
  GemmArgs g{};
  g.A = A;
  g.lda = lda;
  g.W = W;
  g.C = C;
  g.ldc = ldc;
  g.M = 1;
  g.N = N;
  g.K = K;
  g.kt_per_split = (K + kGrpBK - 1) / kGrpBK;
  g.vec_c = true;  // act / y live in the 256-byte aligned work buffer, ldc = I or H (multiples of 32)
  g.vec16_c = true;
  g.grp_off = off;
  g.grp_tiles = tiles;
  g.grp_n = E;
  g.grp_wstride = wstride_bytes;
  g.grp_perm = perm;
  g.grp_k = k;
  g.grp_a_rows = a_rows;
  g.grp_gather = gather;
  g.grp_scatter = scatter;
  auto fn = gemm_kernel<kGrpBM, kGrpBN, kGrpWM, kGrpWN, kGrpStages, EPI, false, true, kGrpBK>;
  const size_t lds = std::max((size_t)kGrpStages * (kGrpBM + kGrpBN) * kGrpBK * 2, gemm_stage_bytes(kGrpBM, kGrpBN));
  constexpr int threads = 64 * kGrpWM * kGrpWN;
  if (hi_blocks_per_cu(reinterpret_cast<const void*>(fn), threads, lds) <= 0) HI_FAIL("moe: grouped GEMM does not fit");
  const int tiles_n = (N + kGrpBN - 1) / kGrpBN;
  hipLaunchKernelGGL(fn, dim3(max_row_tiles * tiles_n), dim3(threads), lds, s, g);
  HI_TRY(hipGetLastError());
  return 0;
}

size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// The largest row count the GEMV path takes: HIPINFER_GEMV_MAX, shared with the decode step.
int gemv_max() { return hi_gemv_max_rows(); }

// The expert workspace (hi_moe_work_bytes), each piece on a 256-byte boundary. The first
// kMoeBarBytes (at a fixed offset, whatever M) hold the one-token launch's arrival counters and the
// grouped router's arrival counter; then perm [n], off and tiles [E+1] int, y [n, H] (pair order)
// and act [n, I] fp16 (sorted order on the grouped path, pair order on the GEMV path).
constexpr int kMoeBarStride = 64;                 // words between two arrival counters (256 bytes)
constexpr size_t kMoeBarBytes = 9 * 256;          // 8 counters, then the 8 expected totals
struct MoeWork {
  unsigned* bar;
  int *perm, *off, *tiles;
  f16 *y, *act;
};
MoeWork moe_work(void* work, int n, int E, int H) {
  char* p = (char*)work;
  MoeWork m;
  m.bar = (unsigned*)p; p += kMoeBarBytes;
  m.perm = (int*)p;   p += al256((size_t)n * 4);
  m.off = (int*)p;    p += al256((size_t)(E + 1) * 4);
  m.tiles = (int*)p;  p += al256((size_t)(E + 1) * 4);
  m.y = (f16*)p;      p += al256((size_t)n * H * 2);
  m.act = (f16*)p;
  return m;
}

// The grouped path after the sort (perm / off / tiles in wk): gate/up + SwiGLU on the rows of xn
// gathered by the tile DMA (act in sorted order), down scattered to pair order (y), the combine.
int moe_grouped(const f16* xn, int ldxn, const f16* Wgu, const f16* Wd, const int* idx, const float* w, int M, int E,
                int k, int H, int I, int flags, float scale, f16* x, int ldx, const MoeWork& wk, hipStream_t st) {
  const int n = M * k;
  // the tile DMA addresses xn's gathered rows, and act's and y's rows, at 32-bit byte offsets
  if ((int64_t)M * ldxn * 2 >= INT32_MAX || (int64_t)n * (H > I ? H : I) * 2 >= INT32_MAX)
    HI_FAIL("moe: %d rows too many for the grouped path's 32-bit offsets", M);
  const int max_row_tiles = (n + kGrpBM - 1) / kGrpBM + E;  // each expert adds at most one partial tile
  if (int r = grouped_gemm<2>(xn, ldxn, M, Wgu, (int64_t)2 * I * H * 2, wk.act, I, 2 * I, H, wk.off, wk.tiles, wk.perm,
                              k, true, false, E, max_row_tiles, st))
    return r;
  if (int r = grouped_gemm<0>(wk.act, I, n, Wd, (int64_t)H * I * 2, wk.y, H, H, I, wk.off, wk.tiles, wk.perm, 1, false,
                              true, E, max_row_tiles, st))
    return r;
  const auto comb = k <= 4 ? moe_combine_kernel<4> : k <= 8 ? moe_combine_kernel<8> : moe_combine_kernel<16>;
  hipLaunchKernelGGL(comb, dim3(M), dim3(128), 0, st, wk.y, idx, w, k, E, H, flags, scale, x, (int64_t)ldx);
  HI_TRY(hipGetLastError());
  return 0;
}

// The GEMV path's down projection + weighted combine + residual.
int moe_down_launch(const f16* act, const f16* Wd, const int* idx, const float* w, int M, int k, int E, int H, int I,
                    int flags, float scale, void* x, int ldx, hipStream_t st) {
  const int64_t dn_waves = (int64_t)M * H;
  const auto dn = k <= 4 ? moe_gemv_down_kernel<4> : k <= 8 ? moe_gemv_down_kernel<8> : moe_gemv_down_kernel<16>;
  hipLaunchKernelGGL(dn, dim3((unsigned)((dn_waves + kMoeWaves - 1) / kMoeWaves)), dim3(kMoeWaves * 64), 0, st, act,
                     Wd, idx, w, M, k, E, H, I, flags, scale, (f16*)x, (int64_t)ldx);
  HI_TRY(hipGetLastError());
  return 0;
}


// ------------------------------------------------------------------ one-launch decode (one token)
// Router, gate/up + SwiGLU, down projection, weighted combine and residual for ONE token in a single
// launch whose blocks are all resident at once (the host checks the occupancy). Phase 1 is
// moe_route_gu_kernel's work (same device functions, same bits). The activations go out with
// agent-coherent stores; a grid handoff (arrival counters, relaxed agent-scope atomics, no L2
// writeback fence) separates the phases. Once a block has arrived, the waves that own its
// down-projection columns issue their k expert rows' loads, so those weights stream while the grid
// waits. Phase 2 copies the token's activations into LDS once per block with agent-coherent 16-byte
// loads and runs moe_gemv_down_kernel's arithmetic, one wave per hidden column.
// The handoff counts arrivals on eight counters in the caller's work buffer (block b on counter
// b % 8, 256 bytes apart so they sit in different memory channels) that are never reset: the
// word after them, expect[x], holds what counter x reads once every launch so far has arrived, so
// a launch's target is that plus its own arrivals on x. Each block adds 1 (no returned value) once
// its activations are complete; one wave per block polls the eight counters (one load each per
// poll); block 0 then advances expect (every block has read it by then: a block reads it before it
// arrives). A zeroed region is consistent (0 == 0) and every launch leaves it consistent; calls that
// share a work buffer must not overlap in time (they share its activations too), calls with their
// own buffers are independent.
constexpr int kMoeOneMaxBlocks = 512;  // 16-wave blocks resident at once: at most 2 per CU, 256 CUs
constexpr int kMoeSpinMax = 1 << 18;  // polls before a block gives up waiting (never reached when resident)
constexpr int kMoeOneMaxAct = kMoeOneMaxBlocks * 16;  // k * I = 16 units per block
constexpr int kMoeRawBuffer = 0x00020000;  // buffer resource word 3: raw (untyped) 32-bit access
constexpr int kMoeSc1 = 16;                // buffer cache policy sc1: agent-coherent, as an agent-scope load

__device__ __forceinline__ uint32_t ld_coherent_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int CH, int KM, int RND>
__global__ void __launch_bounds__(kFusedWaves * 64) moe_decode_one_kernel(
    const f16* __restrict__ xn, const f16* __restrict__ Wr, const f16* __restrict__ wgu,
    const f16* __restrict__ wdown, int k, int E, int H, int I, int flags, float scale, int cols_per_block,
    int* __restrict__ idx_out, float* __restrict__ w_out, uint32_t* act2, f16* x, unsigned* bar, int* fail) {
  __shared__ float logit[kMoeMaxE];
  __shared__ float selv[kMoeMaxK];
  __shared__ int seli[kMoeMaxK];
  __shared__ f16 unit_out[kFusedWaves];
  __shared__ int ridx[kMoeMaxK];
  __shared__ float rw[kMoeMaxK];
  __shared__ u32x4 act_s[kMoeOneMaxAct / 8];  // the token's k * I activations, 8 halves a word
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nb = gridDim.x;
  constexpr int kPoller = kFusedWaves - 1;  // the wave that arrives and polls (a down wave only when
                                            // every wave is one)
  // lane x < 8 of the poller: counter x's target (needed only at the handoff, so the load's latency
  // is hidden)
  const unsigned target =
      (wave == kPoller && lane < 8) ? ld_coherent_u32(&bar[8 * kMoeBarStride + lane]) + (unsigned)((nb - lane + 7) / 8) : 0u;
  // this block's down-projection column (one per wave) and its residual, read early: no other block
  // writes it
  const int h = blockIdx.x * cols_per_block + wave;
  const bool down_wave = wave < cols_per_block && h < H;
  f16 xh = (f16)0.f;
  if (down_wave && lane == 0) xh = x[h];
  // ---- phase 1a: the routing (every block computes the token's own, as moe_route_gu_kernel)
  router_logits<CH>(xn, Wr, E, H, kFusedWaves, wave, lane, logit);
  __syncthreads();
  router_topk(logit, E, k, kFusedWaves, wave, lane, selv, seli);
  __syncthreads();
  // every block forms the weights itself (into LDS; block 0 also writes them out), so phase 2 never
  // reads another block's plain stores
  if (wave == 0) {
    router_weights(logit, selv, seli, E, k, flags, lane, 0, ridx, rw);
    if (blockIdx.x == 0) router_weights(logit, selv, seli, E, k, flags, lane, 0, idx_out, w_out);
  }
  // ---- phase 1b: gate/up + SwiGLU of this block's 16 units (pair p = slot j, units o0 .. o0 + 15)
  {
    const int64_t w0 = (int64_t)blockIdx.x * kFusedWaves;
    const int j = (int)(w0 / I);
    const int o = (int)(w0 - (int64_t)j * I) + wave;
    const int e = seli[j];
    const int r0 = (o >> 4) * 32 + (o & 15);
    const f16* g = wgu + ((int64_t)e * 2 * I + r0) * H;
    const f16* u = g + 16 * (int64_t)H;
    const int H8 = H / 8;
    float ag = 0.f, au = 0.f;
    for (int b = 0; b < H8; b += 64 * CH) {
      u32x4 xv[CH], gv[CH], uv[CH];
#pragma unroll
      for (int q = 0; q < CH; q++) {
        const int c = b + q * 64 + lane, cc = c < H8 ? c : 0;
        xv[q] = *reinterpret_cast<const u32x4*>(xn + 8 * cc);
        gv[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g + 8 * cc));
        uv[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(u + 8 * cc));
      }
#pragma unroll
      for (int q = 0; q < CH; q++) {
        const bool ok = b + q * 64 + lane < H8;
#pragma unroll
        for (int hh = 0; hh < 4; hh++) {
          const f16x2 x2 = as_h2(ok ? xv[q][hh] : 0u);
          ag = dot2(as_h2(gv[q][hh]), x2, ag);
          au = dot2(as_h2(uv[q][hh]), x2, au);
        }
      }
    }
    ag = wave_sum(ag);
    au = wave_sum(au);
    if (lane == 0) unit_out[wave] = silu_mul(ag, au);
    __syncthreads();
    // the block's 16 units leave as 8 agent-coherent words of fp16 pairs
    if (tid < kFusedWaves / 2) {
      const uint32_t pair = as_u32(f16x2{unit_out[2 * tid], unit_out[2 * tid + 1]});
      __hip_atomic_store(act2 + ((int64_t)j * I + (o - wave)) / 2 + tid, pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // ---- grid handoff: the activation words are complete before this block arrives
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  if (wave == kPoller && lane == 0)
    __hip_atomic_fetch_add(&bar[(blockIdx.x & 7) * kMoeBarStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the down waves' weight rows (all k experts of the block's columns) stream during the handoff
  const int I8 = I / 8;  // I <= 64 * 8 * RND (the host's choice of RND)
  u32x4 wv[KM][RND];
#pragma unroll
  for (int j = 0; j < KM; j++)
#pragma unroll
    for (int rr = 0; rr < RND; rr++) wv[j][rr] = u32x4{0u, 0u, 0u, 0u};
  if (down_wave) {
#pragma unroll
    for (int j = 0; j < KM; j++) {
      if (j < k) {
        const int e = seli[j];
#pragma unroll
        for (int rr = 0; rr < RND; rr++) {
          const int c = rr * 64 + lane;
          if (c < I8)
            wv[j][rr] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wdown + ((int64_t)e * H + h) * I + 8 * c));
        }
      }
    }
  }
  // every block waits for every arrival (all blocks are resident, so every wait ends; the poll
  // count is bounded all the same). A block whose polls run out goes on, so the grid still drains,
  // and raises the host-visible fail word: its output is wrong, and the host reports it on the next
  // MoE call or engine step and stops using this path.
  if (wave == kPoller) {
    // one poll in flight: a second one (checked while the next is out) measured slower, the
    // counters' memory channel serving the polls and the arrivals alike
    bool arrived = false;
    for (int it = 0; it < kMoeSpinMax; it++) {
      const bool ok = lane >= 8 || (int)(ld_coherent_u32(&bar[lane * kMoeBarStride]) - target) >= 0;
      if (__all(ok)) {
        arrived = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!arrived && lane == 0) __hip_atomic_store(fail, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (blockIdx.x == 0 && lane < 8) __hip_atomic_store(&bar[8 * kMoeBarStride + lane], target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // ---- phase 2: the activations into LDS once per block (agent-coherent 16-byte loads), then the
  //      down projection + weighted combine (slot order) + residual, one wave per column
  {
    const int n16 = k * I / 8;
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(act2, (short)0, n16 * 16, kMoeRawBuffer);
    for (int i = tid; i < n16; i += kFusedWaves * 64) act_s[i] = __builtin_amdgcn_raw_buffer_load_b128(ar, i * 16, 0, kMoeSc1);
  }
  __syncthreads();
  if (down_wave) {
    float acc[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) acc[j] = 0.f;
#pragma unroll
    for (int rr = 0; rr < RND; rr++) {
      const int c = rr * 64 + lane;
      if (rr * 64 < I8) {  // uniform over the wave
#pragma unroll
        for (int j = 0; j < KM; j++) {
          if (j < k) {
            const u32x4 av = c < I8 ? act_s[j * I8 + c] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int q = 0; q < 4; q++) acc[j] = dot2(as_h2(wv[j][rr][q]), as_h2(av[q]), acc[j]);
          }
        }
      }
    }
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < KM; j++) {
      if (j < k) {
        float c = (float)(f16)wave_sum(acc[j]) * rw[j];
        asm volatile("" : "+v"(c));  // the fp32 product is what gets rounded to fp16
        sum += (flags & kMoeFp16Weights) ? (float)(f16)c : c;
      }
    }
    if (lane == 0) {
      f16 o = (f16)sum;
      if (scale != 1.f) {
        float t = (float)o * scale;
        asm volatile("" : "+v"(t));  // fp32 product, then fp16 (two roundings)
        o = (f16)t;
      }
      x[h] = xh + o;
    }
  }
}

// The one-launch kernel's fail word: one pinned host int (mapped for the GPU, so a kernel's
// system-scope store reaches the host without a copy), allocated on the first one-launch call made
// outside stream capture. Raised by a block whose handoff wait ran out of polls; taken (read and
// cleared) by moe_one_launch_failed, which also turns the one-launch path off for the process.
std::mutex g_moe_fail_mu;
int* g_moe_fail = nullptr;
std::atomic<bool> g_moe_one_off{false};

int* moe_fail_word(hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_moe_fail_mu);
  if (!g_moe_fail) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
    void* p = nullptr;
    if (hipHostMalloc(&p, sizeof(int), hipHostMallocDefault) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    __atomic_store_n((int*)p, 0, __ATOMIC_RELEASE);
    g_moe_fail = (int*)p;
  }
  return g_moe_fail;
}

// Launches moe_decode_one_kernel for one token when its grid can be resident all at once: k * I / 16
// blocks of 16 waves (each 16 gate/up units, then up to 16 down columns). Returns 0 after the
// launch, 1 when the shape or the occupancy does not allow it (the caller takes the two launches),
// or a negative error code.
template <int CH, int KM, int RND>
int moe_decode_one_go(const void* xn, const void* Wr, const void* wgu, const void* wdown, int E, int k, int H, int I,
                      int flags, float scale, void* x, int* idx, float* w, void* act, unsigned* bar, int nb, int cpb,
                      hipStream_t st) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  auto fn = moe_decode_one_kernel<CH, KM, RND>;
  const int bpc = hi_blocks_per_cu(reinterpret_cast<const void*>(fn), kFusedWaves * 64, 0);
  if (bpc < 0) return -2;
  if ((long)bpc * d->cus < nb) return 1;  // not resident at once: the handoff could not be waited for
  int* fail = moe_fail_word(st);
  if (!fail) return 1;  // no fail word (a capture before the first eager call): the two launches
  hipLaunchKernelGGL(fn, dim3(nb), dim3(kFusedWaves * 64), 0, st, (const f16*)xn, (const f16*)Wr, (const f16*)wgu,
                     (const f16*)wdown, k, E, H, I, flags, scale, cpb, idx, w, (uint32_t*)act, (f16*)x, bar, fail);
  HI_TRY(hipGetLastError());
  return 0;
}

template <int CH, int RND>
int moe_decode_one_k(const void* xn, const void* Wr, const void* wgu, const void* wdown, int E, int k, int H, int I,
                     int flags, float scale, void* x, int* idx, float* w, void* act, unsigned* bar, int nb, int cpb,
                     hipStream_t st) {
  if (k <= 4)
    return moe_decode_one_go<CH, 4, RND>(xn, Wr, wgu, wdown, E, k, H, I, flags, scale, x, idx, w, act, bar, nb, cpb, st);
  if (k <= 8 && RND <= 2)
    return moe_decode_one_go<CH, 8, RND <= 2 ? RND : 2>(xn, Wr, wgu, wdown, E, k, H, I, flags, scale, x, idx, w, act, bar,
                                                        nb, cpb, st);
  if (RND == 1)
    return moe_decode_one_go<CH, 16, 1>(xn, Wr, wgu, wdown, E, k, H, I, flags, scale, x, idx, w, act, bar, nb, cpb, st);
  return 1;  // k * (I / 512) above 16 rounds of expert rows per lane: more registers than this kernel holds
}

// HIPINFER_MOE_ONE_LAUNCH=0 turns the one-launch path off (read once): its handoff needs every block
// resident at once, which other kernels running concurrently on the GPU could prevent.
bool moe_one_launch_enabled() {
  static const bool on = [] {
    const char* e = getenv("HIPINFER_MOE_ONE_LAUNCH");
    return !e || atoi(e) != 0;
  }();
  return on && !g_moe_one_off.load();
}

int moe_decode_one(const void* xn, const void* Wr, const void* wgu, const void* wdown, int E, int k, int H, int I,
                   int flags, float scale, void* x, int* idx, float* w, void* act, unsigned* bar, hipStream_t st) {
  if (!moe_one_launch_enabled()) return 1;
  if ((int64_t)k * I % kFusedWaves || I > 2048) return 1;
  const int nb = k * I / kFusedWaves;
  if (nb > kMoeOneMaxBlocks) return 1;
  const int cpb = (H + nb - 1) / nb;
  if (cpb > kFusedWaves) return 1;
  const int rnd = I <= 512 ? 1 : I <= 1024 ? 2 : 4;
  const int ch = chunks_for(H);
#define HI_MOE_ONE(C, R)   \
  if (ch == C && rnd == R) \
    return moe_decode_one_k<C, R>(xn, Wr, wgu, wdown, E, k, H, I, flags, scale, x, idx, w, act, bar, nb, cpb, st);
  HI_MOE_ONE(1, 1) HI_MOE_ONE(1, 2) HI_MOE_ONE(1, 4) HI_MOE_ONE(2, 1) HI_MOE_ONE(2, 2) HI_MOE_ONE(2, 4)
  HI_MOE_ONE(4, 1) HI_MOE_ONE(4, 2) HI_MOE_ONE(4, 4)
#undef HI_MOE_ONE
  return 1;
}

}  // namespace

bool moe_one_launch_failed() {
  std::lock_guard<std::mutex> lk(g_moe_fail_mu);
  if (!g_moe_fail || __atomic_load_n(g_moe_fail, __ATOMIC_ACQUIRE) == 0) return false;
  __atomic_store_n(g_moe_fail, 0, __ATOMIC_RELEASE);
  g_moe_one_off.store(true);
  fprintf(stderr,
          "hipinfer_amd: a one-launch MoE call gave up waiting for its grid (its blocks were not all resident "
          "at once): that call's output is wrong; the one-launch path is off for the rest of this process\n");
  return true;
}

// Router + top-k for M normalised rows xn: idx[M, k] (int) and weights w[M, k] (fp32), descending.
HI_EXPORT int hi_moe_router(const void* xn, int ldx, const void* Wr, int M, int E, int H, int k, int flags, int* idx,
                            float* w, void* s) {
  if (E < 1 || E > kMoeMaxE || k < 1 || k > kMoeMaxK || k > E || H < 8 || H % 8)
    HI_FAIL("hi_moe_router: unsupported E %d / k %d / H %d (E <= %d, k <= %d, H %% 8 == 0)", E, k, H, kMoeMaxE,
            kMoeMaxK);
  if (M < 0) HI_FAIL("hi_moe_router: M %d < 0", M);
  if (M == 0) return 0;
  if (!xn || !Wr || !idx || !w || ((uintptr_t)xn & 15) || ((uintptr_t)Wr & 15) || ldx % 8)
    HI_FAIL("hi_moe_router: xn and Wr must be 16-byte aligned device pointers (ldx %% 8 == 0)");
  const auto kern = chunks_for(H) == 1 ? moe_router_kernel<1> : chunks_for(H) == 2 ? moe_router_kernel<2>
                                                                                     : moe_router_kernel<4>;
  hipLaunchKernelGGL(kern, dim3(M), dim3(kRouterWaves * 64), 0, (hipStream_t)s, (const f16*)xn, (int64_t)ldx,
                     (const f16*)Wr, E, H, k, flags, idx, w);
  HI_TRY(hipGetLastError());
  return 0;
}

// Expert workspace, each piece on a 256-byte boundary: arrival counters (2304 bytes, first,
// whatever M), perm [M*k] int, off, tiles [E+1] int, y [M*k, H] and act [M*k, I] fp16. The GEMV
// path uses only act.
HI_EXPORT size_t hi_moe_work_bytes(int M, int k, int E, int H, int I) {
  const size_t n = (size_t)(M > 0 ? M : 0) * (k > 0 ? k : 0);
  return kMoeBarBytes + al256(n * 4) + 2 * al256((size_t)(E + 1) * 4) + al256(n * H * 2) + al256(n * I * 2);
}

// x[m] += MoE(xn[m]) for M rows given the routing (idx, w from hi_moe_router): wgu [E][2I, H]
// (gate/up interleaved per expert), wdown [E][H, I]. path 0 takes the GEMV path for
// M <= HIPINFER_GEMV_MAX (default 8), else the grouped path; 1 / 2 force GEMV / grouped.
HI_EXPORT int hi_moe_experts(const void* xn, int ldxn, const void* wgu, const void* wdown, const int* idx, const float* w,
                             int M, int E, int k, int H, int I, int flags, float scale, void* x, int ldx, int path,
                             void* work, void* s) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  if (H % 32 || I % 32 || H < 32 || I < 32) HI_FAIL("hi_moe_experts: H %d and I %d must be multiples of 32", H, I);
  if (E < 1 || E > kMoeMaxE || k < 1 || k > kMoeMaxK) HI_FAIL("hi_moe_experts: unsupported E %d / k %d", E, k);
  if (path < 0 || path > 2) HI_FAIL("hi_moe_experts: path must be 0, 1 or 2 (got %d)", path);
  if (M < 0) HI_FAIL("hi_moe_experts: M %d < 0", M);
  if (M == 0) return 0;
  if (!xn || !wgu || !wdown || !idx || !w || !x || !work) HI_FAIL("hi_moe_experts: null pointer");
  if (((uintptr_t)xn & 15) || ((uintptr_t)wgu & 15) || ((uintptr_t)wdown & 15) || ((uintptr_t)x & 15) ||
      ((uintptr_t)work & 255) || ldxn % 8 || ldx % 8)
    HI_FAIL("hi_moe_experts: tensors must be 16-byte aligned (work 256-byte), ldxn and ldx multiples of 8");
  const hipStream_t st = (hipStream_t)s;
  const int n = M * k;
  const MoeWork wk = moe_work(work, n, E, H);
  const f16* Wgu = (const f16*)wgu;
  const f16* Wd = (const f16*)wdown;
  if (path == 1 || (path == 0 && M <= gemv_max())) {
    const int64_t gu_waves = (int64_t)n * I;
    const auto gu = chunks_for(H) == 1 ? moe_gemv_gu_kernel<1> : chunks_for(H) == 2 ? moe_gemv_gu_kernel<2>
                                                                                    : moe_gemv_gu_kernel<4>;
    hipLaunchKernelGGL(gu, dim3((unsigned)((gu_waves + kMoeWaves - 1) / kMoeWaves)), dim3(kMoeWaves * 64),
                       0, st, (const f16*)xn, (int64_t)ldxn, Wgu, idx, n, k, E, H, I, wk.act);
    HI_TRY(hipGetLastError());
    return moe_down_launch(wk.act, Wd, idx, w, M, k, E, H, I, flags, scale, x, ldx, st);
  }
  hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(kSortThreads), 0, st, idx, n, E, wk.off, wk.tiles, wk.perm);
  HI_TRY(hipGetLastError());
  return moe_grouped((const f16*)xn, ldxn, Wgu, Wd, idx, w, M, E, k, H, I, flags, scale, (f16*)x, ldx, wk, st);
}

// Router and experts in one call: x[m] += MoE(xn[m]) for M rows, with the routing computed here and
// written to idx / w as hi_moe_router writes it. The same bits as hi_moe_router followed by
// hi_moe_experts with path 0. One row runs as one launch (moe_decode_one_kernel) when its grid fits
// on the GPU at once; otherwise, on the GEMV path (M <= HIPINFER_GEMV_MAX), the router runs inside
// the gate/up launch (moe_route_gu_kernel), which saves a launch and a dependent memory round trip
// per layer; larger M run the router and the grouped experts as two calls. The work buffer must be
// zeroed once before its first use here (its arrival counters; every call leaves them consistent).
// No counterpart in the reference, whose engine makes the two calls (api.cu:1701-1703); this
// build's engine uses this.
HI_EXPORT int hi_moe_route_experts(const void* xn, int ldxn, const void* Wr, const void* wgu, const void* wdown, int M,
                                   int E, int k, int H, int I, int flags, float scale, void* x, int ldx, int* idx,
                                   float* w, void* work, void* s) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  if (M < 0) HI_FAIL("hi_moe_route_experts: M %d < 0", M);
  if (M == 0) return 0;
  if (E < 1 || E > kMoeMaxE || k < 1 || k > kMoeMaxK || k > E)
    HI_FAIL("hi_moe_route_experts: unsupported E %d / k %d (E <= %d, k <= %d, k <= E)", E, k, kMoeMaxE, kMoeMaxK);
  if (H % 32 || I % 32 || H < 32 || I < 32) HI_FAIL("hi_moe_route_experts: H %d and I %d must be multiples of 32", H, I);
  if (!xn || !Wr || !wgu || !wdown || !idx || !w || !x || !work) HI_FAIL("hi_moe_route_experts: null pointer");
  if (((uintptr_t)xn & 15) || ((uintptr_t)Wr & 15) || ((uintptr_t)wgu & 15) || ((uintptr_t)wdown & 15) ||
      ((uintptr_t)x & 15) || ((uintptr_t)work & 255) || ldxn % 8 || ldx % 8)
    HI_FAIL("hi_moe_route_experts: tensors must be 16-byte aligned (work 256-byte), ldxn and ldx multiples of 8");
  if (moe_one_launch_failed()) return -2;  // an earlier call's output was wrong: report it, launch nothing
  const hipStream_t st = (hipStream_t)s;
  const int n = M * k;
  const MoeWork wk = moe_work(work, n, E, H);
  if (M > gemv_max()) {  // the router, then the grouped experts (sort, two GEMMs, combine)
    if (int r = hi_moe_router(xn, ldxn, Wr, M, E, H, k, flags, idx, w, s)) return r;
    hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(kSortThreads), 0, st, idx, n, E, wk.off, wk.tiles, wk.perm);
    HI_TRY(hipGetLastError());
    return moe_grouped((const f16*)xn, ldxn, (const f16*)wgu, (const f16*)wdown, idx, w, M, E, k, H, I, flags, scale,
                       (f16*)x, ldx, wk, st);
  }
  if (M == 1) {
    const int r = moe_decode_one(xn, Wr, wgu, wdown, E, k, H, I, flags, scale, x, idx, w, wk.act, wk.bar, st);
    if (r <= 0) return r;  // launched (0) or failed (< 0); 1: this shape takes the two launches
  }
  const int64_t gu_waves = (int64_t)n * I;
  const auto gu = chunks_for(H) == 1 ? moe_route_gu_kernel<1> : chunks_for(H) == 2 ? moe_route_gu_kernel<2>
                                                                                  : moe_route_gu_kernel<4>;
  hipLaunchKernelGGL(gu, dim3((unsigned)(gu_waves / kFusedWaves)), dim3(kFusedWaves * 64), 0, st, (const f16*)xn,
                     (int64_t)ldxn, (const f16*)Wr, (const f16*)wgu, n, k, E, H, I, flags, idx, w, wk.act);
  HI_TRY(hipGetLastError());
  return moe_down_launch(wk.act, (const f16*)wdown, idx, w, M, k, E, H, I, flags, scale, x, ldx, st);
}
