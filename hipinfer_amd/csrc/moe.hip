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
//    weighted combine in slot order. Fixed launch shape, the expert choice stays on the device.
//  * grouped (prefill): a counting sort of the M*k (token, slot) pairs by expert, which also
//    writes each expert's row-tile prefix; a gather; two grouped MFMA GEMM launches (gate/up with
//    the SwiGLU epilogue, then down) in which every block finds its expert from the prefix; and
//    the combine. Unlike the reference (which copies the per-expert counts to the host and
//    launches one GEMM per expert, api.cu:901-909) nothing returns to the host, so the grouped
//    path is graph-capturable too.
// Expert ids outside [0, E) are never dereferenced: such a slot contributes nothing.
#include <cstdlib>

#include "gemm.h"

namespace {

constexpr int kMoeMaxE = 256, kMoeMaxK = 16;
constexpr int kMoeNormTopk = 1, kMoeFp16Weights = 2;
constexpr int kGrpBM = 64, kGrpBN = 128;  // grouped GEMM tile (gemm config kGemmGrpCfg)

// v beats (best, bi): NaN above numbers; equal values (and NaN vs NaN) go to the lower index
// (reference argmax_better, kernels.cuh:1886-1890).
__device__ __forceinline__ bool argmax_better(float v, int i, float best, int bi) {
  const bool vn = v != v, bn = best != best;
  if (vn != bn) return vn;
  return (vn || v == best) ? i < bi : v > best;
}

// ------------------------------------------------------------------ router
__global__ void __launch_bounds__(256) moe_router_kernel(const f16* __restrict__ xn, int64_t ldx,
                                                         const f16* __restrict__ Wr, int E, int H, int k, int flags,
                                                         int* __restrict__ idx_out, float* __restrict__ w_out) {
  __shared__ float logit[kMoeMaxE];
  __shared__ float selv[kMoeMaxK];
  __shared__ int seli[kMoeMaxK];
  const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const f16* xr = xn + t * ldx;
  for (int e = wave; e < E; e += 4) {
    const f16* wr = Wr + (int64_t)e * H;
    float acc = 0.f;
    for (int c = lane; c < H / 8; c += 64) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(xr + 8 * c), b = *reinterpret_cast<const u32x4*>(wr + 8 * c);
#pragma unroll
      for (int p = 0; p < 4; p++) acc = dot2(as_h2(a[p]), as_h2(b[p]), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) logit[e] = (float)(f16)acc;  // the router linear is rounded to fp16
  }
  __syncthreads();
  if (wave != 0) return;
  float v[kMoeMaxE / 64];
#pragma unroll
  for (int i = 0; i < kMoeMaxE / 64; i++) {
    const int e = i * 64 + lane;
    v[i] = e < E ? logit[e] : -__builtin_huge_valf();
  }
  unsigned taken = 0;  // bit i: this lane's expert i * 64 + lane is selected
  for (int j = 0; j < k; j++) {
    float best = -__builtin_huge_valf();
    int bi = 0x7fffffff;  // above every expert index: any untaken expert beats it
#pragma unroll
    for (int i = 0; i < kMoeMaxE / 64; i++) {
      const int e = i * 64 + lane;
      if (e < E && !((taken >> i) & 1u) && argmax_better(v[i], e, best, bi)) {
        best = v[i];
        bi = e;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(best, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (argmax_better(ov, oi, best, bi)) {
        best = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);  // every lane holds the winner; its owner marks it
    if (lane == 0) {
      seli[j] = bi;
      selv[j] = best;
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const float mx = selv[0];
  float denom = 0.f;
  if (flags & kMoeNormTopk) {
    for (int j = 0; j < k; j++) denom += expf(selv[j] - mx);
  } else {
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < kMoeMaxE / 64; i++)
      if (i * 64 + lane < E) sum += expf(v[i] - mx);
    denom = wave_sum(sum);
  }
  if (lane < k) {
    float wj = expf(selv[lane] - mx) / denom;
    if (flags & kMoeFp16Weights) wj = (float)(f16)wj;
    idx_out[(int64_t)t * k + lane] = seli[lane];
    w_out[(int64_t)t * k + lane] = wj;
  }
}

// ------------------------------------------------------------------ GEMV expert path
// Gate/up + SwiGLU: block (x, pair p) covers 16 units; wave w takes units 4w..4w+3 of them. Unit o
// of expert e reads rows (o/16)*32 + o%16 and that + 16 of wgu[e] [2I, H].
constexpr int kGuUnitsPerWave = 4;
__global__ void __launch_bounds__(256) moe_gemv_gu_kernel(const f16* __restrict__ xn, int64_t ldx,
                                                          const f16* __restrict__ wgu, const int* __restrict__ idx,
                                                          int k, int E, int H, int I, f16* __restrict__ act) {
  const int p = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = idx[p];
  const int o0 = (blockIdx.x * 4 + wave) * kGuUnitsPerWave;
  if (e < 0 || e >= E) {  // no expert: this slot's activation is zero
    if (lane < kGuUnitsPerWave && o0 + lane < I) act[(int64_t)p * I + o0 + lane] = (f16)0.f;
    return;
  }
  const f16* W = wgu + (int64_t)e * 2 * I * H;
  const f16* xr = xn + (int64_t)(p / k) * ldx;
  float acc[kGuUnitsPerWave][2];
  const f16* rows[kGuUnitsPerWave][2];
#pragma unroll
  for (int u = 0; u < kGuUnitsPerWave; u++) {
    const int o = min(o0 + u, I - 1);
    const int r0 = (o >> 4) * 32 + (o & 15);
    rows[u][0] = W + (int64_t)r0 * H;
    rows[u][1] = W + (int64_t)(r0 + 16) * H;
    acc[u][0] = acc[u][1] = 0.f;
  }
  for (int c = lane; c < H / 8; c += 64) {
    const u32x4 xv = *reinterpret_cast<const u32x4*>(xr + 8 * c);
    u32x4 wv[kGuUnitsPerWave][2];
#pragma unroll
    for (int u = 0; u < kGuUnitsPerWave; u++)
#pragma unroll
      for (int r = 0; r < 2; r++) wv[u][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rows[u][r] + 8 * c));
#pragma unroll
    for (int u = 0; u < kGuUnitsPerWave; u++)
#pragma unroll
      for (int r = 0; r < 2; r++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[u][r] = dot2(as_h2(wv[u][r][q]), as_h2(xv[q]), acc[u][r]);
  }
#pragma unroll
  for (int u = 0; u < kGuUnitsPerWave; u++) {
    const float g = wave_sum(acc[u][0]), up = wave_sum(acc[u][1]);
    if (lane == 0 && o0 + u < I) act[(int64_t)p * I + o0 + u] = silu_mul(g, up);
  }
}

// Down projection + weighted combine + residual: wave (token b, column h) computes the k dot
// products wdown[e_j][h] . act[b*k + j] four at a time and adds them up in slot order.
constexpr int kDownColsPerWave = 2;
__global__ void __launch_bounds__(256) moe_gemv_down_kernel(const f16* __restrict__ act, const f16* __restrict__ wdown,
                                                            const int* __restrict__ idx, const float* __restrict__ wts,
                                                            int k, int E, int H, int I, int flags, float scale, f16* x,
                                                            int64_t ldx) {
  const int b = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h0 = (blockIdx.x * 4 + wave) * kDownColsPerWave;
  float sum[kDownColsPerWave];
#pragma unroll
  for (int u = 0; u < kDownColsPerWave; u++) sum[u] = 0.f;
  for (int j0 = 0; j0 < k; j0 += 4) {
    float acc[4][kDownColsPerWave];
    int ex[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      ex[r] = j0 + r < k ? idx[(int64_t)b * k + j0 + r] : -1;
#pragma unroll
      for (int u = 0; u < kDownColsPerWave; u++) acc[r][u] = 0.f;
    }
    for (int c = lane; c < I / 8; c += 64) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        if (ex[r] < 0 || ex[r] >= E) continue;
        const u32x4 av = *reinterpret_cast<const u32x4*>(act + ((int64_t)b * k + j0 + r) * I + 8 * c);
#pragma unroll
        for (int u = 0; u < kDownColsPerWave; u++) {
          const int h = min(h0 + u, H - 1);
          const u32x4 wv = __builtin_nontemporal_load(
              reinterpret_cast<const u32x4*>(wdown + ((int64_t)ex[r] * H + h) * I + 8 * c));
#pragma unroll
          for (int q = 0; q < 4; q++) acc[r][u] = dot2(as_h2(wv[q]), as_h2(av[q]), acc[r][u]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      if (ex[r] < 0 || ex[r] >= E) continue;  // uniform over the wave
      const float wr = wts[(int64_t)b * k + j0 + r];
#pragma unroll
      for (int u = 0; u < kDownColsPerWave; u++) {
        const float c = (float)(f16)wave_sum(acc[r][u]) * wr;
        sum[u] += (flags & kMoeFp16Weights) ? (float)(f16)c : c;
      }
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int u = 0; u < kDownColsPerWave; u++) {
      const int h = h0 + u;
      if (h >= H) continue;
      f16 o = (f16)sum[u];
      if (scale != 1.f) o = (f16)((float)o * scale);
      f16* dst = x + (int64_t)b * ldx + h;
      *dst = *dst + o;
    }
  }
}

// ------------------------------------------------------------------ grouped path
// Counting sort of the n (token, slot) pairs by expert (one block): off[E+1] exclusive prefix of
// the counts, tiles[E+1] prefix of each expert's row tiles of kGrpBM, perm[q] = pair at sorted
// position q, inv[pair] = q (-1 for an expert id outside [0, E)). The order within an expert
// follows the LDS atomics; every GEMM row is computed on its own, so it changes no result.
__global__ void __launch_bounds__(1024) moe_sort_kernel(const int* __restrict__ idx, int n, int E, int* __restrict__ off,
                                                        int* __restrict__ tiles, int* __restrict__ perm,
                                                        int* __restrict__ inv) {
  __shared__ int cnt[kMoeMaxE], cur[kMoeMaxE];
  for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int p = threadIdx.x; p < n; p += blockDim.x) {
    const int e = idx[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int s = 0, ts = 0;
    for (int e = 0; e < E; e++) {
      off[e] = s;
      cur[e] = s;
      tiles[e] = ts;
      s += cnt[e];
      ts += (cnt[e] + kGrpBM - 1) / kGrpBM;
    }
    off[E] = s;
    tiles[E] = ts;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < n; p += blockDim.x) {
    const int e = idx[p];
    if (e >= 0 && e < E) {
      const int q = atomicAdd(&cur[e], 1);
      perm[q] = p;
      inv[p] = q;
    } else {
      inv[p] = -1;
    }
  }
}

// rows[q] = xn[perm[q] / k] for the sorted pairs (16-byte copies); one block per possible row,
// blocks past the valid count exit.
__global__ void __launch_bounds__(128) moe_gather_kernel(const f16* __restrict__ xn, int64_t ldx, const int* __restrict__ perm,
                                                         const int* __restrict__ off, int E, int k, int H,
                                                         f16* __restrict__ rows) {
  const int q = blockIdx.x;
  if (q >= off[E]) return;
  const u32x4* src = reinterpret_cast<const u32x4*>(xn + (int64_t)(perm[q] / k) * ldx);
  u32x4* dst = reinterpret_cast<u32x4*>(rows + (int64_t)q * H);
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) dst[i] = src[i];
}

// x[t] += scale * fp16(sum_j w_tj * y[inv[t*k + j]]) with the GEMV path's roundings; one block
// per token, 8 columns per thread.
__global__ void __launch_bounds__(128) moe_combine_kernel(const f16* __restrict__ y, const int* __restrict__ inv,
                                                          const float* __restrict__ wts, int k, int H, int flags,
                                                          float scale, f16* x, int64_t ldx) {
  const int t = blockIdx.x;
  f16* xr = x + (int64_t)t * ldx;
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) {
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < k; j++) {
      const int q = inv[(int64_t)t * k + j];
      if (q < 0) continue;
      const float w = wts[(int64_t)t * k + j];
      const f16x8 v = *reinterpret_cast<const f16x8*>(y + (int64_t)q * H + 8 * i);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const float c = (float)v[u] * w;
        s[u] += (flags & kMoeFp16Weights) ? (float)(f16)c : c;
      }
    }
    f16x8 xv = *reinterpret_cast<const f16x8*>(xr + 8 * i);
#pragma unroll
    for (int u = 0; u < 8; u++) {
      f16 o = (f16)s[u];
      if (scale != 1.f) o = (f16)((float)o * scale);
      xv[u] = xv[u] + o;
    }
    *reinterpret_cast<f16x8*>(xr + 8 * i) = xv;
  }
}

template <int EPI>
int grouped_gemm(const f16* A, int lda, const f16* W, int64_t wstride_bytes, f16* C, int ldc, int N, int K,
                 const int* off, const int* tiles, int E, int max_row_tiles, hipStream_t s) {
  constexpr int cfg = kGemmGrpCfg;
  static_assert(kGemmCfgs[cfg].bm == kGrpBM && kGemmCfgs[cfg].bn == kGrpBN, "grouped tile");
  GemmArgs g{};
  g.A = A;
  g.lda = lda;
  g.W = W;
  g.C = C;
  g.ldc = ldc;
  g.M = 1;
  g.N = N;
  g.K = K;
  g.kt_per_split = (K + kGemmBK - 1) / kGemmBK;
  g.vec_c = true;  // act / y live in the 256-byte aligned work buffer, ldc = I or H (multiples of 32)
  g.grp_off = off;
  g.grp_tiles = tiles;
  g.grp_n = E;
  g.grp_wstride = wstride_bytes;
  auto fn = gemm_kernel<kGrpBM, kGrpBN, kGemmCfgs[cfg].wm, kGemmCfgs[cfg].wn, kGemmCfgs[cfg].st, EPI, false, true>;
  const size_t lds = gemm_lds_bytes(cfg, false);
  constexpr int threads = 64 * kGemmCfgs[cfg].wm * kGemmCfgs[cfg].wn;
  if (hi_blocks_per_cu(reinterpret_cast<const void*>(fn), threads, lds) <= 0) HI_FAIL("moe: grouped GEMM does not fit");
  const int tiles_n = (N + kGrpBN - 1) / kGrpBN;
  hipLaunchKernelGGL(fn, dim3(max_row_tiles * tiles_n), dim3(threads), lds, s, g);
  HI_TRY(hipGetLastError());
  return 0;
}

size_t al256(size_t b) { return (b + 255) / 256 * 256; }

// HIPINFER_GEMV_MAX (default 4, at most 8): the largest row count the GEMV path takes
// (reference api.cu:1884-1887).
int gemv_max() {
  static const int v = getenv("HIPINFER_GEMV_MAX") ? atoi(getenv("HIPINFER_GEMV_MAX")) : 4;
  return v < 8 ? v : 8;
}

}  // namespace

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
  hipLaunchKernelGGL(moe_router_kernel, dim3(M), dim3(256), 0, (hipStream_t)s, (const f16*)xn, (int64_t)ldx,
                     (const f16*)Wr, E, H, k, flags, idx, w);
  HI_TRY(hipGetLastError());
  return 0;
}

// Expert workspace, each piece on a 256-byte boundary: perm, inv [M*k] int, off, tiles [E+1] int,
// rows [M*k, H], y [M*k, H] and act [M*k, I] fp16. The GEMV path uses only act.
HI_EXPORT size_t hi_moe_work_bytes(int M, int k, int E, int H, int I) {
  const size_t n = (size_t)(M > 0 ? M : 0) * (k > 0 ? k : 0);
  return 2 * al256(n * 4) + 2 * al256((size_t)(E + 1) * 4) + 2 * al256(n * H * 2) + al256(n * I * 2);
}

// x[m] += MoE(xn[m]) for M rows given the routing (idx, w from hi_moe_router): wgu [E][2I, H]
// (gate/up interleaved per expert), wdown [E][H, I]. path 0 takes the GEMV path for
// M <= HIPINFER_GEMV_MAX (default 4), else the grouped path; 1 / 2 force GEMV / grouped.
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
  char* p = (char*)work;
  int* perm = (int*)p;   p += al256((size_t)n * 4);
  int* inv = (int*)p;    p += al256((size_t)n * 4);
  int* off = (int*)p;    p += al256((size_t)(E + 1) * 4);
  int* tiles = (int*)p;  p += al256((size_t)(E + 1) * 4);
  f16* rows = (f16*)p;   p += al256((size_t)n * H * 2);
  f16* y = (f16*)p;      p += al256((size_t)n * H * 2);
  f16* act = (f16*)p;
  const f16* Wgu = (const f16*)wgu;
  const f16* Wd = (const f16*)wdown;
  if (path == 1 || (path == 0 && M <= gemv_max())) {
    hipLaunchKernelGGL(moe_gemv_gu_kernel, dim3((I + 4 * kGuUnitsPerWave - 1) / (4 * kGuUnitsPerWave), n), dim3(256), 0,
                       st, (const f16*)xn, (int64_t)ldxn, Wgu, idx, k, E, H, I, act);
    HI_TRY(hipGetLastError());
    hipLaunchKernelGGL(moe_gemv_down_kernel, dim3((H + 4 * kDownColsPerWave - 1) / (4 * kDownColsPerWave), M), dim3(256),
                       0, st, act, Wd, idx, w, k, E, H, I, flags, scale, (f16*)x, (int64_t)ldx);
    HI_TRY(hipGetLastError());
    return 0;
  }
  hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(1024), 0, st, idx, n, E, off, tiles, perm, inv);
  HI_TRY(hipGetLastError());
  hipLaunchKernelGGL(moe_gather_kernel, dim3(n), dim3(128), 0, st, (const f16*)xn, (int64_t)ldxn, perm, off, E, k, H, rows);
  HI_TRY(hipGetLastError());
  const int max_row_tiles = (n + kGrpBM - 1) / kGrpBM + E;  // each expert adds at most one partial tile
  if (int r = grouped_gemm<2>(rows, H, Wgu, (int64_t)2 * I * H * 2, act, I, 2 * I, H, off, tiles, E, max_row_tiles, st))
    return r;
  if (int r = grouped_gemm<0>(act, I, Wd, (int64_t)H * I * 2, y, H, H, I, off, tiles, E, max_row_tiles, st)) return r;
  hipLaunchKernelGGL(moe_combine_kernel, dim3(M), dim3(128), 0, st, y, inv, w, k, H, flags, scale, (f16*)x, (int64_t)ldx);
  HI_TRY(hipGetLastError());
  return 0;
}
