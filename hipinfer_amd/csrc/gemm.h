// Prefill GEMM for gfx950: C[M, N'] (epi) A[M, K] @ W[N, K]^T with fp16 MFMA and fp32 accumulation.
//
// Replaces the reference's portable WMMA gemm_kernel<BM, BN, BK, WGM, WGN, EPI, Q8>
// (src/kernels.cuh:305-506) behind the same C-ABI (hi_gemm, hi_gemm_w8; api.cu:566-577).
//
// Design:
//  * a block of 4 waves owns a BM x BN output tile; each wave a (BM/WM) x (BN/WN) sub-tile built
//    from v_mfma_f32_32x32x16_f16 tiles (A and W are both K-contiguous, so each lane's 8-half
//    fragment is one 16-byte LDS read);
//  * K advances in 64-deep tiles, double-buffered in LDS: the next tile's global loads are in
//    flight (in registers) while the MFMAs consume the current one; one barrier per K tile;
//  * LDS rows hold 8 chunks of 16 bytes whose position is XOR-swizzled by the row (chunk ^ row % 8),
//    so the 32 rows an MFMA fragment read touches spread over the banks;
//  * int8 weights are dequantised on their way into LDS: exact int8 -> fp16 unpack, then one
//    packed fp16 multiply by the row scale = fp16(q * s), the weight the reference's int8 GEMM
//    computes with (kernels.cuh:86-94, 336-341);
//  * the tile index is remapped so that the 8 XCDs (blocks are dealt round-robin across them)
//    each get a contiguous run of tiles, rasterised in groups of 8 tile rows, so the A and W
//    panels a run needs stay in that XCD's L2;
//  * epilogues (reference kernels.cuh:454-505): 0 store (+ bias, fp32 before the rounding),
//    1 residual (fp16 add), 2 SwiGLU over 16-column gate/up groups (the partner column sits 16
//    lanes away in the MFMA result and is fetched with one lane swizzle);
//  * split-K: gridDim.y blocks share a tile; each writes its fp32 partial to a workspace, and the
//    last to arrive (device-scope counter, reset for the next launch or graph replay) sums the
//    partials in split order -- deterministic whatever the arrival order -- and runs the epilogue.
#pragma once
#include "hi_common.h"

struct GemmArgs {
  const f16* A;
  int64_t lda;
  const void* W;       // [N, K] fp16 or int8
  const f16* scales;   // int8 row scales [N] or nullptr
  const f16* bias;     // [N] (epilogue 0) or nullptr
  f16* C;
  int64_t ldc;
  int M, N, K;
  int kt_per_split;    // K tiles per split (gridDim.y splits)
  float* ws;           // split-K partials: [splits][tiles][BM * BN] fp32
  int* counters;       // [tiles] arrival counters, zero between launches
};

constexpr int kGemmBK = 64;
constexpr int kGemmThreads = 256;

// element (r, k) of an LDS tile with kGemmBK halves per row, 16-byte chunks XOR-swizzled by row
__device__ __forceinline__ int lds_off(int r, int chunk) { return r * kGemmBK + ((chunk ^ (r & 7)) << 3); }

template <int BM, int BN, int WM, int WN, int EPI, bool Q8>
__global__ void __launch_bounds__(kGemmThreads) gemm_kernel(GemmArgs g) {
  constexpr int TM = BM / WM, TN = BN / WN;       // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;       // MFMA tiles per wave
  constexpr int CH = kGemmBK / 8;                 // 16-byte chunks per LDS row
  constexpr int A_PT = BM * CH / kGemmThreads;    // A chunks per thread per K tile
  constexpr int B_PT = Q8 ? BN * (kGemmBK / 16) / kGemmThreads : BN * CH / kGemmThreads;
  static_assert(WM * WN == 4 && FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tiling");
  static_assert(A_PT >= 1 && B_PT >= 1, "tile too small for the block");
  extern __shared__ f16 smem[];
  f16* As = smem;                     // [2][BM][BK]
  f16* Bs = smem + 2 * BM * kGemmBK;  // [2][BN][BK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int M = g.M, N = g.N, K = g.K;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, ntiles = tiles_m * tiles_n;

  // tile index: blocks are dealt round-robin over the 8 XCDs; give each XCD a contiguous run of
  // tile ids (the part of the grid that divides by 8; the remainder keeps its id)
  int pid = blockIdx.x;
  {
    const int per = ntiles / 8;
    if (pid < per * 8) pid = (pid % 8) * per + pid / 8;
  }
  int tm, tn;
  {
    constexpr int GM = 8;
    const int per_group = GM * tiles_n, first = (pid / per_group) * GM;
    const int gsize = min(tiles_m - first, GM), r = pid % per_group;
    tm = first + r % gsize;
    tn = r / gsize;
  }
  const int bm = tm * BM, bn = tn * BN;

  const int nkt = (K + kGemmBK - 1) / kGemmBK;
  const int kt0 = blockIdx.y * g.kt_per_split;
  const int kt1 = min(nkt, kt0 + g.kt_per_split);

  // ---- global -> register staging
  u32x4 ra[A_PT];
  u32x4 rb[B_PT];
  f16 bscale[B_PT];
  const char* Wb = reinterpret_cast<const char*>(g.W);
#pragma unroll
  for (int i = 0; i < B_PT; i++) {
    bscale[i] = (f16)0.f;
    if constexpr (Q8) {
      const int c = tid + i * kGemmThreads, r = c / (kGemmBK / 16);
      if (bn + r < N) bscale[i] = g.scales[bn + r];
    }
  }
  auto gload = [&](int kt) {
    const int k0 = kt * kGemmBK;
#pragma unroll
    for (int i = 0; i < A_PT; i++) {
      const int c = tid + i * kGemmThreads, r = c / CH, kc = (c % CH) * 8;
      const int row = bm + r, k = k0 + kc;
      ra[i] = (row < M && k < K) ? *reinterpret_cast<const u32x4*>(g.A + row * g.lda + k) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < B_PT; i++) {
      if constexpr (Q8) {  // 16 int8 weights per load
        const int c = tid + i * kGemmThreads, r = c / (kGemmBK / 16), kc = (c % (kGemmBK / 16)) * 16;
        const int row = bn + r, k = k0 + kc;
        rb[i] = (row < N && k < K) ? *reinterpret_cast<const u32x4*>(Wb + (int64_t)row * K + k) : u32x4{0u, 0u, 0u, 0u};
      } else {
        const int c = tid + i * kGemmThreads, r = c / CH, kc = (c % CH) * 8;
        const int row = bn + r, k = k0 + kc;
        rb[i] = (row < N && k < K) ? *reinterpret_cast<const u32x4*>(Wb + ((int64_t)row * K + k) * 2)
                                   : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto sstore = [&](int st) {
    f16* as = As + st * BM * kGemmBK;
    f16* bs = Bs + st * BN * kGemmBK;
#pragma unroll
    for (int i = 0; i < A_PT; i++) {
      const int c = tid + i * kGemmThreads, r = c / CH, ch = c % CH;
      *reinterpret_cast<u32x4*>(as + lds_off(r, ch)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PT; i++) {
      if constexpr (Q8) {
        const int c = tid + i * kGemmThreads, r = c / (kGemmBK / 16), ch = (c % (kGemmBK / 16)) * 2;
        const f16x2 s2 = {bscale[i], bscale[i]};
        u32x4 lo, hi;
#pragma unroll
        for (int p = 0; p < 4; p++) {
          f16x2 a, b;
          i8x4_to_f16(rb[i][p], a, b);
          a = a * s2;  // fp16(q * s), one rounding
          b = b * s2;
          if (p < 2) {
            lo[2 * p] = as_u32(a);
            lo[2 * p + 1] = as_u32(b);
          } else {
            hi[2 * p - 4] = as_u32(a);
            hi[2 * p - 3] = as_u32(b);
          }
        }
        *reinterpret_cast<u32x4*>(bs + lds_off(r, ch)) = lo;
        *reinterpret_cast<u32x4*>(bs + lds_off(r, ch + 1)) = hi;
      } else {
        const int c = tid + i * kGemmThreads, r = c / CH, ch = c % CH;
        *reinterpret_cast<u32x4*>(bs + lds_off(r, ch)) = rb[i];
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  if (kt0 < kt1) {
    gload(kt0);
    sstore(0);
  }
  __syncthreads();
  const int fr = lane & 31, fk = lane >> 5;  // fragment row (or column) and k half
  for (int kt = kt0; kt < kt1; kt++) {
    const int st = (kt - kt0) & 1;
    if (kt + 1 < kt1) gload(kt + 1);
    const f16* as = As + st * BM * kGemmBK;
    const f16* bs = Bs + st * BN * kGemmBK;
#pragma unroll
    for (int ks = 0; ks < kGemmBK / 16; ks++) {
      const int ch = ks * 2 + fk;
      f16x8 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const f16x8*>(as + lds_off(wm * TM + i * 32 + fr, ch));
#pragma unroll
      for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const f16x8*>(bs + lds_off(wn * TN + j * 32 + fr, ch));
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < kt1) sstore(st ^ 1);
    __syncthreads();
  }

  // ---- split-K: partial to the workspace; the last block of the tile reduces in split order
  const int splits = gridDim.y;
  const int tile = tm * tiles_n + tn;
  if (splits > 1) {
    float* part = g.ws + ((int64_t)blockIdx.y * ntiles + tile) * (BM * BN);
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int r = wm * TM + i * 32 + 8 * (e >> 2) + 4 * fk + (e & 3), c = wn * TN + j * 32 + fr;
          part[r * BN + c] = acc[i][j][e];
        }
    __threadfence();
    __syncthreads();
    __shared__ int last;
    if (tid == 0) {
      const int prev = atomicAdd(&g.counters[tile], 1);
      last = prev == splits - 1;
      if (last) g.counters[tile] = 0;  // ready for the next launch / graph replay
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int r = wm * TM + i * 32 + 8 * (e >> 2) + 4 * fk + (e & 3), c = wn * TN + j * 32 + fr;
          float t = 0.f;
          for (int z = 0; z < splits; z++)
            t += __builtin_nontemporal_load(g.ws + ((int64_t)z * ntiles + tile) * (BM * BN) + r * BN + c);
          acc[i][j][e] = t;
        }
  }

  // ---- epilogue straight from the MFMA result layout: lane (fk, fr) of tile (i, j) holds rows
  //      8*(e/4) + 4*fk + e%4 of column fr
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int col = bn + wn * TN + j * 32 + fr;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int row = bm + wm * TM + i * 32 + 8 * (e >> 2) + 4 * fk + (e & 3);
        const float v = acc[i][j][e];
        if constexpr (EPI == 2) {
          const float up = __shfl_xor(v, 16, kWave);  // column fr + 16 of the same 32-column group
          if (fr < 16 && row < M && col < N) {
            const int oc = ((bn + wn * TN + j * 32) >> 1) + fr;
            g.C[row * g.ldc + oc] = silu_mul(v, up);
          }
        } else if (row < M && col < N) {
          f16* dst = g.C + row * g.ldc + col;
          if constexpr (EPI == 1) *dst = *dst + (f16)v;
          else *dst = (f16)(g.bias ? v + (float)g.bias[col] : v);
        }
      }
    }
}

// Tile configurations (all 4 waves, BK = 64): {BM, BN, WM, WN}.
struct GemmCfg {
  int bm, bn, wm, wn;
};
constexpr GemmCfg kGemmCfgs[] = {{256, 128, 2, 2}, {128, 128, 2, 2}, {128, 64, 2, 2},
                                 {64, 128, 2, 2},  {64, 64, 2, 2},   {32, 128, 1, 4}};
constexpr int kGemmNumCfgs = sizeof(kGemmCfgs) / sizeof(kGemmCfgs[0]);
inline size_t gemm_lds_bytes(int cfg) { return (size_t)2 * (kGemmCfgs[cfg].bm + kGemmCfgs[cfg].bn) * kGemmBK * 2; }

template <int BM, int BN, int WM, int WN, int EPI, bool Q8>
int gemm_launch(const GemmArgs& g, int splits, hipStream_t s) {
  const size_t lds = (size_t)2 * (BM + BN) * kGemmBK * 2;
  const void* fn = reinterpret_cast<const void*>(&gemm_kernel<BM, BN, WM, WN, EPI, Q8>);
  const int bpc = hi_blocks_per_cu(fn, kGemmThreads, lds);  // also lifts the dynamic-LDS limit
  if (bpc < 0) return -2;
  if (bpc == 0) HI_FAIL("gemm: tile %dx%d does not fit on a CU", BM, BN);
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, EPI, Q8>), dim3(tiles, splits), dim3(kGemmThreads), lds, s, g);
  HI_TRY(hipGetLastError());
  return 0;
}

template <int EPI>
int gemm_run(const GemmArgs& g, int cfg, int splits, bool q8, hipStream_t s);
// Resident blocks per CU of a config's kernel (occupancy API). Kernels are only ever named in
// their own instance file: naming one elsewhere would instantiate (and register) a second copy.
template <int EPI>
int gemm_blocks_per_cu(int cfg, bool q8);

#define HI_GEMM_CFG(i, q)                                                                              \
  if (cfg == i && q8 == q)                                                                             \
    return gemm_launch<kGemmCfgs[i].bm, kGemmCfgs[i].bn, kGemmCfgs[i].wm, kGemmCfgs[i].wn, EPI, q>(g, splits, s);
#define HI_GEMM_DEFINE_RUN(EPIV)                                                                       \
  template <>                                                                                          \
  int gemm_run<EPIV>(const GemmArgs& g, int cfg, int splits, bool q8, hipStream_t s) {                \
    constexpr int EPI = EPIV;                                                                          \
    HI_GEMM_CFG(0, false) HI_GEMM_CFG(1, false) HI_GEMM_CFG(2, false) HI_GEMM_CFG(3, false)            \
    HI_GEMM_CFG(4, false) HI_GEMM_CFG(5, false)                                                        \
    HI_GEMM_CFG(0, true) HI_GEMM_CFG(1, true) HI_GEMM_CFG(2, true) HI_GEMM_CFG(3, true)                \
    HI_GEMM_CFG(4, true) HI_GEMM_CFG(5, true)                                                          \
    HI_FAIL("gemm: no kernel for config %d", cfg);                                                     \
  }                                                                                                    \
  template <>                                                                                          \
  int gemm_blocks_per_cu<EPIV>(int cfg, bool q8) {                                                     \
    constexpr int EPI = EPIV;                                                                          \
    HI_GEMM_OCC(0) HI_GEMM_OCC(1) HI_GEMM_OCC(2) HI_GEMM_OCC(3) HI_GEMM_OCC(4) HI_GEMM_OCC(5)            \
    return -1;                                                                                         \
  }
#define HI_GEMM_OCC(i)                                                                                 \
  if (cfg == i) {                                                                                      \
    const void* fn = q8 ? reinterpret_cast<const void*>(&gemm_kernel<kGemmCfgs[i].bm, kGemmCfgs[i].bn,  \
                                                                      kGemmCfgs[i].wm, kGemmCfgs[i].wn, EPI, true>) \
                        : reinterpret_cast<const void*>(&gemm_kernel<kGemmCfgs[i].bm, kGemmCfgs[i].bn,  \
                                                                      kGemmCfgs[i].wm, kGemmCfgs[i].wn, EPI, false>); \
    return hi_blocks_per_cu(fn, kGemmThreads, gemm_lds_bytes(i));                                      \
  }
