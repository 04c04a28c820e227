// Prefill GEMM for gfx950: C[M, N'] (epi) A[M, K] @ W[N, K]^T with fp16 MFMA and fp32 accumulation.
//
// Replaces the reference's portable WMMA gemm_kernel<BM, BN, BK, WGM, WGN, EPI, Q8>
// (src/kernels.cuh:305-506) behind the same C-ABI (hi_gemm, hi_gemm_w8; api.cu:566-577).
//
// Design:
//  * a block of 4 waves owns a BM x BN output tile; each wave a (BM/WM) x (BN/WN) sub-tile built
//    from v_mfma_f32_32x32x16_f16 tiles (A and W are both K-contiguous, so each lane's 8-half
//    fragment is one 16-byte LDS read);
//  * K advances in 64-deep tiles through an S-stage ring in LDS fed by gfx950's direct
//    global->LDS loads (global_load_lds_dwordx4): no register staging, S-1 tiles in flight while
//    the MFMAs consume the oldest, one explicit vmcnt wait and one barrier per K tile;
//  * LDS rows hold 16-byte chunks whose position is XOR-swizzled by the row, so the 32 rows one
//    fragment read touches spread over the banks; the swizzle is applied on the global side (each
//    lane fetches the chunk that belongs at its LDS slot), since a DMA lane's LDS slot is fixed;
//  * int8 weights travel to LDS raw (half the bytes) and are dequantised per fragment: exact
//    int8 -> fp16 unpack, then one packed fp16 multiply by the row scale = fp16(q * s), the weight
//    the reference's int8 GEMM computes with (kernels.cuh:86-94, 336-341);
//  * rows past M or N load a clamped (valid) row whose results are never stored; a K tail of 32
//    skips the last two 16-deep MFMA steps;
//  * the tile index is remapped so each of the 8 XCDs (blocks are dealt round-robin across them)
//    gets a contiguous run of tiles, rasterised in groups of 8 tile rows, so the A and W panels a
//    run needs stay in that XCD's L2;
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
  // grouped mode (MoE experts): group e owns A/C rows [grp_off[e], grp_off[e+1]) and the weights
  // at W + e * grp_wstride bytes; its row tiles are [grp_tiles[e], grp_tiles[e+1]) of the global
  // row-tile count (block id / column tiles)
  const int* grp_off;
  const int* grp_tiles;
  int grp_n;
  int64_t grp_wstride;
};

constexpr int kGemmBK = 64;
constexpr int kGemmThreads = 256;
typedef __attribute__((address_space(3))) void lds_void_t;

// Wait until at most N vector-memory operations (global loads, LDS DMA) are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Workgroup barrier without a memory fence (a fence would drain every in-flight LDS DMA); the
// DMA completions it orders are waited for explicitly with wait_vmcnt.
__device__ __forceinline__ void barrier_no_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Half offset of 16-byte chunk `c` of row `r` in an LDS tile of 64-half (128-byte) rows.
__device__ __forceinline__ int lds_off(int r, int c) { return r * kGemmBK + ((c ^ (r & 7)) << 3); }
// Byte offset of 16-byte chunk `c` of row `r` in an LDS tile of 64-byte int8 rows.
__device__ __forceinline__ int lds_off8(int r, int c) { return r * 64 + ((c ^ (r & 3)) << 4); }

template <int BM, int BN, int WM, int WN, int S, int EPI, bool Q8, bool GRP = false>
__global__ void __launch_bounds__(kGemmThreads) gemm_kernel(GemmArgs g) {
  constexpr int TM = BM / WM, TN = BN / WN;          // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;          // MFMA tiles per wave
  constexpr int A_ST = BM * kGemmBK;                 // halves per stage
  constexpr int B_ROWB = Q8 ? 64 : 128;              // bytes of one W row per K tile
  constexpr int B_ST = BN * B_ROWB / 2;              // halves per stage
  constexpr int A_LD = BM / 32;                      // 1 KB DMA instructions per wave per K tile (A)
  constexpr int B_LD = BN * B_ROWB / 4096;           // ... (W)
  constexpr int L = A_LD + B_LD;                     // vector-memory ops per lane per K tile
  static_assert(WM * WN == 4 && FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tiling");
  static_assert(A_LD >= 1 && B_LD >= 1 && (S - 2) * L < 64 && S >= 2 && S <= 4, "pipeline shape");
  static_assert(!(GRP && Q8), "grouped (expert) GEMMs take fp16 weights");
  extern __shared__ f16 smem[];
  f16* As = smem;               // [S][BM][64]
  f16* Bs = smem + S * A_ST;    // [S][BN][64] fp16, or [S][BN][64 bytes] int8

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int N = g.N, K = g.K;
  int M = g.M;
  const f16* Ap = g.A;
  f16* Cp = g.C;
  const char* Wb = reinterpret_cast<const char*>(g.W);
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn, ntiles;
  if constexpr (GRP) {
    // find this block's group: grp_tiles[e] <= row tile < grp_tiles[e + 1]; blocks past the last
    // row tile (the grid is sized for the worst case) exit
    const int mt = blockIdx.x / tiles_n;
    tn = blockIdx.x - mt * tiles_n;
    if (mt >= g.grp_tiles[g.grp_n]) return;
    int lo = 0, hi = g.grp_n;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (g.grp_tiles[mid] <= mt) lo = mid;
      else hi = mid;
    }
    const int r0 = g.grp_off[lo];
    M = g.grp_off[lo + 1] - r0;
    Ap += r0 * g.lda;
    Cp += r0 * g.ldc;
    Wb += lo * g.grp_wstride;
    tm = mt - g.grp_tiles[lo];
    ntiles = 0;
  } else {
    const int tiles_m = (M + BM - 1) / BM;
    ntiles = tiles_m * tiles_n;
    // tile index: blocks are dealt round-robin over the 8 XCDs; give each XCD a contiguous run of
    // tile ids (the part of the grid that divides by 8; the remainder keeps its id)
    int pid = blockIdx.x;
    const int per = ntiles / 8;
    if (pid < per * 8) pid = (pid % 8) * per + pid / 8;
    constexpr int GM = 8;
    const int per_group = GM * tiles_n, first = (pid / per_group) * GM;
    const int gsize = min(tiles_m - first, GM), r = pid % per_group;
    tm = first + r % gsize;
    tn = r / gsize;
  }
  const int bm = tm * BM, bn = tn * BN;

  const int nkt = (K + kGemmBK - 1) / kGemmBK;
  const int kt0 = blockIdx.y * g.kt_per_split;
  const int nloc = min(nkt, kt0 + g.kt_per_split) - kt0;  // K tiles of this split

  // ---- DMA of one K tile into stage st. Lane l of an instruction covering 8 (A, W fp16) or
  //      16 (W int8) rows fills LDS slot l: it fetches the chunk the swizzle puts there.
  auto issue = [&](int kt, int st) {
    const int k0 = kt * kGemmBK;
    f16* as = As + st * A_ST;
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      const int r0 = (wave * A_LD + i) * 8, r = r0 + (lane >> 3), lc = (lane & 7) ^ (lane >> 3);
      const int row = min(bm + r, M - 1);
      const int k = k0 + lc * 8 < K ? k0 + lc * 8 : k0;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(Ap + row * g.lda + k),
                                       (lds_void_t*)(as + r0 * kGemmBK), 16, 0, 0);
    }
    f16* bs = Bs + st * B_ST;
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      if constexpr (Q8) {
        const int r0 = (wave * B_LD + i) * 16, r = r0 + (lane >> 2), lc = (lane & 3) ^ (r & 3);
        const int row = min(bn + r, N - 1);
        const int k = k0 + lc * 16 < K ? k0 + lc * 16 : k0;
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(Wb + (int64_t)row * K + k),
                                         (lds_void_t*)(reinterpret_cast<char*>(bs) + r0 * 64), 16, 0, 0);
      } else {
        const int r0 = (wave * B_LD + i) * 8, r = r0 + (lane >> 3), lc = (lane & 7) ^ (lane >> 3);
        const int row = min(bn + r, N - 1);
        const int k = k0 + lc * 8 < K ? k0 + lc * 8 : k0;
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(Wb + ((int64_t)row * K + k) * 2),
                                         (lds_void_t*)(bs + r0 * kGemmBK), 16, 0, 0);
      }
    }
  };

  const int fr = lane & 31, fk = lane >> 5;  // fragment row (or column) and k half
  f16x2 bsc[FN];                             // int8: the scale of the W row each B fragment reads
#pragma unroll
  for (int j = 0; j < FN; j++) {
    bsc[j] = f16x2{(f16)0.f, (f16)0.f};
    if constexpr (Q8) {
      const f16 sv = g.scales[min(bn + wn * TN + j * 32 + fr, N - 1)];
      bsc[j] = f16x2{sv, sv};
    }
  }

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

#pragma unroll
  for (int s = 0; s < S - 1; s++)
    if (s < nloc) issue(kt0 + s, s);

  for (int t = 0; t < nloc; t++) {
    // tile t has landed once at most `later` tiles' DMA remain outstanding
    const int later = min(S - 2, nloc - 1 - t);
    if (later >= 2) wait_vmcnt<2 * L>();
    else if (later == 1) wait_vmcnt<L>();
    else wait_vmcnt<0>();
    barrier_no_fence();  // every lane's part of tile t is in LDS; every wave is done with tile t-1
    if (t + S - 1 < nloc) issue(kt0 + t + S - 1, (t + S - 1) % S);

    const int st = t % S, k0 = (kt0 + t) * kGemmBK;
    const f16* as = As + st * A_ST;
    const f16* bs = Bs + st * B_ST;
#pragma unroll
    for (int ks = 0; ks < kGemmBK / 16; ks++) {
      if (k0 + ks * 16 < K) {
        const int ch = ks * 2 + fk;
        f16x8 af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const f16x8*>(as + lds_off(wm * TM + i * 32 + fr, ch));
#pragma unroll
        for (int j = 0; j < FN; j++) {
          if constexpr (Q8) {
            const int r = wn * TN + j * 32 + fr;
            const u32x2 q = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(bs) + lds_off8(r, ks) + 8 * fk);
            f16x2 p0, p1, p2, p3;
            i8x4_to_f16(q[0], p0, p1);
            i8x4_to_f16(q[1], p2, p3);
            p0 = p0 * bsc[j];  // fp16(q * s), one rounding each
            p1 = p1 * bsc[j];
            p2 = p2 * bsc[j];
            p3 = p3 * bsc[j];
            bf[j] = f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
          } else {
            bf[j] = *reinterpret_cast<const f16x8*>(bs + lds_off(wn * TN + j * 32 + fr, ch));
          }
        }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      }
    }
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
            Cp[row * g.ldc + oc] = silu_mul(v, up);
          }
        } else if (row < M && col < N) {
          f16* dst = Cp + row * g.ldc + col;
          if constexpr (EPI == 1) *dst = *dst + (f16)v;
          else *dst = (f16)(g.bias ? v + (float)g.bias[col] : v);
        }
      }
    }
}

// Tile configurations (all 4 waves, BK = 64): {BM, BN, WM, WN, stages}.
struct GemmCfg {
  int bm, bn, wm, wn, st;
};
constexpr GemmCfg kGemmCfgs[] = {{256, 128, 2, 2, 3}, {128, 128, 2, 2, 4}, {128, 64, 2, 2, 4}, {64, 128, 2, 2, 4},
                                 {64, 64, 2, 2, 4},   {32, 128, 1, 4, 4},  {256, 256, 2, 2, 2}};
constexpr int kGemmNumCfgs = sizeof(kGemmCfgs) / sizeof(kGemmCfgs[0]);
inline size_t gemm_lds_bytes(int cfg, bool q8) {
  const GemmCfg& c = kGemmCfgs[cfg];
  return (size_t)c.st * (c.bm * kGemmBK * 2 + c.bn * (q8 ? 64 : 128));
}

template <int BM, int BN, int WM, int WN, int S, int EPI, bool Q8>
int gemm_launch(const GemmArgs& g, int cfg, int splits, hipStream_t s) {
  const size_t lds = gemm_lds_bytes(cfg, Q8);
  const void* fn = reinterpret_cast<const void*>(&gemm_kernel<BM, BN, WM, WN, S, EPI, Q8>);
  const int bpc = hi_blocks_per_cu(fn, kGemmThreads, lds);  // also lifts the dynamic-LDS limit
  if (bpc < 0) return -2;
  if (bpc == 0) HI_FAIL("gemm: tile %dx%d does not fit on a CU", BM, BN);
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, S, EPI, Q8>), dim3(tiles, splits), dim3(kGemmThreads), lds, s, g);
  HI_TRY(hipGetLastError());
  return 0;
}

template <int EPI>
int gemm_run(const GemmArgs& g, int cfg, int splits, bool q8, hipStream_t s);
// Resident blocks per CU of a config's kernel (occupancy API). Kernels are only ever named in
// their own instance file: naming one elsewhere would instantiate (and register) a second copy.
template <int EPI>
int gemm_blocks_per_cu(int cfg, bool q8);

#define HI_GEMM_K(i, q) gemm_kernel<kGemmCfgs[i].bm, kGemmCfgs[i].bn, kGemmCfgs[i].wm, kGemmCfgs[i].wn, kGemmCfgs[i].st, EPI, q>
#define HI_GEMM_CFG(i, q)                                                                                      \
  if (cfg == i && q8 == q)                                                                                     \
    return gemm_launch<kGemmCfgs[i].bm, kGemmCfgs[i].bn, kGemmCfgs[i].wm, kGemmCfgs[i].wn, kGemmCfgs[i].st, EPI, q>( \
        g, cfg, splits, s);
#define HI_GEMM_OCC(i)                                                                                         \
  if (cfg == i)                                                                                                \
    return hi_blocks_per_cu(q8 ? reinterpret_cast<const void*>(&HI_GEMM_K(i, true))                            \
                               : reinterpret_cast<const void*>(&HI_GEMM_K(i, false)),                          \
                            kGemmThreads, gemm_lds_bytes(i, q8));
#define HI_GEMM_DEFINE_RUN(EPIV)                                                                               \
  template <>                                                                                                  \
  int gemm_run<EPIV>(const GemmArgs& g, int cfg, int splits, bool q8, hipStream_t s) {                        \
    constexpr int EPI = EPIV;                                                                                  \
    HI_GEMM_CFG(0, false) HI_GEMM_CFG(1, false) HI_GEMM_CFG(2, false) HI_GEMM_CFG(3, false)                    \
    HI_GEMM_CFG(4, false) HI_GEMM_CFG(5, false) HI_GEMM_CFG(6, false)                                          \
    HI_GEMM_CFG(0, true) HI_GEMM_CFG(1, true) HI_GEMM_CFG(2, true) HI_GEMM_CFG(3, true)                        \
    HI_GEMM_CFG(4, true) HI_GEMM_CFG(5, true) HI_GEMM_CFG(6, true)                                             \
    HI_FAIL("gemm: no kernel for config %d", cfg);                                                             \
  }                                                                                                            \
  template <>                                                                                                  \
  int gemm_blocks_per_cu<EPIV>(int cfg, bool q8) {                                                             \
    constexpr int EPI = EPIV;                                                                                  \
    HI_GEMM_OCC(0) HI_GEMM_OCC(1) HI_GEMM_OCC(2) HI_GEMM_OCC(3) HI_GEMM_OCC(4) HI_GEMM_OCC(5) HI_GEMM_OCC(6)    \
    return -1;                                                                                                 \
  }
