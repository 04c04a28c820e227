// Prefill GEMM for gfx950: C[M, N'] (epi) A[M, K] @ W[N, K]^T with fp16 MFMA and fp32 accumulation.
//
// Replaces the reference's portable WMMA gemm_kernel<BM, BN, BK, WGM, WGN, EPI, Q8>
// (src/kernels.cuh:305-506) behind the same C-ABI (hi_gemm, hi_gemm_w8; api.cu:566-577).
//
// Design:
//  * a block of WM x WN waves (4 or 8) owns a BM x BN output tile; each wave a (BM/WM) x (BN/WN)
//    sub-tile built from v_mfma_f32_32x32x16_f16 tiles (A and W are both K-contiguous, so each
//    lane's 8-half fragment is one 16-byte LDS read). The big tiles give each wave a 128 x 128 (or
//    128 x 64) sub-tile, so every 16-byte fragment read feeds four (or two) MFMAs; with 8 waves two
//    share each SIMD, so one wave's MFMAs cover the other's LDS waits, barrier and DMA issue;
//  * K advances in 64-deep tiles through an S-stage ring in LDS fed by gfx950's direct
//    global->LDS loads (global_load_lds_dwordx4): no register staging, the next S-1 tiles in flight
//    while the MFMAs consume the current one;
//  * within a tile the fragments of step s+1 are read from LDS while the MFMAs of step s run (the
//    order is pinned with scheduling-group barriers: MFMA, LDS read, MFMA, ...); the one barrier
//    per tile sits in the last step, after its fragments are in registers, and is followed at once
//    by the DMA that refills the stage just freed and by the first fragment reads of the next tile.
//    The refill is unconditional (past the split's last tile it re-reads the first), so the loop
//    body has no branch and its DMA waits are compile-time counts;
//  * LDS rows hold 16-byte chunks at positions XOR-swizzled by the row (c ^ ((r >> 1) & 7) for
//    128-byte rows, c ^ ((r >> 2) & 3) for 64-byte int8 rows): the 16 lanes one 128-bit read serves
//    per cycle then cover all 64 banks. The swizzle is applied on the global side (each DMA lane
//    fetches the chunk that belongs at its fixed LDS slot);
//  * the k order inside each 32-deep half tile is permuted identically for A and W: step 2j + h
//    gives lane (row, half fk) the k values 32j + 16 fk + 8 h + 0..7. An int8 lane then reads its
//    two steps' 16 weights as one 16-byte chunk (a conflict-free 128-bit read) and dequantises
//    them per fragment: exact int8 -> fp16 unpack, one packed fp16 multiply by the row scale =
//    fp16(q * s), the weight the reference's int8 GEMM computes with (kernels.cuh:86-94, 336-341);
//  * the DMA goes through buffer resources based at the block's first rows, so each lane keeps
//    32-bit offsets only and rows past M or N read zeros (never stored); a K tail of 32
//    (K % 64 == 32) is the last tile's first half only, handled outside the main loop;
//  * the tile index is remapped so each of the 8 XCDs (blocks are dealt round-robin across them)
//    gets a contiguous run of tiles, rasterised in groups of 8 tile rows, so the A and W panels a
//    run needs stay in that XCD's L2;
//  * the W fragment is the MFMA's first operand, so each lane ends with 16 results of ONE output
//    row, four consecutive columns per register quad: the epilogue stores 8 bytes at a time, and
//    a gate column and its up column (16 apart) sit in the same lane -- no cross-lane traffic;
//  * epilogues (reference kernels.cuh:454-505): 0 store (+ bias, fp32 before the rounding),
//    1 residual (fp16 add), 2 SwiGLU over 16-column gate/up groups;
//  * split-K: gridDim.y blocks share a tile and write fp32 partials [split][M][N]; a second kernel
//    sums them in split order (deterministic) and runs the epilogue. The kernel boundary makes the
//    partials visible across XCDs; an in-kernel "last block reduces" handoff would need an
//    agent-scope fence, which writes back and invalidates the XCD's L2 on this part.
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
  float* ws;           // split-K partials: [splits][M][N] fp32
  bool vec_c;          // C (and the residual read) allow 8-byte accesses: C 8-byte aligned, ldc % 4 == 0
  bool vec16_c;        // ... and 16-byte ones (C 16-byte aligned, ldc % 8 == 0): the LDS-staged epilogue
  // grouped mode (MoE experts): group e owns sorted rows [grp_off[e], grp_off[e+1]) and the
  // weights at W + e * grp_wstride bytes; its row tiles are [grp_tiles[e], grp_tiles[e+1]) of the
  // global row-tile count (block id / column tiles). Sorted row q is A row q and C row q, unless
  // grp_perm is given: then with grp_gather A row q is A row grp_perm[q] / grp_k (A has
  // grp_a_rows rows; rows are gathered by the tile DMA itself), and with grp_scatter C row q is
  // C row grp_perm[q]
  const int* grp_off;
  const int* grp_tiles;
  int grp_n;
  int64_t grp_wstride;
  const int* grp_perm;
  int grp_k, grp_a_rows;
  bool grp_gather, grp_scatter;
  // epilogue 1 with split-K only: the second pass also writes norm_y = RMSNorm(C) * norm_w (rows
  // of N <= 8192 halves, C and norm_y contiguous: ldc == N); nullptr: the plain second pass
  const f16* norm_w;
  f16* norm_y;
  float norm_eps;
};

constexpr int kGemmBK = 64;
constexpr int kGemmMaxGroups = 256;  // grouped mode: at most this many groups (MoE experts)
// Wait until every LDS read of this wave has returned.
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Workgroup barrier without a memory fence (a fence would drain every in-flight LDS DMA); the
// DMA completions it orders are waited for explicitly with wait_vmcnt.
__device__ __forceinline__ void barrier_no_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Four consecutive fp16 values at p: one 8-byte access when `vec` (p 8-byte aligned), else four.
__device__ __forceinline__ f16x4 load4(const f16* p, bool vec) {
  if (vec) return *reinterpret_cast<const f16x4*>(p);
  return f16x4{p[0], p[1], p[2], p[3]};
}
__device__ __forceinline__ void store4(f16* p, f16x4 v, bool vec) {
  if (vec) {
    *reinterpret_cast<f16x4*>(p) = v;
  } else {
    p[0] = v[0];
    p[1] = v[1];
    p[2] = v[2];
    p[3] = v[3];
  }
}

// Half offset of logical 16-byte chunk `c` of row `r` in an LDS tile of BK-half rows (256, 128 or
// 64 bytes): the XOR term spreads the 16 rows one 128-bit read serves per cycle over all 64 banks.
template <int BK>
__device__ __forceinline__ int lds_off(int r, int c) {
  if constexpr (BK == 128) return r * 128 + ((c ^ (r & 15)) << 3);
  else if constexpr (BK == 64) return r * 64 + ((c ^ ((r >> 1) & 7)) << 3);
  else return r * 32 + ((c ^ ((r >> 2) & 3)) << 3);
}
// Byte offset of logical 16-byte chunk `c` of row `r` in an LDS tile of BK-byte int8 rows.
template <int BK>
__device__ __forceinline__ int lds_off8(int r, int c) {
  if constexpr (BK == 64) return r * 64 + ((c ^ ((r >> 2) & 3)) << 4);
  else return r * 32 + ((c ^ ((r >> 3) & 1)) << 4);
}

// Scheduling pattern of one step: the step's NM MFMAs alternate with the ND LDS reads of the next
// step's fragments (then whichever is left over), so the reads are issued early and their latency
// hides under the matrix work instead of being sunk next to their first use.
template <int NM, int ND>
__device__ __forceinline__ void sched_step() {
  constexpr int P = ND < NM ? ND : NM;
#pragma unroll
  for (int i = 0; i < P; i++) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
  }
  if constexpr (NM > P) __builtin_amdgcn_sched_group_barrier(0x008, NM - P, 0);
  if constexpr (ND > P) __builtin_amdgcn_sched_group_barrier(0x100, ND - P, 0);
}

template <int BM, int BN, int WM, int WN, int S, int EPI, bool Q8, bool GRP = false, int BK = 64, int KG = 1>
__global__ void __launch_bounds__(64 * WM * WN * KG) gemm_kernel(GemmArgs g) {
  constexpr int TM = BM / WM, TN = BN / WN;          // wave tile
  constexpr int FM = TM / 32, FN = TN / 32;          // MFMA tiles per wave
  constexpr int A_ST = BM * BK;                      // halves per stage
  constexpr int B_ROWB = Q8 ? BK : 2 * BK;           // bytes of one W row per K tile
  constexpr int RPI = 512 / BK;                      // fp16 rows per 1 KB DMA instruction
  constexpr int RPI8 = 1024 / BK;                    // int8 rows per 1 KB DMA instruction
  constexpr int B_ST = BN * B_ROWB / 2;              // halves per stage
  constexpr int NW = WM * WN;                        // waves per block (4 or 8)
  constexpr int A_LD = BM * 2 * BK / 1024 / NW;      // 1 KB DMA instructions per wave per K tile (A)
  constexpr int B_LD = BN * B_ROWB / 1024 / NW;      // ... (W)
  constexpr int L = A_LD + B_LD;                     // vector-memory ops per lane per K tile
  static_assert((NW == 4 || NW == 8) && FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tiling");
  static_assert(A_LD >= 1 && B_LD >= 1 && A_LD * 1024 * NW == BM * 2 * BK && B_LD * 1024 * NW == BN * B_ROWB &&
                    S >= 2 && S <= 8 && (S - 1) * L < 64 && 3 * L < 64,
                "pipeline shape: every wave issues the same whole number of 1 KB DMA instructions");
  static_assert(!(GRP && Q8), "grouped (expert) GEMMs take fp16 weights");
  static_assert(BK == 128 || BK == 64 || BK == 32, "K tile depth");
  static_assert(BK != 128 || (!Q8 && !GRP), "128-deep K tiles take fp16 weights (and K % 128 == 0)");
  static_assert(KG == 1 || (KG == 2 && !GRP), "one or two K groups (not in grouped mode)");
  // The dynamic LDS follows the static (the split-K flag below); a 16-byte element type makes the
  // compiler start it on a 16-byte boundary, which every 128-bit LDS access and DMA here needs.
  extern __shared__ u32x4 smem_raw[];
  // KG K groups of WM x WN waves each run the whole pipeline below on their share of the K tiles,
  // each with its own S-stage ring; group 0 adds the other groups' sums at the end
  const int tid = threadIdx.x, lane = tid & 63;
  const int kg = KG > 1 ? (tid >> 6) / NW : 0;  // this wave's K group
  const int wave = (tid >> 6) - kg * NW;        // its index within the group
  f16* smem = reinterpret_cast<f16*>(smem_raw) + kg * S * (A_ST + B_ST);
  f16* As = smem;               // [S][BM][64]
  f16* Bs = smem + S * A_ST;    // [S][BN][64] fp16, or [S][BN][64 bytes] int8

  const int wm = wave / WN, wn = wave % WN;
  const int N = g.N, K = g.K;
  int M = g.M;
  const f16* Ap = g.A;
  f16* Cp = g.C;
  const char* Wb = reinterpret_cast<const char*>(g.W);
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn, ntiles;
  [[maybe_unused]] int grp_r0 = 0;  // grouped mode: the group's first sorted row
  if constexpr (GRP) {
    // find this block's group: grp_tiles[e] <= row tile < grp_tiles[e + 1] (the prefix is
    // non-decreasing, so e is the number of groups whose tiles start at or before the row tile,
    // minus one); blocks past the last row tile (the grid is sized for the worst case) exit. Every
    // thread loads one group's tile start and first row at once (thread 0 also the totals): one
    // memory round trip, then one counting barrier.
    static_assert(64 * NW * KG >= kGemmMaxGroups, "one thread per group");
    __shared__ int s_tiles[kGemmMaxGroups + 1], s_off[kGemmMaxGroups + 1];
    const int E = g.grp_n, mt = blockIdx.x / tiles_n;
    tn = blockIdx.x - mt * tiles_n;
    int te = 0;
    if (tid < E) {
      te = g.grp_tiles[tid];
      s_tiles[tid] = te;
      s_off[tid] = g.grp_off[tid];
    }
    if (tid == 0) {
      s_tiles[E] = g.grp_tiles[E];
      s_off[E] = g.grp_off[E];
    }
    const int lo = __syncthreads_count(tid < E && te <= mt) - 1;
    if (mt >= s_tiles[E]) return;
    grp_r0 = s_off[lo];
    M = s_off[lo + 1] - grp_r0;
    if (!g.grp_gather) Ap += grp_r0 * g.lda;
    if (!g.grp_scatter) Cp += grp_r0 * g.ldc;
    Wb += lo * g.grp_wstride;
    tm = mt - s_tiles[lo];
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

  const int nkt = (K + BK - 1) / BK;
  // K tiles of this split (>= 1), cut into KG equal runs, one per K group (the host offers KG > 1
  // only when K % BK == 0 and the runs come out equal, so every group loops alike)
  const int nloc = (min(nkt, (int)blockIdx.y * g.kt_per_split + g.kt_per_split) - (int)blockIdx.y * g.kt_per_split) / KG;
  const int kt0 = blockIdx.y * g.kt_per_split + kg * nloc;
  // the last tile holds only 32 k (K % 64 == 32 with 64-deep tiles; K % 32 == 0 always)
  const bool half_tail = BK == 64 && (K & 63) != 0 && kt0 + nloc == nkt;

  // ---- DMA of one K tile into stage st, through buffer resources based at the block's first A
  //      and W rows. Lane l of an instruction covering 8 (A, W fp16) or 16 (W int8) rows fills LDS
  //      slot l: it fetches the chunk the swizzle puts there. Offsets are bounds-checked against
  //      the rows that exist: rows past M or N read zeros (never stored). Chunks past K (the second
  //      half of a half tile) read bytes of the next row or zeros, and are never used.
  const int valid_m = min(M - bm, BM), valid_n = min(N - bn, BN);
  const bool gather = GRP && g.grp_gather;  // A rows through grp_perm: the resource spans all of A
  const int a_bytes = gather ? (int)(((int64_t)(g.grp_a_rows - 1) * g.lda + K) * 2)
                             : (int)(((int64_t)(valid_m - 1) * g.lda + K) * 2);
  const __amdgpu_buffer_rsrc_t a_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<f16*>(gather ? Ap : Ap + (int64_t)bm * g.lda), (short)0, a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(Wb + (int64_t)bn * K * (Q8 ? 1 : 2)), (short)0, (int)((int64_t)valid_n * K * (Q8 ? 1 : 2)),
      0x00020000);
  // this lane's byte offset within an instruction's rows; the swizzle term of a 256-byte row r is
  // (r & 15), which over an instruction's 4 rows depends on the instruction's index mod 4 and
  // lane / 16; of a 128-byte row ((r >> 1) & 7), which over an instruction's 8 rows depends on the
  // instruction's parity and lane / 16; of a 64-byte row ((r >> 2) & 3) and of a 32-byte int8 row
  // ((r >> 3) & 1), which depend on the lane only
  const int a_r = lane / (BK / 8), a_p = lane % (BK / 8);
  int a_lo[4], b_lo[4];  // per instruction index mod 4 (mod 2 for 128-byte rows; unused entries)
#pragma unroll
  for (int par = 0; par < 4; par++) {
    const int sw = BK == 128 ? (par * 4 + a_r) & 15 : BK == 64 ? (par * 4 + (a_r >> 1)) & 7 : (a_r >> 2) & 3;
    a_lo[par] = (int)((int64_t)a_r * g.lda * 2) + ((a_p ^ sw) << 4);
    if constexpr (Q8) {
      b_lo[par] = BK == 64 ? (lane >> 2) * K + (((lane & 3) ^ ((lane >> 4) & 3)) << 4)
                           : (lane >> 1) * K + (((lane & 1) ^ ((lane >> 4) & 1)) << 4);
    } else {
      b_lo[par] = a_r * K * 2 + ((a_p ^ sw) << 4);
    }
  }
  // grouped gather: this lane's row of each A instruction is sorted row grp_r0 + bm + ri + a_r,
  // fetched from A row grp_perm[that] / grp_k; rows past the group's count get an offset past the
  // resource, so they read zeros
  int a_go[A_LD];  // set and read in grouped mode only
  if constexpr (GRP) {
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      const int ri = (wave * A_LD + i) * RPI, r = bm + ri + a_r;
      const int lo_i = a_lo[(ri / RPI) % (BK == 128 ? 4 : 2)] - (int)((int64_t)a_r * g.lda * 2);  // the chunk term
      if (gather)
        a_go[i] = r < M ? (int)((int64_t)(g.grp_perm[grp_r0 + r] / g.grp_k) * g.lda * 2) + lo_i : a_bytes;
      else
        a_go[i] = a_lo[(ri / RPI) % (BK == 128 ? 4 : 2)] + (int)((int64_t)ri * g.lda * 2);
    }
  }
  auto issue = [&](int kt, int st) {
    const int k0 = kt * BK;
    f16* as = As + st * A_ST;
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      const int ri = (wave * A_LD + i) * RPI;
      // (a plain conditional: an `if constexpr` here kept clang from emitting the grouped kernels)
      const int off = GRP ? a_go[i] : a_lo[(ri / RPI) % (BK == 128 ? 4 : 2)] + (int)((int64_t)ri * g.lda * 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, (lds_void_t*)(as + ri * BK), 16, off + k0 * 2, 0, 0, 0);
    }
    char* bs = reinterpret_cast<char*>(Bs + st * B_ST);
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      if constexpr (Q8) {
        const int ri = (wave * B_LD + i) * RPI8;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rs, (lds_void_t*)(bs + ri * BK), 16, b_lo[0] + ri * K + k0, 0, 0, 0);
      } else {
        const int ri = (wave * B_LD + i) * RPI;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rs, (lds_void_t*)(bs + ri * 2 * BK), 16,
                                                 b_lo[(ri / RPI) % (BK == 128 ? 4 : 2)] + ri * K * 2 + k0 * 2, 0, 0, 0);
      }
    }
  };

  const int fr = lane & 31, fk = lane >> 5;  // fragment row (or column) and k half
  // grouped scatter: the C row of each of this lane's fragment rows, requested now so that the
  // epilogue waits for nothing
  int c_row[FM];
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int row = bm + wm * TM + i * 32 + fr;
    c_row[i] = (GRP && g.grp_scatter && row < M) ? g.grp_perm[grp_r0 + row] : row;
  }
  f16x2 bsc[FN];                             // int8: the scale of the W row each B fragment reads
#pragma unroll
  for (int j = 0; j < FN; j++) {
    bsc[j] = f16x2{(f16)0.f, (f16)0.f};
    if constexpr (Q8) {
      const f16 sv = g.scales[min(bn + wn * TN + j * 32 + fr, N - 1)];
      bsc[j] = f16x2{sv, sv};
    }
  }
  // LDS offsets of this lane's fragment rows (halves for A / fp16 W, bytes for int8 W), per chunk
  // parity: the swizzle term of row r is ((r >> 1) & 7) (or (r >> 2) & 3), fixed per lane
  int a_row[FM], b_row[FN];
#pragma unroll
  for (int i = 0; i < FM; i++) a_row[i] = (wm * TM + i * 32 + fr);
#pragma unroll
  for (int j = 0; j < FN; j++) b_row[j] = (wn * TN + j * 32 + fr);

  // fragments of step s = 2 jh + h of the tile in stage st
  auto load_a = [&](int st, int s, f16x8 (&af)[FM]) {
    const int c = 4 * (s >> 1) + 2 * fk + (s & 1);
    const f16* as = As + st * A_ST;
#pragma unroll
    for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const f16x8*>(as + lds_off<BK>(a_row[i], c));
  };
  // fp16 W: one fragment per step
  auto load_b = [&](int st, int s, f16x8 (&bf)[FN]) {
    const int c = 4 * (s >> 1) + 2 * fk + (s & 1);
    const f16* bs = Bs + st * B_ST;
#pragma unroll
    for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const f16x8*>(bs + lds_off<BK>(b_row[j], c));
  };
  // int8 W: both steps of half jh as one raw 16-byte chunk
  auto load_q = [&](int st, int jh, u32x4 (&bq)[FN]) {
    const char* bs = reinterpret_cast<const char*>(Bs + st * B_ST);
    const int c = 2 * jh + fk;
#pragma unroll
    for (int j = 0; j < FN; j++) bq[j] = *reinterpret_cast<const u32x4*>(bs + lds_off8<BK>(b_row[j], c));
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  // the MFMAs of one step; int8 fragments are dequantised from half h of the raw chunk
  auto mfmas = [&](int h, const f16x8 (&af)[FM], const f16x8 (&bf)[FN], const u32x4 (&bq)[FN]) {
    f16x8 b[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
      if constexpr (Q8) {
        f16x2 p0, p1, p2, p3;
        i8x4_to_f16(bq[j][2 * h], p0, p1);
        i8x4_to_f16(bq[j][2 * h + 1], p2, p3);
        p0 = p0 * bsc[j];  // fp16(q * s), one rounding each
        p1 = p1 * bsc[j];
        p2 = p2 * bsc[j];
        p3 = p3 * bsc[j];
        b[j] = f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
      } else {
        b[j] = bf[j];
      }
    }
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b[j], af[i], acc[i][j], 0, 0, 0);
  };

  // ---- prologue: S tiles in flight (past the split's last tile, its first tile again: a stage is
  //      filled every time, so the outstanding-DMA count is the same in every iteration), the
  //      first fragments of tile 0 in registers
  auto tile_or_first = [&](int kt) { return kt < kt0 + nloc ? kt : kt0; };
#pragma unroll
  for (int s = 0; s < S; s++) issue(tile_or_first(kt0 + s), s);
  wait_vmcnt<(S - 1) * L>();
  barrier_no_fence();
  f16x8 af0[FM], af1[FM], bf0[FN], bf1[FN];
  u32x4 bq0[FN], bq1[FN];  // int8: raw chunks of the tile's first and second 32-deep half
  load_a(0, 0, af0);
  if constexpr (Q8) load_q(0, 0, bq0);
  else load_b(0, 0, bf0);

  constexpr int NM = FM * FN;               // MFMAs per step
  constexpr int ND = FM + (Q8 ? 0 : FN);    // LDS reads per step (int8 W: + FN every other step)
  if constexpr (BK == 128) {
    // ---- 128-deep fp16 tiles (K % 128 == 0): 8 steps each, fragments one step ahead, the same
    //      k order as two consecutive 64-deep tiles (so the same sums, bit for bit)
    for (int t = 0; t < nloc - 1; t++) {
      const int st = t % S;
#pragma unroll
      for (int p = 0; p < 3; p++) {
        load_a(st, 2 * p + 1, af1);
        load_b(st, 2 * p + 1, bf1);
        mfmas(0, af0, bf0, bq0);
        sched_step<NM, ND>();
        load_a(st, 2 * p + 2, af0);
        load_b(st, 2 * p + 2, bf0);
        mfmas(0, af1, bf1, bq0);
        sched_step<NM, ND>();
      }
      load_a(st, 7, af1);
      load_b(st, 7, bf1);
      mfmas(0, af0, bf0, bq0);
      sched_step<NM, ND>();
      // the tile's last fragments are in registers: free its stage, refill it, start the next tile
      wait_lgkm0();
      wait_vmcnt<(S - 2) * L>();
      barrier_no_fence();
      issue(tile_or_first(kt0 + t + S), st);
      const int sn = (t + 1) % S;
      load_a(sn, 0, af0);
      load_b(sn, 0, bf0);
      mfmas(0, af1, bf1, bq0);
      sched_step<NM, ND>();
    }
    const int st = (nloc - 1) % S;
#pragma unroll
    for (int p = 0; p < 4; p++) {
      load_a(st, 2 * p + 1, af1);
      load_b(st, 2 * p + 1, bf1);
      mfmas(0, af0, bf0, bq0);
      if (p < 3) {
        load_a(st, 2 * p + 2, af0);
        load_b(st, 2 * p + 2, bf0);
      }
      mfmas(0, af1, bf1, bq0);
    }
  } else if constexpr (BK == 64) {
    // ---- main loop over all tiles but the last: 4 steps each, fragments one step ahead
    for (int t = 0; t < nloc - 1; t++) {
      const int st = t % S;
      load_a(st, 1, af1);
      if constexpr (!Q8) load_b(st, 1, bf1);
      mfmas(0, af0, bf0, bq0);
      sched_step<NM, ND>();
      load_a(st, 2, af0);
      if constexpr (Q8) load_q(st, 1, bq1);
      else load_b(st, 2, bf0);
      mfmas(1, af1, bf1, bq0);
      sched_step<NM, ND + (Q8 ? FN : 0)>();
      load_a(st, 3, af1);
      if constexpr (!Q8) load_b(st, 3, bf1);
      mfmas(0, af0, bf0, bq1);
      sched_step<NM, ND>();
      // the tile's last fragments are in registers: free its stage, refill it, start the next tile
      wait_lgkm0();
      wait_vmcnt<(S - 2) * L>();
      barrier_no_fence();
      issue(tile_or_first(kt0 + t + S), st);
      const int sn = (t + 1) % S;
      load_a(sn, 0, af0);
      if constexpr (Q8) load_q(sn, 0, bq0);
      else load_b(sn, 0, bf0);
      mfmas(1, af1, bf1, bq1);
      sched_step<NM, ND + (Q8 ? FN : 0)>();
    }
    // ---- the last tile (its first half only when K % 64 == 32)
    {
      const int st = (nloc - 1) % S;
      load_a(st, 1, af1);
      if constexpr (!Q8) load_b(st, 1, bf1);
      mfmas(0, af0, bf0, bq0);
      mfmas(1, af1, bf1, bq0);
      if (!half_tail) {
        load_a(st, 2, af0);
        load_a(st, 3, af1);
        if constexpr (Q8) {
          load_q(st, 1, bq1);
        } else {
          load_b(st, 2, bf0);
          load_b(st, 3, bf1);
        }
        mfmas(0, af0, bf0, bq1);
        mfmas(1, af1, bf1, bq1);
      }
    }
  } else {
    // ---- 32-deep tiles: 2 steps each, fragments one step ahead; int8 W holds both steps of a
    //      tile in one raw 16-byte chunk per fragment (bq0), the next tile's read into bqn first
    for (int t = 0; t < nloc - 1; t++) {
      const int st = t % S;
      load_a(st, 1, af1);
      if constexpr (!Q8) load_b(st, 1, bf1);
      mfmas(0, af0, bf0, bq0);
      sched_step<NM, ND>();
      // the tile's last fragments are in registers: free its stage, refill it, start the next tile
      wait_lgkm0();
      wait_vmcnt<(S - 2) * L>();
      barrier_no_fence();
      issue(tile_or_first(kt0 + t + S), st);
      const int sn = (t + 1) % S;
      load_a(sn, 0, af0);
      [[maybe_unused]] u32x4 bqn[FN];
      if constexpr (Q8) load_q(sn, 0, bqn);
      else load_b(sn, 0, bf0);
      mfmas(1, af1, bf1, bq0);
      sched_step<NM, ND + (Q8 ? FN : 0)>();
      if constexpr (Q8) {
#pragma unroll
        for (int j = 0; j < FN; j++) bq0[j] = bqn[j];
      }
    }
    const int st = (nloc - 1) % S;
    load_a(st, 1, af1);
    if constexpr (!Q8) load_b(st, 1, bf1);
    mfmas(0, af0, bf0, bq0);
    mfmas(1, af1, bf1, bq0);
  }
  wait_vmcnt<0>();  // the refills issued past the last tile have landed before the block ends
  if constexpr (KG > 1) {
    // the other group's sums to group 0 through the idle rings (element e of a wave's fragment
    // set as one 256-byte row over its lanes), added in group order: deterministic
    constexpr int NE = FM * FN * 16;
    float* xf = reinterpret_cast<float*>(smem_raw);
    barrier_no_fence();  // every wave's last fragment reads are done with the rings
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
          for (int e = 0; e < 16; e++) xf[((wave * NE) + (i * FN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) acc[i][j][e] += xf[((wave * NE) + (i * FN + j) * 16 + e) * 64 + lane];
  }

  // ---- result layout (W fragment as the MFMA's first operand): lane (fk, fr) of tile (i, j) holds
  //      row fr of the tile's 32 rows, columns 8 g + 4 fk + 0..3 in acc[i][j][4 g .. 4 g + 3]:
  //      four consecutive output columns per register quad

  // ---- staged epilogue (grouped tiles and the one-wave-wide 128 x 96 / 128 x 160 tiles; one K
  //      group, no split, C 16-byte addressable): the finished fp16 tile goes through LDS and leaves
  //      in 16-byte chunks, whole row segments per store instruction. Stored straight from the
  //      fragments, each store instruction writes 16 bytes into each of 32 rows (about 150 ns per
  //      instruction measured on the grouped down GEMM, 16 per lane there, 12-20 on the wide-wave
  //      tiles); staged, four to six rows of contiguous chunks. Other tiles keep the direct path:
  //      there the staged code cost registers (4-12 VGPRs, more spills on 256 x 256) for no gain.
  //      The roundings are the direct path's: the bias is added in fp32 before the fp16 rounding,
  //      SwiGLU is formed from the fp32 sums, and the residual is added (fp16 add) to the rounded
  //      product in the copy.
  constexpr bool kStaged = KG == 1 && (GRP || WN == 1);
  if (kStaged && gridDim.y == 1 && g.vec16_c) {
    constexpr int BNO = EPI == 2 ? BN / 2 : BN;  // output columns of the tile
    // LDS row stride in halves: 16 bytes of padding put the 32 rows one fragment write covers on
    // every bank once per 16 rows (BNO % 16 == 0)
    constexpr int CS = BNO + 8;
    static_assert(BNO % 16 == 0, "staged tile row padding");
    f16* cs = reinterpret_cast<f16*>(smem_raw);
    int* s_row = reinterpret_cast<int*>(cs + BM * CS);  // C row of each tile row
    barrier_no_fence();  // every wave is done with the rings (their DMA landed above)
#pragma unroll
    for (int i = 0; i < FM; i++) {
      const int lr = wm * TM + i * 32 + fr;
      if (wn == 0 && fk == 0) s_row[lr] = c_row[i];
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int lc0 = wn * TN + j * 32;  // the 32-column MFMA tile's first column in the tile
        if constexpr (EPI == 2) {
#pragma unroll
          for (int q = 0; q < 2; q++) {
            f16x4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = silu_mul_fast(acc[i][j][4 * q + e], acc[i][j][4 * q + 8 + e]);
            *reinterpret_cast<f16x4*>(cs + lr * CS + (lc0 >> 1) + 8 * q + 4 * fk) = o;
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const int lc = lc0 + 8 * q + 4 * fk;
            f16x4 o;
            if constexpr (EPI == 1) {
#pragma unroll
              for (int e = 0; e < 4; e++) o[e] = (f16)acc[i][j][4 * q + e];
            } else {
              f16x4 b = {(f16)0.f, (f16)0.f, (f16)0.f, (f16)0.f};
              if (g.bias && bn + lc < N) b = load4(g.bias + bn + lc, ((uintptr_t)g.bias & 7) == 0);
#pragma unroll
              for (int e = 0; e < 4; e++) o[e] = (f16)(acc[i][j][4 * q + e] + (float)b[e]);
            }
            *reinterpret_cast<f16x4*>(cs + lr * CS + lc) = o;
          }
        }
      }
    }
    __syncthreads();
    constexpr int CPR = BNO / 8;  // 16-byte chunks per tile row
    const int bno = EPI == 2 ? bn / 2 : bn, ncol = min((EPI == 2 ? N / 2 : N) - bno, BNO);
    for (int c = tid; c < BM * CPR; c += 64 * NW) {
      const int r = c / CPR, cc = c - r * CPR;
      if (r >= valid_m || cc * 8 >= ncol) continue;  // N % 16 == 0: a chunk is all in or all out
      f16x8 v = *reinterpret_cast<const f16x8*>(cs + r * CS + cc * 8);
      f16* dst = Cp + (int64_t)s_row[r] * g.ldc + bno + cc * 8;
      if constexpr (EPI == 1) {
        const f16x8 rv = *reinterpret_cast<const f16x8*>(dst);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = rv[e] + v[e];  // fp16 add, correctly rounded
      }
      *reinterpret_cast<f16x8*>(dst) = v;
    }
    return;
  }
  if (gridDim.y > 1) {
    // split-K: this split's fp32 partial [split][M][N]; a second kernel (gemm_splitk_reduce) sums
    // the splits in order and runs the epilogue, after the kernel boundary made them visible
    float* part = g.ws + (int64_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < FM; i++) {
      const int row = bm + wm * TM + i * 32 + fr;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int col = bn + wn * TN + j * 32 + 8 * q + 4 * fk;
          if (col < N)
            *reinterpret_cast<f32x4*>(part + (int64_t)row * N + col) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int row = bm + wm * TM + i * 32 + fr;
    if (row >= M) continue;
    f16* crow = Cp + (int64_t)c_row[i] * g.ldc;
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int c0 = bn + wn * TN + j * 32;  // first column of the 32-column MFMA tile
      if (c0 >= N) continue;
      if constexpr (EPI == 2) {
        // gate columns c0 + 0..15 and their up columns c0 + 16..31 sit in the same lane
#pragma unroll
        for (int q = 0; q < 2; q++) {
          f16x4 o;
#pragma unroll
          for (int e = 0; e < 4; e++) o[e] = silu_mul_fast(acc[i][j][4 * q + e], acc[i][j][4 * q + 8 + e]);
          store4(crow + (c0 >> 1) + 8 * q + 4 * fk, o, g.vec_c);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int col = c0 + 8 * q + 4 * fk;
          if (col >= N) continue;  // N % 16 == 0: the last 32-column tile can end 16 columns past N
          f16x4 o;
          if constexpr (EPI == 1) {
            const f16x4 r = load4(crow + col, g.vec_c);
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = r[e] + (f16)acc[i][j][4 * q + e];  // fp16 add, rounded
          } else {
            f16x4 b = {(f16)0.f, (f16)0.f, (f16)0.f, (f16)0.f};
            if (g.bias) b = load4(g.bias + col, ((uintptr_t)g.bias & 7) == 0);
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = (f16)(acc[i][j][4 * q + e] + (float)b[e]);
          }
          store4(crow + col, o, g.vec_c);
        }
      }
    }
  }
}

// Split-K second pass: sum the fp32 partials [splits][M][N] in split order (deterministic) and run
// the epilogue with the main kernel's rounding; each thread owns 4 consecutive output columns.
template <int EPI>
__global__ void __launch_bounds__(256) gemm_splitk_reduce(const float* __restrict__ ws, int splits, int M, int N,
                                                          const f16* __restrict__ bias, f16* C, int64_t ldc,
                                                          bool vec_c) {
  const int n_out = EPI == 2 ? N / 2 : N;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (idx >= (int64_t)M * n_out) return;
  const int row = (int)(idx / n_out), oc = (int)(idx - (int64_t)row * n_out);
  const int64_t plane = (int64_t)M * N;
  f16* dst = C + (int64_t)row * ldc + oc;
  f16x4 o;
  if constexpr (EPI == 2) {
    const int gc = (oc >> 4) * 32 + (oc & 15);  // gate column; its up column is gc + 16
    f32x4 gs = {0.f, 0.f, 0.f, 0.f}, us = gs;
    for (int z = 0; z < splits; z++) {
      gs += *reinterpret_cast<const f32x4*>(ws + z * plane + (int64_t)row * N + gc);
      us += *reinterpret_cast<const f32x4*>(ws + z * plane + (int64_t)row * N + gc + 16);
    }
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = silu_mul_fast(gs[e], us[e]);
  } else {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    for (int z = 0; z < splits; z++) t += *reinterpret_cast<const f32x4*>(ws + z * plane + (int64_t)row * N + oc);
    if constexpr (EPI == 1) {
      const f16x4 r = load4(dst, vec_c);
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = r[e] + (f16)t[e];
    } else {
      f16x4 b = {(f16)0.f, (f16)0.f, (f16)0.f, (f16)0.f};
      if (bias) b = load4(bias + oc, ((uintptr_t)bias & 7) == 0);
#pragma unroll
      for (int e = 0; e < 4; e++) o[e] = (f16)(t[e] + (float)b[e]);
    }
  }
  store4(dst, o, vec_c);
}

// Tile configurations: {BM, BN, WM, WN, stages, BK[, K groups]}; WM x WN waves per K group, BK-deep
// K tiles. The
// 32-deep ones give the big 8-wave tiles four (or six) stages in the same LDS as two 64-deep
// ones: more K tiles in flight to cover the global->LDS latency. 128 x 160 and 128 x 96 (four
// waves stacked along M, each 32 rows by the whole width) cut N = 5120 and N = 3072 at M = 1024
// into exactly 256 tiles, one per CU, with no split-K. 32 x 256 (four waves side by side, 32 x 64
// each) serves batched decode (M <= 32) on the widest projections: 32 KB of weights per stage.
// 256 x 192 (eight waves of 64 x 96) cuts N = 3072 at M = 1024 into 64 big tiles, 256 blocks with
// a 4-way split-K: half the staged bytes of 128 x 96 for the same K range. The two 128-deep small
// tiles (fp16 weights, K % 128 == 0) fetch each W row in 256-byte runs per K tile instead of
// 128-byte ones, for the weight-streaming small-M shapes. The last, 128 x 160 in two K groups
// (eight waves: two 4-wave pipelines on the two halves of the K tiles, each with its own 2-stage
// ring, group 1's sums handed to group 0 through LDS at the end), puts two waves on each SIMD
// for the same one-tile-per-CU cut of N = 5120: QKV of Llama-3.2-3B at M = 1024 in 42.3 against
// 45.6 us. The same split of 128 x 96 (o, down) measured no faster, and neither did four-wave
// tiles whose waves hold 64 rows (37 % fewer LDS fragment reads per MFMA): neither latency nor the
// LDS reads bound the narrow tiles.
struct GemmCfg {
  int bm, bn, wm, wn, st, bk, kg = 1;  // kg: K groups of wm x wn waves (two waves on each SIMD at kg 2)
};
constexpr GemmCfg kGemmCfgs[] = {{256, 256, 2, 2, 2, 64}, {256, 128, 2, 2, 3, 64}, {128, 256, 2, 2, 3, 64},
                                 {64, 128, 2, 2, 4, 64},  {128, 128, 2, 2, 2, 64}, {64, 64, 2, 2, 4, 64},
                                 {32, 128, 1, 4, 4, 64},  {128, 64, 2, 2, 4, 64},  {256, 256, 2, 4, 2, 64},
                                 {256, 128, 2, 4, 3, 64}, {256, 256, 2, 4, 4, 32}, {256, 128, 2, 2, 6, 32},
                                 {128, 256, 2, 4, 6, 32}, {128, 160, 4, 1, 4, 64}, {128, 96, 4, 1, 4, 64},
                                 {32, 256, 1, 4, 4, 64},  {256, 192, 4, 2, 2, 64}, {64, 128, 2, 2, 3, 128},
                                 {128, 64, 2, 2, 3, 128}, {128, 160, 4, 1, 2, 64, 2}};
constexpr int kGemmNumCfgs = sizeof(kGemmCfgs) / sizeof(kGemmCfgs[0]);
// A config exists for a weight format when its A and W tiles split into whole 1 KB DMA
// instructions per wave (int8 W rows are half as wide: 128 x 160 and 128 x 96 are fp16 only).
constexpr bool gemm_cfg_ok(int c, bool q8) {
  const int nw = kGemmCfgs[c].wm * kGemmCfgs[c].wn, bk = kGemmCfgs[c].bk;
  const int a = kGemmCfgs[c].bm * 2 * bk, b = kGemmCfgs[c].bn * (q8 ? bk : 2 * bk);
  return a % (1024 * nw) == 0 && b % (1024 * nw) == 0 && a >= 1024 * nw && b >= 1024 * nw && !(q8 && bk == 128);
}
// ... and for a shape: 128-deep tiles have no K tail, so they need K % 128 == 0.
constexpr bool gemm_cfg_fits(int c, bool q8, int K) {
  return gemm_cfg_ok(c, q8) && (kGemmCfgs[c].bk < 128 || K % 128 == 0) &&
         (kGemmCfgs[c].kg == 1 || (K % kGemmCfgs[c].bk == 0 && (K / kGemmCfgs[c].bk) % kGemmCfgs[c].kg == 0));
}
// The grouped (MoE expert) GEMM's tile: 128 x 128, four 64-deep stages (128 KB of LDS, one block
// per CU). 128 rows hold a whole expert's share of a 256-token prefill (top-8 of 32 experts: about
// 64 rows each), so each expert's weights are streamed once; a 64-row tile split most experts into
// two row tiles, each streaming the same weights.
constexpr int kGrpBM = 128, kGrpBN = 128, kGrpWM = 2, kGrpWN = 2, kGrpStages = 4, kGrpBK = 64;
// LDS of the staged epilogue: the fp16 tile with 16-byte row padding, then one C row index per row
constexpr size_t gemm_stage_bytes(int bm, int bn) { return (size_t)bm * (bn + 8) * 2 + (size_t)bm * 4; }
inline size_t gemm_lds_bytes(int cfg, bool q8) {
  const GemmCfg& c = kGemmCfgs[cfg];
  const size_t ring = (size_t)c.kg * c.st * (c.bm * c.bk * 2 + c.bn * (q8 ? c.bk : 2 * c.bk));
  const bool staged = c.kg == 1 && c.wn == 1;  // the kernel's kStaged (grouped tiles size their own)
  return staged && gemm_stage_bytes(c.bm, c.bn) > ring ? gemm_stage_bytes(c.bm, c.bn) : ring;
}

// Split-K second pass of a residual GEMM fused with the RMSNorm that reads its result: one block
// of kNormThreads per row sums the row's partials in split order and adds the residual exactly as
// gemm_splitk_reduce<1> does, writes the row back, and normalises it as rmsnorm_kernel does (the
// same chunk ownership, summation order and norm_finish), so both outputs are bit-identical to
// the two kernels run in turn. With the split count ZS fixed at compile time (2..8) a thread issues
// all its loads of a chunk's partials before it adds them: with one row per block the pass is
// otherwise one memory round trip per split (ZS = 0: any count, one split at a time). RC chunks
// per thread: 1 for rows of up to 4096 halves (rmsnorm_kernel's second chunk then only adds exact
// zeros), else kNormChunks. Rows of N <= 8192 halves (N % 8 == 0), C and y contiguous.
template <int RC, int ZS>
__global__ void __launch_bounds__(kNormThreads) gemm_splitk_reduce_rmsnorm(const float* __restrict__ ws, int splits,
                                                                           int M, int N, f16* C,
                                                                           const f16* __restrict__ w,
                                                                           f16* __restrict__ y, float eps) {
  static_assert(RC >= 1 && RC <= kNormChunks, "chunks per thread");
  __shared__ float red[kNormThreads / 64];
  const int tid = threadIdx.x, n8 = N / 8, row = blockIdx.x;
  const int64_t plane = (int64_t)M * N;
  f16* xr = C + (int64_t)row * N;
  const float* pr = ws + (int64_t)row * N;
  u32x4 hv[RC], wv[RC];
#pragma unroll
  for (int j = 0; j < RC; j++) {
    const int c = tid + j * kNormThreads;
    hv[j] = wv[j] = u32x4{0u, 0u, 0u, 0u};
    if (c < n8) {
      wv[j] = *reinterpret_cast<const u32x4*>(w + 8 * c);
      const f16x8 r = *reinterpret_cast<const f16x8*>(xr + 8 * c);
      f32x4 t0 = {0.f, 0.f, 0.f, 0.f}, t1 = t0;
      if constexpr (ZS > 0) {
        f32x4 a[ZS], b[ZS];
#pragma unroll
        for (int z = 0; z < ZS; z++) {
          a[z] = *reinterpret_cast<const f32x4*>(pr + z * plane + 8 * c);
          b[z] = *reinterpret_cast<const f32x4*>(pr + z * plane + 8 * c + 4);
        }
#pragma unroll
        for (int z = 0; z < ZS; z++) {
          t0 += a[z];
          t1 += b[z];
        }
      } else {
        for (int z = 0; z < splits; z++) {
          t0 += *reinterpret_cast<const f32x4*>(pr + z * plane + 8 * c);
          t1 += *reinterpret_cast<const f32x4*>(pr + z * plane + 8 * c + 4);
        }
      }
      f16x8 h;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        h[e] = r[e] + (f16)t0[e];
        h[4 + e] = r[4 + e] + (f16)t1[e];
      }
      hv[j] = __builtin_bit_cast(u32x4, h);
      *reinterpret_cast<u32x4*>(xr + 8 * c) = hv[j];
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < RC; j++)
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const f16x2 h = as_h2(hv[j][p]);
      ss = dot2(h, h, ss);
    }
  const float rs = norm_finish(ss, red, N, eps);
  f16* yr = y + (int64_t)row * N;
#pragma unroll
  for (int j = 0; j < RC; j++) {
    const int c = tid + j * kNormThreads;
    if (c >= n8) continue;
    u32x4 o;
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const f16x2 xh = as_h2(hv[j][p]), wh = as_h2(wv[j][p]);
      f16x2 t;
      t.x = wh.x * (f16)((float)xh.x * rs);
      t.y = wh.y * (f16)((float)xh.y * rs);
      o[p] = as_u32(t);
    }
    *reinterpret_cast<u32x4*>(yr + 8 * c) = o;
  }
}

typedef void (*SplitkRmsnormFn)(const float*, int, int, int, f16*, const f16*, f16*, float);
template <int RC>
inline SplitkRmsnormFn splitk_rmsnorm_for(int splits) {
  switch (splits) {
    case 2: return gemm_splitk_reduce_rmsnorm<RC, 2>;
    case 3: return gemm_splitk_reduce_rmsnorm<RC, 3>;
    case 4: return gemm_splitk_reduce_rmsnorm<RC, 4>;
    case 5: return gemm_splitk_reduce_rmsnorm<RC, 5>;
    case 6: return gemm_splitk_reduce_rmsnorm<RC, 6>;
    case 8: return gemm_splitk_reduce_rmsnorm<RC, 8>;
    default: return gemm_splitk_reduce_rmsnorm<RC, 0>;
  }
}
inline SplitkRmsnormFn splitk_rmsnorm_kernel(bool one_chunk, int splits) {
  return one_chunk ? splitk_rmsnorm_for<1>(splits) : splitk_rmsnorm_for<kNormChunks>(splits);
}

template <int BM, int BN, int WM, int WN, int S, int EPI, bool Q8, int BK, int KG>
int gemm_launch(const GemmArgs& g, int cfg, int splits, hipStream_t s) {
  const size_t lds = gemm_lds_bytes(cfg, Q8);
  const void* fn = reinterpret_cast<const void*>(&gemm_kernel<BM, BN, WM, WN, S, EPI, Q8, false, BK, KG>);
  const int bpc = hi_blocks_per_cu(fn, 64 * WM * WN * KG, lds);  // also lifts the dynamic-LDS limit
  if (bpc < 0) return -2;
  if (bpc == 0) HI_FAIL("gemm: tile %dx%d does not fit on a CU", BM, BN);
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, S, EPI, Q8, false, BK, KG>), dim3(tiles, splits),
                     dim3(64 * WM * WN * KG), lds, s, g);
  HI_TRY(hipGetLastError());
  if (splits > 1 && EPI == 1 && g.norm_y) {
    hipLaunchKernelGGL(splitk_rmsnorm_kernel(g.N <= 8 * kNormThreads, splits), dim3(g.M), dim3(kNormThreads), 0, s, g.ws,
                       splits, g.M, g.N, g.C, g.norm_w, g.norm_y, g.norm_eps);
    HI_TRY(hipGetLastError());
  } else if (splits > 1) {
    const int64_t quads = (int64_t)g.M * (EPI == 2 ? g.N / 2 : g.N) / 4;
    hipLaunchKernelGGL(gemm_splitk_reduce<EPI>, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, s, g.ws, splits,
                       g.M, g.N, g.bias, g.C, g.ldc, g.vec_c);
    HI_TRY(hipGetLastError());
  }
  return 0;
}

template <int EPI>
int gemm_run(const GemmArgs& g, int cfg, int splits, bool q8, hipStream_t s);
// Resident blocks per CU of a config's kernel (occupancy API). Kernels are only ever named in
// their own instance file: naming one elsewhere would instantiate (and register) a second copy.
template <int EPI>
int gemm_blocks_per_cu(int cfg, bool q8);

#define HI_GEMM_K(i, q)                                                                                        \
  gemm_kernel<kGemmCfgs[i].bm, kGemmCfgs[i].bn, kGemmCfgs[i].wm, kGemmCfgs[i].wn, kGemmCfgs[i].st, EPI, q, false, \
              kGemmCfgs[i].bk, kGemmCfgs[i].kg>
#define HI_GEMM_CFG(i, q)                                                                                      \
  if constexpr (gemm_cfg_ok(i, q)) {                                                                           \
    if (cfg == i && q8 == q)                                                                                   \
      return gemm_launch<kGemmCfgs[i].bm, kGemmCfgs[i].bn, kGemmCfgs[i].wm, kGemmCfgs[i].wn, kGemmCfgs[i].st, EPI, \
                         q, kGemmCfgs[i].bk, kGemmCfgs[i].kg>(g, cfg, splits, s);                              \
  }
#define HI_GEMM_OCC(i)                                                                                         \
  if constexpr (gemm_cfg_ok(i, true))                                                                          \
    if (cfg == i && q8)                                                                                        \
      return hi_blocks_per_cu(reinterpret_cast<const void*>(&HI_GEMM_K(i, true)),                              \
                              64 * kGemmCfgs[i].wm * kGemmCfgs[i].wn * kGemmCfgs[i].kg, gemm_lds_bytes(i, true)); \
  if constexpr (gemm_cfg_ok(i, false))                                                                         \
    if (cfg == i && !q8)                                                                                       \
      return hi_blocks_per_cu(reinterpret_cast<const void*>(&HI_GEMM_K(i, false)),                             \
                              64 * kGemmCfgs[i].wm * kGemmCfgs[i].wn * kGemmCfgs[i].kg, gemm_lds_bytes(i, false));
#define HI_GEMM_DEFINE_RUN(EPIV)                                                                               \
  template <>                                                                                                  \
  int gemm_run<EPIV>(const GemmArgs& g, int cfg, int splits, bool q8, hipStream_t s) {                        \
    constexpr int EPI = EPIV;                                                                                  \
    HI_GEMM_CFG(0, false) HI_GEMM_CFG(1, false) HI_GEMM_CFG(2, false) HI_GEMM_CFG(3, false)                    \
    HI_GEMM_CFG(4, false) HI_GEMM_CFG(5, false) HI_GEMM_CFG(6, false) HI_GEMM_CFG(7, false)                    \
    HI_GEMM_CFG(8, false) HI_GEMM_CFG(9, false) HI_GEMM_CFG(10, false) HI_GEMM_CFG(11, false)                  \
    HI_GEMM_CFG(12, false) HI_GEMM_CFG(13, false) HI_GEMM_CFG(14, false) HI_GEMM_CFG(15, false)                \
    HI_GEMM_CFG(16, false) HI_GEMM_CFG(17, false) HI_GEMM_CFG(18, false) HI_GEMM_CFG(19, false)                \
    HI_GEMM_CFG(0, true) HI_GEMM_CFG(1, true) HI_GEMM_CFG(2, true) HI_GEMM_CFG(3, true)                        \
    HI_GEMM_CFG(4, true) HI_GEMM_CFG(5, true) HI_GEMM_CFG(6, true) HI_GEMM_CFG(7, true)                        \
    HI_GEMM_CFG(8, true) HI_GEMM_CFG(9, true) HI_GEMM_CFG(10, true) HI_GEMM_CFG(11, true) HI_GEMM_CFG(12, true) \
    HI_GEMM_CFG(13, true) HI_GEMM_CFG(14, true) HI_GEMM_CFG(15, true) HI_GEMM_CFG(16, true)                   \
    HI_GEMM_CFG(19, true)                                                                                      \
    HI_FAIL("gemm: no kernel for config %d", cfg);                                                             \
  }                                                                                                            \
  template <>                                                                                                  \
  int gemm_blocks_per_cu<EPIV>(int cfg, bool q8) {                                                             \
    constexpr int EPI = EPIV;                                                                                  \
    HI_GEMM_OCC(0) HI_GEMM_OCC(1) HI_GEMM_OCC(2) HI_GEMM_OCC(3) HI_GEMM_OCC(4) HI_GEMM_OCC(5) HI_GEMM_OCC(6)    \
    HI_GEMM_OCC(7) HI_GEMM_OCC(8) HI_GEMM_OCC(9) HI_GEMM_OCC(10) HI_GEMM_OCC(11) HI_GEMM_OCC(12)              \
    HI_GEMM_OCC(13) HI_GEMM_OCC(14) HI_GEMM_OCC(15) HI_GEMM_OCC(16) HI_GEMM_OCC(17) HI_GEMM_OCC(18)            \
    HI_GEMM_OCC(19)                                                                                            \
    return -1;                                                                                                 \
  }
