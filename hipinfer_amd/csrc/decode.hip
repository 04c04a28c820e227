// Decode-step kernels around the GEMVs, behind the reference's C-ABI: split-KV decode attention
// (hi_decode_attn, hi_decode_work_bytes; src/api.cu:643-720, ctypes scripts/hipinfer.py:21-22,30)
// and the greedy argmax (hi_argmax; api.cu:838-840, kernels.cuh:1883-1931). hi_embed (the
// reference's internal embed_kernel, kernels.cuh:1876-1881, called from decode_step api.cu:1900)
// is exported as well so that a caller can assemble a whole decode step from C-ABI calls.
//
// Decode attention, one new token per sequence, for gfx950:
//  * block = (split, kv head, sequence), 4 waves; every block serves all G query heads of its kv
//    head, so the cache is read once per GQA group. A split covers a contiguous run of keys; the
//    number of splits in use is derived on the device from pos[b], so a captured graph stays valid
//    while the context grows;
//  * a wave takes 64-key tiles: the tile's K rows go straight into LDS (1 KB per DMA instruction)
//    and its V rows into registers, all in flight at once (the wave's first tile before anything
//    else), so a tile costs one memory round trip; lane l then owns key t0 + l, reads its K row
//    from LDS and computes the key's logit for every query head in fp32 with the query chunks in
//    scalar registers (scalar loads, the same for every lane; q pre-scaled by log2(e) / sqrt(D),
//    the reference's log2-domain softmax, kernels.cuh:1522);
//  * online softmax per wave (max and sum over the 64 lanes), P.V with each lane owning D / 64
//    output dims and the weights as fp16 key pairs through LDS, the 4 waves merged through LDS;
//  * splits hand their partials (o, m, l) to the last-arriving block of their (sequence, kv head)
//    with agent-coherent (sc1) stores and loads and a relaxed agent-scope counter, which the last
//    block resets: no L2 writeback/invalidate fence (gfx950's agent-scope fence costs several
//    microseconds), and the caller's zeroed work buffer stays zeroed, as the reference requires
//    (api.cu:648-650).
#include <type_traits>

#include "hi_common.h"
#include "hi_internal.h"

#ifndef HI_DA_WAVES
#define HI_DA_WAVES 4
#endif

namespace {

constexpr int kDecodeCounters = 4096;  // as api.cu:651: counters at a fixed offset, then partials
constexpr int kDecodeMaxSplits = 64;
constexpr int kDaTile = 64;  // keys per wave tile (one per lane)
constexpr int kDaWaves = HI_DA_WAVES;  // waves per block

__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS of one block: the waves' K tiles and softmax weights while the keys stream, then (after a
// barrier) the waves' partial results and the split merge's tables in the same bytes.
template <int G, int D, int NWV>
struct DaSmem {
  static constexpr int CPR = D / 8;
  struct Loop {
    u32x4 ks[NWV][kDaTile * CPR];      // K tile, chunk c of row r at slot c ^ (r % CPR)
    uint32_t ps[NWV][G][kDaTile / 2];  // softmax weights, fp16 pairs of keys
  };
  struct Merge {
    float wo[NWV][G][D];
    float sm[G][kDecodeMaxSplits], sw[G][kDecodeMaxSplits];
  };
  union {
    Loop loop;
    Merge merge;
  };
};

template <int G, int D, int NWV>
__global__ void __launch_bounds__(NWV * 64) decode_attn_kernel(const f16* __restrict__ q, int ldq,
                                                               const f16* __restrict__ kc, const f16* __restrict__ vc,
                                                               int max_seq, int Hkv, const int* __restrict__ pos,
                                                               float* part, int* counters, int S, f16* __restrict__ out,
                                                               int ldo, float scale_log2, int kv_slot) {
  constexpr int DPL = D / 64;        // output dims per lane
  constexpr int CPR = D / 8;         // 16-byte chunks of a K row
  constexpr int RPI = 64 / CPR;      // K rows per 1 KB DMA instruction
  constexpr int BK = NWV * kDaTile;  // keys per block pass
  constexpr int NT = NWV * 64;
  __shared__ DaSmem<G, D, NWV> sh;
  __shared__ float wm[NWV][G], wl[NWV][G];
  __shared__ int is_last;
  // blocks in split-major order: the splits a sequence uses (split < S_eff) come first in dispatch
  // order, so they spread over the CUs instead of sharing them with blocks that exit at once
  const int nhb = gridDim.x / S;  // (sequence, kv head) pairs
  const int split = blockIdx.x / nhb, hk = blockIdx.x % Hkv, b = (blockIdx.x % nhb) / Hkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int Hq = Hkv * G;
  const int len = min(pos[b] + 1, max_seq);
  const int S_eff = min(S, (len + BK - 1) / BK);
  if (split >= S_eff) return;
  const int chunk = (len + S_eff - 1) / S_eff;
  const int start = split * chunk, end = min(len, start + chunk);
  const int64_t cb = kv_slot >= 0 ? kv_slot : b;
  const f16* Kh = kc + (cb * Hkv + hk) * (int64_t)max_seq * D;
  const f16* Vh = vc + (cb * Hkv + hk) * (int64_t)max_seq * D;
  const __amdgpu_buffer_rsrc_t k_rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(Kh), (short)0, end * D * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(Vh), (short)0, end * D * 2, 0x00020000);

  // a tile's K rows, 1 KB per instruction straight into LDS, swizzled so that the one-key-per-lane
  // reads below are conflict-free; rows at or past the split's end read as zeros through the
  // buffer bounds.
  auto issue_tile = [&](int t0) {
#pragma unroll
    for (int i = 0; i < kDaTile / RPI; i++) {
      const int r = i * RPI + lane / CPR, c = (lane % CPR) ^ (r % CPR);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(k_rs, (__attribute__((address_space(3))) void*)&sh.loop.ks[wave][i * 64],
                                               16, ((t0 + r) * D + 8 * c) * 2, 0, 0, 0);
    }
  };
  const int t_first = start + wave * kDaTile;
  if (t_first < end) issue_tile(t_first);
  // the group's query rows are read in the loop with scalar loads (the same for every lane): no
  // LDS copy, no vector registers, no barrier before a wave's first tile
  const f16* qg = q + (int64_t)b * ldq + hk * G * D;

  float m[G], l[G], o[G][DPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -__builtin_huge_valf();
    l[g] = 0.f;
#pragma unroll
    for (int d = 0; d < DPL; d++) o[g][d] = 0.f;
  }

  for (int t0 = t_first; t0 < end; t0 += BK) {
    // keeps the query loads inside the loop: hoisted, they would need G * D / 2 scalar registers
    asm volatile("" ::: "memory");
    const int n = min(kDaTile, end - t0);
    const bool valid = lane < n;
    if (t0 != t_first) issue_tile(t0);
    // the tile's V rows into registers (lane l: dims l*DPL..), in flight with its K rows
    typedef typename std::conditional<DPL == 2, uint32_t, uint16_t>::type VT;
    VT vv[kDaTile];
#pragma unroll
    for (int jj = 0; jj < kDaTile; jj++) {
      const int off = ((t0 + jj) * D + lane * DPL) * 2;
      if constexpr (DPL == 2) vv[jj] = __builtin_amdgcn_raw_buffer_load_b32(v_rs, off, 0, 0);
      else vv[jj] = __builtin_amdgcn_raw_buffer_load_b16(v_rs, off, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K in LDS, V in registers
    __builtin_amdgcn_wave_barrier();
    u32x4 kv[CPR];
#pragma unroll
    for (int c = 0; c < CPR; c++) kv[c] = sh.loop.ks[wave][lane * CPR + (c ^ (lane % CPR))];

    // logits: fp16 q . fp16 k with exact products and fp32 sums (v_dot2_f32_f16), then the
    // log2(e) / sqrt(D) scale once per logit (the reference's log2-domain softmax, kernels.cuh:1522)
    float s[G];
#pragma unroll
    for (int g = 0; g < G; g++) s[g] = 0.f;
#pragma unroll
    for (int c = 0; c < CPR; c++) {
#pragma unroll
      for (int g = 0; g < G; g++) {
        const u32x4 qv = *reinterpret_cast<const u32x4*>(qg + g * D + 8 * c);
#pragma unroll
        for (int p = 0; p < 4; p++) s[g] = dot2(as_h2(qv[p]), as_h2(kv[c][p]), s[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < G; g++) s[g] *= scale_log2;
    float p_[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float sv = valid ? s[g] : -__builtin_huge_valf();
      const float mn = fmaxf(m[g], wave_max(sv));  // finite: every tile has a valid key
      p_[g] = valid ? exp2f(sv - mn) : 0.f;
      const float a = exp2f(m[g] - mn);  // 0 on the first tile (m = -inf)
      l[g] = l[g] * a + wave_sum(p_[g]);
      m[g] = mn;
#pragma unroll
      for (int d = 0; d < DPL; d++) o[g][d] *= a;
    }
    // P.V: lane l owns dims l*DPL..; the weights go through LDS as fp16 pairs of consecutive keys
    // (the precision of the reference's tensor-core path, which packs P to half for its MMA,
    // kernels.cuh:1455-1460), and each pair of keys meets its two V values per dim in one
    // v_dot2_f32_f16. A wave's LDS accesses complete in order, so its writes are visible to its
    // later reads.
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float hi = __shfl_xor(p_[g], 1, 64);  // the neighbouring key's weight
      if ((lane & 1) == 0) sh.loop.ps[wave][g][lane >> 1] = as_u32(f16x2{(f16)p_[g], (f16)hi});
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j8 = 0; j8 < kDaTile; j8 += 8) {
      if (j8 < n) {  // uniform over the wave; keys past n have p = 0 and V = 0
        u32x4 pw[G];
#pragma unroll
        for (int g = 0; g < G; g++) pw[g] = *reinterpret_cast<const u32x4*>(&sh.loop.ps[wave][g][j8 / 2]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int j = j8 + 2 * k;
          if constexpr (DPL == 2) {
            // (v_j[d0], v_j[d1]), (v_j+1[d0], v_j+1[d1]) -> (v_j[d0], v_j+1[d0]), (v_j[d1], v_j+1[d1])
            const uint32_t a0 = vv[j], a1 = vv[j + 1];
            const f16x2 v0 = as_h2(__builtin_amdgcn_perm(a1, a0, 0x05040100u));
            const f16x2 v1 = as_h2(__builtin_amdgcn_perm(a1, a0, 0x07060302u));
#pragma unroll
            for (int g = 0; g < G; g++) {
              o[g][0] = dot2(as_h2(pw[g][k]), v0, o[g][0]);
              o[g][1] = dot2(as_h2(pw[g][k]), v1, o[g][1]);
            }
          } else {
            const f16x2 v0 = as_h2((uint32_t)vv[j] | ((uint32_t)vv[j + 1] << 16));
#pragma unroll
            for (int g = 0; g < G; g++) o[g][0] = dot2(as_h2(pw[g][k]), v0, o[g][0]);
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the block's waves (a wave without keys has m = -inf and weight 0)
  __syncthreads();  // every wave is done with the loop's LDS before it is reused
#pragma unroll
  for (int g = 0; g < G; g++) {
    if (lane == 0) {
      wm[wave][g] = m[g];
      wl[wave][g] = l[g];
    }
#pragma unroll
    for (int d = 0; d < DPL; d++) sh.merge.wo[wave][g][lane * DPL + d] = o[g][d];
  }
  __syncthreads();
  const bool single = S_eff == 1;
  float* po = part + (int64_t)kDecodeCounters;  // partials follow the counters (floats)
  for (int i = tid; i < G * D; i += NT) {
    const int g = i / D, d = i % D;
    float M = -__builtin_huge_valf();
#pragma unroll
    for (int w = 0; w < NWV; w++) M = fmaxf(M, wm[w][g]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; w++) {
      const float f = wm[w][g] == -__builtin_huge_valf() ? 0.f : exp2f(wm[w][g] - M);
      L = __builtin_fmaf(wl[w][g], f, L);
      O = __builtin_fmaf(sh.merge.wo[w][g][d], f, O);
    }
    if (single) {
      out[(int64_t)b * ldo + (hk * G + g) * D + d] = (f16)(O / L);
    } else {
      const int64_t pi = ((int64_t)b * Hq + hk * G + g) * kDecodeMaxSplits + split;
      st_coherent(po + pi * (D + 2) + d, O);
      if (d == 0) {
        st_coherent(po + pi * (D + 2) + D, M);
        st_coherent(po + pi * (D + 2) + D + 1, L);
      }
    }
  }
  if (single) return;
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this thread's partial stores are complete
  __syncthreads();
  if (tid == 0) {
    int* ctr = counters + b * Hkv + hk;
    const int done = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = done == S_eff - 1;
    if (is_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next launch
  }
  __syncthreads();
  if (!is_last) return;
  // ---- the last block merges the S_eff splits of every head of its group, in split order. The
  //      (m, l) pairs and the first 16 splits' partial outputs are requested in one round; the
  //      split weights exp2(m_s - M) / L are formed once per head while those loads are in flight.
  constexpr int EPT = (G * D + NT - 1) / NT;  // output elements per thread
  float v0[EPT][16];
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    const int i = tid + e * NT;
    const int g = min(i / D, G - 1), d = i % D;
    const float* pp = po + ((int64_t)b * Hq + hk * G + g) * kDecodeMaxSplits * (D + 2) + d;
#pragma unroll
    for (int k = 0; k < 16; k++) v0[e][k] = ld_coherent(pp + (int64_t)min(k, S_eff - 1) * (D + 2));
  }
  for (int i = tid; i < G * S_eff; i += NT) {
    const int g = i / S_eff, s2 = i - g * S_eff;
    const float* pp = po + (((int64_t)b * Hq + hk * G + g) * kDecodeMaxSplits + s2) * (D + 2);
    sh.merge.sm[g][s2] = ld_coherent(pp + D);
    sh.merge.sw[g][s2] = ld_coherent(pp + D + 1);
  }
  __syncthreads();
  for (int g = wave; g < G; g += NWV) {
    float M = -__builtin_huge_valf();
    for (int s2 = lane; s2 < S_eff; s2 += 64) M = fmaxf(M, sh.merge.sm[g][s2]);
    M = wave_max(M);
    float Lp = 0.f;
    for (int s2 = lane; s2 < S_eff; s2 += 64)
      Lp = __builtin_fmaf(sh.merge.sw[g][s2], exp2f(sh.merge.sm[g][s2] - M), Lp);
    const float Lt = wave_sum(Lp);
    for (int s2 = lane; s2 < S_eff; s2 += 64) sh.merge.sw[g][s2] = exp2f(sh.merge.sm[g][s2] - M) / Lt;
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < EPT; e++) {
    const int i = tid + e * NT;
    if (i < G * D) {
      const int g = i / D, d = i % D;
      const float* pp = po + ((int64_t)b * Hq + hk * G + g) * kDecodeMaxSplits * (D + 2) + d;
      float O = 0.f;
#pragma unroll
      for (int k = 0; k < 16; k++) O = __builtin_fmaf(v0[e][k], k < S_eff ? sh.merge.sw[g][k] : 0.f, O);
      for (int s0 = 16; s0 < S_eff; s0 += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = ld_coherent(pp + (int64_t)min(s0 + k, S_eff - 1) * (D + 2));
#pragma unroll
        for (int k = 0; k < 16; k++) O = __builtin_fmaf(v[k], s0 + k < S_eff ? sh.merge.sw[g][s0 + k] : 0.f, O);
      }
      out[(int64_t)b * ldo + (hk * G + g) * D + d] = (f16)O;
    }
  }
}

// Splits per (sequence, kv head): enough blocks for two per CU (as api.cu:643-646), at most 64;
// the kernel uses min(S, ceil(len / 256)) of them.
int decode_splits(int B, int Hkv, int cus) {
  const int S = (2 * cus + B * Hkv - 1) / (B * Hkv);
  return S < 1 ? 1 : S > kDecodeMaxSplits ? kDecodeMaxSplits : S;
}

template <int D>
int decode_attn_d(int G, dim3 grid, hipStream_t s, const f16* q, int ldq, const f16* kc, const f16* vc, int max_seq,
                  int Hkv, const int* pos, float* part, int* counters, int S, f16* out, int ldo, float sl2,
                  int kv_slot) {
#define HI_DA(g)                                                                                                      \
  case g:                                                                                                             \
    hipLaunchKernelGGL((decode_attn_kernel<g, D, kDaWaves>), grid, dim3(kDaWaves * 64), 0, s, q, ldq, kc, vc, max_seq, \
                       Hkv, pos, part, counters, S, out, ldo, sl2, kv_slot);                                          \
    break;
  switch (G) {
    HI_DA(1) HI_DA(2) HI_DA(3) HI_DA(4) HI_DA(5) HI_DA(6) HI_DA(7) HI_DA(8)
    default: HI_FAIL("hi_decode_attn: unsupported GQA group %d (1..8)", G);
  }
#undef HI_DA
  HI_TRY(hipGetLastError());
  return 0;
}

// ---- greedy argmax: largest logit, NaN above every number, lowest index on ties; a row of -inf
//      gives 0 (kernels.cuh:1883-1931)
__device__ __forceinline__ bool argmax_better(float v, int i, float best, int bi) {
  const bool vn = v != v, bn = best != best;
  if (vn != bn) return vn;
  return (vn || v == best) ? i < bi : v > best;
}

constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxLoads = 16;
__global__ void __launch_bounds__(kArgmaxThreads) argmax_kernel(const f16* __restrict__ logits, int V,
                                                                int* __restrict__ tok_out) {
  __shared__ float bv[kArgmaxThreads / 64];
  __shared__ int bi[kArgmaxThreads / 64];
  const f16* row = logits + (int64_t)blockIdx.x * V;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float best = -__builtin_huge_valf();
  int idx = 0;
  auto scan = [&](int i) {  // one logit by the exact rule
    const float v = (float)row[i];
    if (argmax_better(v, i, best, idx)) { best = v; idx = i; }
  };
  if (((uintptr_t)row & 15) == 0) {  // 8 logits per 16-byte chunk, then the tail
    // Thread t takes chunks t, t + kArgmaxThreads, ..., issuing up to kArgmaxLoads loads before
    // looking at any (a 128K vocabulary row in one round trip). Per chunk, packed fp16 max and
    // add only: the chunk's max against the thread's best (strictly greater replaces it, so the
    // thread keeps its lowest chunk holding its max), and a running sum that turns NaN if any
    // logit is NaN (or, harmlessly, if +inf and -inf overflow meet). Afterwards the thread finds
    // its index inside that chunk (reloaded from L2; keeping its words in registers measured no
    // faster); a thread whose sum is NaN rescans its chunks by the exact rule.
    const int V8 = V / 8;
    f16 cbest = (f16)(-__builtin_huge_valf());
    int cidx = tid < V8 ? tid : -1;
    f16x2 nsum = {(f16)0.f, (f16)0.f};
    for (int c0 = tid; c0 < V8; c0 += kArgmaxThreads * kArgmaxLoads) {
      u32x4 v[kArgmaxLoads];
#pragma unroll
      for (int u = 0; u < kArgmaxLoads; u++) {
        const int c = c0 + u * kArgmaxThreads;
        v[u] = c < V8 ? *reinterpret_cast<const u32x4*>(row + 8 * c) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < kArgmaxLoads; u++) {
        const int c = c0 + u * kArgmaxThreads;
        if (c < V8) {
          const f16x2 x0 = as_h2(v[u][0]), x1 = as_h2(v[u][1]), x2 = as_h2(v[u][2]), x3 = as_h2(v[u][3]);
          const f16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(x0, x1), __builtin_elementwise_max(x2, x3));
          const f16 cm = m.x > m.y ? m.x : m.y;
          nsum += (x0 + x1) + (x2 + x3);
          if (cm > cbest) {
            cbest = cm;
            cidx = c;
          }
        }
      }
    }
    if (nsum.x != nsum.x || nsum.y != nsum.y) {
      for (int c = tid; c < V8; c += kArgmaxThreads)
        for (int i = 8 * c; i < 8 * c + 8; i++) scan(i);
    } else if (cidx >= 0) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(row + 8 * cidx);
      best = (float)cbest;
      idx = 8 * cidx + 7;
#pragma unroll
      for (int e = 7; e >= 0; e--)  // the first logit equal to the chunk's max (-0 equals +0)
        if ((float)as_h2(w[e >> 1])[e & 1] == best) idx = 8 * cidx + e;
    }
    for (int i = 8 * V8 + tid; i < V; i += kArgmaxThreads) scan(i);
  } else {
    for (int i = tid; i < V; i += kArgmaxThreads) scan(i);
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (argmax_better(ov, oi, best, idx)) { best = ov; idx = oi; }
  }
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; w++)
      if (argmax_better(bv[w], bi[w], best, idx)) { best = bv[w]; idx = bi[w]; }
    tok_out[blockIdx.x] = idx;
  }
}

// ---- embedding rows: x[b] = table[tok[b]] (H halves), 16 bytes per thread
__global__ void __launch_bounds__(256) embed_kernel(const int* __restrict__ tok, const f16* __restrict__ table, int V,
                                                    int H, f16* __restrict__ x, int64_t ldx) {
  const int b = blockIdx.x;
  const int t = tok[b];
  if (t < 0 || t >= V) return;  // an id outside the vocabulary leaves the row untouched
  const u32x4* src = reinterpret_cast<const u32x4*>(table + (int64_t)t * H);
  u32x4* dst = reinterpret_cast<u32x4*>(x + (int64_t)b * ldx);
  for (int i = threadIdx.x; i < H / 8; i += blockDim.x) dst[i] = src[i];
}

}  // namespace

// Work bytes for hi_decode_attn (as api.cu:651-655): 4096 int counters the caller zeroes once (the
// kernel leaves them zeroed), then B * Hq * 64 * (D + 2) fp32 partials.
HI_EXPORT size_t hi_decode_work_bytes(int B, int Hq, int Hkv, int D) {
  (void)Hkv;
  return (size_t)kDecodeCounters * 4 + (size_t)(B > 0 ? B : 0) * (Hq > 0 ? Hq : 0) * kDecodeMaxSplits * (D + 2) * 4;
}

static int decode_attn_run(const void* q, int ldq, const void* kc, const void* vc, int max_seq, const int* pos,
                           void* out, int ldo, int B, int Hq, int Hkv, int D, void* work, int kv_slot, void* s,
                           const char* who) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  if (D != 64 && D != 128) HI_FAIL("%s: head dim %d (64 or 128)", who, D);
  if (B < 0 || Hkv < 1 || Hq < Hkv || Hq % Hkv || Hq / Hkv > 8 || max_seq < 1)
    HI_FAIL("%s: B %d, Hq %d, Hkv %d (Hq / Hkv in 1..8), max_seq %d", who, B, Hq, Hkv, max_seq);
  if (B == 0) return 0;
  if ((int64_t)max_seq * D * 2 > INT32_MAX)  // a head's cache rows are addressed by 32-bit byte offsets
    HI_FAIL("%s: max_seq %d too long for 32-bit cache offsets (at most %d at D=%d)", who, max_seq,
            (int)(INT32_MAX / (2 * D)), D);
  if (B * Hkv > kDecodeCounters) HI_FAIL("%s: B*Hkv %d > %d", who, B * Hkv, kDecodeCounters);
  if (!q || !kc || !vc || !pos || !out || !work) HI_FAIL("%s: null pointer", who);
  if (((uintptr_t)q & 15) || ldq % 8 || ((uintptr_t)kc & 15) || ((uintptr_t)vc & 15) || ((uintptr_t)work & 3) ||
      (((uintptr_t)out) & 1))
    HI_FAIL("%s: q, kc and vc must be 16-byte aligned and ldq a multiple of 8", who);
  if (ldq < Hq * D || ldo < Hq * D) HI_FAIL("%s: ldq %d / ldo %d < Hq * D = %d", who, ldq, ldo, Hq * D);
  // one sequence (kv_slot >= 0): a batch of one's split count, so every row matches that decode
  const int S = decode_splits(kv_slot >= 0 ? 1 : B, Hkv, d->cus);
  const float sl2 = 1.4426950408889634f / sqrtf((float)D);
  const dim3 grid(S * Hkv * B);  // split-major: (split, sequence, kv head)
  int* counters = (int*)work;
  float* part = (float*)work;
  const hipStream_t st = (hipStream_t)s;
  if (D == 64)
    return decode_attn_d<64>(Hq / Hkv, grid, st, (const f16*)q, ldq, (const f16*)kc, (const f16*)vc, max_seq, Hkv, pos,
                             part, counters, S, (f16*)out, ldo, sl2, kv_slot);
  return decode_attn_d<128>(Hq / Hkv, grid, st, (const f16*)q, ldq, (const f16*)kc, (const f16*)vc, max_seq, Hkv, pos,
                            part, counters, S, (f16*)out, ldo, sl2, kv_slot);
}

// out[b, h*D : (h+1)*D] = softmax(q_h . K[0..pos[b]] / sqrt(D)) V for every query head h of
// sequence b, K/V read from cache slot b ([slots][Hkv][max_seq][D] fp16), the kv head of h being
// h / (Hq / Hkv). work: hi_decode_work_bytes(B, Hq, Hkv, D) bytes, zeroed once by the caller.
HI_EXPORT int hi_decode_attn(const void* q, int ldq, const void* kc, const void* vc, int max_seq, const int* pos,
                             void* out, int ldo, int B, int Hq, int Hkv, int D, void* work, void* s) {
  return decode_attn_run(q, ldq, kc, vc, max_seq, pos, out, ldo, B, Hq, Hkv, D, work, -1, s, "hi_decode_attn");
}

int decode_attn_slot(const void* q, int ldq, const void* kc, const void* vc, int max_seq, const int* pos, void* out,
                     int ldo, int R, int Hq, int Hkv, int D, void* work, int kv_slot, hipStream_t s) {
  if (kv_slot < 0) HI_FAIL("decode_attn_slot: kv_slot %d < 0", kv_slot);
  return decode_attn_run(q, ldq, kc, vc, max_seq, pos, out, ldo, R, Hq, Hkv, D, work, kv_slot, s, "decode_attn_slot");
}

// tok_out[b] = argmax of logits[b, 0:V] (fp16): NaN ranks above every number, ties go to the
// lowest index, an all -inf row gives 0 (api.cu:838-840).
HI_EXPORT int hi_argmax(const void* logits, int B, int V, int* tok_out, void* s) {
  if (!hi_device()) return -2;
  if (B < 0 || V < 1) HI_FAIL("hi_argmax: B %d, V %d", B, V);
  if (B == 0) return 0;
  if (!logits || !tok_out || ((uintptr_t)logits & 1)) HI_FAIL("hi_argmax: null or misaligned pointer");
  hipLaunchKernelGGL(argmax_kernel, dim3(B), dim3(kArgmaxThreads), 0, (hipStream_t)s, (const f16*)logits, V, tok_out);
  HI_TRY(hipGetLastError());
  return 0;
}

// x[b, 0:H] = table[tok[b], 0:H] for b < B (no reference export: the reference's engine runs its
// embed_kernel internally). Token ids outside [0, V) leave the row untouched.
HI_EXPORT int hi_embed(const int* tok, const void* table, int V, int H, void* x, int ldx, int B, void* s) {
  if (!hi_device()) return -2;
  if (B < 0 || V < 1 || H < 8 || H % 8 || ldx % 8 || ldx < H) HI_FAIL("hi_embed: B %d V %d H %d ldx %d", B, V, H, ldx);
  if (B == 0) return 0;
  if (!tok || !table || !x || ((uintptr_t)table & 15) || ((uintptr_t)x & 15))
    HI_FAIL("hi_embed: null pointer or table / x not 16-byte aligned");
  hipLaunchKernelGGL(embed_kernel, dim3(B), dim3(256), 0, (hipStream_t)s, tok, (const f16*)table, V, H, (f16*)x,
                     (int64_t)ldx);
  HI_TRY(hipGetLastError());
  return 0;
}
