// Decode GEMV for gfx950: out[m, n] (epi) sum_k x[m, k] * W[n, k] for M <= 16 activation rows.
//
// Replaces the reference's gemv_kernel<MR, NORM, EPI, Q8> (src/kernels.cuh:164-281) behind the
// same C-ABI (hi_gemv, hi_gemv_w8, hi_gemv_qkv_rope, hi_gemv_qkv_rope_w8; api.cu:181-230).
//
// Design (weight-bandwidth bound; the activation rows are tiny and live in LDS):
//  * the block stages the M activation rows in LDS once, RMSNorm'd on the way when normw is
//    given (fused prologue, HF rounding order);
//  * each wave owns one output unit at a time (one weight row, or the row pair an epilogue
//    combines) and streams it with 128-bit nontemporal buffer loads (the weights are read once),
//    lane l taking 16-byte chunks l, l+64, ...; the unit is cut into steps, and two register sets
//    alternate so that the next step (of this unit or the wave's next one) is always in flight
//    while the current one is computed: the first step (the first two for the one-row fp16
//    gate/up and lm_head launches) goes out before the activation prologue, and the wave's memory
//    pipe never idles behind its own compute, reductions or epilogues;
//  * a step's epilogue inputs (row scales, residual, bias, RoPE table entry) travel with its
//    weights, and every memory instruction runs on every path (buffer bounds turn the tails and
//    the step past a wave's last unit into zero reads, dropped stores replace skipped ones), so
//    the compiler's waits stay exact: each stage waits only for the step it computes;
//  * int8 chunks are unpacked to exact fp16 1152 + q in registers (one v_perm_b32 per two
//    weights; each lane's sums start at -1152 times the activation elements it meets, so the
//    offset is never subtracted per weight) and every pair of weights meets its activation pair
//    in one v_dot2_f32_f16 (fp32 accumulate);
//  * a fixed DPP/swizzle butterfly reduces each row over the wave (from 4 sums on, all of an
//    item's rows at once, scattered over the lanes with the same tree); the int8 row scale is
//    applied once to the reduced sum, then the epilogue runs on lane m for activation row m.
// A row's arithmetic never depends on M, the unit schedule or the grid: row m of an M-row GEMV is
// bit-identical to the 1-row GEMV of that row (the reference's promise, api.cu:153-155, that
// speculative verification relies on).
#pragma once
#include <type_traits>

#include "hi_common.h"

// Weight formats: fp16; int8 streamed 16 weights per 16-byte load (K % 16 == 0); int8 streamed
// 8 weights per 8-byte load (K % 16 == 8, where rows are only 8-byte aligned).
enum { WF_F16 = 0, WF_I8 = 1, WF_I8H = 2 };

struct GemvArgs {
  const f16* x;
  int64_t ldx;
  const f16* normw;  // fused RMSNorm weight [K] or nullptr
  float eps;
  const void* W;     // [N, K] fp16 or int8
  const f16* scales; // [N] int8 row scales, or nullptr
  f16* out;
  int64_t ldo;
  int M, N, K;
  // epilogue 3: QKV + bias + RoPE + KV-cache write
  const f16* bias;   // [(Hq + 2 Hkv) D] or nullptr
  const f16x2* cs;   // [max_seq][D/2] (cos, sin)
  const int* pos;    // [M] position of each row (already offset to this launch's first row)
  f16* kc;
  f16* vc;           // caches [slots][Hkv][max_seq][D]
  int max_seq, Hq, Hkv, D, kv_slot, slot_base;
  int ipb;  // items per block per round: waves 0 .. ipb-1 of block b take items b*ipb + wave + r*grid*ipb
};

template <int WF> struct WLoad { typedef u32x4 T; };
template <> struct WLoad<WF_I8H> { typedef u32x2 T; };

constexpr int kGemvThreads = 512;              // 8 waves per block
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kRawBuffer = 0x00020000;         // buffer resource word 3: raw (untyped) 32-bit access
constexpr int kNT = 2;                         // cache policy: nontemporal

template <int WF>
__device__ __forceinline__ typename WLoad<WF>::T load_w(__amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (WF == WF_I8H) return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNT);
  else return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT);
}

template <int MR, bool NORM, int EPI, int WF, int G>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(GemvArgs a) {
  constexpr int NR = EPI >= 2 ? 2 : 1;                  // weight rows per output unit
  constexpr int R = NR * G;                             // weight rows per item (G consecutive units)
  constexpr int WPL = WF == WF_I8 ? 16 : 8;             // weights per load
  constexpr int XPL = WPL / 8;                          // 16-byte activation chunks per load
  constexpr int WB = WF == WF_F16 ? 16 : WPL;           // bytes per load
  // loads per row per step; two steps are in flight at any time. A step is 64 bytes of the item per
  // lane (32 for 8-byte loads), 128 for the SwiGLU launches and 32 for the int8 residual ones:
  // measured on MI355X, launches whose waves stream several items (gate/up) run fastest on the
  // larger steps, launches of about one item per wave (QKV, o, down) on the smaller ones, which
  // overlap more of the item's latency (int8 o / down: 5.24 / 11.32 us against 5.31 / 11.39). From 4
  // activation rows on, the SwiGLU launches take the smaller step too: it frees the registers for a
  // second block per CU (C4 gate/up at 8 rows: fp16 13.6 against 14.7 us, int8 14.4 against 14.7).
  // The one-row plain launch (lm_head: waves stream about 16 items each) takes the larger step:
  // fp16 152.7 against 156.2 us (a step twice as large again: 153.0; int8 79.9 against 80.2).
  constexpr int UN = (EPI == 2 ? (MR >= 4 ? 4 : 8) : (EPI == 0 && MR == 1) ? 8 : (EPI == 1 && WF == WF_I8) ? 2 : 4) *
                     (WF == WF_I8H ? 2 : 1);
  constexpr int U = UN / R > 0 ? UN / R : 1;
  constexpr int SW = 64 * U;                            // chunks of a row per step
  constexpr int XC = MR <= 8 ? (MR <= 4 ? 4 / MR : 1) : 0;  // activation chunks per row held in registers
  typedef typename WLoad<WF>::T LT;
  typedef __amdgpu_buffer_rsrc_t RS;
  constexpr bool BIAS = WF != WF_F16;                    // int8 weights unpacked with an offset (below)
  extern __shared__ u32x4 xs[];                         // [MR][K / 8] activation chunks
  __shared__ float red[kGemvWaves][MR];
  __shared__ float rinv[MR];
  __shared__ float xp[BIAS ? MR : 1][BIAS ? kGemvThreads : 1];  // per staging thread: its chunks' sum

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = a.K, K8 = K >> 3, M = a.M;
  const int n_units = EPI >= 2 ? a.N / 2 : a.N;
  const int n_items = (n_units + G - 1) / G;
  const int nload = K / WPL;
  const int SPI = (nload + SW - 1) / SW;                // steps per item
  const int row_bytes = K * (WF == WF_F16 ? 2 : 1);
  const char* Wb = reinterpret_cast<const char*>(a.W);
  const int nw = gridDim.x * a.ipb;  // items per round

  // The R weight rows of item t: units t*G .. t*G+G-1 (a unit past the end repeats the last one;
  // its results are never stored).
  auto item_rows = [&](int t, int (&rows)[R]) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      const int u = min(t * G + g, n_units - 1);
      if constexpr (EPI <= 1) {
        rows[g] = u;
      } else if constexpr (EPI == 2) {  // gate/up interleaved in groups of 16 rows
        rows[2 * g] = (u >> 4) * 32 + (u & 15);
        rows[2 * g + 1] = rows[2 * g] + 16;
      } else {  // rows d and d + D/2 of one head
        const int HD = a.D >> 1;
        rows[2 * g] = (u / HD) * a.D + u % HD;
        rows[2 * g + 1] = rows[2 * g] + HD;
      }
    }
  };

  // Epilogue inputs of an item's units (row scales, residual, bias, RoPE table entry), requested
  // with the item's weights so that none of them is a dependent memory round trip at the end of
  // the item. Every lane loads (lanes >= M those of row M-1): the same memory instructions run on
  // every path, which keeps the compiler's waits for each step's weights exact.
  struct Pre {
    f16 s0, s1, r, b0, b1;
    f16x2 cs;
  };
  const int lm = min(lane, M - 1);
  const int my_pos = EPI == 3 ? a.pos[lm] : 0;
  // bias reads through a buffer of 0 bytes when there is no bias: zeros, no memory access
  const RS bias_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<f16*>(a.bias), (short)0,
                                                       (EPI == 3 && a.bias) ? a.N * 2 : 0, kRawBuffer);

  // One step of item t (step s: chunks s*SW .. s*SW+SW-1 of each row) and its epilogue inputs.
  // Chunks past the row's end, and every chunk of an item past the last, read as zeros through
  // the buffer bounds without a memory access.
  auto issue = [&](LT (&wv)[R][U], Pre (&pre)[G], int t, int s) {
    int rows[R];
    item_rows(t, rows);
    const int nbytes = t < n_items ? row_bytes : 0;
    RS rs[R];
#pragma unroll
    for (int j = 0; j < R; j++)
      rs[j] = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(Wb + (int64_t)rows[j] * row_bytes), (short)0, nbytes,
                                                kRawBuffer);
#pragma unroll
    for (int i = 0; i < U; i++) {
      const int off = (s * SW + i * 64 + lane) * WB;
#pragma unroll
      for (int j = 0; j < R; j++) wv[j][i] = load_w<WF>(rs[j], off);
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      const int u = min(t * G + g, n_units - 1);
      if constexpr (WF != WF_F16) {
        pre[g].s0 = a.scales[rows[g * NR]];
        pre[g].s1 = NR == 2 ? a.scales[rows[g * NR + NR - 1]] : pre[g].s0;
      }
      if constexpr (EPI == 1) pre[g].r = a.out[lm * a.ldo + u];
      if constexpr (EPI == 3) {
        const int HD = a.D >> 1;
        pre[g].b0 = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(bias_rs, rows[g * NR] * 2, 0, 0));
        pre[g].b1 = __builtin_bit_cast(f16, __builtin_amdgcn_raw_buffer_load_b16(bias_rs, rows[g * NR + NR - 1] * 2, 0, 0));
        pre[g].cs = a.cs[(int64_t)my_pos * HD + u % HD];
      }
    }
  };

  // ---- 1. activation (and norm-weight) chunks into registers, before any weight load, so
  //         their latency overlaps the first weight step's
  const bool xreg = XC > 0 && K8 <= XC * kGemvThreads;
  u32x4 xr[MR][XC > 0 ? XC : 1];
  u32x4 nr[XC > 0 ? XC : 1];
  if (xreg) {
#pragma unroll
    for (int j = 0; j < XC; j++) {
      const int c = tid + j * kGemvThreads;
      if constexpr (NORM) nr[j] = c < K8 ? *reinterpret_cast<const u32x4*>(a.normw + 8 * c) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int m = 0; m < MR; m++)
        xr[m][j] = (c < K8 && m < M) ? *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  // ---- 2. the first step of this wave's first item
  LT wa[R][U], wb[R][U];
  Pre pa[G] = {}, pb[G] = {};
  int t = wave < a.ipb ? blockIdx.x * a.ipb + wave : n_items, s = 0;  // the step in flight in (wa, pa)
  issue(wa, pa, t, 0);
  // The one-row fp16 SwiGLU and plain launches (gate/up, lm_head: waves stream several items)
  // also issue the step after it here, so two steps are in flight through the prologue: measured
  // on MI355X at Llama-3.1-8B shapes, gate/up 36.7 against 37.2 us. The launches that request
  // their whole share in one or two steps (QKV, o, the int8 ones) ran slower that way (fp16 QKV
  // 10.46 against 10.11 us, int8 QKV 8.57 against 7.42): a larger first burst of requests.
  constexpr bool PRE = MR == 1 && WF == WF_F16 && (EPI == 0 || EPI == 2);
  if constexpr (PRE) {
    int t1 = t, s1 = 1;
    if (s1 == SPI) {
      s1 = 0;
      t1 += nw;
    }
    issue(wb, pb, t1, s1);
  }
  // ---- 3. stage the activation rows in LDS, RMSNorm'd (HF order) when normw is given; rows >= M
  //         are zero so no garbage reaches the sums. Thread t stages chunks t, t + 512, ... of
  //         every row, in that order on every path, and (int8) sums each row's chunks as it goes.
  float xsum[BIAS ? MR : 1];
#pragma unroll
  for (int m = 0; m < (BIAS ? MR : 1); m++) xsum[m] = 0.f;
  auto put = [&](int m, int c, u32x4 v) {
    xs[m * K8 + c] = v;
    if constexpr (BIAS) {
      const f16x2 one = {(f16)1.0f, (f16)1.0f};
#pragma unroll
      for (int p = 0; p < 4; p++) xsum[m] = dot2(as_h2(v[p]), one, xsum[m]);
    }
  };
  if constexpr (NORM) {
    float ss[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) ss[m] = 0.f;
    if (xreg) {
#pragma unroll
      for (int j = 0; j < XC; j++)
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
          for (int p = 0; p < 4; p++) {
            const f16x2 h = as_h2(xr[m][j][p]);
            ss[m] = dot2(h, h, ss[m]);
          }
    } else {
      for (int c = tid; c < K8; c += kGemvThreads)
#pragma unroll
        for (int m = 0; m < MR; m++)
          if (m < M) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * c);
#pragma unroll
            for (int p = 0; p < 4; p++) {
              const f16x2 h = as_h2(v[p]);
              ss[m] = dot2(h, h, ss[m]);
            }
          }
    }
    if constexpr (MR >= 4) {  // one scattered reduction: lane m ends with row m's sum
      // (padded with zero sums to a power of 2: each sum keeps wave_sum's tree, so its bits)
      constexpr int MP = pow2_at_least(MR);
      float sp[MP];
#pragma unroll
      for (int m = 0; m < MP; m++) sp[m] = m < MR ? ss[m] : 0.f;
      wave_sum_scatter<MP>(sp, lane);
      if (lane < MR) red[wave][lane] = sp[0];
    } else {
#pragma unroll
      for (int m = 0; m < MR; m++) ss[m] = wave_sum(ss[m]);
      if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MR; m++) red[wave][m] = ss[m];
      }
    }
    __syncthreads();
    // row m's inverse RMS, formed once (thread m) and read by every thread
    if (tid < MR) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < kGemvWaves; w++) tot += red[w][tid];
      rinv[tid] = 1.0f / __builtin_sqrtf(tot / (float)K + a.eps);
    }
    __syncthreads();
    float r[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) r[m] = rinv[m];
    auto norm_chunk = [&](u32x4 v, u32x4 wv_, float rm) {
      u32x4 o;
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const f16x2 xh = as_h2(v[p]), wh = as_h2(wv_[p]);
        f16x2 y;
        y.x = wh.x * (f16)((float)xh.x * rm);  // w * fp16(x * r): fp16 product (HF order)
        y.y = wh.y * (f16)((float)xh.y * rm);
        o[p] = as_u32(y);
      }
      return o;
    };
    if (xreg) {
#pragma unroll
      for (int j = 0; j < XC; j++) {
        const int c = tid + j * kGemvThreads;
        if (c < K8) {
#pragma unroll
          for (int m = 0; m < MR; m++) put(m, c, m < M ? norm_chunk(xr[m][j], nr[j], r[m]) : u32x4{0u, 0u, 0u, 0u});
        }
      }
    } else {
      for (int c = tid; c < K8; c += kGemvThreads) {
        const u32x4 wn = *reinterpret_cast<const u32x4*>(a.normw + 8 * c);
#pragma unroll
        for (int m = 0; m < MR; m++)
          put(m, c, m < M ? norm_chunk(*reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * c), wn, r[m])
                          : u32x4{0u, 0u, 0u, 0u});
      }
    }
  } else {
    if (xreg) {
#pragma unroll
      for (int j = 0; j < XC; j++) {
        const int c = tid + j * kGemvThreads;
        if (c < K8) {
#pragma unroll
          for (int m = 0; m < MR; m++) put(m, c, xr[m][j]);
        }
      }
    } else {
      // SB chunks of every row per thread are loaded together before any is stored, so a long
      // row costs about one memory round trip, not one per chunk (a row's chunks are still put in
      // increasing order)
      constexpr int SB = MR >= 16 ? 2 : 4;
      for (int c0 = tid; c0 < K8; c0 += SB * kGemvThreads) {
        u32x4 v[SB][MR];
#pragma unroll
        for (int i = 0; i < SB; i++) {
          const int c = c0 + i * kGemvThreads;
#pragma unroll
          for (int m = 0; m < MR; m++)
            v[i][m] = (c < K8 && m < M) ? *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * c) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < SB; i++) {
          const int c = c0 + i * kGemvThreads;
          if (c < K8) {
#pragma unroll
            for (int m = 0; m < MR; m++) put(m, c, v[i][m]);
          }
        }
      }
    }
  }
  if constexpr (BIAS) {
#pragma unroll
    for (int m = 0; m < MR; m++) xp[m][tid] = xsum[m];
  }
  __syncthreads();

  // ---- 4. stream the steps: each stage requests the next step (into the other register set)
  //         before computing its own, so a wave always has a step of weights in flight. Every
  //         activation chunk read from LDS feeds all R rows of the item, and each row's products
  //         are summed in the same order for every G and step size, so neither changes a result.
  // int8 rows are unpacked as 1152 + q (one packed fp16 subtraction fewer per two weights), so a
  // lane's sums carry 1152 times the sum of the activation elements it meets (chunks c = lane mod
  // 64 of each row, whatever the step size); they start at minus that, from the partial sums of
  // the staging threads that hold those elements. The offset depends only on the activation row
  // and the lane, so row independence and the one-hot exactness hold as for unbiased sums.
  float x0[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) x0[m] = 0.f;
  if constexpr (BIAS) {
    // staging thread t holds activation chunks t + 512 j: those of lane (t mod 128) / 2 for
    // 16-byte weight loads (two chunks per load), of lane t mod 64 for 8-byte ones; eight threads
    // per lane, summed in thread order
    static_assert(kGemvThreads == 512, "the partial-sum lanes assume 512 staging threads");
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float v = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) v += xp[m][XPL == 2 ? 2 * lane + (i & 1) + 128 * (i >> 1) : lane + 64 * i];
      x0[m] = v * -1152.0f;
    }
  }
  float acc[R][MR];
#pragma unroll
  for (int j = 0; j < R; j++)
#pragma unroll
    for (int m = 0; m < MR; m++) acc[j][m] = x0[m];
  const bool epi_lane = lane < MR && lane < M;
  const int n_out = EPI == 2 ? a.N / 2 : a.N;
  // epilogues 0-2 store through a buffer: lanes without a row write at its end, where the store
  // is dropped, so every lane runs the same store instructions
  const uint32_t out_bytes = (uint32_t)(((int64_t)(M - 1) * a.ldo + n_out) * 2);
  const RS out_rs = __builtin_amdgcn_make_buffer_rsrc(a.out, (short)0, (int)out_bytes, kRawBuffer);

  auto stage = [&](auto issue_next, LT (&cur)[R][U], Pre (&pc)[G], LT (&nxt)[R][U], Pre (&pn)[G]) {
    t = __builtin_amdgcn_readfirstlane(t);  // wave-uniform: keeps every buffer resource in SGPRs
    s = __builtin_amdgcn_readfirstlane(s);
    int tn = t, sn = s + 1;
    if (sn == SPI) {
      sn = 0;
      tn += nw;
    }
    if constexpr (decltype(issue_next)::value) issue(nxt, pn, tn, sn);
    // this step's weights and epilogue inputs: consumed here, on every path (the compute below
    // skips lanes past the row's end), so no load into a register is still pending when the loop
    // comes round and the compiler's waits at the loop head stay exact
#pragma unroll
    for (int j = 0; j < R; j++)
#pragma unroll
      for (int i = 0; i < U; i++) asm volatile("" ::"v"(cur[j][i]));
#pragma unroll
    for (int g = 0; g < G; g++) {
      if constexpr (WF != WF_F16) asm volatile("" ::"v"(pc[g].s0), "v"(pc[g].s1));
      if constexpr (EPI == 1) asm volatile("" ::"v"(pc[g].r));
      if constexpr (EPI == 3) asm volatile("" ::"v"(pc[g].b0), "v"(pc[g].b1), "v"(pc[g].cs));
    }
    const int base = s * SW;
#pragma unroll
    for (int i = 0; i < U; i++) {
      const int c = base + i * 64 + lane;
      if (c < nload) {
#pragma unroll
        for (int q = 0; q < XPL; q++) {
          u32x4 xv[MR];
#pragma unroll
          for (int m = 0; m < MR; m++) xv[m] = xs[m * K8 + c * XPL + q];
#pragma unroll
          for (int j = 0; j < R; j++) {
            f16x2 w4[4];  // the 8 weights of this row that meet activation chunk q
            if constexpr (WF == WF_F16) {
#pragma unroll
              for (int p = 0; p < 4; p++) w4[p] = as_h2(cur[j][i][p]);
            } else {
              i8x4_to_f16_biased(cur[j][i][2 * q], w4[0], w4[1]);
              i8x4_to_f16_biased(cur[j][i][2 * q + 1], w4[2], w4[3]);
            }
#pragma unroll
            for (int m = 0; m < MR; m++)
#pragma unroll
              for (int p = 0; p < 4; p++) acc[j][m] = dot2(w4[p], as_h2(xv[m][p]), acc[j][m]);
          }
        }
      }
    }
    // epilogues 0-2 store on every stage (a dropped store except on an item's last step), so the
    // stages issue the same memory instructions whichever way the branch below goes
    f16 y[G], y2[G];
#pragma unroll
    for (int g = 0; g < G; g++) y[g] = y2[g] = (f16)0.f;
    const bool last = s == SPI - 1;
    if (last) {
      // the R x MR sums over the wave (wave_sum's tree), then each lane's row: from 4 sums on, one
      // scattered reduction of all of them, padded with zero sums to NP, a power of 2 (accumulator
      // j * MR + m ends in lanes l with l % L == (j * MR + m) % L, slot (j * MR) / L) and a lane read
      // per sum the epilogue needs
      constexpr int NA = R * MR, NP = pow2_at_least(NA), L = NP < 16 ? NP : 16;
      float av0[G], av1[G];
      if constexpr (NA >= 4) {
        float v[NP];
#pragma unroll
        for (int j = 0; j < R; j++)
#pragma unroll
          for (int m = 0; m < MR; m++) v[j * MR + m] = acc[j][m];
#pragma unroll
        for (int a = NA; a < NP; a++) v[a] = 0.f;
        wave_sum_scatter<NP>(v, lane);
        // the total of accumulator a0 + lm (this lane's row of the unit whose rows start at a0):
        // lane (a0 + lm) % L of slot (a0 + lm) / L. A unit's MR rows can straddle two slots when MR
        // does not divide L (5 rows); both candidates are read and the lane's own slot kept
        auto row_sum = [&](int a0) {
          const int a = a0 + lm;
          const float s0 = __shfl(v[a0 / L], a % L, kWave);
          if ((a0 + MR - 1) / L == a0 / L) return s0;
          const float s1 = __shfl(v[(a0 + MR - 1) / L], a % L, kWave);
          return a / L == a0 / L ? s0 : s1;
        };
#pragma unroll
        for (int g = 0; g < G; g++) {
          const int j0 = g * NR * MR, j1 = (g * NR + NR - 1) * MR;
          av0[g] = row_sum(j0);
          av1[g] = NR == 2 ? row_sum(j1) : av0[g];
        }
      } else {
#pragma unroll
        for (int j = 0; j < R; j++)
#pragma unroll
          for (int m = 0; m < MR; m++) acc[j][m] = wave_sum(acc[j][m]);
#pragma unroll
        for (int g = 0; g < G; g++) {
          av0[g] = av1[g] = 0.f;  // this lane's row, selected without dynamic register indexing
#pragma unroll
          for (int m = 0; m < MR; m++)
            if (m == lm) {
              av0[g] = acc[g * NR][m];
              av1[g] = acc[g * NR + NR - 1][m];
            }
        }
      }
#pragma unroll
      for (int g = 0; g < G; g++) {
        const int u = t * G + g;
        float a0 = av0[g], a1 = av1[g];
        if constexpr (WF != WF_F16) {
          a0 *= (float)pc[g].s0;  // the row scale applied once to the reduced sum (reference kernels.cuh:261)
          a1 *= (float)pc[g].s1;
          // the fp32 product is rounded before its conversion to fp16 (two roundings, as the
          // reference's fp32 multiply then __float2half): no fused mixed-precision fma
          asm volatile("" : "+v"(a0), "+v"(a1));
        }
        if constexpr (EPI == 0) {
          y[g] = (f16)a0;
        } else if constexpr (EPI == 1) {
          y[g] = pc[g].r + (f16)a0;  // fp16 add, correctly rounded
        } else if constexpr (EPI == 2) {
          y[g] = silu_mul(a0, a1);
        } else {
          if (a.bias) {
            a0 += (float)pc[g].b0;
            a1 += (float)pc[g].b1;
            asm volatile("" : "+v"(a0), "+v"(a1));  // fp32 sum, then fp16: two roundings
          }
          f16 r1 = (f16)a0, r2 = (f16)a1;
          const int HD = a.D >> 1;
          if (min(u, n_units - 1) / HD < a.Hq + a.Hkv) rope_pair(r1, r2, pc[g].cs);
          y[g] = r1;
          y2[g] = r2;
        }
      }
#pragma unroll
      for (int j = 0; j < R; j++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[j][m] = x0[m];
    }
    if constexpr (EPI <= 2) {
#pragma unroll
      for (int g = 0; g < G; g++) {
        const int u = t * G + g;
        const uint32_t off = (last && epi_lane && u < n_units) ? (uint32_t)((lane * a.ldo + u) * 2) : out_bytes;
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, y[g]), out_rs, (int)off, 0, 0);
      }
    } else {
      // q to out[row, head*D + d], k / v to the cache at (slot, kv head, pos, d), through a buffer
      // whose base is uniform (out, or this launch's first slot's kv head in the cache) and which
      // holds no records except on an item's last step. Lanes past the last row repeat that row's
      // stores (same values, same addresses). The host keeps every offset below 4 GB.
#pragma unroll
      for (int g = 0; g < G; g++) {
        const int u = min(t * G + g, n_units - 1);
        const int D = a.D, HD = D >> 1, head = u / HD, d = u - head * HD;
        const f16* base;
        uint32_t off;
        if (head < a.Hq) {
          base = a.out;
          off = (uint32_t)(lm * a.ldo + head * D + d);
        } else {
          const bool isk = head < a.Hq + a.Hkv;
          const int kvh = head - a.Hq - (isk ? 0 : a.Hkv);
          const int sb = a.kv_slot >= 0 ? a.kv_slot : a.slot_base, dl = a.kv_slot >= 0 ? 0 : lm;
          base = (isk ? a.kc : a.vc) + ((int64_t)sb * a.Hkv + kvh) * a.max_seq * D;
          off = (uint32_t)(((int64_t)dl * a.Hkv * a.max_seq + my_pos) * D + d);
        }
        const uint64_t bp = reinterpret_cast<uint64_t>(base);  // wave-uniform: a resource in SGPRs
        const uint32_t blo = __builtin_amdgcn_readfirstlane((uint32_t)bp), bhi = __builtin_amdgcn_readfirstlane((uint32_t)(bp >> 32));
        const RS rs = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<f16*>(((uint64_t)bhi << 32) | blo), (short)0,
                                                        __builtin_amdgcn_readfirstlane(last ? -1 : 0), kRawBuffer);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, y[g]), rs, (int)(off * 2), 0, 0);
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, y2[g]), rs, (int)((off + HD) * 2), 0, 0);
      }
    }
    t = tn;
    s = sn;
  };
  if constexpr (PRE) {
    if (t < n_items) {
      stage(std::false_type{}, wa, pa, wb, pb);  // the step after it is already in flight
      while (t < n_items) {
        stage(std::true_type{}, wb, pb, wa, pa);
        if (t >= n_items) break;
        stage(std::true_type{}, wa, pa, wb, pb);
      }
    }
  } else {
    while (t < n_items) {
      stage(std::true_type{}, wa, pa, wb, pb);
      if (t >= n_items) break;
      stage(std::true_type{}, wb, pb, wa, pa);
    }
  }
}

// One launch of k blocks per CU, each block's first ipb waves taking one item per round, (k, ipb)
// chosen, among those that keep at least min(16, items per CU) items in flight on a CU (8 for the
// lean launches below), so that the CU streaming the most items streams as few as possible
// (blocks b, b + CUs, ... are taken to share a CU), then for the most items in flight (lean: the
// fewest blocks), then for the fewest blocks (each pays the activation staging once). A block's
// waves take consecutive items: its loads stay on neighbouring rows.
template <int MR, bool NORM, int EPI, int WF, int G>
int gemv_launch(const GemvArgs& a, hipStream_t s) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  const size_t lds = (size_t)MR * a.K * 2;
  const void* fn = reinterpret_cast<const void*>(&gemv_kernel<MR, NORM, EPI, WF, G>);
  const int bpc = hi_blocks_per_cu(fn, kGemvThreads, lds);
  if (bpc < 0) return -2;
  if (bpc == 0) HI_FAIL("gemv: %zu bytes of activation rows do not fit in LDS", lds);
  const int n_units = EPI >= 2 ? a.N / 2 : a.N;
  const int n_items = (n_units + G - 1) / G;
  const int cus = d->cus, per_cu = (n_items + cus - 1) / cus;
  // One-row residual launches (o, down) and int8 plain ones (lm_head) run fastest on fewer,
  // fuller blocks: 8 items in flight per CU suffice, and among shapes of equal load the one with
  // the fewest blocks wins (each block stages the activation row once; measured on MI355X at
  // Llama-3.1-8B shapes: fp16 down 19.14-19.25 against 19.25-19.26 us, int8 lm_head 78.5-78.7
  // against 79.6-79.7, the fp16 token 2504 against 2510 us). The one-row int8 QKV launch does the
  // same with 6 in flight, so that each wave streams two row pairs instead of requesting all of
  // its CU's share at once (7.08 against 7.43 us; the fp16 one ran slower that way, 10.30 against
  // 10.12). Other launches keep 16 in flight.
  const bool qkv8 = MR == 1 && EPI == 3 && WF != WF_F16;
  const bool lean = MR == 1 && (EPI == 1 || qkv8 || (EPI == 0 && WF != WF_F16));
  const int need = std::min(std::min(per_cu, qkv8 ? 6 : lean ? 8 : 16), bpc * kGemvWaves);  // items in flight per CU, at least
  int grid = 1, ipb = 1;
  long best_load = -1;
  int best_fly = 0;
  for (int k = 1; k <= bpc; k++)
    for (int w = kGemvWaves; w >= 1; w--) {
      const long nb = n_items < cus ? n_items : (long)k * cus, nw = nb * w;
      const long full = n_items / nw, last_blocks = (n_items - full * nw + w - 1) / w;
      const long load = full * (nb / std::min<long>(nb, cus)) * w + (last_blocks + cus - 1) / cus * w;
      const int fly = (int)std::min<long>((long)k * w, per_cu);
      if (fly < need) continue;
      if (best_load < 0 || load < best_load || (load == best_load && (lean ? nb < grid : fly > best_fly))) {
        best_load = load;
        best_fly = fly;
        grid = (int)nb;
        ipb = w;
      }
    }
  GemvArgs b = a;
  b.ipb = ipb;
  hipLaunchKernelGGL((gemv_kernel<MR, NORM, EPI, WF, G>), dim3(grid), dim3(kGemvThreads), lds, s, b);
  HI_TRY(hipGetLastError());
  return 0;
}

// Units per item. From 4 activation rows on, each 16-byte weight chunk costs M 16-byte activation
// reads from LDS and M x 4 dot products, and a unit's compute stops overlapping its wave's weight
// stream; G one-row units per item share every activation read. Measured on MI355X at M = 8
// (Qwen2.5-1.5B shapes), this pays only for lm_head-sized launches: 2 units per item for fp16
// weights, 4 for int8. Two-row units (SwiGLU, RoPE) and smaller N ran fastest with one unit per
// wave, since the extra accumulators cost resident waves. At one row, two units per item make a
// wave stream two rows side by side, which the memory system serves a little faster than one: the
// fp16 lm_head (128256 x 4096) takes 156.1 against 160.5 us; o and down (4096 rows) ran slower
// (7.59 / 19.88 against 7.29 / 19.37 us) and the int8 lm_head the same. G never changes a result.
inline int gemv_group(int MR, int epi, int wf, int n_units) {
  if (MR == 1) return (epi == 0 && wf == WF_F16 && n_units >= 32768) ? 2 : 1;
  if (MR < 4 || epi >= 2 || wf == WF_I8H || n_units < 32768) return 1;
  const int G = wf == WF_F16 ? 2 : 4;
  return G * MR > (MR >= 16 ? 32 : 64) ? G / 2 : G;  // 16 rows also hold 64 registers of activations
}

// Template selection for one epilogue (each epilogue's instances live in their own file).
template <int EPI>
int gemv_run(const GemvArgs& a, int MR, bool norm, int wf, hipStream_t s);

#define HI_GEMV_CASE(mr, nm, wfv, g) \
  if (MR == (mr) && norm == (nm) && wf == (wfv) && G == (g)) return gemv_launch<(mr), (nm), EPI, (wfv), (g)>(a, s);
#define HI_GEMV_WF(mr, nm) HI_GEMV_CASE(mr, nm, WF_F16, 1) HI_GEMV_CASE(mr, nm, WF_I8, 1) HI_GEMV_CASE(mr, nm, WF_I8H, 1)
#define HI_GEMV_GROUPED(mr, nm) HI_GEMV_CASE(mr, nm, WF_F16, 2) HI_GEMV_CASE(mr, nm, WF_I8, mr >= 16 ? 2 : 4)
#define HI_GEMV_DEFINE_RUN(EPIV)                                                                  \
  template <>                                                                                     \
  int gemv_run<EPIV>(const GemvArgs& a, int MR, bool norm, int wf, hipStream_t s) {              \
    constexpr int EPI = EPIV;                                                                     \
    const int G = gemv_group(MR, EPI, wf, EPI >= 2 ? a.N / 2 : a.N);                              \
    HI_GEMV_WF(1, true) HI_GEMV_WF(2, true) HI_GEMV_WF(3, true) HI_GEMV_WF(4, true)               \
    HI_GEMV_WF(5, true) HI_GEMV_WF(6, true) HI_GEMV_WF(7, true) HI_GEMV_WF(8, true)               \
    HI_GEMV_WF(1, false) HI_GEMV_WF(2, false) HI_GEMV_WF(3, false) HI_GEMV_WF(4, false)           \
    HI_GEMV_WF(5, false) HI_GEMV_WF(6, false) HI_GEMV_WF(7, false) HI_GEMV_WF(8, false)           \
    HI_GEMV_WF(16, false)                                                                         \
    if constexpr (EPI <= 1) {                                                                     \
      HI_GEMV_CASE(1, true, WF_F16, 2) HI_GEMV_CASE(1, false, WF_F16, 2)                          \
      HI_GEMV_GROUPED(4, true) HI_GEMV_GROUPED(5, true) HI_GEMV_GROUPED(6, true)                  \
      HI_GEMV_GROUPED(7, true) HI_GEMV_GROUPED(8, true) HI_GEMV_GROUPED(4, false)                 \
      HI_GEMV_GROUPED(5, false) HI_GEMV_GROUPED(6, false) HI_GEMV_GROUPED(7, false)               \
      HI_GEMV_GROUPED(8, false) HI_GEMV_GROUPED(16, false)                                        \
    }                                                                                             \
    HI_FAIL("gemv: no kernel for %d rows (norm %d, format %d, group %d)", MR, (int)norm, wf, G);  \
  }
