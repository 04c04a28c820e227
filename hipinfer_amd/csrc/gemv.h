// Decode GEMV for gfx950: out[m, n] (epi) sum_k x[m, k] * W[n, k] for M <= 16 activation rows.
//
// Replaces the reference's gemv_kernel<MR, NORM, EPI, Q8> (src/kernels.cuh:164-281) behind the
// same C-ABI (hi_gemv, hi_gemv_w8, hi_gemv_qkv_rope, hi_gemv_qkv_rope_w8; api.cu:181-230).
//
// Design (weight-bandwidth bound; the activation rows are tiny and live in LDS):
//  * the block stages the M activation rows in LDS once, RMSNorm'd on the way when normw is
//    given (fused prologue, HF rounding order);
//  * each wave owns one output unit at a time (one weight row, or the row pair an epilogue
//    combines) and streams it with 128-bit nontemporal loads (the weights are read once), lane l
//    taking 16-byte chunks l, l+64, ...; the first unit's loads are issued before the activation
//    prologue and every next unit's before the current unit's reduction, so the prologue and the
//    reductions hide under weight traffic; a unit's epilogue inputs (row scales, residual, bias,
//    RoPE table entry) are read right after its first weights, so the epilogue waits for no
//    dependent memory round trip;
//  * int8 chunks are unpacked to exact fp16 in registers (v_perm_b32 + one packed fp16 sub per
//    two weights) and every pair of weights meets its activation pair in one v_dot2_f32_f16
//    (fp32 accumulate);
//  * a fixed DPP/swizzle butterfly reduces each row over the wave; the int8 row scale is applied
//    once to the reduced sum, then the epilogue runs on lane m for activation row m.
// A row's arithmetic never depends on M, the unit schedule or the grid: row m of an M-row GEMV is
// bit-identical to the 1-row GEMV of that row (the reference's promise, api.cu:153-155, that
// speculative verification relies on).
#pragma once
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
};

template <int WF> struct WLoad { typedef u32x4 T; };
template <> struct WLoad<WF_I8H> { typedef u32x2 T; };

constexpr int kGemvThreads = 512;              // 8 waves per block
constexpr int kGemvWaves = kGemvThreads / kWave;

template <int MR, bool NORM, int EPI, int WF, int G>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(GemvArgs a) {
  constexpr int NR = EPI >= 2 ? 2 : 1;                  // weight rows per output unit
  constexpr int R = NR * G;                             // weight rows per item (G consecutive units)
  constexpr int WPL = WF == WF_I8 ? 16 : 8;             // weights per load
  constexpr int XPL = WPL / 8;                          // 16-byte activation chunks per load
  constexpr int WB = WF == WF_F16 ? 16 : WPL;           // bytes per load
  constexpr int U = R >= 8 ? 1 : 8 / R;                 // loads per row per step (8 per lane in flight)
  constexpr int XC = MR <= 8 ? (MR <= 4 ? 4 / MR : 1) : 0;  // activation chunks per row held in registers
  typedef typename WLoad<WF>::T LT;
  extern __shared__ u32x4 xs[];                         // [MR][K / 8] activation chunks
  __shared__ float red[kGemvWaves][MR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = a.K, K8 = K >> 3, M = a.M;
  const int n_units = EPI >= 2 ? a.N / 2 : a.N;
  const int n_items = (n_units + G - 1) / G;
  const int nload = K / WPL;
  const int64_t row_bytes = (int64_t)K * (WF == WF_F16 ? 2 : 1);
  const char* Wb = reinterpret_cast<const char*>(a.W);
  const int nw = gridDim.x * kGemvWaves;

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
  // One step of an item: U 16-byte (or 8-byte) chunks of each of its rows, streamed past the
  // caches (nontemporal: the weights are read exactly once).
  auto load_step = [&](LT (&wv)[R][U], const int (&rows)[R], int base) {
#pragma unroll
    for (int i = 0; i < U; i++) {
      const int c = base + i * 64 + lane;
#pragma unroll
      for (int j = 0; j < R; j++) {
        if (c < nload)
          wv[j][i] = __builtin_nontemporal_load(reinterpret_cast<const LT*>(Wb + rows[j] * row_bytes + (int64_t)c * WB));
        else
          wv[j][i] = LT{};
      }
    }
  };

  // Epilogue inputs of an item's units (row scales, residual, bias, RoPE table entry), read right
  // after the item's first weights so that none of them is a dependent memory round trip at the
  // end of the item; kept as the raw loaded values. Lane m < M reads those of activation row m.
  struct Pre {
    f16 s0, s1, r, b0, b1;
    f16x2 cs;
  };
  const bool epi_lane = lane < MR && lane < M;
  const int my_pos = (EPI == 3 && epi_lane) ? a.pos[lane] : 0;
  auto load_pre = [&](Pre (&pre)[G], int t, const int (&rows)[R]) {
    if (!epi_lane) return;
#pragma unroll
    for (int g = 0; g < G; g++) {
      const int u = min(t * G + g, n_units - 1);
      if constexpr (WF != WF_F16) {
        pre[g].s0 = a.scales[rows[g * NR]];
        pre[g].s1 = a.scales[rows[g * NR + NR - 1]];
      }
      if constexpr (EPI == 1) pre[g].r = a.out[lane * a.ldo + u];
      if constexpr (EPI == 3) {
        const int HD = a.D >> 1;
        if (a.bias) {
          pre[g].b0 = a.bias[rows[g * NR]];
          pre[g].b1 = a.bias[rows[g * NR + NR - 1]];
        }
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
  LT wv[R][U];
  int rows[R];
  Pre pn[G] = {};  // the epilogue inputs of the item whose first step is in flight
  const int t0 = blockIdx.x * kGemvWaves + wave;
  bool have = t0 < n_items;
  if (have) {
    item_rows(t0, rows);
    load_step(wv, rows, 0);
    load_pre(pn, t0, rows);
  }
  // ---- 3. stage the activation rows in LDS, RMSNorm'd (HF order) when normw is given; rows >= M
  //         are zero so no garbage reaches the sums
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
#pragma unroll
    for (int m = 0; m < MR; m++) ss[m] = wave_sum(ss[m]);
    if (lane == 0) {
#pragma unroll
      for (int m = 0; m < MR; m++) red[wave][m] = ss[m];
    }
    __syncthreads();
    float r[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < kGemvWaves; w++) tot += red[w][m];
      r[m] = 1.0f / __builtin_sqrtf(tot / (float)K + a.eps);
    }
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
          for (int m = 0; m < MR; m++) xs[m * K8 + c] = m < M ? norm_chunk(xr[m][j], nr[j], r[m]) : u32x4{0u, 0u, 0u, 0u};
        }
      }
    } else {
      for (int c = tid; c < K8; c += kGemvThreads) {
        const u32x4 wn = *reinterpret_cast<const u32x4*>(a.normw + 8 * c);
#pragma unroll
        for (int m = 0; m < MR; m++)
          xs[m * K8 + c] = m < M ? norm_chunk(*reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * c), wn, r[m])
                                 : u32x4{0u, 0u, 0u, 0u};
      }
    }
  } else {
    if (xreg) {
#pragma unroll
      for (int j = 0; j < XC; j++) {
        const int c = tid + j * kGemvThreads;
        if (c < K8) {
#pragma unroll
          for (int m = 0; m < MR; m++) xs[m * K8 + c] = xr[m][j];
        }
      }
    } else {
      for (int i = tid; i < MR * K8; i += kGemvThreads) {
        const int m = i / K8, c = i - m * K8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (m < M) v = *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + 8 * c);
        xs[i] = v;
      }
    }
  }
  __syncthreads();

  // ---- 4. stream the items; each item's next-item prefetch is issued before its reduction.
  //         Every activation chunk read from LDS feeds all R rows of the item, and each row's
  //         products are summed in the same order for every G, so G never changes a result.
  for (int t = t0; t < n_items; t += nw) {
    Pre pc[G];
#pragma unroll
    for (int g = 0; g < G; g++) pc[g] = pn[g];
    float acc[R][MR];
#pragma unroll
    for (int j = 0; j < R; j++)
#pragma unroll
      for (int m = 0; m < MR; m++) acc[j][m] = 0.f;

    for (int base = 0; base < nload; base += 64 * U) {
      if (!have) load_step(wv, rows, base);
      have = false;
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
                for (int p = 0; p < 4; p++) w4[p] = as_h2(wv[j][i][p]);
              } else {
                i8x4_to_f16(wv[j][i][2 * q], w4[0], w4[1]);
                i8x4_to_f16(wv[j][i][2 * q + 1], w4[2], w4[3]);
              }
#pragma unroll
              for (int m = 0; m < MR; m++)
#pragma unroll
                for (int p = 0; p < 4; p++) acc[j][m] = dot2(w4[p], as_h2(xv[m][p]), acc[j][m]);
            }
          }
        }
      }
    }

    if (t + nw < n_items) {
      item_rows(t + nw, rows);
      load_step(wv, rows, 0);
      load_pre(pn, t + nw, rows);
      have = true;
    }

#pragma unroll
    for (int j = 0; j < R; j++)
#pragma unroll
      for (int m = 0; m < MR; m++) acc[j][m] = wave_sum(acc[j][m]);

    if (epi_lane) {
#pragma unroll
      for (int g = 0; g < G; g++) {
        const int u = t * G + g;
        if (u >= n_units) break;
        float a0 = 0.f, a1 = 0.f;  // this lane's row, selected without dynamic register indexing
#pragma unroll
        for (int m = 0; m < MR; m++)
          if (m == lane) {
            a0 = acc[g * NR][m];
            a1 = acc[g * NR + NR - 1][m];
          }
        if constexpr (WF != WF_F16) {
          a0 *= (float)pc[g].s0;  // the row scale applied once to the reduced sum (reference kernels.cuh:261)
          a1 *= (float)pc[g].s1;
        }
        f16* orow = a.out + lane * a.ldo;
        if constexpr (EPI == 0) {
          orow[u] = (f16)a0;
        } else if constexpr (EPI == 1) {
          orow[u] = pc[g].r + (f16)a0;  // fp16 add, correctly rounded
        } else if constexpr (EPI == 2) {
          orow[u] = silu_mul(a0, a1);
        } else {
          const int D = a.D, HD = D >> 1, head = u / HD, d = u - head * HD;
          const int p = my_pos;
          const int slot = a.kv_slot >= 0 ? a.kv_slot : a.slot_base + lane;
          if (a.bias) {
            a0 += (float)pc[g].b0;
            a1 += (float)pc[g].b1;
          }
          f16 y1 = (f16)a0, y2 = (f16)a1;
          if (head < a.Hq + a.Hkv) rope_pair(y1, y2, pc[g].cs);
          f16* dst;
          if (head < a.Hq) dst = orow + head * D;
          else if (head < a.Hq + a.Hkv) dst = a.kc + (((int64_t)slot * a.Hkv + head - a.Hq) * a.max_seq + p) * D;
          else dst = a.vc + (((int64_t)slot * a.Hkv + head - a.Hq - a.Hkv) * a.max_seq + p) * D;
          dst[d] = y1;
          dst[d + HD] = y2;
        }
      }
    }
  }
}

// One launch: the grid fills the resident block slots once, every wave taking the same number
// of items (within one), so the fused-norm prologue is paid once per block.
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
  const int slots = bpc * d->cus * kGemvWaves;
  const int per_wave = (n_items + slots - 1) / slots;
  int grid = (n_items + kGemvWaves * per_wave - 1) / (kGemvWaves * per_wave);
  // An equal split that would leave CUs idle (items just above the resident slots) gives way to
  // every resident block, the waves taking items in grid stride (counts within one of each other).
  if (grid < d->cus) {
    const int all = (n_items + kGemvWaves - 1) / kGemvWaves;
    grid = all < bpc * d->cus ? all : bpc * d->cus;
  }
  hipLaunchKernelGGL((gemv_kernel<MR, NORM, EPI, WF, G>), dim3(grid), dim3(kGemvThreads), lds, s, a);
  HI_TRY(hipGetLastError());
  return 0;
}

// Units per item. From 4 activation rows on, each 16-byte weight chunk costs M 16-byte activation
// reads from LDS and M x 4 dot products, and a unit's compute stops overlapping its wave's weight
// stream; G one-row units per item share every activation read. Measured on MI355X at M = 8
// (Qwen2.5-1.5B shapes), this pays only for lm_head-sized launches: 2 units per item for fp16
// weights, 4 for int8. Two-row units (SwiGLU, RoPE) and smaller N ran fastest with one unit per
// wave, since the extra accumulators cost resident waves. G never changes a result.
inline int gemv_group(int MR, int epi, int wf, int n_units) {
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
    HI_GEMV_WF(1, true) HI_GEMV_WF(2, true) HI_GEMV_WF(4, true) HI_GEMV_WF(8, true)               \
    HI_GEMV_WF(1, false) HI_GEMV_WF(2, false) HI_GEMV_WF(4, false) HI_GEMV_WF(8, false)           \
    HI_GEMV_WF(16, false)                                                                         \
    if constexpr (EPI <= 1) {                                                                     \
      HI_GEMV_GROUPED(4, true) HI_GEMV_GROUPED(8, true) HI_GEMV_GROUPED(4, false)                 \
      HI_GEMV_GROUPED(8, false) HI_GEMV_GROUPED(16, false)                                        \
    }                                                                                             \
    HI_FAIL("gemv: no kernel for %d rows (norm %d, format %d, group %d)", MR, (int)norm, wf, G);  \
  }
