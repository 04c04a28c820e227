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

template <int MR, bool NORM, int EPI, int WF>
__global__ void __launch_bounds__(kGemvThreads) gemv_kernel(GemvArgs a) {
  constexpr int NR = EPI >= 2 ? 2 : 1;                  // weight rows per output unit
  constexpr int WPL = WF == WF_I8 ? 16 : 8;             // weights per load
  constexpr int XPL = WPL / 8;                          // 16-byte activation chunks per load
  constexpr int WB = WF == WF_F16 ? 16 : WPL;           // bytes per load
  constexpr int U = 8 / NR;                             // loads per row per step (128 B per lane)
  constexpr int XC = MR <= 8 ? (MR <= 4 ? 4 / MR : 1) : 0;  // activation chunks per row held in registers
  typedef typename WLoad<WF>::T LT;
  extern __shared__ u32x4 xs[];                         // [MR][K / 8] activation chunks
  __shared__ float red[kGemvWaves][MR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = a.K, K8 = K >> 3, M = a.M;
  const int n_units = EPI >= 2 ? a.N / 2 : a.N;
  const int nload = K / WPL;
  const int64_t row_bytes = (int64_t)K * (WF == WF_F16 ? 2 : 1);
  const char* Wb = reinterpret_cast<const char*>(a.W);
  const int nw = gridDim.x * kGemvWaves;

  auto unit_rows = [&](int u, int (&rows)[NR]) {
    if constexpr (EPI <= 1) {
      rows[0] = u;
    } else if constexpr (EPI == 2) {  // gate/up interleaved in groups of 16 rows
      rows[0] = (u >> 4) * 32 + (u & 15);
      rows[NR - 1] = rows[0] + 16;
    } else {  // rows d and d + D/2 of one head
      const int HD = a.D >> 1;
      rows[0] = (u / HD) * a.D + u % HD;
      rows[NR - 1] = rows[0] + HD;
    }
  };
  // One step of a unit: U 16-byte (or 8-byte) chunks of each of its rows, streamed past the
  // caches (nontemporal: the weights are read exactly once).
  auto load_step = [&](LT (&wv)[NR][U], const int (&rows)[NR], int base) {
#pragma unroll
    for (int i = 0; i < U; i++) {
      const int c = base + i * 64 + lane;
#pragma unroll
      for (int j = 0; j < NR; j++) {
        if (c < nload)
          wv[j][i] = __builtin_nontemporal_load(reinterpret_cast<const LT*>(Wb + rows[j] * row_bytes + (int64_t)c * WB));
        else
          wv[j][i] = LT{};
      }
    }
  };

  // Epilogue inputs of a unit (row scales, residual, bias, RoPE table entry), read right after the
  // unit's first weights so that none of them is a dependent memory round trip at the end of the
  // unit; kept as the raw loaded values. Lane m < M reads those of activation row m.
  struct Pre {
    f16 s0, s1, r, b0, b1;
    f16x2 cs;
  };
  const bool epi_lane = lane < MR && lane < M;
  const int my_pos = (EPI == 3 && epi_lane) ? a.pos[lane] : 0;
  auto load_pre = [&](Pre& pre, int u, const int (&rows)[NR]) {
    if (!epi_lane) return;
    if constexpr (WF != WF_F16) {
      pre.s0 = a.scales[rows[0]];
      pre.s1 = a.scales[rows[NR - 1]];
    }
    if constexpr (EPI == 1) pre.r = a.out[lane * a.ldo + u];
    if constexpr (EPI == 3) {
      const int HD = a.D >> 1;
      if (a.bias) {
        pre.b0 = a.bias[rows[0]];
        pre.b1 = a.bias[rows[NR - 1]];
      }
      pre.cs = a.cs[(int64_t)my_pos * HD + u % HD];
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
  // ---- 2. the first step of this wave's first unit
  LT wv[NR][U];
  int rows[NR];
  Pre pn{};  // the epilogue inputs of the unit whose first step is in flight
  const int u0 = blockIdx.x * kGemvWaves + wave;
  bool have = u0 < n_units;
  if (have) {
    unit_rows(u0, rows);
    load_step(wv, rows, 0);
    load_pre(pn, u0, rows);
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

  // ---- 4. stream the units; each unit's next-unit prefetch is issued before its reduction
  for (int u = u0; u < n_units; u += nw) {
    const Pre pc = pn;
    float acc[NR][MR];
#pragma unroll
    for (int j = 0; j < NR; j++)
#pragma unroll
      for (int m = 0; m < MR; m++) acc[j][m] = 0.f;

    for (int base = 0; base < nload; base += 64 * U) {
      if (!have) load_step(wv, rows, base);
      have = false;
#pragma unroll
      for (int i = 0; i < U; i++) {
        const int c = base + i * 64 + lane;
        if (c < nload) {
          f16x2 wp[NR][WPL / 2];
#pragma unroll
          for (int j = 0; j < NR; j++) {
            if constexpr (WF == WF_F16) {
#pragma unroll
              for (int p = 0; p < 4; p++) wp[j][p] = as_h2(wv[j][i][p]);
            } else {
#pragma unroll
              for (int p = 0; p < WPL / 4; p++) i8x4_to_f16(wv[j][i][p], wp[j][2 * p], wp[j][2 * p + 1]);
            }
          }
#pragma unroll
          for (int m = 0; m < MR; m++) {
#pragma unroll
            for (int t = 0; t < XPL; t++) {
              const u32x4 xv = xs[m * K8 + c * XPL + t];
#pragma unroll
              for (int p = 0; p < 4; p++) {
                const f16x2 xp = as_h2(xv[p]);
#pragma unroll
                for (int j = 0; j < NR; j++) acc[j][m] = dot2(wp[j][4 * t + p], xp, acc[j][m]);
              }
            }
          }
        }
      }
    }

    if (u + nw < n_units) {
      unit_rows(u + nw, rows);
      load_step(wv, rows, 0);
      load_pre(pn, u + nw, rows);
      have = true;
    }

#pragma unroll
    for (int j = 0; j < NR; j++)
#pragma unroll
      for (int m = 0; m < MR; m++) acc[j][m] = wave_sum(acc[j][m]);

    if (epi_lane) {
      float a0 = 0.f, a1 = 0.f;  // this lane's row, selected without dynamic register indexing
#pragma unroll
      for (int m = 0; m < MR; m++)
        if (m == lane) {
          a0 = acc[0][m];
          a1 = acc[NR - 1][m];
        }
      if constexpr (WF != WF_F16) {
        a0 *= (float)pc.s0;  // the row scale applied once to the reduced sum (reference kernels.cuh:261)
        a1 *= (float)pc.s1;
      }
      f16* orow = a.out + lane * a.ldo;
      if constexpr (EPI == 0) {
        orow[u] = (f16)a0;
      } else if constexpr (EPI == 1) {
        orow[u] = pc.r + (f16)a0;  // fp16 add, correctly rounded
      } else if constexpr (EPI == 2) {
        orow[u] = silu_mul(a0, a1);
      } else {
        const int D = a.D, HD = D >> 1, head = u / HD, d = u - head * HD;
        const int p = my_pos;
        const int slot = a.kv_slot >= 0 ? a.kv_slot : a.slot_base + lane;
        if (a.bias) {
          a0 += (float)pc.b0;
          a1 += (float)pc.b1;
        }
        f16 y1 = (f16)a0, y2 = (f16)a1;
        if (head < a.Hq + a.Hkv) rope_pair(y1, y2, pc.cs);
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

// One launch: the grid fills the resident block slots once, every wave taking the same number
// of units (within one), so the fused-norm prologue is paid once per block.
template <int MR, bool NORM, int EPI, int WF>
int gemv_launch(const GemvArgs& a, hipStream_t s) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  const size_t lds = (size_t)MR * a.K * 2;
  const void* fn = reinterpret_cast<const void*>(&gemv_kernel<MR, NORM, EPI, WF>);
  const int bpc = hi_blocks_per_cu(fn, kGemvThreads, lds);
  if (bpc < 0) return -2;
  if (bpc == 0) HI_FAIL("gemv: %zu bytes of activation rows do not fit in LDS", lds);
  const int n_units = EPI >= 2 ? a.N / 2 : a.N;
  const int slots = bpc * d->cus * kGemvWaves;
  const int per_wave = (n_units + slots - 1) / slots;
  const int grid = (n_units + kGemvWaves * per_wave - 1) / (kGemvWaves * per_wave);
  hipLaunchKernelGGL((gemv_kernel<MR, NORM, EPI, WF>), dim3(grid), dim3(kGemvThreads), lds, s, a);
  HI_TRY(hipGetLastError());
  return 0;
}

// Template selection for one epilogue (each epilogue's instances live in their own file).
template <int EPI>
int gemv_run(const GemvArgs& a, int MR, bool norm, int wf, hipStream_t s);

#define HI_GEMV_CASE(mr, nm, wfv) \
  if (MR == mr && norm == nm && wf == wfv) return gemv_launch<mr, nm, EPI, wfv>(a, s);
#define HI_GEMV_WF(mr, nm) HI_GEMV_CASE(mr, nm, WF_F16) HI_GEMV_CASE(mr, nm, WF_I8) HI_GEMV_CASE(mr, nm, WF_I8H)
#define HI_GEMV_DEFINE_RUN(EPIV)                                                                  \
  template <>                                                                                     \
  int gemv_run<EPIV>(const GemvArgs& a, int MR, bool norm, int wf, hipStream_t s) {              \
    constexpr int EPI = EPIV;                                                                     \
    HI_GEMV_WF(1, true) HI_GEMV_WF(2, true) HI_GEMV_WF(4, true) HI_GEMV_WF(8, true)               \
    HI_GEMV_WF(1, false) HI_GEMV_WF(2, false) HI_GEMV_WF(4, false) HI_GEMV_WF(8, false)           \
    HI_GEMV_WF(16, false)                                                                         \
    HI_FAIL("gemv: no kernel for %d rows (norm %d, format %d)", MR, (int)norm, wf);               \
  }
