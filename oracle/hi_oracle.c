/* CPU oracle for the hipinfer matmul hot path -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker (or, for cpu_baseline, as the timed CPU restatement of the reference's CPU
 * path). The HIP library never links it.
 *
 * Each function restates one piece of the reference's arithmetic, written from the formulas and
 * rounding points below, not translated from its code:
 *   or_quantize_rows    scripts/export.py:54-68 (docs/quantization.md:24-31)
 *   or_dequantize_rows  scripts/export.py:71-73, src/kernels.cuh:86-94
 *   or_interleave_*     scripts/export.py:97-101, scripts/ref_engine.py:32-36
 *   or_rmsnorm          src/kernels.cuh:182-200 (HF order: w * fp16(x * rsqrt(mean x^2 + eps)))
 *   or_silu_mul         src/kernels.cuh:100-105 = scripts/ref_engine.py:39-42
 *   or_rope_pair        src/kernels.cuh:132-136
 *   or_gemv             src/kernels.cuh:164-281 (epilogues 256-264), int8 scaling kernels.cuh:261;
 *                       CPU reference form tests/test_kernels.py:47-65, 382-407
 *   or_gemv_qkv_rope    src/kernels.cuh:210,265-278 with RopeArgs 139-147
 *   or_gemm             src/kernels.cuh:305-506 (epilogues 454-505, split-K 406-452);
 *                       int8 = fp32 math on fp16(q*s), tests/test_kernels.py:447
 *   or_moe_router       src/kernels.cuh:2091-2147, argmax_better 1886-1890, docs/moe-design.md:186-201
 *   or_moe_experts      src/kernels.cuh:2156-2209 and 2250-2276, scripts/ref_engine.py:60-73
 *   or_decode_attn      src/kernels.cuh:1486-1660 (decode_attn_kernel), api.cu:694-720;
 *                       CPU reference form tests/test_kernels.py:298-307 (ref_attn)
 *   or_argmax           src/kernels.cuh:1883-1931 (argmax_better, block_argmax, argmax_kernel)
 *   or_rope_cache       src/kernels.cuh:1120-1158 (rope_cache_kernel), api.cu:579-586;
 *                       CPU reference form tests/test_kernels.py:230-261 (hf_rope)
 *   or_flash_prefill    src/kernels.cuh:1160-1329 (flash_prefill_kernel), api.cu:594-623;
 *                       CPU reference form tests/test_kernels.py:288-309 (ref_attn, causal on
 *                       absolute positions p0 + t)
 *
 * fp16 conversions are this file's own IEEE binary16 routines (round to nearest even, subnormals,
 * overflow to inf). Accumulation is fp64; the reference accumulates in fp32 in kernel-specific
 * orders, so outputs agree to tolerance, with every fp16 rounding point at the same place.
 * Build with -ffp-contract=off and without -ffast-math (oracle/Makefile). */
#include "hi_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------ fp16 */
uint16_t or_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf, or NaN (quiet, payload kept where it fits) */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: the tie above 65504 goes to inf */
  const uint32_t e = ax >> 23;
  if (e >= 113) { /* normal binary16 (>= 2^-14) */
    uint32_t h = ((e - 112) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* a carry moves into the exponent correctly */
    return (uint16_t)(sign | h);
  }
  if (e < 102) return (uint16_t)sign; /* below 2^-25 (2^-25 itself is a tie that goes to 0) */
  const uint32_t mant = (ax & 0x7fffffu) | 0x800000u, shift = 126 - e; /* subnormal: n * 2^-24 */
  uint32_t n = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (n & 1u))) n++;
  return (uint16_t)(sign | n);
}

float or_h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    const float f = (float)mant * 0x1p-24f; /* exact */
    memcpy(&x, &f, 4);
    x |= sign;
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (mant << 13);
  } else {
    x = sign | ((exp + 112) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void or_f2h_array(const float* f, uint16_t* h, int64_t n) {
  for (int64_t i = 0; i < n; i++) h[i] = or_f2h(f[i]);
}
void or_h2f_array(const uint16_t* h, float* f, int64_t n) {
  for (int64_t i = 0; i < n; i++) f[i] = or_h2f(h[i]);
}
static inline float r16(float f) { return or_h2f(or_f2h(f)); }

void or_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n > 0 ? n : 1);
#else
  (void)n;
#endif
}
int or_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ int8 weight format */
/* s[n] = fp16(fp32(max_k |w| / 127)); q = clamp(round_half_even(fp32(w / s)), -127, 127); q = 0 when s == 0. */
int or_quantize_rows(const uint16_t* w, int64_t N, int64_t K, int8_t* q, uint16_t* s) {
  if (N < 0 || K <= 0) return -1;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    const uint16_t* wr = w + n * K;
    float amax = 0.f;
    for (int64_t k = 0; k < K; k++) {
      const float a = fabsf(or_h2f(wr[k]));
      if (a > amax) amax = a;
    }
    const float sc = amax / 127.0f;
    const uint16_t sh = or_f2h(sc);
    const float sf = or_h2f(sh);
    for (int64_t k = 0; k < K; k++) {
      float v = 0.f;
      if (sf > 0.f) {
        v = nearbyintf(or_h2f(wr[k]) / sf);
        if (v > 127.f) v = 127.f;
        if (v < -127.f) v = -127.f;
      }
      q[n * K + k] = (int8_t)v;
    }
    s[n] = sh;
  }
  return 0;
}

/* fp16(q * s): q * s is exact in fp32 (8 x 11 significant bits), so this is one rounding. */
int or_dequantize_rows(const int8_t* q, const uint16_t* s, int64_t N, int64_t K, uint16_t* out) {
  if (N < 0 || K <= 0) return -1;
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    const float sf = or_h2f(s[n]);
    for (int64_t k = 0; k < K; k++) out[n * K + k] = or_f2h((float)q[n * K + k] * sf);
  }
  return 0;
}

/* [2I, *] rows in groups of 16: rows 32j..32j+15 are gate rows 16j.., rows 32j+16..32j+31 the same up rows. */
int or_interleave_gate_up(const void* g, const void* u, int64_t I, int64_t row_bytes, void* out) {
  if (I % 16 || row_bytes <= 0) return -1;
  const char* gp = (const char*)g;
  const char* up = (const char*)u;
  char* op = (char*)out;
  for (int64_t r = 0; r < 2 * I; r++) {
    const int64_t grp = r / 32, within = r % 32, src = grp * 16 + (within % 16);
    memcpy(op + r * row_bytes, (within < 16 ? gp : up) + src * row_bytes, (size_t)row_bytes);
  }
  return 0;
}
int or_deinterleave_gate_up(const void* gu, int64_t I, int64_t row_bytes, void* g, void* u) {
  if (I % 16 || row_bytes <= 0) return -1;
  const char* ip = (const char*)gu;
  for (int64_t r = 0; r < 2 * I; r++) {
    const int64_t grp = r / 32, within = r % 32, dst = grp * 16 + (within % 16);
    memcpy((char*)(within < 16 ? g : u) + dst * row_bytes, ip + r * row_bytes, (size_t)row_bytes);
  }
  return 0;
}

/* ------------------------------------------------------------------ elementwise pieces */
static void rms_row(const uint16_t* x, const uint16_t* w, int K, float eps, uint16_t* y) {
  double ss = 0.0;
  for (int k = 0; k < K; k++) {
    const double v = or_h2f(x[k]);
    ss += v * v;
  }
  const float r = 1.0f / sqrtf((float)(ss / K) + eps);
  for (int k = 0; k < K; k++) y[k] = or_f2h(or_h2f(w[k]) * r16(or_h2f(x[k]) * r));
}

int or_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* w, int M, int K, float eps, uint16_t* y, int64_t ldy) {
  if (M < 0 || K <= 0) return -1;
  for (int m = 0; m < M; m++) rms_row(x + m * ldx, w, K, eps, y + m * ldy);
  return 0;
}

/* fp16(g); fp16(silu(g)); fp16(silu * fp16(u)) */
uint16_t or_silu_mul(float g, float u) {
  const float gh = r16(g);
  const float sh = r16(gh / (1.0f + expf(-gh)));
  return or_f2h(sh * r16(u));
}

/* y1 = x1 c - x2 s, y2 = x2 c + x1 s, each product and each result rounded to fp16 */
void or_rope_pair(uint16_t x1, uint16_t x2, uint16_t c, uint16_t s, uint16_t* y1, uint16_t* y2) {
  const float cf = or_h2f(c), sf = or_h2f(s), f1 = or_h2f(x1), f2 = or_h2f(x2);
  *y1 = or_f2h(r16(f1 * cf) - r16(f2 * sf));
  *y2 = or_f2h(r16(f2 * cf) + r16(f1 * sf));
}

/* ------------------------------------------------------------------ dot products */
static inline double dot_h(const uint16_t* x, const uint16_t* w, int K) {
  double a = 0.0;
  for (int k = 0; k < K; k++) a += (double)or_h2f(x[k]) * (double)or_h2f(w[k]);
  return a;
}
static inline double dot_q(const uint16_t* x, const int8_t* q, int K) {
  double a = 0.0;
  for (int k = 0; k < K; k++) a += (double)or_h2f(x[k]) * (double)q[k];
  return a;
}

/* Activation rows as the GEMV consumes them: x, or its RMSNorm (fp16) when normw is given. */
static uint16_t* gemv_rows(const uint16_t* x, int64_t ldx, const uint16_t* normw, float eps, int M, int K) {
  uint16_t* xs = (uint16_t*)malloc((size_t)M * K * 2);
  if (!xs) return NULL;
  for (int m = 0; m < M; m++) {
    if (normw) rms_row(x + m * ldx, normw, K, eps, xs + (size_t)m * K);
    else memcpy(xs + (size_t)m * K, x + m * ldx, (size_t)K * 2);
  }
  return xs;
}

/* GEMV row n for activation row m, as fp32: fp16 weights, or (sum q x) * s for int8. */
static inline float gemv_dot(const uint16_t* xm, const void* W, const uint16_t* scales, int64_t n, int K) {
  if (scales) return (float)dot_q(xm, (const int8_t*)W + n * (int64_t)K, K) * or_h2f(scales[n]); /* fp32 sum x fp32 s */
  return (float)dot_h(xm, (const uint16_t*)W + n * (int64_t)K, K);
}

/* out[m, :] (epi) x[m, :] @ W^T. epi 0: store; 1: out = fp16(out + fp16(y)); 2: SwiGLU over rows
 * interleaved in groups of 16 (N/2 outputs). */
int or_gemv(const uint16_t* x, int64_t ldx, const uint16_t* normw, float eps, const void* W, const uint16_t* scales,
            uint16_t* out, int64_t ldo, int M, int N, int K, int epi) {
  if (M < 1 || N < 1 || K < 1 || epi < 0 || epi > 2 || (epi == 2 && N % 32)) return -1;
  uint16_t* xs = gemv_rows(x, ldx, normw, eps, M, K);
  if (!xs) return -1;
  const int n_out = epi == 2 ? N / 2 : N;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < n_out; o++) {
    for (int m = 0; m < M; m++) {
      const uint16_t* xm = xs + (size_t)m * K;
      uint16_t* dst = out + m * ldo + o;
      if (epi == 2) {
        const int64_t r0 = (int64_t)(o / 16) * 32 + o % 16;
        *dst = or_silu_mul(gemv_dot(xm, W, scales, r0, K), gemv_dot(xm, W, scales, r0 + 16, K));
      } else {
        const float y = gemv_dot(xm, W, scales, o, K);
        *dst = epi == 0 ? or_f2h(y) : or_f2h(or_h2f(*dst) + r16(y));
      }
    }
  }
  free(xs);
  return 0;
}

/* Fused QKV (+bias) + RoPE + KV-cache write. Unit (head, d < D/2) pairs rows head*D + d and +D/2;
 * q heads go to out[m, head*D + ...], k/v heads to cache [slot][Hkv][max_seq][D] at pos[m]
 * (slot = kv_slot if >= 0, else m). cs is [max_seq][D/2] of (cos, sin) fp16 pairs. */
int or_gemv_qkv_rope(const uint16_t* x, int64_t ldx, const uint16_t* normw, float eps, const void* W,
                     const uint16_t* scales, const uint16_t* bias, uint16_t* out, int64_t ldo, int M, int K, int Hq,
                     int Hkv, int D, const uint16_t* cs, const int32_t* pos, uint16_t* kc, uint16_t* vc, int max_seq,
                     int kv_slot) {
  if (M < 1 || K < 1 || Hq < 1 || Hkv < 0 || D < 2 || D % 2) return -1;
  uint16_t* xs = gemv_rows(x, ldx, normw, eps, M, K);
  if (!xs) return -1;
  const int HD = D / 2, heads = Hq + 2 * Hkv;
  for (int m = 0; m < M; m++) {
    const uint16_t* xm = xs + (size_t)m * K;
    const int p = pos[m], slot = kv_slot >= 0 ? kv_slot : m;
#pragma omp parallel for schedule(static)
    for (int u = 0; u < heads * HD; u++) {
      const int head = u / HD, d = u % HD;
      const int64_t r0 = (int64_t)head * D + d, r1 = r0 + HD;
      float a0 = gemv_dot(xm, W, scales, r0, K), a1 = gemv_dot(xm, W, scales, r1, K);
      if (bias) {
        a0 += or_h2f(bias[r0]);
        a1 += or_h2f(bias[r1]);
      }
      uint16_t y1 = or_f2h(a0), y2 = or_f2h(a1);
      if (head < Hq + Hkv) {
        const uint16_t* t = cs + ((int64_t)p * HD + d) * 2;
        or_rope_pair(y1, y2, t[0], t[1], &y1, &y2);
      }
      uint16_t* dst;
      if (head < Hq) dst = out + m * ldo + (int64_t)head * D;
      else if (head < Hq + Hkv) dst = kc + (((int64_t)slot * Hkv + head - Hq) * max_seq + p) * D;
      else dst = vc + (((int64_t)slot * Hkv + head - Hq - Hkv) * max_seq + p) * D;
      dst[d] = y1;
      dst[d + HD] = y2;
    }
  }
  free(xs);
  return 0;
}

/* C (epi) A @ W^T; int8 weights enter as fp16(q * s) (the tile dequantisation). epi 0 adds bias[N]
 * (fp32, before the single rounding) when given; 1 residual; 2 SwiGLU (N/2 output columns). */
int or_gemm(const uint16_t* A, int64_t lda, const void* W, const uint16_t* scales, const uint16_t* bias, uint16_t* C,
            int64_t ldc, int M, int N, int K, int epi) {
  if (M < 1 || N < 1 || K < 1 || epi < 0 || epi > 2 || (epi == 2 && N % 32)) return -1;
  const uint16_t* Wh = (const uint16_t*)W;
  uint16_t* deq = NULL;
  if (scales) {
    deq = (uint16_t*)malloc((size_t)N * K * 2);
    if (!deq) return -1;
    or_dequantize_rows((const int8_t*)W, scales, N, K, deq);
    Wh = deq;
  }
  const int n_out = epi == 2 ? N / 2 : N;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; m++) {
    for (int o = 0; o < n_out; o++) {
      const uint16_t* am = A + m * lda;
      uint16_t* dst = C + m * ldc + o;
      if (epi == 2) {
        const int64_t c = (int64_t)(o / 16) * 32 + o % 16;
        *dst = or_silu_mul((float)dot_h(am, Wh + c * K, K), (float)dot_h(am, Wh + (c + 16) * K, K));
      } else {
        const float y = (float)dot_h(am, Wh + (int64_t)o * K, K);
        if (epi == 1) *dst = or_f2h(or_h2f(*dst) + r16(y));
        else *dst = or_f2h(y + (bias ? or_h2f(bias[o]) : 0.f));
      }
    }
  }
  free(deq);
  return 0;
}

/* ------------------------------------------------------------------ mixture of experts */
enum { OR_MOE_NORM_TOPK = 1, OR_MOE_FP16_WEIGHTS = 2 };

/* v beats (best, bi): NaN above numbers, ties (and NaN vs NaN) to the lower index. */
static int argmax_better(float v, int i, float best, int bi) {
  const int vn = v != v, bn = best != best;
  if (vn != bn) return vn;
  return (vn || v == best) ? i < bi : v > best;
}

int or_moe_router(const uint16_t* xn, int64_t ldx, const uint16_t* Wr, int M, int E, int H, int k, int flags,
                  int32_t* idx, float* w) {
  if (M < 0 || E < 1 || E > 256 || k < 1 || k > 16 || k > E || H < 1) return -1;
#pragma omp parallel for schedule(static)
  for (int t = 0; t < M; t++) {
    float logit[256], sel_v[16] = {0};
    int sel_i[16], taken[256];
    for (int e = 0; e < E; e++) {
      logit[e] = r16((float)dot_h(xn + t * ldx, Wr + (int64_t)e * H, H));
      taken[e] = 0;
    }
    for (int j = 0; j < k; j++) {
      float best = -INFINITY;
      int bi = 0x7fffffff;
      for (int e = 0; e < E; e++)
        if (!taken[e] && argmax_better(logit[e], e, best, bi)) {
          best = logit[e];
          bi = e;
        }
      taken[bi] = 1;
      sel_i[j] = bi;
      sel_v[j] = best;
    }
    const float mx = sel_v[0];
    float denom = 0.f;
    if (flags & OR_MOE_NORM_TOPK)
      for (int j = 0; j < k; j++) denom += expf(sel_v[j] - mx);
    else
      for (int e = 0; e < E; e++) denom += expf(logit[e] - mx);
    for (int j = 0; j < k; j++) {
      float wj = expf(sel_v[j] - mx) / denom;
      if (flags & OR_MOE_FP16_WEIGHTS) wj = r16(wj);
      idx[t * k + j] = sel_i[j];
      w[t * k + j] = wj;
    }
  }
  return 0;
}

/* x[t] += scale * fp16(sum_j w_tj * fp16(down_e(SwiGLU_e(xn[t])))) with the reference's roundings:
 * the SwiGLU activation per silu_mul, each expert output rounded, the weighted term rounded when
 * routing weights are fp16, fp32 sum in j order, one rounding, optional scale (rounded), fp16 add. */
int or_moe_experts(const uint16_t* xn, int64_t ldxn, const uint16_t* wgu, const uint16_t* wdown, const int32_t* idx,
                   const float* w, int M, int E, int k, int H, int I, int flags, float scale, uint16_t* x,
                   int64_t ldx) {
  if (M < 0 || E < 1 || k < 1 || H < 1 || I < 16 || I % 16) return -1;
  for (int p = 0; p < M * k; p++)
    if (idx[p] < 0 || idx[p] >= E) return -1;
#pragma omp parallel for schedule(static)
  for (int t = 0; t < M; t++) {
    uint16_t* act = (uint16_t*)malloc((size_t)I * 2);
    float* sum = (float*)calloc((size_t)H, sizeof(float));
    for (int j = 0; j < k; j++) {
      const int e = idx[t * k + j];
      const uint16_t* G = wgu + (int64_t)e * 2 * I * H;
      const uint16_t* Dn = wdown + (int64_t)e * H * I;
      for (int i = 0; i < I; i++) {
        const int64_t r0 = (int64_t)(i / 16) * 32 + i % 16;
        act[i] = or_silu_mul((float)dot_h(xn + t * ldxn, G + r0 * H, H), (float)dot_h(xn + t * ldxn, G + (r0 + 16) * H, H));
      }
      const float wt = w[t * k + j];
      for (int h = 0; h < H; h++) {
        float c = r16((float)dot_h(act, Dn + (int64_t)h * I, I)) * wt;
        if (flags & OR_MOE_FP16_WEIGHTS) c = r16(c);
        sum[h] += c;
      }
    }
    for (int h = 0; h < H; h++) {
      uint16_t o = or_f2h(sum[h]);
      if (scale != 1.f) o = or_f2h(or_h2f(o) * scale);
      x[t * ldx + h] = or_f2h(or_h2f(x[t * ldx + h]) + or_h2f(o));
    }
    free(act);
    free(sum);
  }
  return 0;
}

/* Decode attention (the reference's decode_attn_kernel, src/kernels.cuh:1486-1660, host
 * api.cu:694-720; CPU reference form tests/test_kernels.py:298-307 ref_attn): for query head h of
 * sequence b, kv head h / (Hq / Hkv), keys and values 0..pos[b] of cache slot b:
 * out = fp16(sum_j softmax_j(q . k_j / sqrt(D)) v_j), in fp64 (an upper bound on the reference's
 * fp32 log2-domain online softmax). */
int or_decode_attn(const uint16_t* q, int64_t ldq, const uint16_t* kc, const uint16_t* vc, int max_seq,
                   const int32_t* pos, uint16_t* out, int64_t ldo, int B, int Hq, int Hkv, int D) {
  if (B < 0 || Hkv < 1 || Hq < Hkv || Hq % Hkv || D < 1 || max_seq < 1) return -1;
  for (int b = 0; b < B; b++)
    if (pos[b] < 0 || pos[b] >= max_seq) return -1;
  const int G = Hq / Hkv;
#pragma omp parallel for schedule(static)
  for (int bh = 0; bh < B * Hq; bh++) {
    const int b = bh / Hq, h = bh % Hq, hk = h / G, L = pos[b] + 1;
    const uint16_t* qh = q + (int64_t)b * ldq + (int64_t)h * D;
    const uint16_t* K = kc + ((int64_t)b * Hkv + hk) * max_seq * D;
    const uint16_t* V = vc + ((int64_t)b * Hkv + hk) * max_seq * D;
    double* s = (double*)malloc((size_t)L * sizeof(double));
    double mx = -INFINITY;
    for (int j = 0; j < L; j++) {
      double acc = 0.0;
      for (int d = 0; d < D; d++) acc += (double)or_h2f(qh[d]) * (double)or_h2f(K[(int64_t)j * D + d]);
      s[j] = acc / sqrt((double)D);
      if (s[j] > mx) mx = s[j];
    }
    double den = 0.0;
    for (int j = 0; j < L; j++) {
      s[j] = exp(s[j] - mx);
      den += s[j];
    }
    for (int d = 0; d < D; d++) {
      double o = 0.0;
      for (int j = 0; j < L; j++) o += s[j] * (double)or_h2f(V[(int64_t)j * D + d]);
      out[(int64_t)b * ldo + (int64_t)h * D + d] = or_f2h((float)(o / den));
    }
    free(s);
  }
  return 0;
}

/* Greedy token of each row (src/kernels.cuh:1883-1931): the largest logit, NaN above every number,
 * the lowest index on ties, starting from (-inf, 0) so a row of -inf gives 0. */
int or_argmax(const uint16_t* logits, int B, int V, int32_t* tok) {
  if (B < 0 || V < 1) return -1;
  for (int b = 0; b < B; b++) {
    float best = -INFINITY;
    int bi = 0;
    for (int i = 0; i < V; i++) {
      const float v = or_h2f(logits[(int64_t)b * V + i]);
      if (argmax_better(v, i, best, bi)) {
        best = v;
        bi = i;
      }
    }
    tok[b] = bi;
  }
  return 0;
}

/* RoPE of the q and k heads of each qkv row and the KV-cache write (src/kernels.cuh:1120-1158):
 * row m sits at position pos[m] in slot slot_base + m (decode form, pos non-null) or at position
 * pos_base + m in slot slot_base (prefill form). q heads are rotated in place; rotated k heads and
 * the raw v heads go to cache [slot][Hkv][max_seq][D]. */
int or_rope_cache(uint16_t* qkv, int64_t ldq, int M, int Hq, int Hkv, int D, const uint16_t* cs, const int32_t* pos,
                  int pos_base, int slot_base, uint16_t* kc, uint16_t* vc, int max_seq) {
  if (M < 0 || Hq < 1 || Hkv < 1 || D < 2 || D % 2 || max_seq < 1) return -1;
  const int HD = D / 2;
  for (int m = 0; m < M; m++) {
    const int p = pos ? pos[m] : pos_base + m, slot = pos ? slot_base + m : slot_base;
    if (p < 0 || p >= max_seq || slot < 0) return -1;
    uint16_t* row = qkv + (int64_t)m * ldq;
    for (int head = 0; head < Hq + Hkv; head++)
      for (int d = 0; d < HD; d++) {
        uint16_t* x = row + (int64_t)head * D;
        const uint16_t* t = cs + ((int64_t)p * HD + d) * 2;
        uint16_t y1, y2;
        or_rope_pair(x[d], x[d + HD], t[0], t[1], &y1, &y2);
        uint16_t* dst = head < Hq ? x : kc + (((int64_t)slot * Hkv + head - Hq) * max_seq + p) * D;
        dst[d] = y1;
        dst[d + HD] = y2;
      }
    for (int i = 0; i < Hkv * D; i++)
      vc[(((int64_t)slot * Hkv + i / D) * max_seq + p) * D + i % D] = row[(int64_t)(Hq + Hkv) * D + i];
  }
  return 0;
}

/* Causal prefill attention over a cache slot (src/kernels.cuh:1160-1329): query row t (head h at
 * columns h*D of q) sits at position p0 + t and attends to keys 0..p0+t of kv head h / (Hq/Hkv),
 * softmax(q.k / sqrt(D)) v in fp64, one rounding to fp16. lse (optional, [Hq][T] fp32) is each
 * row's log-sum-exp in the log2 domain of the scaled logits, log2(sum_j 2^(s_j log2(e)/sqrt(D))). */
int or_flash_prefill(const uint16_t* q, int64_t ldq, const uint16_t* kc, const uint16_t* vc, int max_seq,
                     uint16_t* out, int64_t ldo, int T, int p0, int Hq, int Hkv, int D, float* lse) {
  if (T < 0 || p0 < 0 || p0 + T > max_seq || Hkv < 1 || Hq < Hkv || Hq % Hkv || D < 1) return -1;
  const int G = Hq / Hkv;
#pragma omp parallel for schedule(dynamic)
  for (int th = 0; th < T * Hq; th++) {
    const int t = th / Hq, h = th % Hq, L = p0 + t + 1;
    const uint16_t* qh = q + (int64_t)t * ldq + (int64_t)h * D;
    const uint16_t* K = kc + (int64_t)(h / G) * max_seq * D;
    const uint16_t* V = vc + (int64_t)(h / G) * max_seq * D;
    double* s = (double*)malloc((size_t)L * sizeof(double));
    double mx = -INFINITY;
    for (int j = 0; j < L; j++) {
      double acc = 0.0;
      for (int d = 0; d < D; d++) acc += (double)or_h2f(qh[d]) * (double)or_h2f(K[(int64_t)j * D + d]);
      s[j] = acc / sqrt((double)D);
      if (s[j] > mx) mx = s[j];
    }
    double den = 0.0;
    for (int j = 0; j < L; j++) {
      s[j] = exp(s[j] - mx);
      den += s[j];
    }
    for (int d = 0; d < D; d++) {
      double o = 0.0;
      for (int j = 0; j < L; j++) o += s[j] * (double)or_h2f(V[(int64_t)j * D + d]);
      out[(int64_t)t * ldo + (int64_t)h * D + d] = or_f2h((float)(o / den));
    }
    if (lse) lse[(int64_t)h * T + t] = (float)((mx + log(den)) / log(2.0));
    free(s);
  }
  return 0;
}
