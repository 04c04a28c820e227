// C-ABI of the decode GEMV (the reference's hi_gemv, hi_gemv_w8, hi_gemv_qkv_rope,
// hi_gemv_qkv_rope_w8; src/api.cu:181-230, ctypes argtypes scripts/hipinfer.py:14-18).
//
// Same signatures and argument meaning; the launchers return 0, or a negative code after printing
// the reason where the reference would print and exit(1). Rows are processed in launches of at most
// 8 (fused RMSNorm) or 16 rows, fewer when the activation rows would not fit in LDS; rows are
// independent, so chunking never changes a result.
#include "gemv.h"
#include "hi_internal.h"

template <> int gemv_run<0>(const GemvArgs&, int, bool, int, hipStream_t);
template <> int gemv_run<1>(const GemvArgs&, int, bool, int, hipStream_t);
template <> int gemv_run<2>(const GemvArgs&, int, bool, int, hipStream_t);
template <> int gemv_run<3>(const GemvArgs&, int, bool, int, hipStream_t);

static bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// LDS per activation row: the row, its per-wave norm partials and inverse RMS, and for int8
// weights one partial sum per staging thread
static size_t gemv_row_lds(int K, bool int8) {
  return (size_t)K * 2 + (kGemvWaves + 1) * sizeof(float) + (int8 ? kGemvThreads * sizeof(float) : 0);
}

static int rows_per_launch(size_t row_lds, bool norm, int lds_max) {
  if (row_lds > (size_t)lds_max) return 0;
  int cap = norm ? 8 : 16;
  while (cap > 1 && (size_t)cap * row_lds > (size_t)lds_max) cap >>= 1;
  return cap;
}

int gemv_rows_per_launch(int K, bool norm, bool int8) {
  const HiDevice* d = hi_device();
  return d ? rows_per_launch(gemv_row_lds(K, int8), norm, d->lds_max) : 0;
}

HI_EXPORT int hi_gemv_rows_per_launch(int K, int norm, int int8) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  return K < 8 ? 0 : rows_per_launch(gemv_row_lds(K, int8 != 0), norm != 0, d->lds_max);
}

static int gemv_common(GemvArgs a, int epi, hipStream_t s, const char* who) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  if (a.M < 0 || a.N < 1 || a.K < 8) HI_FAIL("%s: bad shape M=%d N=%d K=%d", who, a.M, a.N, a.K);
  if (a.M == 0) return 0;
  if (a.K % 8) HI_FAIL("%s: K must be a multiple of 8 (K=%d)", who, a.K);
  if (!a.x || !a.W || !a.out) HI_FAIL("%s: null tensor pointer", who);
  if (!aligned(a.x, 16) || a.ldx % 8 || a.ldx < a.K)
    HI_FAIL("%s: x must be 16-byte aligned with ldx >= K and ldx %% 8 == 0 (ldx=%lld)", who, (long long)a.ldx);
  if (a.normw && !aligned(a.normw, 16)) HI_FAIL("%s: normw must be 16-byte aligned", who);
  const int wf = !a.scales ? WF_F16 : (a.K % 16 == 0 ? WF_I8 : WF_I8H);
  if (!aligned(a.W, wf == WF_I8H ? 8 : 16)) HI_FAIL("%s: W must be %d-byte aligned", who, wf == WF_I8H ? 8 : 16);
  if (a.scales && !aligned(a.scales, 2)) HI_FAIL("%s: scales must be 2-byte aligned", who);
  const int n_out = epi == 2 ? a.N / 2 : a.N;
  if (epi != 3 && a.ldo < n_out) HI_FAIL("%s: ldo %lld < %d output columns", who, (long long)a.ldo, n_out);
  const bool norm = a.normw != nullptr;
  int cap = rows_per_launch(gemv_row_lds(a.K, wf != WF_F16), norm, d->lds_max);
  if (!cap) HI_FAIL("%s: K=%d activation row exceeds LDS", who, a.K);
  if (epi == 3) {
    // the fused QKV epilogue writes a launch's cache rows at 32-bit byte offsets from its first
    // slot (and q rows from out): fewer rows per launch when a slot is large
    const uint64_t lim = 0xFFFFFFFFull, pos_bytes = (uint64_t)a.max_seq * a.D * 2;
    const uint64_t slot_bytes = pos_bytes * a.Hkv;
    if (pos_bytes > lim) HI_FAIL("%s: a cache head of %d x %d fp16 exceeds 4 GB", who, a.max_seq, a.D);
    if (a.kv_slot < 0)
      while (cap > 1 && (uint64_t)(cap - 1) * slot_bytes + pos_bytes > lim) cap >>= 1;
    if (((uint64_t)(cap - 1) * a.ldo + (uint64_t)a.Hq * a.D) * 2 > lim) HI_FAIL("%s: ldo %lld too large", who, (long long)a.ldo);
  } else if (((uint64_t)(cap - 1) * a.ldo + (uint64_t)n_out) * 2 > 0xFFFFFFFFull) {
    // epilogues 0-2 store through a buffer at 32-bit byte offsets from a launch's first row
    HI_FAIL("%s: ldo %lld too large (a launch's output rows must span under 4 GB)", who, (long long)a.ldo);
  }
  const int M = a.M;
  for (int m0 = 0; m0 < M; m0 += cap) {
    GemvArgs c = a;
    c.M = M - m0 < cap ? M - m0 : cap;
    c.x = a.x + m0 * a.ldx;
    c.out = a.out + m0 * a.ldo;
    if (epi == 3) {
      c.pos = a.pos + m0;
      c.slot_base = a.slot_base + m0;
    }
    // rows of the kernel instance: 1-8 exactly, 16 above (dot products of padding rows cost as much
    // as real ones: 5 rows on the 8-row instance had run 60 % more of them)
    const int MR = c.M <= 8 ? c.M : 16;
    int r;
    switch (epi) {
      case 0: r = gemv_run<0>(c, MR, norm, wf, s); break;
      case 1: r = gemv_run<1>(c, MR, norm, wf, s); break;
      case 2: r = gemv_run<2>(c, MR, norm, wf, s); break;
      default: r = gemv_run<3>(c, MR, norm, wf, s); break;
    }
    if (r) return r;
  }
  return 0;
}

static int gemv_plain(const void* x, int ldx, const void* normw, float eps, const void* W, const void* scales, void* out,
                      int ldo, int M, int N, int K, int epi, void* s, const char* who) {
  if (epi < 0 || epi > 2) HI_FAIL("%s: epi must be 0, 1 or 2 (got %d)", who, epi);
  if (epi == 2 && N % 32) HI_FAIL("%s: the SwiGLU epilogue needs N %% 32 == 0 (N=%d)", who, N);
  GemvArgs a{};
  a.x = (const f16*)x;
  a.ldx = ldx;
  a.normw = (const f16*)normw;
  a.eps = eps;
  a.W = W;
  a.scales = (const f16*)scales;
  a.out = (f16*)out;
  a.ldo = ldo;
  a.M = M;
  a.N = N;
  a.K = K;
  return gemv_common(a, epi, (hipStream_t)s, who);
}

// out[M, *] (epi) x[M, K] @ W[N, K]^T, fp16 weights; normw != null fuses RMSNorm of x.
HI_EXPORT int hi_gemv(const void* x, int ldx, const void* normw, float eps, const void* W, void* out, int ldo, int M,
                      int N, int K, int epi, void* s) {
  return gemv_plain(x, ldx, normw, eps, W, nullptr, out, ldo, M, N, K, epi, s, "hi_gemv");
}

// The same with int8 weights W [N, K] and fp16 row scales [N].
HI_EXPORT int hi_gemv_w8(const void* x, int ldx, const void* normw, float eps, const void* W, const void* scales,
                         void* out, int ldo, int M, int N, int K, int epi, void* s) {
  if (!scales) HI_FAIL("hi_gemv_w8: scales must not be null");
  return gemv_plain(x, ldx, normw, eps, W, scales, out, ldo, M, N, K, epi, s, "hi_gemv_w8");
}

static int qkv_common(const void* x, int ldx, const void* normw, float eps, const void* W, const void* scales,
                      const void* bias, void* out, int ldo, int M, int K, int Hq, int Hkv, int D, const void* cs,
                      const int* pos, void* kc, void* vc, int max_seq, int kv_slot, void* s, const char* who) {
  if (Hq < 1 || Hkv < 1 || D < 2 || D % 2 || max_seq < 1) HI_FAIL("%s: bad heads Hq=%d Hkv=%d D=%d", who, Hq, Hkv, D);
  if (!cs || !pos || !kc || !vc) HI_FAIL("%s: null cs / pos / cache pointer", who);
  if (ldo < Hq * D) HI_FAIL("%s: ldo %d < Hq * D = %d", who, ldo, Hq * D);
  GemvArgs a{};
  a.x = (const f16*)x;
  a.ldx = ldx;
  a.normw = (const f16*)normw;
  a.eps = eps;
  a.W = W;
  a.scales = (const f16*)scales;
  a.out = (f16*)out;
  a.ldo = ldo;
  a.M = M;
  a.N = (Hq + 2 * Hkv) * D;
  a.K = K;
  a.bias = (const f16*)bias;
  a.cs = (const f16x2*)cs;
  a.pos = pos;
  a.kc = (f16*)kc;
  a.vc = (f16*)vc;
  a.max_seq = max_seq;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = D;
  a.kv_slot = kv_slot;
  a.slot_base = 0;
  return gemv_common(a, 3, (hipStream_t)s, who);
}

// QKV projection (RMSNorm fused when normw != null) with bias, RoPE and the KV-cache write fused
// into the epilogue: q to out[m, 0:Hq*D], k/v to cache slot m at position pos[m].
HI_EXPORT int hi_gemv_qkv_rope(const void* x, int ldx, const void* normw, float eps, const void* W, const void* bias,
                               void* out, int ldo, int M, int K, int Hq, int Hkv, int D, const void* cs, const int* pos,
                               void* kc, void* vc, int max_seq, void* s) {
  return qkv_common(x, ldx, normw, eps, W, nullptr, bias, out, ldo, M, K, Hq, Hkv, D, cs, pos, kc, vc, max_seq, -1, s,
                    "hi_gemv_qkv_rope");
}

// The same with int8 weights and fp16 row scales.
HI_EXPORT int hi_gemv_qkv_rope_w8(const void* x, int ldx, const void* normw, float eps, const void* W,
                                  const void* scales, const void* bias, void* out, int ldo, int M, int K, int Hq,
                                  int Hkv, int D, const void* cs, const int* pos, void* kc, void* vc, int max_seq,
                                  void* s) {
  if (!scales) HI_FAIL("hi_gemv_qkv_rope_w8: scales must not be null");
  return qkv_common(x, ldx, normw, eps, W, scales, bias, out, ldo, M, K, Hq, Hkv, D, cs, pos, kc, vc, max_seq, -1, s,
                    "hi_gemv_qkv_rope_w8");
}

// The verify form: every row's k / v to cache slot kv_slot.
int gemv_qkv_rope_slot(const void* x, int ldx, const void* normw, float eps, const void* W, const void* scales,
                       const void* bias, void* out, int ldo, int M, int K, int Hq, int Hkv, int D, const void* cs,
                       const int* pos, void* kc, void* vc, int max_seq, int kv_slot, hipStream_t s) {
  if (kv_slot < 0) HI_FAIL("gemv_qkv_rope_slot: kv_slot %d < 0", kv_slot);
  return qkv_common(x, ldx, normw, eps, W, scales, bias, out, ldo, M, K, Hq, Hkv, D, cs, pos, kc, vc, max_seq, kv_slot,
                    s, "gemv_qkv_rope_slot");
}
