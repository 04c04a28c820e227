// C-ABI of the prefill GEMM (the reference's hi_gemm, hi_gemm_w8 and its benchmarking hooks
// hi_gemm_force_config, hi_gemm_force_splits, hi_gemm_num_configs, hi_gemm_config_desc;
// src/api.cu:276-577, ctypes argtypes scripts/hipinfer.py:23-28).
//
// Shape rules as the reference's (api.cu:555-557): K % 32 == 0, N % 16 == 0 (N % 32 with the
// SwiGLU epilogue); M is free. Launchers return 0, or a negative code after printing the reason.
//
// Tile choice: without a forced config, a model of the MI355X picks the (tile, split-K) pair with
// the least estimated time: the grid is dealt out in rounds of (CUs x resident blocks), a round
// costs its tile's MFMA work divided by that tile's measured efficiency, and split-K pays for its
// fp32 partial round trip. Split-K workspace is grown only outside stream capture and never freed
// while the process runs, so a captured graph keeps a valid pointer (reference api.cu:54-73).
#include <cmath>
#include <mutex>
#include <vector>

#include "gemm.h"

template <> int gemm_run<0>(const GemmArgs&, int, int, bool, hipStream_t);
template <> int gemm_run<1>(const GemmArgs&, int, int, bool, hipStream_t);
template <> int gemm_run<2>(const GemmArgs&, int, int, bool, hipStream_t);
template <> int gemm_blocks_per_cu<0>(int, bool);

namespace {

constexpr int kMaxTiles = 1 << 16;
struct SplitWs {
  float* ws = nullptr;
  size_t bytes = 0;
  int* cnt = nullptr;
  std::vector<float*> retired;  // outgrown buffers, still referenced by captured graphs
};
std::mutex g_ws_mu;
SplitWs g_ws[64];
int g_force_cfg = -1, g_force_splits = -1;

// Resident blocks per CU of a config (LDS and registers), from the occupancy API.
int cfg_blocks_per_cu(int cfg, bool q8) {
  static int cache[2][kGemmNumCfgs] = {};
  int& v = cache[q8][cfg];
  if (!v) {
    const int n = gemm_blocks_per_cu<0>(cfg, q8);  // the epilogues share the main loop's footprint
    v = n > 0 ? n : 1;
  }
  return v;
}

// Relative MFMA efficiency of each tile shape (bigger tiles reuse more of what they stage).
constexpr double kCfgEff[kGemmNumCfgs] = {1.0, 0.85, 0.7, 0.7, 0.5, 0.45};

struct Choice {
  int cfg, splits;
};

Choice gemm_pick(int M, int N, int K, bool q8, int cus) {
  Choice best{1, 1};
  double best_t = 1e300;
  const int nkt = (K + kGemmBK - 1) / kGemmBK;
  for (int c = 0; c < kGemmNumCfgs; c++) {
    const int bm = kGemmCfgs[c].bm, bn = kGemmCfgs[c].bn;
    const double tiles = (double)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int slots = cus * cfg_blocks_per_cu(c, q8);
    for (int sp = 1; sp <= 16; sp *= 2) {
      if (sp > nkt || (sp > 1 && tiles * sp > 8.0 * cus) || tiles > kMaxTiles) continue;
      const int kps = (nkt + sp - 1) / sp;
      const double rounds = std::ceil(tiles * sp / slots);
      double t = rounds * (double)bm * bn * kps * kGemmBK / kCfgEff[c];
      if (sp > 1) t += tiles * sp * bm * bn * 24.0;  // partial write + read back, per element
      t += (double)bm * bn * kGemmBK * 2.0;          // prologue / epilogue per round
      if (t < best_t) {
        best_t = t;
        best = {c, sp};
      }
    }
  }
  return best;
}

// Workspace for `bytes` of partials (and the tile counters); false when it would have to grow
// inside stream capture.
int ensure_ws(size_t bytes, hipStream_t s, bool* ok) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  SplitWs& w = g_ws[d->id];
  *ok = true;
  if (w.cnt && bytes <= w.bytes) return 0;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HI_TRY(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone) {
    *ok = false;
    return 0;
  }
  if (!w.cnt) {
    HI_TRY(hipMalloc(&w.cnt, kMaxTiles * sizeof(int)));
    HI_TRY(hipMemset(w.cnt, 0, kMaxTiles * sizeof(int)));
  }
  if (bytes > w.bytes) {
    size_t nb = bytes > 2 * w.bytes ? bytes : 2 * w.bytes;
    if (w.ws) w.retired.push_back(w.ws);
    HI_TRY(hipMalloc(&w.ws, nb));
    w.bytes = nb;
  }
  HI_TRY(hipDeviceSynchronize());  // the counters' zeroing is complete before any kernel uses them
  return 0;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int gemm_entry(const void* A, int lda, const void* W, const void* scales, const void* bias, void* C, int ldc, int M,
               int N, int K, int epi, void* stream, const char* who) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  if (epi < 0 || epi > 2) HI_FAIL("%s: epi must be 0, 1 or 2 (got %d)", who, epi);
  if (M < 0 || N < 16 || K < 32 || K % 32 || N % (epi == 2 ? 32 : 16))
    HI_FAIL("%s: unsupported shape M=%d N=%d K=%d epi=%d (K %% 32 == 0, N %% %d == 0)", who, M, N, K, epi,
            epi == 2 ? 32 : 16);
  if (M == 0) return 0;
  if (!A || !W || !C) HI_FAIL("%s: null tensor pointer", who);
  if (!aligned(A, 16) || lda % 8 || lda < K) HI_FAIL("%s: A must be 16-byte aligned with lda >= K, lda %% 8 == 0", who);
  if (!aligned(W, 16)) HI_FAIL("%s: W must be 16-byte aligned", who);
  const int n_out = epi == 2 ? N / 2 : N;
  if (ldc < n_out) HI_FAIL("%s: ldc %d < %d output columns", who, ldc, n_out);
  const bool q8 = scales != nullptr;
  const hipStream_t s = (hipStream_t)stream;

  Choice ch = gemm_pick(M, N, K, q8, d->cus);
  if (g_force_cfg >= 0 && g_force_cfg < kGemmNumCfgs) ch.cfg = g_force_cfg;
  if (g_force_splits >= 1) ch.splits = g_force_splits;
  const int nkt = (K + kGemmBK - 1) / kGemmBK;
  if (ch.splits > nkt) ch.splits = nkt;
  const int kps = (nkt + ch.splits - 1) / ch.splits;
  ch.splits = (nkt + kps - 1) / kps;  // no empty splits
  const int bm = kGemmCfgs[ch.cfg].bm, bn = kGemmCfgs[ch.cfg].bn;
  const int tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);

  GemmArgs g{};
  g.A = (const f16*)A;
  g.lda = lda;
  g.W = W;
  g.scales = (const f16*)scales;
  g.bias = epi == 0 ? (const f16*)bias : nullptr;  // the bias belongs to epilogue 0 (reference api.cu:416-420)
  g.C = (f16*)C;
  g.ldc = ldc;
  g.M = M;
  g.N = N;
  g.K = K;
  g.kt_per_split = kps;
  if (ch.splits > 1) {
    bool ok = false;
    if (tiles > kMaxTiles) ok = false;
    else {
      const int r = ensure_ws((size_t)ch.splits * tiles * bm * bn * sizeof(float), s, &ok);
      if (r) return r;
    }
    if (ok) {
      std::lock_guard<std::mutex> lk(g_ws_mu);
      g.ws = g_ws[d->id].ws;
      g.counters = g_ws[d->id].cnt;
    } else {  // cannot grow under capture: run unsplit
      ch.splits = 1;
      g.kt_per_split = nkt;
    }
  }
  switch (epi) {
    case 0: return gemm_run<0>(g, ch.cfg, ch.splits, q8, s);
    case 1: return gemm_run<1>(g, ch.cfg, ch.splits, q8, s);
    default: return gemm_run<2>(g, ch.cfg, ch.splits, q8, s);
  }
}

}  // namespace

// C (epi) A[M, K] @ W[N, K]^T (+ bias[N] for epi 0 when non-null), fp16 weights.
HI_EXPORT int hi_gemm(const void* A, int lda, const void* W, const void* bias, void* C, int ldc, int M, int N, int K,
                      int epi, void* s) {
  return gemm_entry(A, lda, W, nullptr, bias, C, ldc, M, N, K, epi, s, "hi_gemm");
}

// The same with int8 weights W [N, K] and fp16 row scales [N]; each W tile is dequantised to
// fp16(q * s) on its way into LDS.
HI_EXPORT int hi_gemm_w8(const void* A, int lda, const void* W, const void* scales, const void* bias, void* C, int ldc,
                         int M, int N, int K, int epi, void* s) {
  if (!scales) HI_FAIL("hi_gemm_w8: scales must not be null");
  return gemm_entry(A, lda, W, scales, bias, C, ldc, M, N, K, epi, s, "hi_gemm_w8");
}

// Benchmark / test hooks: force a tile config (-1: automatic) or a split-K factor (-1: automatic).
HI_EXPORT int hi_gemm_force_config(int c) {
  g_force_cfg = c;
  return 0;
}
HI_EXPORT int hi_gemm_force_splits(int sp) {
  g_force_splits = sp;
  return 0;
}
HI_EXPORT int hi_gemm_num_configs() { return kGemmNumCfgs; }
HI_EXPORT int hi_gemm_config_desc(int c, char* out, int n) {
  if (c < 0 || c >= kGemmNumCfgs || !out || n < 1) return -1;
  snprintf(out, n, "mfma 32x32x16 %dx%dx%d waves %dx%d", kGemmCfgs[c].bm, kGemmCfgs[c].bn, kGemmBK, kGemmCfgs[c].wm,
           kGemmCfgs[c].wn);
  return 0;
}
