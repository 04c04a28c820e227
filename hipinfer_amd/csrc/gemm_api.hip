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
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "../../include/hipinfer.h"
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
  std::vector<float*> retired;  // outgrown buffers, still referenced by captured graphs
};
// Split-K partials per host thread and device, as the reference keeps them (api.cu:54-73, 471):
// GEMMs issued at the same time from different host threads never share a buffer.
thread_local SplitWs g_ws[64];
int g_force_cfg = -1, g_force_splits = -1;

// Resident blocks per CU of a config (LDS and registers), from the occupancy API. One value per
// config for the process: every device it runs on is a gfx950 with the same CU resources.
int cfg_blocks_per_cu(int cfg, bool q8) {
  static std::atomic<int> cache[2][kGemmNumCfgs];  // 0 until first asked
  std::atomic<int>& v = cache[q8][cfg];
  int n = v.load(std::memory_order_relaxed);
  if (!n) {
    n = gemm_blocks_per_cu<0>(cfg, q8);  // the epilogues share the main loop's footprint
    n = n > 0 ? n : 1;
    v.store(n, std::memory_order_relaxed);
  }
  return n;
}

// Relative MFMA efficiency of each tile shape (bigger tiles reuse more of what they stage).
constexpr double kCfgEff[kGemmNumCfgs] = {0.9, 0.85, 0.85, 0.6, 0.8, 0.45, 0.4, 0.6,
                                           1.0, 0.9, 1.05, 0.85, 0.95, 0.85, 0.8, 0.5, 0.95, 0.6, 0.6, 0.95};

struct Choice {
  int cfg, splits;
};
thread_local Choice g_last{-1, 0};  // the (tile, split) of this thread's last launch (hi_gemm_last_choice)

// Fallback model (stream capture, autotuning off): rounds of resident blocks times the tile's
// MFMA time at its efficiency, or the L2/MALL time of everything the tiles stage, whichever is
// longer, plus the split-K partial round trip.
Choice gemm_pick(int M, int N, int K, bool q8, int cus) {
  Choice best{1, 1};
  double best_t = 1e300;
  const double mfma_per_cu = 4069.0 * 2.4e9;  // fp16 flop/s per CU at the datasheet peak
  const double l2_bw = 20e12;                 // aggregate L2/MALL bytes/s the staging can draw
  for (int c = 0; c < kGemmNumCfgs; c++) {
    if (!gemm_cfg_fits(c, q8, K)) continue;
    const int bm = kGemmCfgs[c].bm, bn = kGemmCfgs[c].bn, bk = kGemmCfgs[c].bk;
    const int nkt = (K + bk - 1) / bk;
    const double tiles = (double)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int slots = cus * cfg_blocks_per_cu(c, q8);
    for (int sp = 1; sp <= 8; sp += sp < 6 ? 1 : 2) {
      if (sp > nkt || (sp > 1 && (tiles * sp > 4.0 * cus || kGemmCfgs[c].kg > 1)) || tiles > kMaxTiles) continue;
      const int kps = (nkt + sp - 1) / sp;
      const double rounds = std::ceil(tiles * sp / slots);
      const double t_mfma = rounds * 2.0 * bm * bn * kps * bk / (mfma_per_cu * kCfgEff[c]);
      const double t_l2 = tiles * sp * kps * (double)(bm * 2 * bk + bn * (q8 ? bk : 2 * bk)) / l2_bw;
      double t = std::max(t_mfma, t_l2) + 2e-6;
      if (sp > 1) t += (double)M * N * sp * 8.0 / 4e12 + 3e-6;  // partials out and back, second launch
      if (t < best_t) {
        best_t = t;
        best = {c, sp};
      }
    }
  }
  return best;
}

// Workspace for `bytes` of split-K partials; *ok = false when it would have to grow inside stream
// capture (the caller then runs one split). Every partial is written before it is read, so the
// buffer needs no clearing.
int ensure_ws(size_t bytes, hipStream_t s, bool* ok) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  SplitWs& w = g_ws[d->id];
  *ok = true;
  if (w.ws && bytes <= w.bytes) return 0;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HI_TRY(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone) {
    *ok = false;
    return 0;
  }
  size_t nb = bytes > 2 * w.bytes ? bytes : 2 * w.bytes;
  if (w.ws) w.retired.push_back(w.ws);
  HI_TRY(hipMalloc(&w.ws, nb));
  w.bytes = nb;
  return 0;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int launch_choice(const GemmArgs& g0, Choice ch, int epi, bool q8, hipStream_t s, float* fixed_ws = nullptr,
                  int* used_splits = nullptr);

// First-call autotuning per (M bucket, N, K, SwiGLU, int8) and device, as the reference's
// gemm_choose (api.cu:465-552): every valid (tile, split) is timed on the real activations into a
// scratch output, with the weights streamed cold (below); the three fastest are re-timed in
// interleaved rounds and the best median kept. Skipped under stream capture and with
// HIPINFER_GEMM_AUTOTUNE=0 (the model above decides then).
std::mutex g_tune_mu;
std::map<std::tuple<int, int, int, int, bool, bool, bool>, Choice> g_tuned;

// norm: the call is a residual GEMM followed by the RMSNorm of its result (hi_gemm_residual_rmsnorm):
// each candidate is timed with that norm as it would run, inside the split-K second pass or as a
// separate kernel after an unsplit launch, and the choice is kept apart from plain GEMMs'.
int gemm_choose(const GemmArgs& g, int epi, bool q8, hipStream_t s, Choice* out, bool norm = false) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  int mb = 16;
  while (mb < g.M && mb < 4096) mb *= 2;
  const auto key = std::make_tuple(d->id, mb, g.N, g.K, epi == 2, q8, norm);
  {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    auto it = g_tuned.find(key);
    if (it != g_tuned.end()) {
      *out = it->second;
      return 0;
    }
  }
  *out = gemm_pick(g.M, g.N, g.K, q8, d->cus);
  static const bool enabled = !getenv("HIPINFER_GEMM_AUTOTUNE") || atoi(getenv("HIPINFER_GEMM_AUTOTUNE")) != 0;
  // 1: the choice per shape; 2: also every candidate's first timing
  static const int verbose = getenv("HIPINFER_GEMM_VERBOSE") ? atoi(getenv("HIPINFER_GEMM_VERBOSE")) : 0;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  HI_TRY(hipStreamIsCapturing(s, &cap));
  if (!enabled || cap != hipStreamCaptureStatusNone) return 0;

  const int n_out = epi == 2 ? g.N / 2 : g.N;
  f16* scratch = nullptr;
  HI_TRY(hipMalloc(&scratch, (size_t)g.M * n_out * sizeof(f16) * (norm ? 2 : 1) + (norm ? (size_t)g.N * sizeof(f16) : 0)));
  HI_TRY(hipMemsetAsync(scratch, 0, (size_t)g.M * n_out * sizeof(f16) * (norm ? 2 : 1) + (norm ? (size_t)g.N * sizeof(f16) : 0), s));
  hipEvent_t e0, e1;
  HI_TRY(hipEventCreate(&e0));
  HI_TRY(hipEventCreate(&e1));
  GemmArgs t = g;
  t.C = scratch;
  t.ldc = n_out;
  f16* norm_y = scratch + (size_t)g.M * n_out;  // norm: its output, then its (zero) weights
  const f16* norm_w = norm_y + (size_t)g.M * n_out;
  if (norm) {
    t.norm_w = norm_w;
    t.norm_y = norm_y;
    t.norm_eps = 1e-5f;
  }
  auto launch = [&](Choice c) -> int {
    int used = 1;
    if (int rc = launch_choice(t, c, epi, q8, s, nullptr, &used)) return rc;
    return norm && used == 1 ? hi_rmsnorm(t.C, norm_w, norm_y, g.M, g.N, 1e-5f, s) : 0;
  };
  // Candidates are timed on rotating scratch weight buffers (at least ~640 MB in all, so neither
  // the L2s nor the 256 MB MALL hold them): a prefill streams each layer's weights once, and
  // timing on the same, cache-resident weights would favour tiles that re-read more. The scratch
  // contents are never initialised: MFMA timing does not depend on the values, and the results
  // go to the scratch output.
  const size_t wstride = ((size_t)g.N * g.K * (q8 ? 1 : 2) + 255) / 256 * 256;
  int nrot = (int)std::min<size_t>(32, std::max<size_t>(2, ((size_t)640 << 20) / wstride + 1));
  char* wrot = nullptr;
  if (hipMalloc(&wrot, nrot * wstride) != hipSuccess) {
    (void)hipGetLastError();
    wrot = nullptr;
    nrot = 1;
  }
  auto time_it = [&](Choice c, int reps, float* us) -> int {
    t.W = wrot ? wrot : g.W;
    if (int rc = launch(c)) return rc;
    HI_TRY(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++) {
      if (wrot) t.W = wrot + (size_t)((r + 1) % nrot) * wstride;
      if (int rc = launch(c)) return rc;
    }
    HI_TRY(hipEventRecord(e1, s));
    HI_TRY(hipEventSynchronize(e1));
    float ms = 0.f;
    HI_TRY(hipEventElapsedTime(&ms, e0, e1));
    *us = ms * 1e3f / reps;
    return 0;
  };
  std::vector<std::pair<float, Choice>> timed;
  int rc = 0;
  for (int c = 0; c < kGemmNumCfgs && !rc; c++) {
    if (!gemm_cfg_fits(c, q8, g.K)) continue;
    const int bm = kGemmCfgs[c].bm, bn = kGemmCfgs[c].bn;
    const int nkt = (g.K + kGemmCfgs[c].bk - 1) / kGemmCfgs[c].bk;
    const long tiles = (long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
    if (bm > 2 * mb && kGemmCfgs[c].bm != 32) continue;  // a tile far taller than M only stages padding
    for (int sp = 1; sp <= 8 && !rc; sp += sp < 6 ? 1 : 2) {
      if (sp > nkt || (sp > 1 && (tiles * sp > 4L * d->cus || kGemmCfgs[c].kg > 1)) || tiles > kMaxTiles) continue;
      float us = 0.f;
      rc = time_it({c, sp}, std::max(nrot, 4), &us);
      if (!rc) timed.push_back({us, {c, sp}});
      if (!rc && verbose >= 2)
        fprintf(stderr, "hipinfer_amd gemm autotune M=%d N=%d K=%d epi=%d%s%s   cfg %d (%dx%d) split %d: %.1f us\n",
                g.M, g.N, g.K, epi, q8 ? " int8" : "", norm ? " +norm" : "", c, bm, kGemmCfgs[c].bn, sp, us);
    }
  }
  if (!rc && !timed.empty()) {
    // the three fastest are re-timed in three interleaved rounds (a clock ramp or a transient
    // then touches every finalist alike) and the one with the lowest median kept
    const size_t nfin = std::min<size_t>(3, timed.size());
    std::partial_sort(timed.begin(), timed.begin() + nfin, timed.end(),
                      [](const auto& a, const auto& b) { return a.first < b.first; });
    constexpr int kRounds = 3;
    float fin[3][kRounds];
    for (int r = 0; r < kRounds && !rc; r++)
      for (size_t f = 0; f < nfin && !rc; f++) rc = time_it(timed[f].second, std::max(nrot, 8), &fin[f][r]);
    float best = 1e30f;
    for (size_t f = 0; f < nfin && !rc; f++) {
      std::sort(fin[f], fin[f] + kRounds);
      const float us = fin[f][kRounds / 2];
      if (us < best) {
        best = us;
        *out = timed[f].second;
      }
    }
    if (verbose && !rc)
      fprintf(stderr, "hipinfer_amd gemm autotune M=%d N=%d K=%d epi=%d%s%s -> cfg %d split %d: %.1f us, %.1f TFLOP/s\n",
              g.M, g.N, g.K, epi, q8 ? " int8" : "", norm ? " +norm" : "", out->cfg, out->splits, best,
              2.0 * g.M * g.N * g.K / (best * 1e-6) / 1e12);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipStreamSynchronize(s);
  (void)hipFree(scratch);
  if (wrot) (void)hipFree(wrot);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_tune_mu);
  g_tuned[key] = *out;
  return 0;
}

// Launch with a chosen (tile, split): sets up the split-K workspace (or falls back to one split
// when it would have to grow inside stream capture). With fixed_ws the partials go there instead,
// and the caller has checked that they fit.
int launch_choice(const GemmArgs& g0, Choice ch, int epi, bool q8, hipStream_t s, float* fixed_ws, int* used_splits) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  GemmArgs g = g0;
  const int nkt = (g.K + kGemmCfgs[ch.cfg].bk - 1) / kGemmCfgs[ch.cfg].bk;  // K tiles of the chosen depth
  if (ch.splits > nkt) ch.splits = nkt;
  if (kGemmCfgs[ch.cfg].kg > 1) ch.splits = 1;  // a K-group tile splits K inside the block
  int kps = (nkt + ch.splits - 1) / ch.splits;
  ch.splits = (nkt + kps - 1) / kps;  // no empty splits
  const int bm = kGemmCfgs[ch.cfg].bm, bn = kGemmCfgs[ch.cfg].bn;
  const long tiles = (long)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
  if (ch.splits > 1) {
    bool ok = false;
    if (tiles <= kMaxTiles && fixed_ws) {
      ok = true;
      g.ws = fixed_ws;
    } else if (tiles <= kMaxTiles) {
      const int r = ensure_ws((size_t)ch.splits * g.M * g.N * sizeof(float), s, &ok);
      if (r) return r;
      if (ok) g.ws = g_ws[d->id].ws;
    }
    if (!ok) {
      ch.splits = 1;
      kps = nkt;
    }
  }
  g.kt_per_split = kps;
  g_last = ch;
  if (used_splits) *used_splits = ch.splits;
  switch (epi) {
    case 0: return gemm_run<0>(g, ch.cfg, ch.splits, q8, s);
    case 1: return gemm_run<1>(g, ch.cfg, ch.splits, q8, s);
    default: return gemm_run<2>(g, ch.cfg, ch.splits, q8, s);
  }
}


// Shape and pointer checks shared by the entry points; fills g. Returns 0, or a negative code.
int gemm_args(const void* A, int lda, const void* W, const void* scales, const void* bias, void* C, int ldc, int M,
              int N, int K, int epi, const char* who, GemmArgs& g) {
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
  g = GemmArgs{};
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
  g.vec_c = aligned(C, 8) && ldc % 4 == 0;
  g.vec16_c = aligned(C, 16) && ldc % 8 == 0;
  return 0;
}

// norm_y non-null (epilogue 1, ldc == N): afterwards norm_y = RMSNorm(C) * norm_w, inside the
// split-K second pass when the launch splits K and N <= 8192, else by hi_rmsnorm.
int gemm_entry(const void* A, int lda, const void* W, const void* scales, const void* bias, void* C, int ldc, int M,
               int N, int K, int epi, void* stream, const char* who, const void* norm_w = nullptr,
               void* norm_y = nullptr, float eps = 0.f) {
  const HiDevice* d = hi_device();
  if (!d) return -2;
  GemmArgs g;
  if (int r = gemm_args(A, lda, W, scales, bias, C, ldc, M, N, K, epi, who, g)) return r;
  if (M == 0) return 0;
  const bool q8 = scales != nullptr;
  const hipStream_t s = (hipStream_t)stream;
  Choice ch{1, 1};
  if (g_force_cfg >= 0 && g_force_cfg < kGemmNumCfgs && gemm_cfg_fits(g_force_cfg, q8, K)) {  // else: automatic
    ch = gemm_pick(M, N, K, q8, d->cus);
    ch.cfg = g_force_cfg;
  } else if (int r = gemm_choose(g, epi, q8, s, &ch, norm_y != nullptr && N <= 8192)) {
    return r;
  }
  if (g_force_splits >= 1) ch.splits = g_force_splits;
  if (!norm_y) return launch_choice(g, ch, epi, q8, s);
  const bool fuse = N <= 8192;
  if (fuse) {  // the tuner timed each candidate with its norm; the norm fields go on g for the final launch only
    g.norm_w = (const f16*)norm_w;
    g.norm_y = (f16*)norm_y;
    g.norm_eps = eps;
  }
  int used = 1;
  if (int r = launch_choice(g, ch, epi, q8, s, nullptr, &used)) return r;
  return fuse && used > 1 ? 0 : hi_rmsnorm(C, norm_w, norm_y, M, N, eps, stream);
}

}  // namespace

// ---------------------------------------------------------------- the entry point that allocates nothing
// hi_gemm_noalloc keeps its split-K partials in this file-scope device array instead of the
// workspace hi_gemm grows with hipMalloc. Each GPU the library runs on holds its own 64 MB copy
// from the first launch until the process ends. In host code `scratch` is only the host-side
// handle of the array: its device address on the current GPU comes from hipGetSymbolAddress and
// is kept per device in g_scratch, and only that address is ever given to a kernel.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kScratchDevices] = {};

// The current device's copy of `scratch`, looked up once per device (with that device current).
float* scratch_on(const HiDevice* d) {
  if (d->id < 0 || d->id >= kScratchDevices) {
    fprintf(stderr, "hipinfer_amd: hi_gemm_noalloc: device id %d outside the %d devices it keeps scratch for\n", d->id,
            kScratchDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[d->id]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fprintf(stderr, "hipinfer_amd: hipGetSymbolAddress(scratch) failed on device %d: %s\n", d->id,
              hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[d->id] = (float*)p;
  }
  return g_scratch[d->id];
}
}  // namespace

// C (epi) A[M, K] @ W[N, K]^T like hi_gemm (scales == NULL) or hi_gemm_w8 (scales given), without any
// allocation: no hipMalloc / hipFree, no first-call autotuning (which times candidates on scratch
// copies). The tile is the one the autotuner already chose for this shape on this device, else the
// cost model's, or a forced one (hi_gemm_force_config / hi_gemm_force_splits); split-K partials
// ([splits][M][N] fp32) live in the library's 64 MB static scratch. An automatic split is lowered
// until its partials fit; a forced split that does not fit is rejected (-1). Every call on a GPU
// shares that GPU's scratch: calls that overlap in time on one GPU (two streams, two host threads)
// race. Every partial is written before it is read, so nothing needs clearing between calls.
HI_EXPORT int hi_gemm_noalloc(const void* A, int lda, const void* W, const void* scales, const void* bias, void* C,
                              int ldc, int M, int N, int K, int epi, void* stream) {
  const char* who = "hi_gemm_noalloc";
  const HiDevice* d = hi_device();
  if (!d) return -2;
  GemmArgs g;
  if (int r = gemm_args(A, lda, W, scales, bias, C, ldc, M, N, K, epi, who, g)) return r;
  if (M == 0) return 0;
  float* ws = scratch_on(d);
  if (!ws) return -2;
  const bool q8 = scales != nullptr;
  Choice ch = gemm_pick(M, N, K, q8, d->cus);
  if (g_force_cfg >= 0 && g_force_cfg < kGemmNumCfgs && gemm_cfg_fits(g_force_cfg, q8, K)) {
    ch.cfg = g_force_cfg;
  } else {
    int mb = 16;
    while (mb < M && mb < 4096) mb *= 2;
    std::lock_guard<std::mutex> lk(g_tune_mu);
    auto it = g_tuned.find(std::make_tuple(d->id, mb, N, K, epi == 2, q8, false));
    if (it != g_tuned.end()) ch = it->second;
  }
  const size_t per_split = (size_t)M * N * sizeof(float);
  if (g_force_splits >= 1) {
    ch.splits = g_force_splits;
    const int nkt = (K + kGemmCfgs[ch.cfg].bk - 1) / kGemmCfgs[ch.cfg].bk;
    const int sp = std::min(ch.splits, nkt);
    if (sp > 1 && (size_t)sp * per_split > kScratchBytes)
      HI_FAIL("%s: %d splits of %d x %d fp32 partials need %zu bytes, over the %zu-byte static scratch", who, sp, M, N,
              (size_t)sp * per_split, kScratchBytes);
  } else {
    while (ch.splits > 1 && (size_t)ch.splits * per_split > kScratchBytes) ch.splits--;
  }
  return launch_choice(g, ch, epi, q8, (hipStream_t)stream, ws);
}

// X[M, N] += A[M, K] @ W[N, K]^T (epilogue 1, X contiguous), then Y = RMSNorm(X) * norm_w, as
// hi_gemm / hi_gemm_w8 (scales non-null) followed by hi_rmsnorm, with the same results bit for bit.
// When the launch splits K, the norm runs inside the split-K second pass (one kernel instead of
// two, one read of X fewer). No counterpart in the reference, whose engine runs the two in turn.
HI_EXPORT int hi_gemm_residual_rmsnorm(const void* A, int lda, const void* W, const void* scales, void* X, int M, int N,
                                       int K, const void* norm_w, float eps, void* Y, void* stream) {
  const char* who = "hi_gemm_residual_rmsnorm";
  if (M < 0) HI_FAIL("%s: M %d < 0", who, M);
  if (M == 0) return 0;
  if (!X || !Y || !norm_w || !aligned(X, 16) || !aligned(Y, 16) || !aligned(norm_w, 16))
    HI_FAIL("%s: X, Y and norm_w must be 16-byte aligned device pointers", who);
  return gemm_entry(A, lda, W, scales, nullptr, X, N, M, N, K, 1, stream, who, norm_w, Y, eps);
}

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
// Test hook: the tile config and split count the calling thread's last hi_gemm / hi_gemm_w8 launch
// ran with (after a forced config that does not fit fell back to the automatic choice, and splits
// were capped to the K tiles); -1 and 0 before any launch.
HI_EXPORT int hi_gemm_last_choice(int* cfg, int* splits) {
  if (cfg) *cfg = g_last.cfg;
  if (splits) *splits = g_last.splits;
  return 0;
}
HI_EXPORT int hi_gemm_config_desc(int c, char* out, int n) {
  if (c < 0 || c >= kGemmNumCfgs || !out || n < 1) return -1;
  snprintf(out, n, "mfma 32x32x16 %dx%dx%d waves %dx%dx%d stages %d", kGemmCfgs[c].bm, kGemmCfgs[c].bn, kGemmCfgs[c].bk,
           kGemmCfgs[c].wm, kGemmCfgs[c].wn, kGemmCfgs[c].kg, kGemmCfgs[c].st);
  return 0;
}
