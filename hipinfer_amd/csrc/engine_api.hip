// The reference's engine entry points over this library's launchers: weight-file loader
// (hi_load / hi_load_tp, api.cu:1235-1499), prefill (hi_prefill / hi_prefill_logits,
// api.cu:1807-1855), graph-captured greedy decode (hi_decode, api.cu:1891-2003), and the state
// accessors the reference's Python Engine uses (hi_config, hi_moe_config, hi_weight_bytes,
// hi_weight_quant, hi_history, hi_logits, hi_set_state, hi_rewind, hi_sync, hi_stream, hi_free;
// api.cu:1501-1546, 2110-2178), and speculative verification (hi_verify, hi_verify_max_rows;
// api.cu:2018-2108). One GPU: hi_load_tp accepts world = 1 only.
//
// Design for MI355X:
//  * the weight file (scripts/export.py format, versions 2 / 3 / 4) puts every tensor on a 256-byte
//    step after the header, so the file from the header on IS the device layout: it is streamed
//    verbatim into one device arena (double-buffered pinned staging, the disk read of one chunk
//    overlapping the copy of the previous), and tensor pointers are file offsets into the arena;
//  * all per-step state lives on the device (next token, position, history per slot), and every
//    state change is a kernel on the engine's stream, so a decode step is one captured hipGraph per
//    batch size, replayed;
//  * 1..HIPINFER_GEMV_MAX (default 8) sequences decode on the GEMV path (fused RMSNorm, fused
//    QKV+RoPE+cache write); more on the GEMM path. From 2 sequences on, the gate/up, down and
//    lm_head projections each take whichever path the first step of that batch size times faster
//    (the GEMM with a separate RMSNorm where the GEMV fuses it): at 5-8 rows the GEMV streams the
//    weights twice once the rows no longer fit in LDS (Llama-3.1-8B down, K = 14336), and int8
//    weights make it instruction-bound on the long launches. The first step of a batch size runs
//    eagerly (it tunes the GEMM tiles and these paths, and sets kernel attributes, which capture
//    cannot), the rest replay the graph captured after it.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <vector>

#include "../../include/hipinfer.h"
#include "hi_common.h"
#include "hi_internal.h"

namespace {

constexpr int32_t kMagic = 0x48495046;
// rows per verify (k + 1 for k draft tokens), the reference's kGemvMaxRows (api.cu:156). The GEMV
// host runs fused-norm launches of at most 8 rows, so 9..16 rows take two launches per projection;
// a row's arithmetic does not depend on the launch it is in.
constexpr int kVerifyMaxRows = 16;

struct Cfg {
  int vocab = 0, hidden = 0, inter = 0, layers = 0, heads = 0, kv = 0, head_dim = 0, max_pos = 0, window = 0;
  float eps = 1e-5f, attn_scaling = 1.f;
  bool tied = false, qkv_bias = false, moe = false, qk_norm = false;
  int n_experts = 0, top_k = 0, moe_flags = 0, quant = 0;
  float moe_scale = 1.f;
};

struct Wt {  // a projection [N, K]: fp16, or int8 with fp16 row scales
  const void* w = nullptr;
  const f16* s = nullptr;
};

struct Layer {
  const f16 *n1 = nullptr, *n2 = nullptr, *bqkv = nullptr;
  Wt qkv, o, gu, down;
  const f16 *router = nullptr, *ewgu = nullptr, *ewdown = nullptr;  // MoE
};

}  // namespace

struct Engine {
  int dev = 0;
  Cfg c;
  int maxB = 0, max_seq = 0, max_pf = 0, Mmax = 0, qkv_dim = 0, gemv_max = 8;
  char* arena = nullptr;  // the weight file after its header
  size_t arena_bytes = 0;
  const f16 *embed = nullptr, *final_norm = nullptr;
  Wt lm;
  std::vector<Layer> L;
  f16 *kc = nullptr, *vc = nullptr;
  size_t layer_cache = 0;  // elements per layer per cache (maxB * Hkv * max_seq * D)
  f16 *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *act = nullptr, *logits = nullptr;
  int *tok = nullptr, *pos = nullptr, *hist = nullptr, *ptok = nullptr, *moe_idx = nullptr;
  float* moe_w = nullptr;
  void *work = nullptr, *moe_work = nullptr;
  f16x2* rope = nullptr;
  hipStream_t st = nullptr;
  std::vector<hipGraphExec_t> graphs;
  // per batch size of 2..gemv_max sequences: the projections that run on the GEMM path (bit 0
  // gate/up, bit 1 down, bit 2 lm_head), timed on the first eager step of that size
  std::map<int, int> small_gemm;
  std::map<std::pair<int, int>, hipGraphExec_t> vgraphs;  // verify step per (slot, rows)
  int *v_tok = nullptr, *v_pos = nullptr, *v_out = nullptr;
  f16* v_logits = nullptr;
  void* v_work = nullptr;
  std::vector<void*> allocs;
};

namespace {

#define EN_REQ(cond, ...)             \
  do {                                \
    if (!(cond)) {                    \
      fprintf(stderr, __VA_ARGS__);   \
      fputc('\n', stderr);            \
      return false;                   \
    }                                 \
  } while (0)
// A launcher or HIP call inside an engine step: on failure the reason is on stderr already.
#define EN_TRY(call)                                                                    \
  do {                                                                                  \
    const int en_rc_ = (call);                                                          \
    if (en_rc_) {                                                                       \
      fprintf(stderr, "hipinfer_amd engine: %s failed (%d) at %s:%d\n", #call, en_rc_, \
              __FILE__, __LINE__);                                                      \
      return en_rc_;                                                                    \
    }                                                                                   \
  } while (0)

__global__ void set_int_kernel(int* p, int i, int v) { p[i] = v; }

// Greedy emit for slots [b0, b0 + B): the token tok[b] (written by the argmax) is the input of the
// next step at position pos[b] + 1, and is recorded in the slot's history there (the reference's
// emit_token, kernels.cuh:1916-1923).
__global__ void emit_kernel(const int* tok, int* pos, int* hist, int b0, int B, int max_seq) {
  const int b = b0 + (int)threadIdx.x;
  if ((int)threadIdx.x >= B) return;
  const int p = pos[b] + 1;
  pos[b] = p;
  if (p < max_seq) hist[(int64_t)b * max_seq + p] = tok[b];
}

void* dalloc(Engine* e, size_t bytes) {
  void* p = nullptr;
  if (hipMalloc(&p, bytes ? bytes : 256) != hipSuccess) {
    (void)hipGetLastError();
    fprintf(stderr, "hi_load: device allocation of %zu bytes failed\n", bytes);
    return nullptr;
  }
  e->allocs.push_back(p);
  return p;
}

void free_engine(Engine* e) {
  if (!e) return;
  (void)hipSetDevice(e->dev);
  if (e->st) (void)hipStreamSynchronize(e->st);
  for (auto g : e->graphs)
    if (g) (void)hipGraphExecDestroy(g);
  for (auto& g : e->vgraphs)
    if (g.second) (void)hipGraphExecDestroy(g.second);
  for (void* p : e->allocs) (void)hipFree(p);
  if (e->st) (void)hipStreamDestroy(e->st);
  delete e;
}

// Stream file bytes [from, to) into dst through two pinned staging buffers.
bool stream_file(FILE* f, size_t from, size_t to, char* dst, hipStream_t s) {
  constexpr size_t kChunk = 64 << 20;
  char* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  bool ok = true;
  for (int i = 0; i < 2 && ok; i++) {
    ok = hipHostMalloc((void**)&stage[i], kChunk, hipHostMallocDefault) == hipSuccess &&
         hipEventCreateWithFlags(&done[i], hipEventDisableTiming) == hipSuccess;
  }
  if (ok && fseek(f, (long)from, SEEK_SET)) ok = false;
  int k = 0;
  for (size_t o = from; ok && o < to; o += kChunk, k ^= 1) {
    const size_t n = to - o < kChunk ? to - o : kChunk;
    ok = hipEventSynchronize(done[k]) == hipSuccess;  // the copy that last used this buffer is done
    if (ok && fread(stage[k], 1, n, f) != n) {
      fprintf(stderr, "hi_load: weight file too small\n");
      ok = false;
    }
    ok = ok && hipMemcpyAsync(dst + (o - from), stage[k], n, hipMemcpyHostToDevice, s) == hipSuccess &&
         hipEventRecord(done[k], s) == hipSuccess;
  }
  if (hipStreamSynchronize(s) != hipSuccess) ok = false;
  for (int i = 0; i < 2; i++) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  if (!ok) (void)hipGetLastError();
  return ok;
}

bool parse_header(FILE* f, Cfg& c, size_t& base) {
  int32_t hdr[32] = {0};
  EN_REQ(fread(hdr, 4, 16, f) == 16 && hdr[0] == kMagic, "hi_load: bad weight file");
  const int ver = hdr[1];
  EN_REQ(ver >= 2 && ver <= 4, "hi_load: weight file version %d (2 dense, 3 MoE, 4 int8)", ver);
  if (ver == 3) EN_REQ(fread(hdr + 16, 4, 16, f) == 16, "hi_load: bad weight file");
  base = ver == 3 ? 128 : 64;
  c.vocab = hdr[2], c.hidden = hdr[3], c.inter = hdr[4], c.layers = hdr[5];
  c.heads = hdr[6], c.kv = hdr[7], c.head_dim = hdr[8], c.max_pos = hdr[9];
  memcpy(&c.eps, &hdr[10], 4);
  memcpy(&c.attn_scaling, &hdr[11], 4);
  c.tied = hdr[12] & 1, c.qkv_bias = (hdr[12] & 2) != 0, c.moe = (hdr[12] & 4) != 0, c.qk_norm = (hdr[12] & 8) != 0;
  c.window = hdr[13];
  if (c.moe) {
    c.n_experts = hdr[16], c.top_k = hdr[17], c.moe_flags = hdr[18];
    memcpy(&c.moe_scale, &hdr[19], 4);
  }
  if (ver == 4) {
    EN_REQ(hdr[14] == 1, "hi_load: unknown quantization type %d", hdr[14]);
    EN_REQ(!c.moe && !c.tied, "hi_load: version-4 file with the MoE or tied flag set");
    c.quant = 1;
  }
  EN_REQ(c.moe == (ver == 3), "hi_load: MoE flag does not match file version %d", ver);
  EN_REQ(!c.qk_norm, "hi_load: QK-norm models are not supported");
  EN_REQ(c.vocab > 0 && c.hidden > 0 && c.inter > 0 && c.layers > 0 && c.heads > 0 && c.kv > 0,
         "hi_load: bad model shape in the header");
  EN_REQ(c.head_dim == 64 || c.head_dim == 128, "hi_load: head_dim %d not supported (64 or 128)", c.head_dim);
  EN_REQ(c.heads % c.kv == 0 && c.heads / c.kv <= 8, "hi_load: unsupported GQA group %d/%d", c.heads, c.kv);
  EN_REQ(c.hidden % 32 == 0 && c.inter % 16 == 0 && c.vocab % 16 == 0,
         "hi_load: hidden %% 32, intermediate %% 16 and vocab %% 16 must be 0 (%d, %d, %d)", c.hidden, c.inter,
         c.vocab);
  if (c.moe)
    EN_REQ(c.n_experts >= 1 && c.n_experts <= kMoeMaxE && c.top_k >= 1 && c.top_k <= c.n_experts &&
               c.top_k <= kMoeMaxK && c.inter % 32 == 0,
           "hi_load: unsupported MoE shape: %d experts, top-%d, expert inter %d (at most %d experts, top-%d)",
           c.n_experts, c.top_k, c.inter, kMoeMaxE, kMoeMaxK);
  return true;
}

// Walk the file layout (scripts/export.py:269-297) and point every tensor into the arena; returns
// the bytes the layout spans after the header.
size_t place(Engine* e, size_t base) {
  const Cfg& c = e->c;
  const size_t H = c.hidden, I = c.inter, D = c.head_dim, V = c.vocab, wsz = c.quant ? 1 : 2;
  const size_t QKV = (size_t)(c.heads + 2 * c.kv) * D;
  size_t off = base;
  auto next = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return e->arena + (o - base);
  };
  auto proj = [&](size_t N, size_t K) {
    Wt t;
    t.w = next(N * K * wsz);
    if (c.quant) t.s = (const f16*)next(N * 2);
    return t;
  };
  next(D / 2 * 4);  // inv_freq, read on the host
  e->embed = (const f16*)next(V * H * 2);
  e->final_norm = (const f16*)next(H * 2);
  e->lm = c.tied ? Wt{e->embed, nullptr} : proj(V, H);
  e->L.assign(c.layers, Layer{});
  for (auto& l : e->L) {
    l.n1 = (const f16*)next(H * 2);
    l.qkv = proj(QKV, H);
    if (c.qkv_bias) l.bqkv = (const f16*)next(QKV * 2);
    l.o = proj(H, (size_t)c.heads * D);
    l.n2 = (const f16*)next(H * 2);
    if (c.moe) {
      const size_t E = c.n_experts;
      l.router = (const f16*)next(E * H * 2);
      l.ewgu = (const f16*)next(E * 2 * I * H * 2);
      l.ewdown = (const f16*)next(E * H * I * 2);
    } else {
      l.gu = proj(2 * I, H);
      l.down = proj(H, I);
    }
  }
  return off - base;
}

// ---- the launchers a step needs, fp16 or int8 by the weight
int gemv(Engine* e, const void* x, int ldx, const f16* normw, const Wt& W, void* out, int ldo, int M, int N, int K,
         int epi) {
  if (W.s) return hi_gemv_w8(x, ldx, normw, e->c.eps, W.w, W.s, out, ldo, M, N, K, epi, e->st);
  return hi_gemv(x, ldx, normw, e->c.eps, W.w, out, ldo, M, N, K, epi, e->st);
}
int gemm(Engine* e, const void* A, int lda, const Wt& W, const f16* bias, void* C, int ldc, int M, int N, int K,
         int epi) {
  if (W.s) return hi_gemm_w8(A, lda, W.w, W.s, bias, C, ldc, M, N, K, epi, e->st);
  return hi_gemm(A, lda, W.w, bias, C, ldc, M, N, K, epi, e->st);
}

// X += A @ W^T, then Y = RMSNorm(X; nw): the residual GEMM and the norm that reads its result in
// one call (the norm inside the split-K second pass when the GEMM splits K)
int gemm_norm(Engine* e, const void* A, int lda, const Wt& W, f16* X, int M, int N, int K, const f16* nw, f16* Y) {
  return hi_gemm_residual_rmsnorm(A, lda, W.w, W.s, X, M, N, K, nw, e->c.eps, Y, e->st);
}

// x[rows] += MoE(RMSNorm(x; n2)) (router + experts; api.cu:1694-1703)
int moe_rows(Engine* e, const Layer& w, f16* x, f16* xn, int m) {
  const Cfg& c = e->c;
  const int H = c.hidden;
  EN_TRY(hi_rmsnorm(x, w.n2, xn, m, H, c.eps, e->st));
  // router and experts in one call: the same bits as the reference's two calls, with the router
  // inside the gate/up launch on the GEMV path
  EN_TRY(hi_moe_route_experts(xn, H, w.router, w.ewgu, w.ewdown, m, c.n_experts, c.top_k, H, c.inter, c.moe_flags,
                              c.moe_scale, x, H, e->moe_idx, e->moe_w, e->moe_work, e->st));
  return 0;
}

enum { kGuGemm = 1, kDownGemm = 2, kLmGemm = 4 };

// The projections of a B-sequence decode step (2 <= B <= gemv_max) that run on the GEMM path, by a
// fixed rule on the shapes (from step times measured both ways on Llama-3.1-8B and Qwen2.5-1.5B,
// fp16 and int8, at 2-8 sequences):
//  - down, when its B activation rows (K = inter) do not fit one GEMV launch's LDS together (the
//    GEMV would run in row chunks, each streaming the weights), or with int8 weights from 5 rows
//    on, where the int8 GEMV's per-row dot products make it instruction-bound;
//  - lm_head with int8 weights at 8 rows, for the same reason (with the GEMV's exact 5-7-row
//    instances the GEMV lm_head is as fast or faster below that).
// gate/up, QKV and o stay on the GEMV. The choice depends only on the model's shapes, its weight
// format and B, so every process and every box runs the same kernels for a batch size. A row of a
// B-sequence step whose down or lm_head runs on the GEMM is not bit-identical to a batch-of-one
// step of that sequence (the verify path keeps the GEMVs for that reason).
int small_paths_rule(const Engine* e, int B) {
  const Cfg& c = e->c;
  if (B < 2) return 0;
  const bool q8 = e->lm.s != nullptr;
  int mask = 0;
  if (!c.moe) {
    const bool dq8 = e->L[0].down.s != nullptr;
    const int fit = gemv_rows_per_launch(c.inter, false, dq8);
    if (B > fit || (dq8 && B >= 5)) mask |= kDownGemm;
  }
  if (q8 && B >= 8) mask |= kLmGemm;
  return mask;
}

// The same choice made by timing: each of gate/up, down and lm_head is timed both ways on scratch
// rows (the weights of up to 8 layers in turn, so they stream from HBM as in a step), the GEMM side
// with the RMSNorm the GEMV fuses; the GEMM must win by 3 %. Used with HIPINFER_SMALL_GEMM=tune;
// HIPINFER_SMALL_GEMM=<mask> sets the mask; unset, small_paths_rule decides.
int tune_small_paths(Engine* e, int B, int* mask) {
  if (const char* env = getenv("HIPINFER_SMALL_GEMM")) {
    if (strcmp(env, "tune") != 0) {
      *mask = atoi(env) & 7;
      return 0;
    }
  } else {
    *mask = small_paths_rule(e, B);
    return 0;
  }
  const Cfg& c = e->c;
  const int H = c.hidden, I = c.inter, V = c.vocab;
  hipStream_t s = e->st;
  f16 *xs = nullptr, *xn = nullptr, *act = nullptr, *x2 = nullptr, *lg = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  const size_t hb = (size_t)B * H * 2, ib = (size_t)B * (c.moe ? 1 : I) * 2, vb = (size_t)B * V * 2;
  if (hipMalloc(&xs, hb) != hipSuccess || hipMalloc(&xn, hb) != hipSuccess || hipMalloc(&x2, hb) != hipSuccess ||
      hipMalloc(&act, ib) != hipSuccess || hipMalloc(&lg, vb) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess || hipMemsetAsync(xs, 0, hb, s) != hipSuccess ||
      hipMemsetAsync(x2, 0, hb, s) != hipSuccess || hipMemsetAsync(act, 0, ib, s) != hipSuccess)
    rc = -2;
  const int nl = std::min<int>(c.layers, 8), reps = std::max(8, 2 * nl);
  // microseconds per call of fn(layer), after one untimed call on each of two layers (which also
  // tunes the GEMM tiles of these shapes)
  auto time_us = [&](auto fn, float* us) -> int {
    for (int l = 0; l < std::min(nl, 2); l++)
      if (int r = fn(l)) return r;
    if (hipEventRecord(e0, s) != hipSuccess) return -2;
    for (int r = 0; r < reps; r++)
      if (int rr = fn(r % nl)) return rr;
    float ms = 0.f;
    if (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
      return -2;
    *us = ms * 1e3f / reps;
    return 0;
  };
  auto pick = [&](int bit, auto gemv_fn, auto gemm_fn) -> int {
    float tv = 0.f, tm = 0.f;
    if (int r = time_us(gemv_fn, &tv)) return r;
    if (int r = time_us(gemm_fn, &tm)) return r;
    if (tm < 0.97f * tv) *mask |= bit;
    return 0;
  };
  *mask = 0;
  if (!rc && !c.moe) {
    rc = pick(
        kGuGemm, [&](int l) { return gemv(e, xs, H, e->L[l].n2, e->L[l].gu, act, I, B, 2 * I, H, 2); },
        [&](int l) {
          const int r = hi_rmsnorm(xs, e->L[l].n2, xn, B, H, c.eps, s);
          return r ? r : gemm(e, xn, H, e->L[l].gu, nullptr, act, I, B, 2 * I, H, 2);
        });
    if (!rc)
      rc = pick(
          kDownGemm, [&](int l) { return gemv(e, act, I, nullptr, e->L[l].down, x2, H, B, H, I, 1); },
          [&](int l) { return gemm(e, act, I, e->L[l].down, nullptr, x2, H, B, H, I, 1); });
  }
  if (!rc)
    rc = pick(
        kLmGemm, [&](int) { return gemv(e, xs, H, e->final_norm, e->lm, lg, V, B, V, H, 0); },
        [&](int) {
          const int r = hi_rmsnorm(xs, e->final_norm, xn, B, H, c.eps, s);
          return r ? r : gemm(e, xn, H, e->lm, nullptr, lg, V, B, V, H, 0);
        });
  (void)hipStreamSynchronize(s);
  for (void* p : {(void*)xs, (void*)xn, (void*)act, (void*)x2, (void*)lg})
    if (p) (void)hipFree(p);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  return rc;
}

// One greedy decode step for slots [0, B) (api.cu:1891-1952): reads tok / pos, writes the next
// token, advances pos, appends to the history.
int decode_step(Engine* e, int B) {
  const Cfg& c = e->c;
  const int H = c.hidden, D = c.head_dim, Hq = c.heads, Hkv = c.kv, HD = Hq * D, I = c.inter, V = c.vocab;
  const bool small = B <= e->gemv_max;
  hipStream_t s = e->st;
  int sg = 0;  // projections of this batch size on the GEMM path (the GEMV path's are the rest)
  if (small && B > 1) {
    auto it = e->small_gemm.find(B);
    if (it != e->small_gemm.end()) {
      sg = it->second;
    } else {
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      EN_TRY(hipStreamIsCapturing(s, &cap));
      if (cap == hipStreamCaptureStatusNone) {  // chosen once, eagerly; a capture keeps the GEMVs
        EN_TRY(tune_small_paths(e, B, &sg));
        e->small_gemm[B] = sg;
      }
    }
  }
  EN_TRY(hi_embed(e->tok, e->embed, V, H, e->x, H, B, s));
  bool xn_ready = false;  // xn already holds RMSNorm(x) for the next consumer (from a down GEMM)
  for (int l = 0; l < c.layers; l++) {
    const Layer& w = e->L[l];
    f16* kc = e->kc + e->layer_cache * l;
    f16* vc = e->vc + e->layer_cache * l;
    if (small) {
      if (w.qkv.s)
        EN_TRY(hi_gemv_qkv_rope_w8(e->x, H, w.n1, c.eps, w.qkv.w, w.qkv.s, w.bqkv, e->qkv, e->qkv_dim, B, H, Hq, Hkv, D,
                                   e->rope, e->pos, kc, vc, e->max_seq, s));
      else
        EN_TRY(hi_gemv_qkv_rope(e->x, H, w.n1, c.eps, w.qkv.w, w.bqkv, e->qkv, e->qkv_dim, B, H, Hq, Hkv, D, e->rope,
                                e->pos, kc, vc, e->max_seq, s));
    } else {
      if (!xn_ready) EN_TRY(hi_rmsnorm(e->x, w.n1, e->xn, B, H, c.eps, s));
      EN_TRY(gemm(e, e->xn, H, w.qkv, w.bqkv, e->qkv, e->qkv_dim, B, e->qkv_dim, H, 0));
      EN_TRY(hi_rope_cache(e->qkv, e->qkv_dim, B, Hq, Hkv, D, e->rope, e->pos, 0, 0, kc, vc, e->max_seq, s));
    }
    xn_ready = false;
    EN_TRY(hi_decode_attn(e->qkv, e->qkv_dim, kc, vc, e->max_seq, e->pos, e->att, HD, B, Hq, Hkv, D, e->work, s));
    if (small) EN_TRY(gemv(e, e->att, HD, nullptr, w.o, e->x, H, B, H, HD, 1));
    else if (c.moe) EN_TRY(gemm(e, e->att, HD, w.o, nullptr, e->x, H, B, H, HD, 1));
    else EN_TRY(gemm_norm(e, e->att, HD, w.o, e->x, B, H, HD, w.n2, e->xn));
    if (c.moe) {
      EN_TRY(moe_rows(e, w, e->x, e->xn, B));
      continue;
    }
    if (small) {
      if (sg & kGuGemm) {
        EN_TRY(hi_rmsnorm(e->x, w.n2, e->xn, B, H, c.eps, s));
        EN_TRY(gemm(e, e->xn, H, w.gu, nullptr, e->act, I, B, 2 * I, H, 2));
      } else {
        EN_TRY(gemv(e, e->x, H, w.n2, w.gu, e->act, I, B, 2 * I, H, 2));
      }
      if (sg & kDownGemm) EN_TRY(gemm(e, e->act, I, w.down, nullptr, e->x, H, B, H, I, 1));
      else EN_TRY(gemv(e, e->act, I, nullptr, w.down, e->x, H, B, H, I, 1));
    } else {  // xn = RMSNorm(x; n2) from the o GEMM's call
      EN_TRY(gemm(e, e->xn, H, w.gu, nullptr, e->act, I, B, 2 * I, H, 2));
      const f16* nn = l + 1 < c.layers ? e->L[l + 1].n1 : e->final_norm;
      EN_TRY(gemm_norm(e, e->act, I, w.down, e->x, B, H, I, nn, e->xn));
      xn_ready = true;
    }
  }
  if (small && !(sg & kLmGemm)) {
    EN_TRY(gemv(e, e->x, H, e->final_norm, e->lm, e->logits, V, B, V, H, 0));
  } else {
    if (!xn_ready) EN_TRY(hi_rmsnorm(e->x, e->final_norm, e->xn, B, H, c.eps, s));
    EN_TRY(gemm(e, e->xn, H, e->lm, nullptr, e->logits, V, B, V, H, 0));
  }
  EN_TRY(hi_argmax(e->logits, B, V, e->tok, s));
  hipLaunchKernelGGL(emit_kernel, dim3(1), dim3(64), 0, s, e->tok, e->pos, e->hist, 0, B, e->max_seq);
  EN_TRY(hipGetLastError());
  return 0;
}

// Speculative verification rows (api.cu:2018-2067): R tokens of slot `slot` at positions v_pos
// through the kernels of a batch-of-one decode step, R activation rows: the GEMVs (row r's
// arithmetic does not depend on the row count) and decode attention with every query reading this
// slot, at a batch of one's split count. All rows' k / v are written before any attention runs and
// row r reads positions <= v_pos[r] only, so row r's logits, and the k / v it leaves, are
// bit-identical to a plain decode step at v_pos[r]. v_out[r] = the greedy token after row r.
int verify_step(Engine* e, int slot, int R) {
  const Cfg& c = e->c;
  const int H = c.hidden, D = c.head_dim, Hq = c.heads, Hkv = c.kv, HD = Hq * D, I = c.inter, V = c.vocab;
  hipStream_t s = e->st;
  EN_TRY(hi_embed(e->v_tok, e->embed, V, H, e->x, H, R, s));
  for (int l = 0; l < c.layers; l++) {
    const Layer& w = e->L[l];
    f16* kc = e->kc + e->layer_cache * l;
    f16* vc = e->vc + e->layer_cache * l;
    EN_TRY(gemv_qkv_rope_slot(e->x, H, w.n1, c.eps, w.qkv.w, w.qkv.s, w.bqkv, e->qkv, e->qkv_dim, R, H, Hq, Hkv, D,
                              e->rope, e->v_pos, kc, vc, e->max_seq, slot, s));
    EN_TRY(decode_attn_slot(e->qkv, e->qkv_dim, kc, vc, e->max_seq, e->v_pos, e->att, HD, R, Hq, Hkv, D, e->v_work, slot,
                            s));
    EN_TRY(gemv(e, e->att, HD, nullptr, w.o, e->x, H, R, H, HD, 1));
    EN_TRY(gemv(e, e->x, H, w.n2, w.gu, e->act, I, R, 2 * I, H, 2));
    EN_TRY(gemv(e, e->act, I, nullptr, w.down, e->x, H, R, H, I, 1));
  }
  EN_TRY(gemv(e, e->x, H, e->final_norm, e->lm, e->v_logits, V, R, V, H, 0));
  EN_TRY(hi_argmax(e->v_logits, R, V, e->v_out, s));
  return 0;
}

template <class F>
int capture(Engine* e, F step, hipGraphExec_t* out) {
  hipGraph_t g = nullptr;
  EN_TRY(hipStreamBeginCapture(e->st, hipStreamCaptureModeThreadLocal));
  const int rc = step();
  const hipError_t end = hipStreamEndCapture(e->st, &g);
  if (rc || end != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return rc ? rc : -2;
  }
  const hipError_t ins = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  return ins == hipSuccess ? 0 : -2;
}

int capture_step(Engine* e, int B, hipGraphExec_t* out) {
  return capture(e, [&] { return decode_step(e, B); }, out);
}

bool tokens_ok(const Engine* e, const int* tok, int n, const char* who) {
  EN_REQ(tok || n == 0, "%s: null token array", who);
  for (int i = 0; i < n; i++)
    EN_REQ(tok[i] >= 0 && tok[i] < e->c.vocab, "%s: token %d at %d outside vocab %d", who, tok[i], i, e->c.vocab);
  return true;
}

bool prefill_ok(const Engine* e, int slot, const int* tokens, int T, int p0, const char* who) {
  EN_REQ(e, "%s: null engine", who);
  EN_REQ(slot >= 0 && slot < e->maxB, "%s: slot %d outside [0, max_batch %d)", who, slot, e->maxB);
  EN_REQ(T >= 1 && p0 >= 0 && (long long)p0 + T <= e->max_seq, "%s: T %d at p0 %d outside max_seq %d", who, T, p0,
         e->max_seq);
  return tokens_ok(e, tokens, T, who);
}

// Prefill T tokens into slot at positions p0.. (api.cu:1807-1845); all_logits (device, [T, vocab])
// optional. Leaves the greedy next token in tok[slot], its position in pos[slot].
int prefill(Engine* e, int slot, const int* tokens, int T, int p0, f16* all_logits) {
  const Cfg& c = e->c;
  const int H = c.hidden, D = c.head_dim, Hq = c.heads, Hkv = c.kv, HD = Hq * D, I = c.inter, V = c.vocab;
  hipStream_t s = e->st;
  int n = 0;
  for (int t0 = 0; t0 < T; t0 += e->max_pf) {
    n = T - t0 < e->max_pf ? T - t0 : e->max_pf;
    const int pb = p0 + t0;
    EN_TRY(hipMemcpyAsync(e->ptok, tokens + t0, (size_t)n * 4, hipMemcpyHostToDevice, s));
    EN_TRY(hi_embed(e->ptok, e->embed, V, H, e->x, H, n, s));
    bool xn_ready = false;  // xn already holds RMSNorm(x) for the next consumer (from a down GEMM)
    for (int l = 0; l < c.layers; l++) {
      const Layer& w = e->L[l];
      f16* kc = e->kc + e->layer_cache * l;
      f16* vc = e->vc + e->layer_cache * l;
      if (!xn_ready) EN_TRY(hi_rmsnorm(e->x, w.n1, e->xn, n, H, c.eps, s));
      xn_ready = false;
      EN_TRY(gemm(e, e->xn, H, w.qkv, w.bqkv, e->qkv, e->qkv_dim, n, e->qkv_dim, H, 0));
      EN_TRY(hi_rope_cache(e->qkv, e->qkv_dim, n, Hq, Hkv, D, e->rope, nullptr, pb, slot, kc, vc, e->max_seq, s));
      const size_t so = (size_t)slot * Hkv * e->max_seq * D;
      EN_TRY(hi_flash_prefill(e->qkv, e->qkv_dim, kc + so, vc + so, e->max_seq, e->att, HD, n, pb, Hq, Hkv, D, s));
      if (c.moe) {
        EN_TRY(gemm(e, e->att, HD, w.o, nullptr, e->x, H, n, H, HD, 1));
        EN_TRY(moe_rows(e, w, e->x, e->xn, n));
        continue;
      }
      EN_TRY(gemm_norm(e, e->att, HD, w.o, e->x, n, H, HD, w.n2, e->xn));
      EN_TRY(gemm(e, e->xn, H, w.gu, nullptr, e->act, I, n, 2 * I, H, 2));
      const f16* nn = l + 1 < c.layers ? e->L[l + 1].n1 : e->final_norm;
      EN_TRY(gemm_norm(e, e->act, I, w.down, e->x, n, H, I, nn, e->xn));
      xn_ready = true;
    }
    if (all_logits) {
      if (!xn_ready) EN_TRY(hi_rmsnorm(e->x, e->final_norm, e->xn, n, H, c.eps, s));
      EN_TRY(gemm(e, e->xn, H, e->lm, nullptr, all_logits + (size_t)t0 * V, V, n, V, H, 0));
    }
  }
  f16* lg = e->logits + (size_t)slot * V;
  EN_TRY(gemv(e, e->x + (size_t)(n - 1) * H, H, e->final_norm, e->lm, lg, V, 1, V, H, 0));
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, s, e->pos, slot, p0 + T - 1);
  EN_TRY(hi_argmax(lg, 1, V, e->tok + slot, s));
  hipLaunchKernelGGL(emit_kernel, dim3(1), dim3(64), 0, s, e->tok, e->pos, e->hist, slot, 1, e->max_seq);
  EN_TRY(hipGetLastError());
  return 0;
}

Engine* load(const char* path, int maxB, int max_seq, int max_pf) {
  if (!hi_device()) return nullptr;
  if (!path || maxB < 1 || max_seq < 1 || max_pf < 1) {
    fprintf(stderr, "hi_load: a path, max_batch (%d), max_seq (%d) and max_prefill (%d) >= 1 are required\n", maxB,
            max_seq, max_pf);
    return nullptr;
  }
  FILE* f = fopen(path, "rb");
  if (!f) {
    fprintf(stderr, "hi_load: cannot open %s\n", path);
    return nullptr;
  }
  Engine* e = new Engine();
  auto fail = [&]() -> Engine* {
    fclose(f);
    free_engine(e);
    return nullptr;
  };
  (void)hipGetDevice(&e->dev);
  size_t base = 0;
  if (!parse_header(f, e->c, base)) return fail();
  const Cfg& c = e->c;
  if (c.window > 0 && max_seq > c.window) {
    fprintf(stderr, "hi_load: sliding-window model (%d tokens): max_seq %d must be <= %d\n", c.window, max_seq,
            c.window);
    return fail();
  }
  if ((long long)maxB * c.kv > 4096 || maxB > 64) {
    fprintf(stderr, "hi_load: max_batch %d (x %d kv heads) too large (at most 64 sequences, 4096 sequence-heads)\n",
            maxB, c.kv);
    return fail();
  }
  if (hipStreamCreate(&e->st) != hipSuccess) return fail();
  e->maxB = maxB, e->max_seq = max_seq, e->max_pf = max_pf, e->gemv_max = hi_gemv_max_rows();
  const int H = c.hidden, D = c.head_dim, Hq = c.heads, Hkv = c.kv, I = c.inter, V = c.vocab;
  e->qkv_dim = (Hq + 2 * Hkv) * D;
  std::vector<float> inv(D / 2);
  if (fseek(f, (long)base, SEEK_SET) || fread(inv.data(), 4, D / 2, f) != (size_t)D / 2) {
    fprintf(stderr, "hi_load: weight file too small\n");
    return fail();
  }
  // size the layout with a dry walk, then stream the file into the arena
  e->arena = nullptr;
  const size_t span = place(e, base);
  e->arena = (char*)dalloc(e, span);
  if (!e->arena) return fail();
  e->arena_bytes = span;
  place(e, base);
  if (fseek(f, 0, SEEK_END) || (size_t)ftell(f) < base + span - 255) {
    fprintf(stderr, "hi_load: weight file too small for its header's model\n");
    return fail();
  }
  const size_t fend = (size_t)ftell(f) < base + span ? (size_t)ftell(f) : base + span;
  if (!stream_file(f, base, fend, e->arena, e->st)) return fail();
  fclose(f);
  f = nullptr;
  auto fail2 = [&]() -> Engine* {
    free_engine(e);
    return nullptr;
  };

  e->Mmax = ((max_pf > maxB ? max_pf : maxB) + 127) / 128 * 128;
  e->layer_cache = (size_t)maxB * Hkv * max_seq * D;
  const size_t M = e->Mmax;
  bool ok = (e->kc = (f16*)dalloc(e, e->layer_cache * c.layers * 2)) && (e->vc = (f16*)dalloc(e, e->layer_cache * c.layers * 2)) &&
            (e->x = (f16*)dalloc(e, M * H * 2)) && (e->xn = (f16*)dalloc(e, M * H * 2)) &&
            (e->qkv = (f16*)dalloc(e, M * e->qkv_dim * 2)) && (e->att = (f16*)dalloc(e, M * Hq * D * 2)) &&
            (e->act = (f16*)dalloc(e, M * I * 2)) && (e->logits = (f16*)dalloc(e, (size_t)maxB * V * 2)) &&
            (e->tok = (int*)dalloc(e, maxB * 4)) && (e->pos = (int*)dalloc(e, maxB * 4)) &&
            (e->hist = (int*)dalloc(e, (size_t)maxB * max_seq * 4)) && (e->ptok = (int*)dalloc(e, M * 4)) &&
            (e->work = dalloc(e, hi_decode_work_bytes(maxB, Hq, Hkv, D)));
  if (ok && c.moe)
    ok = (e->moe_idx = (int*)dalloc(e, M * c.top_k * 4)) && (e->moe_w = (float*)dalloc(e, M * c.top_k * 4)) &&
         (e->moe_work = dalloc(e, hi_moe_work_bytes((int)M, c.top_k, c.n_experts, H, I)));
  if (!ok) return fail2();
  // zeroed state (the decode and MoE work buffers' counters must start consistent); caches too, so an
  // unwritten position reads as zero, never as stale memory
  ok = hipMemsetAsync(e->kc, 0, e->layer_cache * c.layers * 2, e->st) == hipSuccess &&
       hipMemsetAsync(e->vc, 0, e->layer_cache * c.layers * 2, e->st) == hipSuccess &&
       hipMemsetAsync(e->work, 0, hi_decode_work_bytes(maxB, Hq, Hkv, D), e->st) == hipSuccess &&
       hipMemsetAsync(e->tok, 0, maxB * 4, e->st) == hipSuccess && hipMemsetAsync(e->pos, 0, maxB * 4, e->st) == hipSuccess &&
       hipMemsetAsync(e->hist, 0, (size_t)maxB * max_seq * 4, e->st) == hipSuccess &&
       (!c.moe || hipMemsetAsync(e->moe_work, 0, hi_moe_work_bytes((int)M, c.top_k, c.n_experts, H, I), e->st) == hipSuccess);
  if (!ok) return fail2();
  // RoPE table as HF computes it: fp32 inv_freq (from the export) times the fp32 position, cos and
  // sin of that fp32 angle times attention_scaling, rounded to fp16 (api.cu:1421-1431)
  std::vector<f16x2> rt((size_t)max_seq * (D / 2));
  for (int i = 0; i < D / 2; i++)
    for (int p = 0; p < max_seq; p++) {
      const float a = (float)p * inv[i];
      rt[(size_t)p * (D / 2) + i] = f16x2{(f16)((float)cos((double)a) * c.attn_scaling),
                                          (f16)((float)sin((double)a) * c.attn_scaling)};
    }
  if (!(e->rope = (f16x2*)dalloc(e, rt.size() * 4)) ||
      hipMemcpy(e->rope, rt.data(), rt.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipStreamSynchronize(e->st) != hipSuccess)
    return fail2();
  e->graphs.assign(maxB + 1, nullptr);
  return e;
}

}  // namespace

// Load a weight file (scripts/export.py versions 2, 3, 4) onto the current GPU for up to max_batch
// sequences of max_seq positions, prefilling at most max_prefill rows per chunk. world must be 1
// (this build runs one GPU); devs (optional) names the GPU. Returns null after a message on stderr
// for a bad file or unsupported model / setting. Replaces api.cu:1475-1497 (hi_load_tp).
HI_EXPORT Engine* hi_load_tp(const char* path, int max_batch, int max_seq, int max_prefill, int world,
                             const int* devs) {
  if (world != 1) {
    fprintf(stderr, "hi_load_tp: this build runs one GPU per engine (world %d requested)\n", world);
    return nullptr;
  }
  if (devs && hipSetDevice(devs[0]) != hipSuccess) {
    (void)hipGetLastError();
    fprintf(stderr, "hi_load_tp: cannot select device %d\n", devs[0]);
    return nullptr;
  }
  return load(path, max_batch, max_seq, max_prefill);
}

// The same on the current GPU. Replaces api.cu:1499 (hi_load).
HI_EXPORT Engine* hi_load(const char* path, int max_batch, int max_seq, int max_prefill) {
  return load(path, max_batch, max_seq, max_prefill);
}

// Release everything the engine holds. Replaces api.cu:1501-1507 (hi_free).
HI_EXPORT void hi_free(Engine* e) { free_engine(e); }

// out[11] = vocab, hidden, inter, layers, heads, kv_heads, head_dim, max_pos, tied, qkv_bias,
// sliding window. Replaces api.cu:1509-1515 (hi_config).
HI_EXPORT void hi_config(Engine* e, int* out) {
  const Cfg& c = e->c;
  const int v[11] = {c.vocab, c.hidden, c.inter, c.layers, c.heads, c.kv, c.head_dim, c.max_pos, c.tied, c.qkv_bias, c.window};
  memcpy(out, v, sizeof(v));
}

// out[3] = experts, top_k, MoE flags (zeros for a dense model). Replaces api.cu:1517-1523.
HI_EXPORT void hi_moe_config(Engine* e, int* out) {
  out[0] = e->c.n_experts, out[1] = e->c.top_k, out[2] = e->c.moe_flags;
}

// Device bytes of the model's weights. Replaces api.cu:1525-1538 (hi_weight_bytes).
HI_EXPORT size_t hi_weight_bytes(Engine* e) { return e->arena_bytes; }

// 0: fp16 projections, 1: int8 with fp16 row scales. Replaces api.cu:1540 (hi_weight_quant).
HI_EXPORT int hi_weight_quant(Engine* e) { return e->c.quant; }

// Prefill `T` prompt tokens (host array) into cache slot `slot` at positions p0..; returns the
// greedy next token (also left in the slot's state and history at p0 + T), or -1 for bad
// arguments. Replaces api.cu:1841-1846 (hi_prefill).
HI_EXPORT int hi_prefill(Engine* e, int slot, const int* tokens, int T, int p0) {
  if (!prefill_ok(e, slot, tokens, T, p0, "hi_prefill")) return -1;
  if (hipSetDevice(e->dev) != hipSuccess || prefill(e, slot, tokens, T, p0, nullptr)) return -1;
  int tok = -1;
  if (hipMemcpyAsync(&tok, e->tok + slot, 4, hipMemcpyDeviceToHost, e->st) != hipSuccess ||
      hipStreamSynchronize(e->st) != hipSuccess || (e->c.moe && moe_one_launch_failed()))
    return -1;
  return tok;
}

// The same, and the fp16 logits of every position into dst (device, [T, vocab]). Replaces
// api.cu:1848-1855 (hi_prefill_logits).
HI_EXPORT int hi_prefill_logits(Engine* e, int slot, const int* tokens, int T, int p0, void* dst) {
  if (!prefill_ok(e, slot, tokens, T, p0, "hi_prefill_logits")) return -1;
  if (!dst) {
    fprintf(stderr, "hi_prefill_logits: null destination\n");
    return -1;
  }
  if (hipSetDevice(e->dev) != hipSuccess || prefill(e, slot, tokens, T, p0, (f16*)dst)) return -1;
  int tok = -1;
  if (hipMemcpyAsync(&tok, e->tok + slot, 4, hipMemcpyDeviceToHost, e->st) != hipSuccess ||
      hipStreamSynchronize(e->st) != hipSuccess || (e->c.moe && moe_one_launch_failed()))
    return -1;
  return tok;
}

// Run `steps` greedy decode steps on slots [0, B) (one hipGraph per B, captured on first use when
// use_graph). Returns the elapsed GPU milliseconds, or -1 for bad arguments (a slot whose position
// would pass max_seq) or a failed launch. Replaces api.cu:1996-2003 (hi_decode).
HI_EXPORT float hi_decode(Engine* e, int B, int steps, int use_graph) {
  if (!e || B < 1 || B > e->maxB || steps < 0) {
    fprintf(stderr, "hi_decode: B %d outside [1, max_batch] or steps %d < 0\n", B, steps);
    return -1.f;
  }
  if (hipSetDevice(e->dev) != hipSuccess) return -1.f;
  std::vector<int> pos(B);
  if (hipStreamSynchronize(e->st) != hipSuccess ||
      hipMemcpy(pos.data(), e->pos, (size_t)B * 4, hipMemcpyDeviceToHost) != hipSuccess)
    return -1.f;
  for (int b = 0; b < B; b++)
    if (pos[b] < 0 || (long long)pos[b] + steps > e->max_seq) {
      fprintf(stderr, "hi_decode: slot %d at position %d + %d steps exceeds max_seq %d\n", b, pos[b], steps,
              e->max_seq);
      return -1.f;
    }
  hipEvent_t ev[4];
  for (auto& v : ev)
    if (hipEventCreate(&v) != hipSuccess) return -1.f;
  float ms = 0.f, part = 0.f;
  bool ok = true;
  if (use_graph && !e->graphs[B] && steps > 0) {
    // the first step of this batch size eagerly (tiles tuned, attributes set), then the capture
    ok = hipEventRecord(ev[0], e->st) == hipSuccess && decode_step(e, B) == 0 &&
         hipEventRecord(ev[1], e->st) == hipSuccess && hipEventSynchronize(ev[1]) == hipSuccess &&
         hipEventElapsedTime(&part, ev[0], ev[1]) == hipSuccess && capture_step(e, B, &e->graphs[B]) == 0;
    ms += part;
    steps--;
  }
  ok = ok && hipEventRecord(ev[2], e->st) == hipSuccess;
  for (int i = 0; ok && i < steps; i++)
    ok = use_graph ? hipGraphLaunch(e->graphs[B], e->st) == hipSuccess : decode_step(e, B) == 0;
  ok = ok && hipEventRecord(ev[3], e->st) == hipSuccess && hipEventSynchronize(ev[3]) == hipSuccess &&
       hipEventElapsedTime(&part, ev[2], ev[3]) == hipSuccess;
  if (ok && e->c.moe && moe_one_launch_failed()) ok = false;  // a step's MoE output was wrong
  ms += part;
  for (auto& v : ev) (void)hipEventDestroy(v);
  if (!ok) (void)hipGetLastError();
  return ok ? ms : -1.f;
}

// Tokens hist[slot][from, from + n) (positions) to host. Replaces api.cu:2127-2142 (hi_history).
HI_EXPORT int hi_history(Engine* e, int slot, int from, int n, int* out) {
  if (!e || slot < 0 || slot >= e->maxB || from < 0 || n < 0 || (long long)from + n > e->max_seq || (n && !out)) {
    fprintf(stderr, "hi_history: slot %d range [%d, %d + %d) outside the engine\n", slot, from, from, n);
    return -1;
  }
  if (hipSetDevice(e->dev) != hipSuccess || hipStreamSynchronize(e->st) != hipSuccess) return -1;
  if (n && hipMemcpy(out, e->hist + (size_t)slot * e->max_seq + from, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess)
    return -1;
  return 0;
}

// The latest logits of slots [0, B) (fp16 [B, vocab]) to dst (host or device). Replaces
// api.cu:2145-2161 (hi_logits).
HI_EXPORT int hi_logits(Engine* e, int B, void* dst) {
  if (!e || B < 1 || B > e->maxB || !dst) {
    fprintf(stderr, "hi_logits: B %d outside [1, max_batch] or null destination\n", B);
    return -1;
  }
  if (hipSetDevice(e->dev) != hipSuccess || hipStreamSynchronize(e->st) != hipSuccess ||
      hipMemcpy(dst, e->logits, (size_t)B * e->c.vocab * 2, hipMemcpyDefault) != hipSuccess)
    return -1;
  return 0;
}

// Next input token and its position for slots [0, B). Replaces api.cu:2163-2176 (hi_set_state).
HI_EXPORT int hi_set_state(Engine* e, int B, const int* tok, const int* pos) {
  if (!e || B < 1 || B > e->maxB || !pos || !tokens_ok(e, tok, B, "hi_set_state")) {
    fprintf(stderr, "hi_set_state: bad arguments (B %d)\n", B);
    return -1;
  }
  for (int b = 0; b < B; b++)
    if (pos[b] < 0 || pos[b] >= e->max_seq) {
      fprintf(stderr, "hi_set_state: slot %d position %d outside max_seq %d\n", b, pos[b], e->max_seq);
      return -1;
    }
  if (hipSetDevice(e->dev) != hipSuccess || hipStreamSynchronize(e->st) != hipSuccess ||
      hipMemcpy(e->tok, tok, (size_t)B * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(e->pos, pos, (size_t)B * 4, hipMemcpyHostToDevice) != hipSuccess)
    return -1;
  return 0;
}

// Cut slot's cache to `len` positions; the next decode step feeds `tok` at position len.
// Replaces api.cu:2110-2123 (hi_rewind).
HI_EXPORT int hi_rewind(Engine* e, int slot, int len, int tok) {
  if (!e || slot < 0 || slot >= e->maxB || len < 0 || len >= e->max_seq || !tokens_ok(e, &tok, 1, "hi_rewind")) {
    fprintf(stderr, "hi_rewind: bad arguments (slot %d, length %d)\n", slot, len);
    return -1;
  }
  if (hipSetDevice(e->dev) != hipSuccess || hipStreamSynchronize(e->st) != hipSuccess ||
      hipMemcpy(e->tok + slot, &tok, 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(e->pos + slot, &len, 4, hipMemcpyHostToDevice) != hipSuccess)
    return -1;
  return 0;
}

// Wait for the engine's stream. Replaces api.cu:2125 (hi_sync).
HI_EXPORT void hi_sync(Engine* e) {
  if (e && hipSetDevice(e->dev) == hipSuccess) (void)hipStreamSynchronize(e->st);
}

// The engine's stream (hipStream_t). Replaces api.cu:2178 (hi_stream).
HI_EXPORT void* hi_stream(Engine* e) { return e ? (void*)e->st : nullptr; }

// Rows per hi_verify call (k + 1 for k draft tokens). Replaces api.cu:2070.
HI_EXPORT int hi_verify_max_rows() { return kVerifyMaxRows; }

// Speculative verification (verify_step): the greedy next token after each of the R host tokens
// fed at positions p0 .. p0 + R - 1 of `slot` (whose cache holds the positions below p0), into
// out[0, R) (host); with logits_dst (device, [R, vocab] fp16) non-null the rows' logits too. The
// rows' k / v are written to the cache; the slot's next token, position and history are left alone
// (hi_rewind sets them). Dense models. Returns 0, or -1 for bad arguments. Replaces
// api.cu:2077-2108 (hi_verify).
HI_EXPORT int hi_verify(Engine* e, int slot, const int* tokens, int R, int p0, int* out, void* logits_dst,
                        int use_graph) {
  if (!e || e->c.moe) {
    fprintf(stderr, "hi_verify: dense models only\n");
    return -1;
  }
  if (e->gemv_max < 1) {
    fprintf(stderr, "hi_verify: a batch of one must decode on the GEMV path (HIPINFER_GEMV_MAX >= 1)\n");
    return -1;
  }
  if (R < 1 || R > kVerifyMaxRows || !out) {
    fprintf(stderr, "hi_verify: R %d outside [1, %d] or null output\n", R, kVerifyMaxRows);
    return -1;
  }
  if (!prefill_ok(e, slot, tokens, R, p0, "hi_verify") || hipSetDevice(e->dev) != hipSuccess) return -1;
  hipStream_t s = e->st;
  if (!e->v_tok) {
    const size_t wb = hi_decode_work_bytes(kVerifyMaxRows, e->c.heads, e->c.kv, e->c.head_dim);
    if (!(e->v_tok = (int*)dalloc(e, kVerifyMaxRows * 4)) || !(e->v_pos = (int*)dalloc(e, kVerifyMaxRows * 4)) ||
        !(e->v_out = (int*)dalloc(e, kVerifyMaxRows * 4)) ||
        !(e->v_logits = (f16*)dalloc(e, (size_t)kVerifyMaxRows * e->c.vocab * 2)) || !(e->v_work = dalloc(e, wb)) ||
        hipMemsetAsync(e->v_work, 0, wb, s) != hipSuccess) {
      e->v_tok = nullptr;
      return -1;
    }
  }
  int pos[kVerifyMaxRows];
  for (int i = 0; i < R; i++) pos[i] = p0 + i;
  if (hipMemcpyAsync(e->v_tok, tokens, (size_t)R * 4, hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(e->v_pos, pos, (size_t)R * 4, hipMemcpyHostToDevice, s) != hipSuccess)
    return -1;
  hipGraphExec_t& g = e->vgraphs[{slot, R}];
  if (use_graph && g) {
    if (hipGraphLaunch(g, s) != hipSuccess) return -1;
  } else {
    // eagerly (the first call of a (slot, rows) pair sets kernel attributes outside capture);
    // the graph is captured after it for the next call
    if (verify_step(e, slot, R)) return -1;
    if (use_graph && (hipStreamSynchronize(s) != hipSuccess || capture(e, [&] { return verify_step(e, slot, R); }, &g)))
      return -1;
  }
  if (logits_dst &&
      hipMemcpyAsync(logits_dst, e->v_logits, (size_t)R * e->c.vocab * 2, hipMemcpyDeviceToDevice, s) != hipSuccess)
    return -1;
  if (hipMemcpyAsync(out, e->v_out, (size_t)R * 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return -1;
  return 0;
}
