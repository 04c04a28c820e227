/* libhipinfer.so -- MI355X (gfx950) matmul hot path of hipinfer, C ABI.
 *
 * Drop-in for the kernel launchers of the reference's src/api.cu that scripts/hipinfer.py binds
 * over ctypes (argtypes at scripts/hipinfer.py:12-31, 66-71). Same symbol names, argument order
 * and meaning. Conventions (reference api.cu:18, as scripts/hipinfer.py:101-161 uses them):
 *   - every tensor is a caller-owned device pointer; leading dimensions are in elements;
 *   - fp16 data is IEEE binary16; int8 weights [N, K] carry one fp16 scale per output row
 *     (W[n, k] ~ q[n, k] * s[n], docs/quantization.md);
 *   - epi: 0 store (+ bias where a bias argument exists), 1 residual (out += y, fp16 add),
 *     2 SwiGLU over gate/up rows interleaved in groups of 16 (out is N/2 wide);
 *   - `stream` is a hipStream_t (torch's current stream); launches are asynchronous.
 * Return value: 0 on success; -1 when the arguments are outside what the path supports (the
 * reason is printed on stderr; the reference prints and calls exit(1) there, api.cu:205-211,557);
 * -2 on a HIP runtime error. ctypes callers that ignore the return value (the reference's
 * argtypes declare no restype) keep working unchanged.
 */
#ifndef HIPINFER_AMD_H
#define HIPINFER_AMD_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- decode GEMV, M <= 16 rows (M <= 8 with the fused RMSNorm per launch; more rows are chunked) */

/* out[M, *] (epi) x[M, K] @ W[N, K]^T with fp16 W; normw != NULL fuses RMSNorm(x; normw, eps).
 * Replaces api.cu:181-185 (hi_gemv); binding hipinfer.py:14. */
int hi_gemv(const void* x, int ldx, const void* normw, float eps, const void* W, void* out, int ldo, int M, int N,
            int K, int epi, void* stream);

/* The same with int8 W and fp16 row scales [N]. Replaces api.cu:187-191 (hi_gemv_w8); hipinfer.py:17. */
int hi_gemv_w8(const void* x, int ldx, const void* normw, float eps, const void* W, const void* scales, void* out,
               int ldo, int M, int N, int K, int epi, void* stream);

/* Fused QKV projection (+ bias) + RoPE + KV-cache write: q to out[m, 0:Hq*D]; k and v to
 * kc/vc [slots][Hkv][max_seq][D] at slot m, position pos[m]; cs is [max_seq][D/2] (cos, sin) fp16.
 * Replaces api.cu:216-222 (hi_gemv_qkv_rope); hipinfer.py:16. */
int hi_gemv_qkv_rope(const void* x, int ldx, const void* normw, float eps, const void* W, const void* bias, void* out,
                     int ldo, int M, int K, int Hq, int Hkv, int D, const void* cs, const int* pos, void* kc, void* vc,
                     int max_seq, void* stream);

/* The same with int8 W and row scales. Replaces api.cu:224-230 (hi_gemv_qkv_rope_w8); hipinfer.py:18. */
int hi_gemv_qkv_rope_w8(const void* x, int ldx, const void* normw, float eps, const void* W, const void* scales,
                        const void* bias, void* out, int ldo, int M, int K, int Hq, int Hkv, int D, const void* cs,
                        const int* pos, void* kc, void* vc, int max_seq, void* stream);

/* ---- prefill GEMM (fp16 MFMA, fp32 accumulate); K % 32 == 0, N % 16 == 0 (N % 32 for epi 2)
 * C[M, *] (epi) A[M, K] @ W[N, K]^T, + bias[N] for epi 0 when bias != NULL. Replaces api.cu:566-571
 * (hi_gemm); binding hipinfer.py:24. */
int hi_gemm(const void* A, int lda, const void* W, const void* bias, void* C, int ldc, int M, int N, int K, int epi,
            void* stream);

/* The same with int8 W and fp16 row scales; W tiles enter the MFMAs as fp16(q * s).
 * Replaces api.cu:573-577 (hi_gemm_w8); hipinfer.py:19. */
int hi_gemm_w8(const void* A, int lda, const void* W, const void* scales, const void* bias, void* C, int ldc, int M,
               int N, int K, int epi, void* stream);

/* Benchmark and test hooks: force a tile config (-1 automatic), force a split-K factor (-1 automatic),
 * the number of tile configs and a description of one. Replace api.cu:300-305 and 463
 * (hi_gemm_force_config, hi_gemm_num_configs, hi_gemm_config_desc, hi_gemm_force_splits);
 * hipinfer.py:22-28. */
int hi_gemm_force_config(int cfg);
int hi_gemm_force_splits(int splits);
int hi_gemm_num_configs(void);
int hi_gemm_config_desc(int cfg, char* out, int n);
/* Test hook, no counterpart in the reference: the (tile config, split count) the calling thread's
 * last hi_gemm / hi_gemm_w8 launch ran with, so a test can tell a forced config that ran from one
 * that did not fit the shape or weight format and fell back to the automatic choice. */
int hi_gemm_last_choice(int* cfg, int* splits);

/* hi_gemm (scales == NULL) or hi_gemm_w8 (scales given) for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * No counterpart in the reference. It allocates nothing and never autotunes. The tile is the one the
 * autotuner already chose for the shape on this GPU, else the cost model's, or a forced one. Split-K
 * partials live in a 64 MB static device array per GPU, which the GPU holds until the process
 * ends. An automatic split count is lowered until its splits * M * N fp32 partials fit; a forced
 * split count that does not fit is rejected (-1). Calls that overlap in time on one GPU share that
 * array and race. Returns 0, -1 (bad argument, reason on stderr) or -2 (HIP error). */
int hi_gemm_noalloc(const void* A, int lda, const void* W, const void* scales, const void* bias, void* C, int ldc,
                    int M, int N, int K, int epi, void* stream);

/* X[M, N] += A[M, K] @ W[N, K]^T (the residual epilogue 1, X contiguous: ldc == N), then
 * Y[M, N] = RMSNorm(X) * norm_w (hi_rmsnorm's rule); scales NULL for fp16 W, else int8 W with fp16
 * row scales. No counterpart in the reference: its engine runs the residual GEMM and the RMSNorm
 * that reads it in turn (api.cu:1668-1690). This entry gives the same bits as hi_gemm(epi 1) then
 * hi_rmsnorm, and when the GEMM splits K it runs the norm inside the split-K second pass (one
 * kernel fewer, one read of X fewer). X, Y, norm_w 16-byte aligned. Returns 0, -1 or -2. */
int hi_gemm_residual_rmsnorm(const void* A, int lda, const void* W, const void* scales, void* X, int M, int N, int K,
                             const void* norm_w, float eps, void* Y, void* stream);

/* ---- mixture of experts (fp16 experts, E <= 256, k <= 16)
 * Router + top-k of M normalised rows xn[M, H] under Wr[E, H]: idx[M, k] int, w[M, k] fp32, descending;
 * flags bit 0 = softmax over the k (else over all E), bit 1 = weights rounded to fp16.
 * Replaces api.cu:849-857 (hi_moe_router); hipinfer.py:68. */
int hi_moe_router(const void* xn, int ldx, const void* Wr, int M, int E, int H, int k, int flags, int* idx, float* w,
                  void* stream);
/* Bytes of the workspace hi_moe_experts and hi_moe_route_experts need (the first 2304 bytes hold
 * hi_moe_route_experts' arrival counters). Replaces api.cu:862-865 (hi_moe_work_bytes); hipinfer.py:69. */
size_t hi_moe_work_bytes(int M, int k, int E, int H, int I);
/* x[m] += MoE(xn[m]) given the routing: wgu [E][2I, H] (gate/up interleaved per expert), wdown [E][H, I];
 * scale multiplies the combined output (rounded); path 0 auto (GEMV for M <= HIPINFER_GEMV_MAX, default 8),
 * 1 GEMV, 2 grouped MFMA GEMMs (device-side expert grouping, no host round trip). H % 32 == 0, I % 32 == 0.
 * Replaces api.cu:872-911 (hi_moe_experts); hipinfer.py:71. */
int hi_moe_experts(const void* xn, int ldxn, const void* wgu, const void* wdown, const int* idx, const float* w, int M,
                   int E, int k, int H, int I, int flags, float scale, void* x, int ldx, int path, void* work,
                   void* stream);
/* Router and experts in one call: x[m] += MoE(xn[m]) with the routing computed here and written to
 * idx[M, k] / w[M, k] as hi_moe_router writes it; the same bits as hi_moe_router followed by
 * hi_moe_experts(path 0). M = 1 runs as one launch (router, gate/up, a grid-wide handoff, down and
 * combine) when that grid fits on the GPU at once; otherwise, for M <= HIPINFER_GEMV_MAX, the router
 * runs inside the gate/up launch. work: hi_moe_work_bytes(M, k, E, H, I), zeroed once before its
 * first use with this function (the one-launch path keeps arrival counters in it and leaves them
 * consistent); calls that share a work buffer must not overlap in time. Returns -2, launching
 * nothing, when an earlier one-launch call gave up waiting for its grid (its output was wrong; the
 * one-launch path is then off for the rest of the process).
 * No counterpart in the reference (its engine makes the two calls, api.cu:1701-1703); for callers
 * that run a whole MoE layer, such as this library's engine. */
int hi_moe_route_experts(const void* xn, int ldxn, const void* Wr, const void* wgu, const void* wdown, int M, int E,
                         int k, int H, int I, int flags, float scale, void* x, int ldx, int* idx, float* w, void* work,
                         void* stream);

/* ---- decode-step kernels around the GEMVs
 * Bytes of the workspace hi_decode_attn needs: 4096 int counters (zeroed once by the caller, left
 * zeroed by every launch), then B * Hq * 64 * (D + 2) fp32 split partials. Replaces api.cu:651-656
 * (hi_decode_work_bytes); hipinfer.py:21-22. */
size_t hi_decode_work_bytes(int B, int Hq, int Hkv, int D);
/* Decode attention of B new tokens: out[b, h*D:(h+1)*D] = softmax(q_h . K_slot_b[0..pos[b]] / sqrt(D)) V,
 * caches kc / vc [slots][Hkv][max_seq][D] fp16, query head h reading kv head h / (Hq / Hkv); D 64 or 128,
 * Hq / Hkv in 1..8, B * Hkv <= 4096. Split over the keys on the device (graph-capturable while pos grows).
 * Replaces api.cu:715-720 (hi_decode_attn); hipinfer.py:30. */
int hi_decode_attn(const void* q, int ldq, const void* kc, const void* vc, int max_seq, const int* pos, void* out,
                   int ldo, int B, int Hq, int Hkv, int D, void* work, void* stream);
/* Greedy token of each row of logits [B, V] fp16: the largest value, NaN above every number, the lowest
 * index on ties, 0 for a row of -inf. Replaces api.cu:838-840 (hi_argmax); kernels.cuh:1883-1931. */
int hi_argmax(const void* logits, int B, int V, int* tok_out, void* stream);
/* Embedding rows x[b, 0:H] = table[tok[b], 0:H] (table [V, H] fp16, H % 8 == 0); ids outside [0, V)
 * leave the row untouched. No reference export: the reference's engine runs the same gather
 * (embed_kernel, kernels.cuh:1876-1881) inside decode_step (api.cu:1900); exported here so that a
 * caller can build the whole decode step from C-ABI calls. */
int hi_embed(const int* tok, const void* table, int V, int H, void* x, int ldx, int B, void* stream);

/* ---- prefill kernels around the GEMM
 * RoPE + KV-cache write of M qkv rows [M, ldq] = [q (Hq*D) | k (Hkv*D) | v (Hkv*D)]: q rotated in
 * place (HF order, per-op fp16 rounding), rotated k and raw v to kc / vc [slots][Hkv][max_seq][D].
 * Row m sits at pos[m] in slot slot_base + m (pos non-null), else at pos_base + m in slot slot_base.
 * cs [max_seq][D/2] (cos, sin) fp16. Replaces api.cu:584-586 (hi_rope_cache); hipinfer.py:164-168. */
int hi_rope_cache(void* qkv, int ldq, int M, int Hq, int Hkv, int D, const void* cs, const int* pos, int pos_base,
                  int slot_base, void* kc, void* vc, int max_seq, void* stream);
/* Causal prefill attention: row t of q [T, ldq] (head h at columns h*D) sits at position p0 + t and
 * attends to keys 0..p0+t of one cache slot kc / vc [Hkv][max_seq][D] (kv head h / (Hq / Hkv));
 * out [T, ldo] fp16. D 64 or 128, p0 + T <= max_seq. Replaces api.cu:614-617 (hi_flash_prefill);
 * hipinfer.py:171-177. */
int hi_flash_prefill(const void* q, int ldq, const void* kc, const void* vc, int max_seq, void* out, int ldo, int T,
                     int p0, int Hq, int Hkv, int D, void* stream);
/* The same, and each row's log2-domain log-sum-exp of the scaled logits into lse [Hq][T] fp32.
 * Replaces api.cu:619-623 (hi_flash_prefill_lse); hipinfer.py:193-202. */
int hi_flash_prefill_lse(const void* q, int ldq, const void* kc, const void* vc, int max_seq, void* out, int ldo,
                         int T, int p0, int Hq, int Hkv, int D, float* lse, void* stream);

/* ---- RMSNorm (unfused form of the GEMV prologue; the reference's tests build references with it)
 * y[M, H] = w * fp16(x * rsqrt(mean(x^2) + eps)), rows contiguous. Replaces api.cu:76-79
 * (hi_rmsnorm); hipinfer.py:13. */
int hi_rmsnorm(const void* x, const void* w, void* y, int M, int H, float eps, void* stream);

/* ---- int8 weight format on the GPU (the reference does this on the host in Python)
 * q[N, K] int8, s[N] fp16 from fp16 w[N, K], bit-exact with scripts/export.py:54-68 quantize_rows. */
int hi_quantize_rows(const void* w, long long N, int K, void* q, void* s, void* stream);
/* out[N, K] = fp16(q * s), bit-exact with scripts/export.py:71-73 dequantize_rows. */
int hi_dequantize_rows(const void* q, const void* s, long long N, int K, void* out, void* stream);

/* Compute units of the current device (diagnostics; the launchers size their grids from it). */
int hi_device_cus(void);
/* Largest dynamic LDS (bytes) a block may opt into on the current device: 160 KB on MI355X.
 * Replaces api.cu:49 (hi_max_smem, the CUDA shared-memory opt-in). */
int hi_max_smem(void);
/* Activation rows one GEMV launch takes at K (norm: fused RMSNorm, int8: int8 weights) on the
 * current device; more rows run in row chunks, each streaming the weights again. 0 when one row does
 * not fit, -2 on a HIP error. No counterpart in the reference; for hosts choosing between the GEMV and
 * the GEMM for small batches, such as hipinfer_amd.engine.DecodeStep. */
int hi_gemv_rows_per_launch(int K, int norm, int int8);

/* ---- engine: weight-file loader, prefill, graph-captured greedy decode (one GPU)
 * An opaque engine over a weight file in the reference's export format (scripts/export.py:5-38;
 * versions 2 dense fp16, 3 MoE, 4 int8 projections). Per slot it keeps the next input token, its
 * position and the token history on the device. */
typedef struct Engine Engine;
/* Load `path` onto the current GPU for max_batch slots of max_seq positions and prefill chunks of
 * max_prefill rows; null (reason on stderr) for a bad file or setting. Replaces api.cu:1499. */
Engine* hi_load(const char* path, int max_batch, int max_seq, int max_prefill);
/* The same with a device list; world must be 1 (no tensor parallelism in this build).
 * Replaces api.cu:1475-1497 (hi_load_tp). */
Engine* hi_load_tp(const char* path, int max_batch, int max_seq, int max_prefill, int world, const int* devs);
/* Replaces api.cu:1501-1507. */
void hi_free(Engine* e);
/* out[11]: vocab, hidden, inter, layers, heads, kv_heads, head_dim, max_pos, tied, qkv_bias,
 * sliding window. Replaces api.cu:1509-1515. */
void hi_config(Engine* e, int* out);
/* out[3]: experts, top_k, MoE flags (zeros when dense). Replaces api.cu:1517-1523. */
void hi_moe_config(Engine* e, int* out);
/* Replaces api.cu:1525-1538. */
size_t hi_weight_bytes(Engine* e);
/* 0 fp16 projections, 1 int8 with fp16 row scales. Replaces api.cu:1540. */
int hi_weight_quant(Engine* e);
/* Prefill T host tokens into `slot` at positions p0..; returns the greedy next token (left in the
 * slot's state, and in its history at p0 + T), or -1. Replaces api.cu:1841-1846. */
int hi_prefill(Engine* e, int slot, const int* tokens, int T, int p0);
/* The same, and every position's fp16 logits into dst (device, [T, vocab]). Replaces
 * api.cu:1848-1855. */
int hi_prefill_logits(Engine* e, int slot, const int* tokens, int T, int p0, void* dst);
/* `steps` greedy decode steps on slots [0, B), one captured hipGraph per B when use_graph;
 * returns GPU milliseconds, or -1. Replaces api.cu:1996-2003. */
float hi_decode(Engine* e, int B, int steps, int use_graph);
/* History tokens of `slot` at positions [from, from + n) to host. Replaces api.cu:2127-2142. */
int hi_history(Engine* e, int slot, int from, int n, int* out);
/* Latest logits of slots [0, B), fp16 [B, vocab], to host or device. Replaces api.cu:2145-2161. */
int hi_logits(Engine* e, int B, void* dst);
/* Next input token and position of slots [0, B). Replaces api.cu:2163-2176. */
int hi_set_state(Engine* e, int B, const int* tok, const int* pos);
/* Keep positions [0, len) of `slot`; the next step feeds tok at len. Replaces api.cu:2110-2123. */
int hi_rewind(Engine* e, int slot, int len, int tok);
/* Replaces api.cu:2125. */
void hi_sync(Engine* e);
/* The engine's hipStream_t. Replaces api.cu:2178. */
void* hi_stream(Engine* e);
/* Rows per hi_verify call (k + 1 for k draft tokens): 16 (the reference returns 8). Replaces api.cu:2070. */
int hi_verify_max_rows(void);
/* Speculative verification of a dense model: the greedy token after each of R host tokens fed at
 * positions p0.. of `slot`, through a batch-of-one decode step's kernels with R rows, so entry i
 * equals plain greedy decoding at p0 + i bit for bit; out[R] (host), logits_dst ([R, vocab] fp16,
 * device) optional; the slot's state is left alone (see hi_rewind). Replaces api.cu:2077-2108. */
int hi_verify(Engine* e, int slot, const int* tokens, int R, int p0, int* out, void* logits_dst, int use_graph);

#ifdef __cplusplus
}
#endif
#endif
