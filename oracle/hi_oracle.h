/* CPU oracle for the hipinfer matmul hot path: a plain-C restatement of the reference's
 * arithmetic, used ONLY as the checker (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline).
 * No product code may link or call it.
 *
 * Conventions follow the reference C-ABI (src/api.cu): fp16 values travel as their IEEE binary16
 * bit patterns (uint16_t), weights are [N, K] row-major, leading dimensions are in elements,
 * int8 weights carry one fp16 scale per output row. Accumulation is fp64 (an upper bound on the
 * accuracy of the reference's fp32 accumulation); every fp16 rounding point of the reference's
 * kernels is reproduced at the same place. Functions return 0, or -1 on an argument the reference
 * rejects. */
#ifndef HI_ORACLE_H
#define HI_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint16_t or_f2h(float f);
float or_h2f(uint16_t h);
void or_f2h_array(const float* f, uint16_t* h, int64_t n);
void or_h2f_array(const uint16_t* h, float* f, int64_t n);

void or_set_threads(int n);
int or_get_threads(void);

int or_quantize_rows(const uint16_t* w, int64_t N, int64_t K, int8_t* q, uint16_t* s);
int or_dequantize_rows(const int8_t* q, const uint16_t* s, int64_t N, int64_t K, uint16_t* out);
int or_interleave_gate_up(const void* g, const void* u, int64_t I, int64_t row_bytes, void* out);
int or_deinterleave_gate_up(const void* gu, int64_t I, int64_t row_bytes, void* g, void* u);

int or_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* w, int M, int K, float eps, uint16_t* y, int64_t ldy);
uint16_t or_silu_mul(float g, float u);
void or_rope_pair(uint16_t x1, uint16_t x2, uint16_t c, uint16_t s, uint16_t* y1, uint16_t* y2);

int or_gemv(const uint16_t* x, int64_t ldx, const uint16_t* normw, float eps, const void* W, const uint16_t* scales,
            uint16_t* out, int64_t ldo, int M, int N, int K, int epi);
int or_gemv_qkv_rope(const uint16_t* x, int64_t ldx, const uint16_t* normw, float eps, const void* W,
                     const uint16_t* scales, const uint16_t* bias, uint16_t* out, int64_t ldo, int M, int K, int Hq,
                     int Hkv, int D, const uint16_t* cs, const int32_t* pos, uint16_t* kc, uint16_t* vc, int max_seq,
                     int kv_slot);
int or_gemm(const uint16_t* A, int64_t lda, const void* W, const uint16_t* scales, const uint16_t* bias, uint16_t* C,
            int64_t ldc, int M, int N, int K, int epi);

int or_moe_router(const uint16_t* xn, int64_t ldx, const uint16_t* Wr, int M, int E, int H, int k, int flags,
                  int32_t* idx, float* w);
int or_moe_experts(const uint16_t* xn, int64_t ldxn, const uint16_t* wgu, const uint16_t* wdown, const int32_t* idx,
                   const float* w, int M, int E, int k, int H, int I, int flags, float scale, uint16_t* x,
                   int64_t ldx);

int or_decode_attn(const uint16_t* q, int64_t ldq, const uint16_t* kc, const uint16_t* vc, int max_seq,
                   const int32_t* pos, uint16_t* out, int64_t ldo, int B, int Hq, int Hkv, int D);
int or_argmax(const uint16_t* logits, int B, int V, int32_t* tok);
int or_rope_cache(uint16_t* qkv, int64_t ldq, int M, int Hq, int Hkv, int D, const uint16_t* cs, const int32_t* pos,
                  int pos_base, int slot_base, uint16_t* kc, uint16_t* vc, int max_seq);
int or_flash_prefill(const uint16_t* q, int64_t ldq, const uint16_t* kc, const uint16_t* vc, int max_seq,
                     uint16_t* out, int64_t ldo, int T, int p0, int Hq, int Hkv, int D, float* lse);

#ifdef __cplusplus
}
#endif
#endif
