// Library-internal entry points (hidden; not part of the C-ABI): the verify forms of the fused
// QKV GEMV and of decode attention, where every activation row belongs to one sequence.
#pragma once
#include "hi_common.h"

// hi_gemv_qkv_rope(_w8) with every row's k / v written to cache slot kv_slot (rows m at pos[m]);
// scales null for fp16 weights.
int gemv_qkv_rope_slot(const void* x, int ldx, const void* normw, float eps, const void* W, const void* scales,
                       const void* bias, void* out, int ldo, int M, int K, int Hq, int Hkv, int D, const void* cs,
                       const int* pos, void* kc, void* vc, int max_seq, int kv_slot, hipStream_t s);

// hi_decode_attn for R query rows of ONE sequence: every row reads cache slot kv_slot (row r up
// to pos[r]) with the split count a batch of one uses, so row r is bit-identical to a decode step
// of that sequence at pos[r]. work: hi_decode_work_bytes(R, Hq, Hkv, D) bytes, zeroed once.
int decode_attn_slot(const void* q, int ldq, const void* kc, const void* vc, int max_seq, const int* pos, void* out,
                     int ldo, int R, int Hq, int Hkv, int D, void* work, int kv_slot, hipStream_t s);
