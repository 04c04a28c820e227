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

// Activation rows one GEMV launch takes at K (fused RMSNorm or not, int8 weights or fp16) on the
// current device: 8 (norm) or 16 rows, halved while they do not fit the LDS together; 0 when a
// single row does not fit. More rows than this run in row chunks, each streaming the weights.
int gemv_rows_per_launch(int K, bool norm, bool int8);

// The MoE calls' limits: at most kMoeMaxE experts, each token routed to at most kMoeMaxK of them.
constexpr int kMoeMaxE = 256, kMoeMaxK = 16;

// True once after a one-launch MoE call (hi_moe_route_experts at M = 1) gave up waiting for its
// grid, which leaves that call's output wrong; the flag is cleared, a message printed, and the
// one-launch path turned off for the rest of the process. hi_moe_route_experts checks it before
// launching anything (and returns -2), the engine after each prefill or decode call.
bool moe_one_launch_failed();
