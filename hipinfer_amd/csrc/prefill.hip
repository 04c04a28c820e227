// Prefill kernels around the GEMM, behind the reference's C-ABI: the RoPE + KV-cache write that
// follows a QKV GEMM (hi_rope_cache; src/api.cu:579-586, kernels.cuh:1120-1158, ctypes
// scripts/hipinfer.py:164-168) and causal prefill attention over a cache slot (hi_flash_prefill,
// hi_flash_prefill_lse; api.cu:594-623, kernels.cuh:1160-1329, ctypes hipinfer.py:171-202).
//
// Flash prefill for gfx950 (D = 64 or 128):
//  * block = 128 query rows of one query head, 4 waves of 32 rows; the wave's Q rows stay in
//    registers as v_mfma_f32_32x32x16_f16 operands for the whole kernel;
//  * 64-key K/V tiles of the head's cache rows are loaded once per block (global -> registers ->
//    LDS, the next tile's loads in flight while the current one is computed). K is stored with its
//    16-byte chunks XOR-swizzled by the key so fragment reads are conflict-free; V is stored
//    transposed (V^T[d][key]), because the P.V product contracts over keys;
//  * S^T = K Q^T: with the K fragment as first operand each lane ends with 32 keys of ONE query
//    row (16 keys x 2 halves of the tile, split between lanes l and l + 32), so the row max and sum
//    of the online softmax are the lane's own values plus one exchange with lane l ^ 32;
//  * logits are scaled by log2(e) / sqrt(D) and the softmax runs in base 2 (the reference's
//    log2-domain form, kernels.cuh:1236-1262); P is rounded to fp16 for P.V, the row sum l keeps
//    fp32 p, as the reference does;
//  * O^T += V^T P^T: the P registers of a lane are already a B fragment of the next product once
//    the key order inside each 16-key step is permuted identically for P and V^T (lane half fk
//    takes keys 4 fk + 0..3 and 8 + 4 fk + 0..3), so P never goes through LDS; O^T keeps the
//    lane -> query row map, so the per-row rescale by exp2(m_old - m_new) is per lane;
//  * causal mask on absolute positions (row t at p0 + t sees keys 0..p0+t); a wave skips tiles
//    that lie wholly above its rows' diagonal; cache rows past the block's last key read as zeros.
#include "hi_common.h"

namespace {

constexpr int kFpWaves = 4;
constexpr int kFpBQ = 32 * kFpWaves;  // query rows per block
constexpr int kFpBKV = 64;            // keys per tile
constexpr int kVtStride = kFpBKV + 4;  // halves per V^T row: 136 bytes keeps 8-byte reads aligned

// Slot of 16-byte chunk c of key r in the K tile (D / 8 chunks per key): the XOR term spreads the
// 16 keys one 128-bit read serves per cycle over all 64 banks.
template <int D>
__device__ __forceinline__ int k_slot(int r, int c) {
  if constexpr (D == 128) return r * 16 + (c ^ (r & 15));
  else return r * 8 + (c ^ ((r >> 1) & 7));
}

template <int D>
struct FpSmem {
  u32x4 k[kFpBKV * D / 8];
  f16 vt[D * kVtStride];
};

template <int D>
__global__ void __launch_bounds__(64 * kFpWaves)
    flash_prefill_kernel(const f16* __restrict__ q, int64_t ldq, const f16* __restrict__ kc,
                         const f16* __restrict__ vc, int max_seq, f16* __restrict__ out, int64_t ldo, int T, int p0,
                         int Hq, int Hkv, float scale_log2, float* __restrict__ lse) {
  constexpr int CPR = D / 8;                    // 16-byte chunks per key row
  constexpr int NT = 64 * kFpWaves;
  constexpr int LPT = kFpBKV * CPR / NT;        // chunks of K (and of V) each thread loads per tile
  constexpr int DT = D / 32;                    // 32-row output tiles of O^T
  static_assert(LPT * NT == kFpBKV * CPR, "tile load split");
  __shared__ FpSmem<D> sm;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, fk = lane >> 5;
  const int q0 = blockIdx.x * kFpBQ, h = blockIdx.y, hk = h / (Hq / Hkv);
  const int qw = q0 + wave * 32;                // this wave's first query row
  const int qi = qw + fr;                       // this lane's query row
  const int qpos = p0 + qi;
  const int kv_end = p0 + min(q0 + kFpBQ, T);   // keys any row of the block can see
  const f16* Kh = kc + (int64_t)hk * max_seq * D;
  const f16* Vh = vc + (int64_t)hk * max_seq * D;

  // this lane's Q fragments: row qi, d = 16 ks + 8 fk + 0..7 (zero past T)
  f16x8 qf[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ks++) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (qi < T) v = *reinterpret_cast<const u32x4*>(q + (int64_t)qi * ldq + h * D + 16 * ks + 8 * fk);
    qf[ks] = __builtin_bit_cast(f16x8, v);
  }

  u32x4 kreg[LPT], vreg[LPT];
  auto gload = [&](int j0) {
#pragma unroll
    for (int i = 0; i < LPT; i++) {
      const int ci = tid + i * NT, r = ci / CPR, c = ci % CPR;
      const bool ok = j0 + r < kv_end;
      kreg[i] = ok ? *reinterpret_cast<const u32x4*>(Kh + (int64_t)(j0 + r) * D + 8 * c) : u32x4{0u, 0u, 0u, 0u};
      vreg[i] = ok ? *reinterpret_cast<const u32x4*>(Vh + (int64_t)(j0 + r) * D + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
  };

  float m_i = -__builtin_huge_valf(), l_i = 0.f;
  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; dt++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[dt][e] = 0.f;

  gload(0);
  for (int j0 = 0; j0 < kv_end; j0 += kFpBKV) {
    __syncthreads();  // every wave is done with the previous tile
#pragma unroll
    for (int i = 0; i < LPT; i++) {
      const int ci = tid + i * NT, r = ci / CPR, c = ci % CPR;
      sm.k[k_slot<D>(r, c)] = kreg[i];
      const f16x8 v = __builtin_bit_cast(f16x8, vreg[i]);
#pragma unroll
      for (int e = 0; e < 8; e++) sm.vt[(8 * c + e) * kVtStride + r] = v[e];
    }
    __syncthreads();
    if (j0 + kFpBKV < kv_end) gload(j0 + kFpBKV);
    if (j0 > p0 + qw + 31) continue;  // the whole tile is above this wave's diagonal

    // ---- S^T = K Q^T: two 32-key halves; lane (row fr, half fk) gets keys 8 g + 4 fk + e
    f32x16 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
#pragma unroll
      for (int e = 0; e < 16; e++) s[kt][e] = 0.f;
      const int r = kt * 32 + fr;
#pragma unroll
      for (int ks = 0; ks < D / 16; ks++) {
        const f16x8 kf = __builtin_bit_cast(f16x8, sm.k[k_slot<D>(r, 2 * ks + fk)]);
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[kt], 0, 0, 0);
      }
    }
    // ---- online softmax of row qi over this tile (base 2)
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int kp = j0 + kt * 32 + 8 * (e >> 2) + 4 * fk + (e & 3);
        const float v = (kp <= qpos && kp < kv_end) ? s[kt][e] * scale_log2 : -__builtin_huge_valf();
        s[kt][e] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_i, mx);
    const float alpha = m_new == -__builtin_huge_valf() ? 1.f : exp2f(m_i - m_new);
    float sum = 0.f;
    f16x8 pf[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float p = s[kt][e] == -__builtin_huge_valf() ? 0.f : exp2f(s[kt][e] - m_new);
        sum += p;
        pf[kt][e >> 3][e & 7] = (f16)p;
      }
    sum += __shfl_xor(sum, 32);
    l_i = l_i * alpha + sum;
    m_i = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int e = 0; e < 16; e++) o[dt][e] *= alpha;
    // ---- O^T += V^T P^T; step st of half kt: lane half fk holds keys 16 st + 4 fk + 0..3 and
    //      16 st + 8 + 4 fk + 0..3 of that half, in P's registers and in the V^T reads alike
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
      const f16* vrow = sm.vt + (dt * 32 + fr) * kVtStride;
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int st = 0; st < 2; st++) {
          const int kk = kt * 32 + 16 * st + 4 * fk;
          const f16x4 a = *reinterpret_cast<const f16x4*>(vrow + kk);
          const f16x4 b = *reinterpret_cast<const f16x4*>(vrow + kk + 8);
          const f16x8 vf = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[kt][st], o[dt], 0, 0, 0);
        }
    }
  }

  if (qi >= T) return;
  if (lse && fk == 0) lse[(int64_t)h * T + qi] = m_i + log2f(l_i);
  const float inv = 1.f / l_i;
  f16* orow = out + (int64_t)qi * ldo + h * D;
#pragma unroll
  for (int dt = 0; dt < DT; dt++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      f16x4 v;
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = (f16)(o[dt][4 * g + e] * inv);
      *reinterpret_cast<f16x4*>(orow + dt * 32 + 8 * g + 4 * fk) = v;
    }
}

// One qkv row per block: q heads rotated in place, rotated k and raw v to the cache.
__global__ void __launch_bounds__(256)
    rope_cache_kernel(f16* qkv, int64_t ldq, int Hq, int Hkv, int D, const f16x2* __restrict__ cs,
                      const int* __restrict__ pos, int pos_base, int slot_base, f16* kc, f16* vc, int max_seq) {
  const int HD = D / 2, row = blockIdx.x;
  const int p = pos ? pos[row] : pos_base + row;
  const int slot = pos ? slot_base + row : slot_base;
  f16* base = qkv + (int64_t)row * ldq;
  for (int i = threadIdx.x; i < (Hq + Hkv) * HD; i += blockDim.x) {
    const int hh = i / HD, d = i % HD;
    f16* x = base + hh * D;
    f16 y1 = x[d], y2 = x[d + HD];
    rope_pair(y1, y2, cs[(int64_t)p * HD + d]);
    f16* dst = hh < Hq ? x : kc + (((int64_t)slot * Hkv + hh - Hq) * max_seq + p) * D;
    dst[d] = y1;
    dst[d + HD] = y2;
  }
  const f16* v = base + (Hq + Hkv) * D;
  for (int i = threadIdx.x; i < Hkv * D; i += blockDim.x)
    vc[(((int64_t)slot * Hkv + i / D) * max_seq + p) * D + i % D] = v[i];
}

// The same with 16-byte accesses: a thread step rotates 8 pairs of one head (the 8 elements at d
// and the 8 at d + D/2, and their 8 table entries) or copies 8 elements of v. Used when D/2 is a
// multiple of 8 and every row, cache and the table are 16-byte aligned; each pair is rotated by
// rope_pair, as above, so the two kernels give the same bits.
__global__ void __launch_bounds__(256)
    rope_cache_v8_kernel(f16* qkv, int64_t ldq, int Hq, int Hkv, int D, const f16x2* __restrict__ cs,
                         const int* __restrict__ pos, int pos_base, int slot_base, f16* kc, f16* vc, int max_seq) {
  const int HD = D / 2, C = HD / 8, row = blockIdx.x;
  const int p = pos ? pos[row] : pos_base + row;
  const int slot = pos ? slot_base + row : slot_base;
  f16* base = qkv + (int64_t)row * ldq;
  const int nrot = (Hq + Hkv) * C, nv = Hkv * D / 8;
  for (int i = threadIdx.x; i < nrot + nv; i += blockDim.x) {
    if (i < nrot) {
      const int hh = i / C, d = (i - hh * C) * 8;
      f16* x = base + hh * D;
      f16x8 a = *reinterpret_cast<const f16x8*>(x + d), b = *reinterpret_cast<const f16x8*>(x + d + HD);
      const u32x4* tp = reinterpret_cast<const u32x4*>(cs + (int64_t)p * HD + d);
      const u32x4 c0 = tp[0], c1 = tp[1];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        f16 y1 = a[j], y2 = b[j];
        rope_pair(y1, y2, as_h2(j < 4 ? c0[j] : c1[j - 4]));
        a[j] = y1;
        b[j] = y2;
      }
      f16* dst = hh < Hq ? x : kc + (((int64_t)slot * Hkv + hh - Hq) * max_seq + p) * D;
      *reinterpret_cast<f16x8*>(dst + d) = a;
      *reinterpret_cast<f16x8*>(dst + d + HD) = b;
    } else {
      const int c = i - nrot, h = c / (D / 8), e = (c - h * (D / 8)) * 8;
      *reinterpret_cast<u32x4*>(vc + (((int64_t)slot * Hkv + h) * max_seq + p) * D + e) =
          *reinterpret_cast<const u32x4*>(base + (Hq + Hkv + h) * D + e);
    }
  }
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

int flash_prefill(const void* q, int ldq, const void* kc, const void* vc, int max_seq, void* out, int ldo, int T,
                  int p0, int Hq, int Hkv, int D, float* lse, void* stream, const char* who) {
  if (!hi_device()) return -2;
  if (D != 64 && D != 128) HI_FAIL("%s: head_dim %d not supported (64 or 128)", who, D);
  if (T < 0 || p0 < 0 || Hkv < 1 || Hq < Hkv || Hq % Hkv || max_seq < 1 || (int64_t)p0 + T > max_seq)
    HI_FAIL("%s: bad shape T=%d p0=%d Hq=%d Hkv=%d max_seq=%d", who, T, p0, Hq, Hkv, max_seq);
  if (T == 0) return 0;
  if (!q || !kc || !vc || !out) HI_FAIL("%s: null tensor pointer", who);
  if (!aligned(q, 16) || ldq % 8 || ldq < Hq * D) HI_FAIL("%s: q must be 16-byte aligned, ldq %% 8 == 0, ldq >= Hq*D", who);
  if (!aligned(kc, 16) || !aligned(vc, 16)) HI_FAIL("%s: kc / vc must be 16-byte aligned", who);
  if (!aligned(out, 8) || ldo % 4 || ldo < Hq * D) HI_FAIL("%s: out must be 8-byte aligned, ldo %% 4 == 0, ldo >= Hq*D", who);
  const float scale_log2 = 1.4426950408889634f / sqrtf((float)D);
  const dim3 grid((T + kFpBQ - 1) / kFpBQ, Hq);
  const hipStream_t s = (hipStream_t)stream;
  if (D == 128)
    hipLaunchKernelGGL(flash_prefill_kernel<128>, grid, dim3(64 * kFpWaves), 0, s, (const f16*)q, (int64_t)ldq,
                       (const f16*)kc, (const f16*)vc, max_seq, (f16*)out, (int64_t)ldo, T, p0, Hq, Hkv, scale_log2, lse);
  else
    hipLaunchKernelGGL(flash_prefill_kernel<64>, grid, dim3(64 * kFpWaves), 0, s, (const f16*)q, (int64_t)ldq,
                       (const f16*)kc, (const f16*)vc, max_seq, (f16*)out, (int64_t)ldo, T, p0, Hq, Hkv, scale_log2, lse);
  HI_TRY(hipGetLastError());
  return 0;
}

}  // namespace

// RoPE + KV-cache write for M qkv rows [M, ldq] = [q (Hq*D) | k (Hkv*D) | v (Hkv*D)]: q rotated in
// place, rotated k and raw v to kc / vc [slots][Hkv][max_seq][D]. Row m sits at position pos[m] in
// slot slot_base + m (pos non-null: decode) or at pos_base + m in slot slot_base (prefill).
// cs: [max_seq][D/2] (cos, sin) fp16 pairs. Positions must lie in [0, max_seq).
HI_EXPORT int hi_rope_cache(void* qkv, int ldq, int M, int Hq, int Hkv, int D, const void* cs, const int* pos,
                            int pos_base, int slot_base, void* kc, void* vc, int max_seq, void* stream) {
  if (!hi_device()) return -2;
  if (M < 0 || Hq < 1 || Hkv < 1 || D < 2 || D % 2 || max_seq < 1 || slot_base < 0)
    HI_FAIL("hi_rope_cache: bad shape M=%d Hq=%d Hkv=%d D=%d max_seq=%d", M, Hq, Hkv, D, max_seq);
  if (M == 0) return 0;
  if (!qkv || !cs || !kc || !vc) HI_FAIL("hi_rope_cache: null tensor pointer");
  if (ldq < (Hq + 2 * Hkv) * D) HI_FAIL("hi_rope_cache: ldq %d < (Hq + 2 Hkv) D", ldq);
  if (!pos && (pos_base < 0 || (int64_t)pos_base + M > max_seq))
    HI_FAIL("hi_rope_cache: positions %d..%d outside the cache (max_seq %d)", pos_base, pos_base + M - 1, max_seq);
  if (!aligned(cs, 4)) HI_FAIL("hi_rope_cache: cs must be 4-byte aligned");
  const bool v8 = D % 16 == 0 && ldq % 8 == 0 && aligned(qkv, 16) && aligned(cs, 16) && aligned(kc, 16) && aligned(vc, 16);
  hipLaunchKernelGGL(v8 ? rope_cache_v8_kernel : rope_cache_kernel, dim3(M), dim3(256), 0, (hipStream_t)stream, (f16*)qkv,
                     (int64_t)ldq, Hq, Hkv, D, (const f16x2*)cs, pos, pos_base, slot_base, (f16*)kc, (f16*)vc, max_seq);
  HI_TRY(hipGetLastError());
  return 0;
}

// Causal prefill attention of T query rows (row t at position p0 + t; head h at columns h*D of
// q [T, ldq]) over one cache slot kc / vc [Hkv][max_seq][D], keys 0..p0+t; out [T, ldo].
HI_EXPORT int hi_flash_prefill(const void* q, int ldq, const void* kc, const void* vc, int max_seq, void* out, int ldo,
                               int T, int p0, int Hq, int Hkv, int D, void* stream) {
  return flash_prefill(q, ldq, kc, vc, max_seq, out, ldo, T, p0, Hq, Hkv, D, nullptr, stream, "hi_flash_prefill");
}

// The same, and each row's log2-domain log-sum-exp of the scaled logits into lse [Hq][T] fp32.
HI_EXPORT int hi_flash_prefill_lse(const void* q, int ldq, const void* kc, const void* vc, int max_seq, void* out,
                                   int ldo, int T, int p0, int Hq, int Hkv, int D, float* lse, void* stream) {
  if (!lse) HI_FAIL("hi_flash_prefill_lse: lse must not be null");
  return flash_prefill(q, ldq, kc, vc, max_seq, out, ldo, T, p0, Hq, Hkv, D, lse, stream, "hi_flash_prefill_lse");
}
