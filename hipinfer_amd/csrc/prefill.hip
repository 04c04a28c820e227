// Prefill kernels around the GEMM, behind the reference's C-ABI: the RoPE + KV-cache write that
// follows a QKV GEMM (hi_rope_cache; src/api.cu:579-586, kernels.cuh:1120-1158, ctypes
// scripts/hipinfer.py:164-168) and causal prefill attention over a cache slot (hi_flash_prefill,
// hi_flash_prefill_lse; api.cu:594-623, kernels.cuh:1160-1329, ctypes hipinfer.py:171-202).
//
// Flash prefill for gfx950 (D = 64 or 128):
//  * block = 32 RG query rows of one query head and 2 RG waves: the waves of row group g (g and
//    g + RG) share its 32 rows and split every 128-key tile, keys 0..63 and 64..127, each with its
//    own online-softmax state; the pair merges (m, l, O) through LDS at the end. Two waves per
//    SIMD let one wave's softmax run beside the other's matrix work. The wave's Q rows stay in
//    registers as v_mfma_f32_32x32x16_f16 operands for the whole kernel;
//  * 128-key K/V tiles of the head's cache rows go straight from global memory into LDS by buffer
//    DMA (no register staging), two LDS stages: tile j + 1 streams in while tile j is computed,
//    one barrier per tile. Both tiles keep the cache's row-major order with their 16-byte chunks
//    XOR-swizzled by the key; the swizzle is applied to the DMA's per-lane source address, since
//    a DMA instruction writes 64 consecutive 16-byte LDS slots;
//  * S^T = K Q^T over the wave's 64 keys, in 32-key MFMA blocks: with the K fragment as first
//    operand each lane ends with 16 keys per block of ONE query row (split between lanes l and
//    l + 32), so the row max and sum of the online softmax are the lane's own values plus one
//    exchange with lane l ^ 32;
//  * logits are scaled by log2(e) / sqrt(D) and the softmax runs in base 2 (the reference's
//    log2-domain form, kernels.cuh:1236-1262); P is rounded to fp16 for P.V, the row sum l keeps
//    fp32 p, as the reference does. exp2 is the hardware's v_exp_f32, whose results below 2^-126
//    flush to zero: such p round to fp16 zero anyway and vanish against l >= 1 in fp32. A row's
//    reference max moves only when the row's max passes it by more than 2^8 (p <= 256), and O is
//    rescaled only then;
//  * O^T += V^T P^T: the P registers of a lane are already a B fragment of the next product once
//    the key order inside each 16-key step is permuted identically for P and V^T (lane half fk
//    takes keys 4 fk + 0..3 and 8 + 4 fk + 0..3), so P never goes through LDS. The V^T fragments
//    come from the row-major V tile through ds_read_tr16_b64, which transposes 4 keys x 16 d
//    blocks within each 16-lane group; O^T keeps the lane -> query row map, so the per-row
//    rescale by exp2(m_old - m_new) is per lane;
//  * causal mask on absolute positions (row t at p0 + t sees keys 0..p0+t); a wave skips key
//    halves that lie wholly above its rows' diagonal and drops the mask on halves wholly below
//    it; cache rows past the block's last key read as zeros (the DMA's buffer range ends there);
//  * blocks run the longest query tiles (the most keys) first, across all heads.
#include "hi_common.h"

namespace {

constexpr int kFpRG = 4;              // 32-row groups per block (2 waves each)
constexpr int kFpBQ = 32 * kFpRG;     // query rows per block
constexpr int kFpKPW = 64;            // keys per wave per tile (32-key MFMA blocks of the wave's half)
constexpr int kFpBKV = 2 * kFpKPW;    // keys per tile
constexpr int kFpStages = 2;          // LDS stages of K/V tiles
constexpr float kFpMaxLag = 8.f;      // log2 of how far a row's reference max may trail its max

// XOR term of key r's 16-byte chunks in the K tile: the 16 keys (D = 128) or 8 key pairs (D = 64)
// that one 128-bit fragment read serves per cycle land on distinct banks.
template <int D>
__device__ __forceinline__ int k_swz(int r) {
  if constexpr (D == 128) return r & 15;
  else return (r >> 1) & 7;
}
// XOR term of key r's chunks in the V tile. A transpose read covers keys r..r+3 (r % 4 == 0) at
// 4 consecutive chunks per 32 lanes and 2 per 16 lanes; the terms 0, 6, 12, 10 (D = 128) or 0, 6,
// 4, 2 (D = 64) for r % 4 = 0..3 move those chunks to distinct banks at either width.
template <int D>
__device__ __forceinline__ int v_swz(int r) {
  const int a = r & 3;
  return ((2 * a) ^ (4 * a)) & (D / 8 - 1);
}

template <int D>
struct FpStage {
  u32x4 k[kFpBKV * D / 8];
  u32x4 v[kFpBKV * D / 8];
};
// The O^T accumulators the second wave of each row group hands to the first at the end (in the
// stages' LDS).
template <int D, int RG>
struct FpMerge {
  f32x16 o[RG][D / 32][64];
};

typedef short i16x4 __attribute__((ext_vector_type(4)));

// The two builtins below sit in the device pass only: in this kernel's host pass they made the
// compiler drop the kernel's launch stub without a diagnostic (an undefined symbol at load).
// 16-byte buffer DMA of each lane's chunk at byte offset voff into LDS slot lane of `lds`.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, void* lds, int voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)lds, 16, voff, 0, 0, 0);
#endif
}
// ds_read_tr16_b64 at LDS address p: within each 16-lane group, lane i receives element i % 4 of
// the 4 halves lane 4 e + i / 4 addresses, as its element e.
__device__ __forceinline__ f16x4 lds_read_tr16(const f16* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p));
#else
  return f16x4{};
#endif
}

template <int D, int RG>
__global__ void __launch_bounds__(128 * RG)
    flash_prefill_kernel(const f16* __restrict__ q, int64_t ldq, const f16* __restrict__ kc,
                         const f16* __restrict__ vc, int max_seq, f16* __restrict__ out, int64_t ldo, int T, int p0,
                         int Hq, int Hkv, float scale_log2, float* __restrict__ lse) {
  constexpr int NW = 2 * RG, BQ = 32 * RG;
  constexpr int CPR = D / 8;                   // 16-byte chunks per key row
  constexpr int IPW = kFpBKV * CPR / 64 / NW;  // DMA instructions per wave per tile and operand
  constexpr int DT = D / 32;                   // 32-row output tiles of O^T
  static_assert(IPW * 64 * NW == kFpBKV * CPR, "tile DMA split");
  static_assert(sizeof(FpMerge<D, RG>) <= sizeof(FpStage<D>) * kFpStages, "merge fits the stages");
  __shared__ FpStage<D> sm[kFpStages];
  __shared__ float ml[2][RG][64];  // the second waves' m and l

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = wave % RG, kh = wave / RG;     // row group, key half
  const int fr = lane & 31, fk = lane >> 5;
  // grid (Hq, query tiles), dispatched x first: all heads' longest query tile first; block x runs
  // on XCD x % 8, which takes a contiguous range of query heads (those sharing a KV head)
  const int q0 = (gridDim.y - 1 - blockIdx.y) * BQ;
  const int h = Hq % 8 ? blockIdx.x : (blockIdx.x % 8) * (Hq / 8) + blockIdx.x / 8, hk = h / (Hq / Hkv);
  const int qw = q0 + rg * 32;                  // this wave's first query row
  const int qi = qw + fr;                       // this lane's query row
  const int qpos = p0 + qi;
  const int kv_end = p0 + min(q0 + BQ, T);      // keys any row of the block can see
  // the head's cache rows 0..kv_end-1: loads past them return zeros
  const __amdgpu_buffer_rsrc_t k_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<f16*>(kc + (int64_t)hk * max_seq * D), (short)0, kv_end * D * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<f16*>(vc + (int64_t)hk * max_seq * D), (short)0, kv_end * D * 2, 0x00020000);

  // DMA instruction i of this wave fills slots (wave IPW + i) * 64 + lane of a tile: slot s holds
  // key s / CPR, physical chunk s % CPR, i.e. logical chunk (s % CPR) ^ swz(key)
  int koff[IPW], voff[IPW];
#pragma unroll
  for (int i = 0; i < IPW; i++) {
    const int s = (wave * IPW + i) * 64 + lane, r = s / CPR, p = s % CPR;
    koff[i] = (r * D + 8 * (p ^ k_swz<D>(r))) * 2;
    voff[i] = (r * D + 8 * (p ^ v_swz<D>(r))) * 2;
  }
  auto issue = [&](int j0, int st) {
#pragma unroll
    for (int i = 0; i < IPW; i++) {
      lds_dma16(k_rs, &sm[st].k[(wave * IPW + i) * 64], koff[i] + j0 * D * 2);
      lds_dma16(v_rs, &sm[st].v[(wave * IPW + i) * 64], voff[i] + j0 * D * 2);
    }
  };
  issue(0, 0);

  // this lane's Q fragments: row qi, d = 16 ks + 8 fk + 0..7 (zero past T)
  f16x8 qf[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ks++) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (qi < T) v = *reinterpret_cast<const u32x4*>(q + (int64_t)qi * ldq + h * D + 16 * ks + 8 * fk);
    qf[ks] = __builtin_bit_cast(f16x8, v);
  }

  // transpose reads of V: lane j of each 16-lane group g reads 4 d of key 4 (g / 2) + j / 4 (+ the
  // step's key base), d = 16 (g % 2) + 4 (j % 4) (+ the output tile's d base); the group's lane i
  // then holds d = 16 (g % 2) + i of those 4 keys. Keys of one read are 4-aligned, so the swizzle
  // term is the lane's own.
  const int vr = 4 * fk + ((lane & 15) >> 2);                  // key within a 16-key step
  const int vc0 = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);   // logical chunk within a 32-d tile
  const int vsw = v_swz<D>(vr), vh = 4 * (lane & 1);           // swizzle term, half within the chunk
  constexpr int KT = kFpKPW / 32;                              // 32-key blocks per wave per tile
  const int kr = kFpKPW * kh + fr;                             // K row of this lane's first fragments
  const int ksw = k_swz<D>(kr);                                // the same for every block (kr % 16)
  const int xaddr = (lane ^ 32) << 2;                          // lane l ^ 32, for ds_bpermute
  auto xor32 = [&](float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(xaddr, __builtin_bit_cast(int, v)));
  };

  float m_i = -__builtin_huge_valf(), l_i = 0.f;
  f32x16 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; dt++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[dt][e] = 0.f;

  int st = 0;
  for (int j0 = 0; j0 < kv_end; j0 += kFpBKV, st ^= 1) {
    wait_vmcnt<0>();  // this wave's share of tile j0 is in LDS
    __syncthreads();  // every share is, and every wave is done with the other stage
    if (j0 + kFpBKV < kv_end) issue(j0 + kFpBKV, st ^ 1);
    const int k0 = j0 + kFpKPW * kh;                // this wave's first key
    if (k0 > p0 + qw + 31 || k0 >= kv_end) continue;  // every key of the half is masked for every row
    const bool full = k0 + kFpKPW - 1 <= p0 + qw && k0 + kFpKPW <= kv_end;  // no key of the half is masked
    const u32x4* ks_ = sm[st].k;
    const f16* vs_ = reinterpret_cast<const f16*>(sm[st].v);

    // ---- S^T = K Q^T over the wave's keys, 32 per block kt; lane (row fr, half fk) gets keys
    //      32 kt + 8 g + 4 fk + e
    f32x16 s[KT];
#pragma unroll
    for (int kt = 0; kt < KT; kt++) {
#pragma unroll
      for (int e = 0; e < 16; e++) s[kt][e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < D / 16; ks++) {
        const f16x8 kf = __builtin_bit_cast(f16x8, ks_[(kr + 32 * kt) * CPR + ((2 * ks + fk) ^ ksw)]);
        s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ks], s[kt], 0, 0, 0);
      }
    }
    // ---- online softmax of row qi over these keys (base 2). The row's reference max m_i moves
    //      only when the tile's scaled max exceeds it by more than 2^8, so p = exp2(c s - m_i) stays
    //      at most 256 (exact range for fp16 P and fp32 sums) and O is rescaled only then; the
    //      max of the raw logits is scaled once (c > 0 keeps the order) and c s - m_i is one fma
    float mx = -__builtin_huge_valf();
    if (full) {
#pragma unroll
      for (int kt = 0; kt < KT; kt++)
#pragma unroll
        for (int e = 0; e < 16; e++) mx = fmaxf(mx, s[kt][e]);
    } else {
#pragma unroll
      for (int kt = 0; kt < KT; kt++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int kp = k0 + 32 * kt + 8 * (e >> 2) + 4 * fk + (e & 3);
          const float v = (kp <= qpos && kp < kv_end) ? s[kt][e] : -__builtin_huge_valf();
          s[kt][e] = v;
          mx = fmaxf(mx, v);
        }
    }
    mx = fmaxf(mx, xor32(mx)) * scale_log2;
    const bool move = mx > m_i + kFpMaxLag;  // m_i = -inf: moves to the first finite max
    const float alpha = move ? __builtin_amdgcn_exp2f(m_i - mx) : 1.f;
    if (move) m_i = mx;
    // m_i is -inf only for a row that has seen no key yet (a row past T, or one whose first key
    // lies in the other half): every logit is then -inf and every p 0
    const float m_use = m_i == -__builtin_huge_valf() ? 0.f : m_i;
    float sum = 0.f;
    f16x8 pf[KT][2];
#pragma unroll
    for (int kt = 0; kt < KT; kt++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][e], scale_log2, -m_use));
        sum += p;
        pf[kt][e >> 3][e & 7] = (f16)p;
      }
    sum += xor32(sum);
    l_i = l_i * alpha + sum;
    if (__any(move)) {
#pragma unroll
      for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[dt][e] *= alpha;
    }
    // ---- O^T += V^T P^T; step ss of block kt: lane half fk holds keys 32 kt + 16 ss + 4 fk + 0..3
    //      and 32 kt + 16 ss + 8 + 4 fk + 0..3 of the wave's keys, in P's registers and in the V^T
    //      reads alike
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int kt = 0; kt < KT; kt++)
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {
          const int key = kFpKPW * kh + 32 * kt + 16 * ss + vr;
          const f16* pa = vs_ + key * D + 8 * ((4 * dt + vc0) ^ vsw) + vh;
          const f16x4 fa = lds_read_tr16(pa), fb = lds_read_tr16(pa + 8 * D);  // key + 8: same swizzle term
          const f16x8 vf = {fa[0], fa[1], fa[2], fa[3], fb[0], fb[1], fb[2], fb[3]};
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[kt][ss], o[dt], 0, 0, 0);
        }
  }

  // ---- merge the two key halves of each row group: the second wave hands (m, l, O) over
  __syncthreads();  // every wave is done with the stages (no DMA is in flight after the last tile)
  FpMerge<D, RG>& mg = *reinterpret_cast<FpMerge<D, RG>*>(sm);
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; dt++) mg.o[rg][dt][lane] = o[dt];
    ml[0][rg][lane] = m_i;
    ml[1][rg][lane] = l_i;
  }
  __syncthreads();
  if (kh == 1 || qi >= T) return;
  const float m1 = ml[0][rg][lane], l1 = ml[1][rg][lane];
  const float m = fmaxf(m_i, m1);  // finite: key 0 is visible to every row
  const float a0 = __builtin_amdgcn_exp2f(m_i - m), a1 = __builtin_amdgcn_exp2f(m1 - m);
  const float l = l_i * a0 + l1 * a1;
  if (lse && fk == 0) lse[(int64_t)h * T + qi] = m + log2f(l);
  const float inv = 1.f / l;
  f16* orow = out + (int64_t)qi * ldo + h * D;
#pragma unroll
  for (int dt = 0; dt < DT; dt++) {
    const f32x16 o1 = mg.o[rg][dt][lane];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      f16x4 v;
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = (f16)((o[dt][4 * g + e] * a0 + o1[4 * g + e] * a1) * inv);
      *reinterpret_cast<f16x4*>(orow + dt * 32 + 8 * g + 4 * fk) = v;
    }
  }
}

// Any alignment (2-byte accesses only): block (row, head group), one wave per head of the row's
// Hq + 2 Hkv heads. A q head is rotated in place, a k head rotated into the cache, a v head copied
// into the cache; lane j takes the pairs (j, j + D/2), (j + 64, j + 64 + D/2), ... of its head.
// Each pair goes through rope_pair, as in the 16-byte kernel below, so both give the same bits.
constexpr int kRopeHeadsPerBlock = 4;

__global__ void __launch_bounds__(64 * kRopeHeadsPerBlock)
    rope_cache_heads_kernel(f16* qkv, int64_t ldq, int Hq, int Hkv, int D, const f16x2* __restrict__ cs,
                            const int* __restrict__ pos, int pos_base, int slot_base, f16* kc, f16* vc, int max_seq) {
  const int r = blockIdx.x, lane = threadIdx.x & 63;
  const int head = blockIdx.y * kRopeHeadsPerBlock + (threadIdx.x >> 6);
  if (head >= Hq + 2 * Hkv) return;
  const int at = pos ? pos[r] : pos_base + r;                  // position in the cache
  const int64_t cslot = pos ? (int64_t)slot_base + r : slot_base;
  f16* src = qkv + (int64_t)r * ldq + (int64_t)head * D;
  if (head >= Hq + Hkv) {
    f16* dst = vc + ((cslot * Hkv + (head - Hq - Hkv)) * max_seq + at) * D;
    for (int e = lane; e < D; e += 64) dst[e] = src[e];
    return;
  }
  f16* dst = head < Hq ? src : kc + ((cslot * Hkv + (head - Hq)) * max_seq + at) * D;
  const int half = D >> 1;
  const f16x2* tab = cs + (int64_t)at * half;
  for (int j = lane; j < half; j += 64) {
    f16 lo = src[j], hi = src[j + half];
    rope_pair(lo, hi, tab[j]);
    dst[j] = lo;
    dst[j + half] = hi;
  }
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
  if ((int64_t)max_seq * D * 2 > INT32_MAX)  // a head's cache rows are addressed by 32-bit byte offsets
    HI_FAIL("%s: max_seq %d too long for 32-bit cache offsets (at most %d at D=%d)", who, max_seq,
            (int)(INT32_MAX / (2 * D)), D);
  if (!q || !kc || !vc || !out) HI_FAIL("%s: null tensor pointer", who);
  if (!aligned(q, 16) || ldq % 8 || ldq < Hq * D) HI_FAIL("%s: q must be 16-byte aligned, ldq %% 8 == 0, ldq >= Hq*D", who);
  if (!aligned(kc, 16) || !aligned(vc, 16)) HI_FAIL("%s: kc / vc must be 16-byte aligned", who);
  if (!aligned(out, 8) || ldo % 4 || ldo < Hq * D) HI_FAIL("%s: out must be 8-byte aligned, ldo %% 4 == 0, ldo >= Hq*D", who);
  const float scale_log2 = 1.4426950408889634f / sqrtf((float)D);
  if ((T + kFpBQ - 1) / kFpBQ > 65535) HI_FAIL("%s: T=%d exceeds %d query rows", who, T, 65535 * kFpBQ);
  const dim3 grid(Hq, (T + kFpBQ - 1) / kFpBQ);
  const hipStream_t s = (hipStream_t)stream;
  if (D == 128)
    hipLaunchKernelGGL((flash_prefill_kernel<128, kFpRG>), grid, dim3(128 * kFpRG), 0, s, (const f16*)q, (int64_t)ldq,
                       (const f16*)kc, (const f16*)vc, max_seq, (f16*)out, (int64_t)ldo, T, p0, Hq, Hkv, scale_log2, lse);
  else
    hipLaunchKernelGGL((flash_prefill_kernel<64, kFpRG>), grid, dim3(128 * kFpRG), 0, s, (const f16*)q, (int64_t)ldq,
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
  if ((Hq + 2 * Hkv + kRopeHeadsPerBlock - 1) / kRopeHeadsPerBlock > 65535)
    HI_FAIL("hi_rope_cache: %d heads per row exceed the launch grid", Hq + 2 * Hkv);
  if (!pos && (pos_base < 0 || (int64_t)pos_base + M > max_seq))
    HI_FAIL("hi_rope_cache: positions %d..%d outside the cache (max_seq %d)", pos_base, pos_base + M - 1, max_seq);
  if (!aligned(cs, 4)) HI_FAIL("hi_rope_cache: cs must be 4-byte aligned");
  const bool v8 = D % 16 == 0 && ldq % 8 == 0 && aligned(qkv, 16) && aligned(cs, 16) && aligned(kc, 16) && aligned(vc, 16);
  if (v8)
    hipLaunchKernelGGL(rope_cache_v8_kernel, dim3(M), dim3(256), 0, (hipStream_t)stream, (f16*)qkv, (int64_t)ldq, Hq, Hkv,
                       D, (const f16x2*)cs, pos, pos_base, slot_base, (f16*)kc, (f16*)vc, max_seq);
  else
    hipLaunchKernelGGL(rope_cache_heads_kernel, dim3(M, (Hq + 2 * Hkv + kRopeHeadsPerBlock - 1) / kRopeHeadsPerBlock),
                       dim3(64 * kRopeHeadsPerBlock), 0, (hipStream_t)stream, (f16*)qkv, (int64_t)ldq, Hq, Hkv, D,
                       (const f16x2*)cs, pos, pos_base, slot_base, (f16*)kc, (f16*)vc, max_seq);
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
