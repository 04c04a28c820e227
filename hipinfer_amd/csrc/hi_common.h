// Shared device/host pieces of the MI355X (gfx950, CDNA4, wave64) matmul hot path.
// fp16 storage, fp32 accumulation; every fp16 rounding point of the reference kernels
// (src/kernels.cuh:1-3) is kept at the same place.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdio>

#define HI_EXPORT extern "C" __attribute__((visibility("default")))

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ------------------------------------------------------------------ host-side error reporting
// Entry points return 0 on success and a negative code otherwise, after printing the reason:
// -1 an argument the path does not support (the reference prints and exits, api.cu:205-211),
// -2 a HIP runtime error.
#define HI_FAIL(...)                                  \
  do {                                                \
    fprintf(stderr, "hipinfer_amd: " __VA_ARGS__);    \
    fputc('\n', stderr);                              \
    return -1;                                        \
  } while (0)
#define HI_TRY(call)                                                                                 \
  do {                                                                                               \
    hipError_t e_ = (call);                                                                          \
    if (e_ != hipSuccess) {                                                                          \
      fprintf(stderr, "hipinfer_amd: %s failed: %s (%s:%d)\n", #call, hipGetErrorString(e_), __FILE__, \
              __LINE__);                                                                             \
      return -2;                                                                                     \
    }                                                                                                \
  } while (0)

// Per-device properties, read once per device (hi_runtime.hip).
struct HiDevice {
  int id = -1, cus = 0, lds_max = 0, xcds = 8;
  std::atomic<bool> ready{false};  // set (release) once the fields above are filled in
};
const HiDevice* hi_device();  // current device; nullptr on a HIP error (already reported)
// Largest number of resident blocks of `fn` per CU at `block` threads and `lds` dynamic bytes
// (cached per device and kernel); sets the kernel's dynamic-LDS limit first when lds > 64 KB.
int hi_blocks_per_cu(const void* fn, int block, size_t lds);
// HIPINFER_GEMV_MAX (default 8, clamped to 0..8): the largest batch the decode step and the MoE
// experts run on the GEMV path; larger batches take the GEMM path. One value for both callers, as
// in the reference (api.cu:1884-1887), whose default is 4: on MI355X the GEMV stays ahead of the
// small-M GEMM tiles through 8 rows. Read once per process.
int hi_gemv_max_rows();

// ------------------------------------------------------------------ device helpers
typedef __attribute__((address_space(3))) void lds_void_t;

// Wait until at most N vector-memory operations (global loads, LDS DMA) are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// DPP lane moves with compile-time controls (gfx9 encodings): quad_perm, row_half_mirror, row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Sum over the 64 lanes of a wave (called with the whole wave active); every lane receives the
// same total. The tree is fixed: pairs 1, 2, then half-row and row mirrors leave every lane of a
// 16-lane row holding that row's sum; the four row sums r0..r3 (read from lanes 0, 16, 32, 48, no
// LDS round trip) combine as (r0 + r1) + (r2 + r3). IEEE addition is commutative, so a value's
// sum never depends on which lane asks or on how many values the caller reduces.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// RMSNorm rows (rmsnorm_kernel, and the split-K second pass that normalises its result): one block
// of kNormThreads per row; thread t holds chunks t + kNormThreads j (j < kNormChunks: rows of up
// to 8192 halves) and sums their squares chunk by chunk. Both kernels finish with norm_finish, so
// they round alike.
constexpr int kNormThreads = 512;
constexpr int kNormChunks = 2;
// 1 / sqrt(mean(x^2) + eps) of the block's row from each thread's partial sum of squares: wave
// sums, then the 8 wave partials pairwise. red: 8 floats of LDS.
__device__ __forceinline__ float norm_finish(float ss, float* red, int H, float eps) {
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float t = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  return 1.0f / __builtin_sqrtf(t / (float)H + eps);
}

// DPP row_ror:N (rotate right: data moves to higher lanes) into the lanes of the banks (groups of 4
// lanes of a 16-lane row) in BANKS; the other lanes return old. Lane l reads lane
// (l & ~15) | ((l - N) & 15).
template <int N, int BANKS>
__device__ __forceinline__ float dpp_ror(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               0x120 + N, 0xF, BANKS, false));
}

// The partner value of butterfly stage S: lanes 1, 2, 4 and 8 apart within a row (for 4: lanes 4-7
// and 12-15 read 4 lanes down, lanes 0-3 and 8-11 read 4 lanes up, a rotate by 12).
template <int S>
__device__ __forceinline__ float stage_partner(float v) {
  if constexpr (S == 0) return dpp<0xB1>(v);  // quad_perm [1,0,3,2]
  else if constexpr (S == 1) return dpp<0x4E>(v);  // quad_perm [2,3,0,1]
  else if constexpr (S == 2) return dpp_ror<12, 0x5>(dpp_ror<4, 0xA>(0.f, v), v);
  else return dpp_ror<8, 0xF>(0.f, v);
}

template <int S, int NA>
__device__ __forceinline__ void scatter_stage(float (&v)[NA], int n, int lane) {
  const bool b = (lane >> S) & 1;
#pragma unroll
  for (int k = 0; k < NA / 2; k++)
    if (2 * k < n) {
      const float x = v[2 * k], y = v[2 * k + 1];
      v[k] = (b ? y : x) + stage_partner<S>(b ? x : y);
    }
}

// wave_sum of NA accumulators at once (NA a power of 2, called with the whole wave active). The
// tree is wave_sum's: within a row, the partners 1, 2, 4 and 8 lanes apart (a partner in the other
// quad or half-row holds the same partial as wave_sum's mirrored one), then the rows 16 and 32
// apart, (r0 + r1) + (r2 + r3). It is scattered: at stage s < log2(NA) (at most 4) a lane keeps the
// accumulators whose index bit s equals its lane bit s, adds its partner's partials of those and
// hands over the others, so each stage does half the adds of the one before. Every total has
// exactly wave_sum's bits (IEEE addition is commutative). On return, with L = min(NA, 16),
// v[k] (k < NA / L) of every lane l holds the total of accumulator k * L + (l % L).
// The least power of 2 >= n (n >= 1).
constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }

template <int NA>
__device__ __forceinline__ void wave_sum_scatter(float (&v)[NA], int lane) {
  constexpr int S = NA >= 16 ? 4 : NA >= 8 ? 3 : NA >= 4 ? 2 : NA >= 2 ? 1 : 0;
  if constexpr (S > 0) scatter_stage<0>(v, NA, lane);
  if constexpr (S > 1) scatter_stage<1>(v, NA / 2, lane);
  if constexpr (S > 2) scatter_stage<2>(v, NA / 4, lane);
  if constexpr (S > 3) scatter_stage<3>(v, NA / 8, lane);
  // the stages left over when NA < 16 act on the one value each lane holds
  if constexpr (S < 1) v[0] += stage_partner<0>(v[0]);
  if constexpr (S < 2) v[0] += stage_partner<1>(v[0]);
  if constexpr (S < 3) v[0] += stage_partner<2>(v[0]);
  if constexpr (S < 4) v[0] += stage_partner<3>(v[0]);
  constexpr int K = NA > 16 ? NA / 16 : 1;
#pragma unroll
  for (int k = 0; k < K; k++) {
    v[k] += __shfl_xor(v[k], 16, kWave);
    v[k] += __shfl_xor(v[k], 32, kWave);
  }
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// Four int8 weights (one 32-bit word, k order) as two exact fp16 pairs. Each byte, offset by
// 128, becomes the low mantissa byte of the fp16 1024.0 (0x6400 | b = 1024 + b exactly, one
// v_perm_b32 builds two halves), and one packed fp16 subtraction of 1152 leaves q exactly
// (|q| <= 128 is an integer, representable in fp16). Two VALU ops per two weights.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, f16x2& lo, f16x2& hi) {
  const uint32_t b = w ^ 0x80808080u;
  const uint32_t l = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);  // [b0, 0x64, b1, 0x64]
  const uint32_t h = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);  // [b2, 0x64, b3, 0x64]
  const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
  lo = __builtin_bit_cast(f16x2, l) - bias;
  hi = __builtin_bit_cast(f16x2, h) - bias;
}

__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// The same four weights offset by 1152: 1152 + q exactly, without the subtraction (one v_xor and
// two v_perm_b32 per four weights). A dot product over them carries 1152 times the sum of the
// activations it met, which the caller removes (the GEMV starts each sum at -1152 * that sum).
__device__ __forceinline__ void i8x4_to_f16_biased(uint32_t w, f16x2& lo, f16x2& hi) {
  const uint32_t b = w ^ 0x80808080u;
  lo = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u));
  hi = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u));
}

// A 32-bit word as two fp16 values. Always go through this (a scalar parameter): this clang folds
// __builtin_bit_cast applied directly to a vector element `v[p]` to element 0 of `v`.
__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// HF's act_fn(gate) * up with every step rounded to fp16 (reference src/kernels.cuh:100-105).
__device__ __forceinline__ f16 silu_mul(float g, float u) {
  const float gh = (float)(f16)g;
  const f16 s = (f16)(gh / (1.0f + __expf(-gh)));
  return s * (f16)u;  // fp16 product, correctly rounded
}

// The same rounding points with the division done as gh * rcp(1 + e) (v_rcp_f32, 1 ulp): the
// fp32 quotient differs from the IEEE one by at most ~1.5 ulp before its rounding to fp16, so the
// fp16 result matches except when that quotient lies within 1.5 fp32 ulp of an fp16 rounding
// boundary (then it is one fp16 ulp off). For epilogues that produce thousands of values per lane.
__device__ __forceinline__ f16 silu_mul_fast(float g, float u) {
  const float gh = (float)(f16)g;
  float q = gh * __builtin_amdgcn_rcpf(1.0f + __expf(-gh));
  asm volatile("" : "+v"(q));  // fp32 product, then fp16: not one fused mixed-precision rounding
  const f16 s = (f16)q;
  return s * (f16)u;
}

// One RoPE pair with PyTorch's per-op fp16 rounding (reference src/kernels.cuh:132-136).
__device__ __forceinline__ void rope_pair(f16& y1, f16& y2, f16x2 cs) {
  const float c = (float)cs.x, sn = (float)cs.y, f1 = (float)y1, f2 = (float)y2;
  const f16 a = (f16)((float)(f16)(f1 * c) - (float)(f16)(f2 * sn));
  const f16 b = (f16)((float)(f16)(f2 * c) + (float)(f16)(f1 * sn));
  y1 = a;
  y2 = b;
}
