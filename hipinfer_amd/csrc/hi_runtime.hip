// Per-device state, the int8 weight quantiser (on the GPU), and the standalone RMSNorm.
//
// hi_quantize_rows / hi_dequantize_rows move the reference's host-side quantiser
// (scripts/export.py:54-73, spec docs/quantization.md:24-31) onto the GPU, bit-exact:
//   s[n] = fp16(fp32(max_k |w[n, k]| / 127)), q = clamp(round_half_even(fp32(w / s)), -127, 127),
//   q = 0 when s == 0;  dequantised weight = fp16(q * s).
// hi_rmsnorm is the unfused form of the GEMV prologue (reference api.cu hi_rmsnorm,
// kernels.cuh:110-125), kept because the reference's fused-QKV tests build their expected values
// from it.
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

#include "hi_common.h"

static std::mutex g_mu;
static HiDevice g_dev[64];

const HiDevice* hi_device() {
  int id = 0;
  hipError_t e = hipGetDevice(&id);
  if (e != hipSuccess || id < 0 || id >= 64) {
    fprintf(stderr, "hipinfer_amd: no usable HIP device (%s)\n", hipGetErrorString(e));
    return nullptr;
  }
  HiDevice& d = g_dev[id];
  if (d.ready.load(std::memory_order_acquire)) return &d;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!d.ready.load(std::memory_order_relaxed)) {
    int cus = 0, lds = 0, optin = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, id) != hipSuccess ||
        hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, id) != hipSuccess) {
      fprintf(stderr, "hipinfer_amd: cannot read the properties of device %d\n", id);
      return nullptr;
    }
    if (hipDeviceGetAttribute(&optin, hipDeviceAttributeSharedMemPerBlockOptin, id) != hipSuccess) optin = 0;
    d.cus = cus;
    d.lds_max = optin > 0 ? (optin < lds ? optin : lds) : lds;
    d.xcds = 8;
    d.id = id;
    d.ready.store(true, std::memory_order_release);
  }
  return &d;
}

int hi_blocks_per_cu(const void* fn, int block, size_t lds) {
  const HiDevice* d = hi_device();
  if (!d) return -1;
  static std::map<std::tuple<int, const void*, int, size_t>, int> cache;
  const auto key = std::make_tuple(d->id, fn, block, lds);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  hipFuncAttributes fa{};
  hipError_t e = hipFuncGetAttributes(&fa, fn);
  if (e != hipSuccess) {
    fprintf(stderr, "hipinfer_amd: hipFuncGetAttributes failed: %s\n", hipGetErrorString(e));
    return -1;
  }
  const size_t dyn_max = (size_t)d->lds_max - fa.sharedSizeBytes;  // static LDS counts against the CU's
  if (lds > dyn_max) return 0;
  if (lds > 48 * 1024) {
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn_max);
    if (e != hipSuccess) {
      fprintf(stderr, "hipinfer_amd: hipFuncSetAttribute failed: %s\n", hipGetErrorString(e));
      return -1;
    }
  }
  int n = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, block, lds);
  if (e != hipSuccess) {
    fprintf(stderr, "hipinfer_amd: occupancy query failed: %s\n", hipGetErrorString(e));
    return -1;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  cache[key] = n;
  return n;
}

int hi_gemv_max_rows() {
  static const int v = [] {
    const char* e = getenv("HIPINFER_GEMV_MAX");
    const int n = e ? atoi(e) : 8;
    return n < 0 ? 0 : n > 8 ? 8 : n;
  }();
  return v;
}

HI_EXPORT int hi_device_cus() {
  const HiDevice* d = hi_device();
  return d ? d->cus : -2;
}

// The largest dynamic LDS one block may opt into on the current device (the reference's
// hi_max_smem, api.cu:49: its shared-memory opt-in, which sizes the fused-norm GEMV's rows; on
// MI355X the CU's 160 KB LDS); -2 on a HIP error.
HI_EXPORT int hi_max_smem() {
  const HiDevice* d = hi_device();
  return d ? d->lds_max : -2;
}

// ------------------------------------------------------------------ quantiser
// One wave per row. VEC: 16-byte loads (K % 8 == 0, 16-byte aligned rows), else 2-byte loads.
template <bool VEC>
__global__ void __launch_bounds__(256) quantize_rows_kernel(const f16* __restrict__ w, int64_t N, int K,
                                                           int8_t* __restrict__ q, f16* __restrict__ s) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const f16* wr = w + n * K;
  int8_t* qr = q + n * K;
  float amax = 0.f;
  if constexpr (VEC) {
    for (int c = lane; c < K / 8; c += 64) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(wr + 8 * c);
#pragma unroll
      for (int i = 0; i < 8; i++) amax = fmaxf(amax, __builtin_fabsf((float)v[i]));
    }
  } else {
    for (int k = lane; k < K; k += 64) amax = fmaxf(amax, __builtin_fabsf((float)wr[k]));
  }
  amax = wave_max(amax);
  const f16 sh = (f16)(amax / 127.0f);  // IEEE division, then round to nearest even
  const float sf = (float)sh;
  auto code = [&](f16 x) -> int8_t {
    if (!(sf > 0.f)) return 0;
    float v = __builtin_rintf((float)x / sf);
    v = fminf(fmaxf(v, -127.f), 127.f);
    return (int8_t)(int)v;
  };
  if constexpr (VEC) {
    for (int c = lane; c < K / 8; c += 64) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(wr + 8 * c);
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        lo |= (uint32_t)(uint8_t)code(v[i]) << (8 * i);
        hi |= (uint32_t)(uint8_t)code(v[i + 4]) << (8 * i);
      }
      *reinterpret_cast<u32x2*>(qr + 8 * c) = u32x2{lo, hi};
    }
  } else {
    for (int k = lane; k < K; k += 64) qr[k] = code(wr[k]);
  }
  if (lane == 0) s[n] = sh;
}

HI_EXPORT int hi_quantize_rows(const void* w, long long N, int K, void* q, void* s, void* stream) {
  if (N < 0 || K < 1) HI_FAIL("hi_quantize_rows: bad shape N=%lld K=%d", N, K);
  if (N == 0) return 0;
  if (!w || !q || !s) HI_FAIL("hi_quantize_rows: null pointer");
  const dim3 grid((unsigned)((N + 3) / 4));
  const bool vec = K % 8 == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)q & 7) == 0;
  if (vec)
    hipLaunchKernelGGL(quantize_rows_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, (const f16*)w, (int64_t)N,
                       K, (int8_t*)q, (f16*)s);
  else
    hipLaunchKernelGGL(quantize_rows_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, (const f16*)w,
                       (int64_t)N, K, (int8_t*)q, (f16*)s);
  HI_TRY(hipGetLastError());
  return 0;
}

// fp16(q * s): the weights the int8 GEMM computes with. Exact int8 -> fp16, then one correctly
// rounded fp16 product (q * s is exact before that rounding).
__global__ void __launch_bounds__(256) dequantize_rows_kernel(const int8_t* __restrict__ q, const f16* __restrict__ s,
                                                             int64_t N, int K, f16* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;  // 4 weights per thread
  const int64_t total = N * K;
  if (i >= total) return;
  if (i + 4 <= total && (K & 3) == 0) {
    const int64_t n = i / K;
    const f16 sc = s[n];
    const f16x2 s2 = {sc, sc};
    f16x2 lo, hi;
    i8x4_to_f16(*reinterpret_cast<const uint32_t*>(q + i), lo, hi);
    lo = lo * s2;
    hi = hi * s2;
    *reinterpret_cast<f16x4*>(out + i) = f16x4{lo.x, lo.y, hi.x, hi.y};
  } else {
    for (int64_t j = i; j < i + 4 && j < total; j++) out[j] = (f16)(int)q[j] * s[j / K];
  }
}

HI_EXPORT int hi_dequantize_rows(const void* q, const void* s, long long N, int K, void* out, void* stream) {
  if (N < 0 || K < 1) HI_FAIL("hi_dequantize_rows: bad shape N=%lld K=%d", N, K);
  if (N == 0) return 0;
  if (!q || !s || !out) HI_FAIL("hi_dequantize_rows: null pointer");
  if (((uintptr_t)q & 3) || ((uintptr_t)out & 7)) HI_FAIL("hi_dequantize_rows: q must be 4-byte and out 8-byte aligned");
  const int64_t threads = (N * (int64_t)K + 3) / 4;
  hipLaunchKernelGGL(dequantize_rows_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const int8_t*)q, (const f16*)s, (int64_t)N, K, (f16*)out);
  HI_TRY(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------------ standalone RMSNorm
// y = w * fp16(x * (1 / sqrt(mean x^2 + eps))), one block of kNormThreads per row, rows contiguous.
// Rows of up to kNormChunks * kNormThreads chunks stay in registers between the sum of squares and
// the scaling (one read of the row), and the norm weight is requested before the reduction; the
// sums run in the same chunk order either way.
__global__ void __launch_bounds__(kNormThreads) rmsnorm_kernel(const f16* __restrict__ x, const f16* __restrict__ w,
                                                              f16* __restrict__ y, int H, float eps) {
  constexpr int RC = kNormChunks;
  __shared__ float red[kNormThreads / 64];
  const int tid = threadIdx.x, n8 = H / 8;
  const f16* xr = x + (int64_t)blockIdx.x * H;
  f16* yr = y + (int64_t)blockIdx.x * H;
  const bool held = n8 <= RC * kNormThreads;
  u32x4 xv[RC], wv[RC];
  float ss = 0.f;
  if (held) {
#pragma unroll
    for (int j = 0; j < RC; j++) {
      const int c = tid + j * kNormThreads;
      xv[j] = c < n8 ? *reinterpret_cast<const u32x4*>(xr + 8 * c) : u32x4{0u, 0u, 0u, 0u};
      wv[j] = c < n8 ? *reinterpret_cast<const u32x4*>(w + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < RC; j++)
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const f16x2 h = as_h2(xv[j][p]);
        ss = dot2(h, h, ss);
      }
  } else {
    for (int i = tid; i < n8; i += kNormThreads) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(xr + 8 * i);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const f16x2 h = as_h2(v[p]);
        ss = dot2(h, h, ss);
      }
    }
  }
  const float r = norm_finish(ss, red, H, eps);
  auto scale = [&](u32x4 xc, u32x4 wc) {
    u32x4 o;
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const f16x2 xh = as_h2(xc[p]), wh = as_h2(wc[p]);
      f16x2 t;
      t.x = wh.x * (f16)((float)xh.x * r);
      t.y = wh.y * (f16)((float)xh.y * r);
      o[p] = as_u32(t);
    }
    return o;
  };
  if (held) {
#pragma unroll
    for (int j = 0; j < RC; j++) {
      const int c = tid + j * kNormThreads;
      if (c < n8) *reinterpret_cast<u32x4*>(yr + 8 * c) = scale(xv[j], wv[j]);
    }
  } else {
    for (int i = tid; i < n8; i += kNormThreads)
      *reinterpret_cast<u32x4*>(yr + 8 * i) =
          scale(*reinterpret_cast<const u32x4*>(xr + 8 * i), *reinterpret_cast<const u32x4*>(w + 8 * i));
  }
}

HI_EXPORT int hi_rmsnorm(const void* x, const void* w, void* y, int M, int H, float eps, void* stream) {
  if (M < 0 || H < 8 || H % 8) HI_FAIL("hi_rmsnorm: H must be a positive multiple of 8 (H=%d)", H);
  if (M == 0) return 0;
  if (!x || !w || !y || ((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)y & 15))
    HI_FAIL("hi_rmsnorm: x, w, y must be 16-byte aligned device pointers");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(kNormThreads), 0, (hipStream_t)stream, (const f16*)x, (const f16*)w,
                     (f16*)y, H, eps);
  HI_TRY(hipGetLastError());
  return 0;
}
