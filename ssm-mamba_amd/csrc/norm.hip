// RMSNorm over the channel axis of channel-major activations (batch, C, L),
// for gfx950:
//
//   out[b, c, t] = x[b, c, t] * rsqrt(mean_c x[b, c, t]^2 + eps) * (1 + w[c])
//
// the reference's RMSNorm (modules/rms_norm.py:11-31: fp32 statistics, scale
// 1 + weight, result cast back to the input type) applied to the layout the
// scan streams, so the Mamba stack needs no (B, L, C) <-> (B, C, L) copies.
//
// A workgroup owns 128 positions of one batch row; its 16 waves split the
// channels, each lane holding two adjacent positions, so every wave load is a
// contiguous 256- or 512-byte row segment.  Pass 1 accumulates x^2 per
// position and the waves combine their sums through LDS; pass 2 re-reads x
// (cache-resident) and writes the scaled result.
#include "ss_common.cuh"
#include "ss_prof.h"

namespace ssm {

namespace {

constexpr int kNormThreads = 1024;
constexpr int kNormWaves = kNormThreads / 64;
constexpr int kNormPos = 128;  // positions per workgroup (2 per lane)

template <typename T>
struct Pair;

template <>
struct Pair<float> {
  __device__ static __forceinline__ float2 load(const float* p) {
    return *reinterpret_cast<const float2*>(p);
  }
  __device__ static __forceinline__ void store(float* p, float a, float b) {
    *reinterpret_cast<float2*>(p) = make_float2(a, b);
  }
};

template <>
struct Pair<__hip_bfloat16> {
  __device__ static __forceinline__ float2 load(const __hip_bfloat16* p) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    return make_float2(bf16_lo(w), bf16_hi(w));
  }
  __device__ static __forceinline__ void store(__hip_bfloat16* p, float a, float b) {
    *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(a, b);
  }
};

// kPair: L even and rows 4-byte (bf16) / 8-byte (fp32) aligned, so a lane's two
// positions load and store as one element pair.
template <typename T, bool kPair>
__global__ __launch_bounds__(kNormThreads) void rms_norm_cm_kernel(
    const T* __restrict__ x, const T* __restrict__ w, float eps, T* __restrict__ out, int C, int L,
    int tiles) {
  __shared__ float s_ss[kNormWaves][kNormPos];
  const int b = blockIdx.x / tiles;
  const int t0 = (blockIdx.x - b * tiles) * kNormPos;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int t = t0 + 2 * lane;
  const bool ok0 = t < L, ok1 = t + 1 < L;
  const int cpw = (C + kNormWaves - 1) / kNormWaves;
  const int c_lo = min(C, wave * cpw), c_hi = min(C, c_lo + cpw);
  const T* __restrict__ xb = x + (size_t)b * C * L;
  T* __restrict__ ob = out + (size_t)b * C * L;

  auto load2 = [&](int c) -> float2 {
    const T* p = xb + (size_t)c * L + t;
    if constexpr (kPair) {
      return ok0 ? Pair<T>::load(p) : make_float2(0.f, 0.f);
    } else {
      return make_float2(ok0 ? Elem<T>::load1(p) : 0.f, ok1 ? Elem<T>::load1(p + 1) : 0.f);
    }
  };

  float s0 = 0.f, s1 = 0.f;
#pragma unroll 16
  for (int c = c_lo; c < c_hi; ++c) {
    const float2 v = load2(c);
    s0 = fmaf(v.x, v.x, s0);
    s1 = fmaf(v.y, v.y, s1);
  }
  s_ss[wave][2 * lane] = s0;
  s_ss[wave][2 * lane + 1] = s1;
  __syncthreads();
  float q0 = 0.f, q1 = 0.f;
#pragma unroll
  for (int i = 0; i < kNormWaves; ++i) {
    q0 += s_ss[i][2 * lane];
    q1 += s_ss[i][2 * lane + 1];
  }
  const float r0 = rsqrtf(q0 / (float)C + eps);
  const float r1 = rsqrtf(q1 / (float)C + eps);
#pragma unroll 16
  for (int c = c_lo; c < c_hi; ++c) {
    const float2 v = load2(c);
    const float g = 1.0f + Elem<T>::load1(w + c);
    T* p = ob + (size_t)c * L + t;
    if constexpr (kPair) {
      if (ok0) Pair<T>::store(p, v.x * r0 * g, v.y * r1 * g);
    } else {
      if (ok0) Elem<T>::store1(p, v.x * r0 * g);
      if (ok1) Elem<T>::store1(p + 1, v.y * r1 * g);
    }
  }
}

template <typename T>
hipError_t launch_norm_t(const void* x, const void* w, float eps, void* out, int B, int C, int L,
                         bool pair, hipStream_t st) {
  ProfScope prof("rms_norm_cm", st);
  const int tiles = (L + kNormPos - 1) / kNormPos;
  const dim3 grid((unsigned)((size_t)B * tiles));
  auto* xp = static_cast<const T*>(x);
  auto* wp = static_cast<const T*>(w);
  auto* op = static_cast<T*>(out);
  if (pair)
    hipLaunchKernelGGL((rms_norm_cm_kernel<T, true>), grid, dim3(kNormThreads), 0, st, xp, wp, eps,
                       op, C, L, tiles);
  else
    hipLaunchKernelGGL((rms_norm_cm_kernel<T, false>), grid, dim3(kNormThreads), 0, st, xp, wp, eps,
                       op, C, L, tiles);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rms_norm_cm(int bf16, const void* x, const void* w, float eps, void* out, int B,
                              int C, int L, bool pair, hipStream_t st) {
  return bf16 ? launch_norm_t<__hip_bfloat16>(x, w, eps, out, B, C, L, pair, st)
              : launch_norm_t<float>(x, w, eps, out, B, C, L, pair, st);
}

}  // namespace ssm
