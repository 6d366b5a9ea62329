// Causal depthwise conv1d (+ SiLU) over channel-major rows, forward and
// backward, for gfx950.
//
//   pre[b,c,t] = bias[c] + sum_{j<K} w[c,j] * x[b,c,t-(K-1)+j]   (x = 0 for t < 0)
//   out        = silu(pre) (or pre)
//
// This is the prefill convolution of the Mamba layer (nn.Conv1d with
// groups = channels, padding K-1, first L outputs kept, then SiLU;
// modules/mamba.py:37-44,138-139 of the reference), computed in the
// (batch, channels, seqlen) layout the scan reads, with the activation fused.
//
// Memory-bound: one workgroup streams one (b, c) row; each thread owns chunks
// of 8 consecutive positions (one 16-byte load for bf16, two for fp32) plus
// the previous chunk's last K-1 elements, which the cache serves.  The
// backward recomputes pre over the K-1 positions past its chunk, writes dx,
// and leaves per-row partial sums of dw / dbias that a second kernel adds
// over the batch in a fixed order (deterministic, no atomics).
#include "ss_common.cuh"
#include "ss_io.cuh"
#include "ss_prof.h"

namespace ssm {

namespace {

constexpr int kConvThreads = 256;
constexpr int kConvChunk = 8;
constexpr int kMaxWidth = 8;

template <typename T>
__device__ __forceinline__ void load8(const T* __restrict__ p, float* v);

template <>
__device__ __forceinline__ void load8<float>(const float* __restrict__ p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

template <>
__device__ __forceinline__ void load8<__hip_bfloat16>(const __hip_bfloat16* __restrict__ p, float* v) {
  const uint4 x = *reinterpret_cast<const uint4*>(p);
  v[0] = bf16_lo(x.x); v[1] = bf16_hi(x.x); v[2] = bf16_lo(x.y); v[3] = bf16_hi(x.y);
  v[4] = bf16_lo(x.z); v[5] = bf16_hi(x.z); v[6] = bf16_lo(x.w); v[7] = bf16_hi(x.w);
}

template <typename T>
__device__ __forceinline__ void store8(T* __restrict__ p, const float* v);

template <>
__device__ __forceinline__ void store8<float>(float* __restrict__ p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

template <>
__device__ __forceinline__ void store8<__hip_bfloat16>(__hip_bfloat16* __restrict__ p, const float* v) {
  uint4 x;
  x.x = pack_bf16x2(v[0], v[1]);
  x.y = pack_bf16x2(v[2], v[3]);
  x.z = pack_bf16x2(v[4], v[5]);
  x.w = pack_bf16x2(v[6], v[7]);
  *reinterpret_cast<uint4*>(p) = x;
}

template <int K, typename T>
__device__ __forceinline__ void load_taps(const T* __restrict__ w, const T* __restrict__ bias, int c,
                                          float (&wk)[K], float& bs) {
#pragma unroll
  for (int j = 0; j < K; ++j) wk[j] = Elem<T>::load1(w + (size_t)c * K + j);
  // an absent bias reads a valid stand-in and is dropped: a load in a branch
  // would be waited for there
  bs = Elem<T>::load1(bias ? bias + c : w);
  if (!bias) bs = 0.0f;
}

// Sum of K+1 per-thread values over the workgroup; thread 0 gets the totals.
template <int K>
__device__ __forceinline__ void block_sum(float (&v)[K + 1], float* red) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j <= K; ++j) {
    float s = v[j];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) red[wave * (K + 1) + j] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int j = 0; j <= K; ++j) {
      float s = 0.0f;
      for (int q = 0; q < kConvThreads / 64; ++q) s += red[q * (K + 1) + j];
      v[j] = s;
    }
  }
}

// window (nullable): the decode cache of the row, the K-1 inputs ending at
// position len-1 (len = lengths[b] clamped to [0, L], or L), zero where the
// window starts before the row (the conv context the reference keeps after a
// prefill, modules/mamba.py:113-135).  x's batch rows are xbs elements apart
// (a channel slice of a larger activation); out is contiguous.
template <typename T, int K, bool kVec>
__global__ __launch_bounds__(kConvThreads) void causal_conv1d_fwd_kernel(
    const T* __restrict__ x, int64_t xbs, const T* __restrict__ w, const T* __restrict__ bias,
    T* __restrict__ out, int dim, int L, int silu, const int64_t* __restrict__ lengths,
    T* __restrict__ window) {
  const size_t row = blockIdx.x;
  const int c = (int)(row % (size_t)dim);
  const T* __restrict__ xr = x + (row / (size_t)dim) * (size_t)xbs + (size_t)c * L;
  T* __restrict__ orow = out + row * (size_t)L;
  float wk[K], bs;
  // the decode cache's row length, fetched now and used after the main loop
  const int64_t len_in = lengths ? lengths[row / (size_t)dim] : (int64_t)L;
  if (kVec && L <= kConvThreads * kConvChunk) {
    // one chunk per thread (L <= 2048): its row loads issue before the taps
    // are waited for, so the workgroup pays one memory round trip
    const int t0 = threadIdx.x * kConvChunk;
    const int tc = min(t0, L - kConvChunk);
    float v[2 * kConvChunk];
    load8<T>(xr + tc, v + kConvChunk);
    load8<T>(xr + max(tc - kConvChunk, 0), v);
    load_taps<K>(w, bias, c, wk, bs);
    if (tc == 0) {
#pragma unroll
      for (int i = 0; i < kConvChunk; ++i) v[i] = 0.0f;
    }
    float o[kConvChunk];
#pragma unroll
    for (int i = 0; i < kConvChunk; ++i) {
      float acc = bs;
#pragma unroll
      for (int j = 0; j < K; ++j) acc = fmaf(wk[j], v[kConvChunk + i - (K - 1) + j], acc);
      o[i] = silu ? silu_f(acc) : acc;
    }
    if (t0 < L) store8<T>(orow + t0, o);
  } else if constexpr (kVec) {
    load_taps<K>(w, bias, c, wk, bs);
    for (int t0 = threadIdx.x * kConvChunk; t0 < L; t0 += kConvThreads * kConvChunk) {
      float v[2 * kConvChunk];
      load8<T>(xr + t0, v + kConvChunk);
      // the previous chunk from a clamped address, zeroed at the row start
      // (no load in a branch)
      load8<T>(xr + max(t0 - kConvChunk, 0), v);
      if (t0 == 0) {
#pragma unroll
        for (int i = 0; i < kConvChunk; ++i) v[i] = 0.0f;
      }
      float o[kConvChunk];
#pragma unroll
      for (int i = 0; i < kConvChunk; ++i) {
        float acc = bs;
#pragma unroll
        for (int j = 0; j < K; ++j) acc = fmaf(wk[j], v[kConvChunk + i - (K - 1) + j], acc);
        o[i] = silu ? silu_f(acc) : acc;
      }
      store8<T>(orow + t0, o);
    }
  } else {
    load_taps<K>(w, bias, c, wk, bs);
    for (int t = threadIdx.x; t < L; t += kConvThreads) {
      float acc = bs;
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int tt = t - (K - 1) + j;
        if (tt >= 0) acc = fmaf(wk[j], Elem<T>::load1(xr + tt), acc);
      }
      Elem<T>::store1(orow + t, silu ? silu_f(acc) : acc);
    }
  }
  // the decode cache last, off the main stream's path
  if (K > 1 && window && threadIdx.x < K - 1) {
    const int len = (int)min<int64_t>(max<int64_t>(len_in, 0), L);
    const int idx = len - (K - 1) + (int)threadIdx.x;
    const float v = Elem<T>::load1(xr + max(idx, 0));
    Elem<T>::store1(window + row * (K - 1) + threadIdx.x, idx >= 0 ? v : 0.0f);
  }
}

// dx and per-row partials part[row*(K+1) + j] = sum_t g_t x_{t-(K-1)+j} (j < K)
// and part[row*(K+1) + K] = sum_t g_t, with g = dout * dact(pre).
template <typename T, int K, bool kVec>
__global__ __launch_bounds__(kConvThreads) void causal_conv1d_bwd_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
    const T* __restrict__ dout, T* __restrict__ dx, float* __restrict__ part, int dim, int L,
    int silu) {
  __shared__ float red[(kConvThreads / 64) * (kMaxWidth + 1)];
  const size_t row = blockIdx.x;
  const int c = (int)(row % (size_t)dim);
  const T* __restrict__ xr = x + row * (size_t)L;
  const T* __restrict__ gr = dout + row * (size_t)L;
  T* __restrict__ dxr = dx + row * (size_t)L;
  float wk[K], bs;
  load_taps<K>(w, bias, c, wk, bs);
  float acc[K + 1];
#pragma unroll
  for (int j = 0; j <= K; ++j) acc[j] = 0.0f;

  auto act_grad = [&](float pre) { return silu ? silu_grad_f(pre) : 1.0f; };

  if constexpr (kVec) {
    constexpr int E = kConvChunk;
    for (int t0 = threadIdx.x * E; t0 < L; t0 += kConvThreads * E) {
      // x over [t0-E, t0+2E), dout over [t0, t0+2E)
      float xv[3 * E], dv[2 * E];
      load8<T>(xr + t0, xv + E);
      load8<T>(gr + t0, dv);
      if (t0 > 0) {
        load8<T>(xr + t0 - E, xv);
      } else {
#pragma unroll
        for (int i = 0; i < E; ++i) xv[i] = 0.0f;
      }
      if (t0 + E < L) {
        load8<T>(xr + t0 + E, xv + 2 * E);
        load8<T>(gr + t0 + E, dv + E);
      } else {
#pragma unroll
        for (int i = 0; i < E; ++i) xv[2 * E + i] = dv[E + i] = 0.0f;
      }
      // g at positions t0 + m, m < E + K - 1 (zero past the row end: dv = 0 there)
      float g[E + K - 1];
#pragma unroll
      for (int m = 0; m < E + K - 1; ++m) {
        float pre = bs;
#pragma unroll
        for (int j = 0; j < K; ++j) pre = fmaf(wk[j], xv[E + m - (K - 1) + j], pre);
        g[m] = dv[m] * act_grad(pre);
      }
      float o[E];
#pragma unroll
      for (int i = 0; i < E; ++i) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < K; ++j) s = fmaf(wk[j], g[i + (K - 1) - j], s);
        o[i] = s;
#pragma unroll
        for (int j = 0; j < K; ++j) acc[j] = fmaf(g[i], xv[E + i - (K - 1) + j], acc[j]);
        acc[K] += g[i];
      }
      store8<T>(dxr + t0, o);
    }
  } else {
    for (int t = threadIdx.x; t < L; t += kConvThreads) {
      float g[K];  // g at t + m, m < K
#pragma unroll
      for (int m = 0; m < K; ++m) {
        const int tm = t + m;
        float gm = 0.0f;
        if (tm < L) {
          float pre = bs;
#pragma unroll
          for (int j = 0; j < K; ++j) {
            const int tt = tm - (K - 1) + j;
            if (tt >= 0) pre = fmaf(wk[j], Elem<T>::load1(xr + tt), pre);
          }
          gm = Elem<T>::load1(gr + tm) * act_grad(pre);
        }
        g[m] = gm;
      }
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < K; ++j) s = fmaf(wk[j], g[K - 1 - j], s);
      Elem<T>::store1(dxr + t, s);
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int tt = t - (K - 1) + j;
        if (tt >= 0) acc[j] = fmaf(g[0], Elem<T>::load1(xr + tt), acc[j]);
      }
      acc[K] += g[0];
    }
  }
  block_sum<K>(acc, red);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int j = 0; j <= K; ++j) part[row * (K + 1) + j] = acc[j];
  }
}

// dw[c,j] = sum_b part[(b*dim + c)*(K+1) + j]; dbias[c] likewise at j = K.
template <typename T>
__global__ __launch_bounds__(256) void causal_conv1d_wgrad_kernel(const float* __restrict__ part,
                                                                  T* __restrict__ dw,
                                                                  T* __restrict__ dbias, int batch,
                                                                  int dim, int K) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;  // c*(K+1) + j
  if (i >= dim * (K + 1)) return;
  const int c = i / (K + 1);
  const int j = i - c * (K + 1);
  float s = 0.0f;
  for (int b = 0; b < batch; ++b) s += part[((size_t)b * dim + c) * (K + 1) + j];
  if (j < K) {
    Elem<T>::store1(dw + (size_t)c * K + j, s);
  } else if (dbias) {
    Elem<T>::store1(dbias + c, s);
  }
}

template <typename T, int K>
hipError_t launch_fwd_k(int batch, int dim, int L, const void* x, int64_t xbs, const void* w,
                        const void* bias, int silu, void* out, const int64_t* lengths, void* window,
                        bool vec, hipStream_t st) {
  ProfScope prof("causal_conv1d_fwd", st);
  const dim3 grid((unsigned)((size_t)batch * dim));
  auto* xp = static_cast<const T*>(x);
  auto* wp = static_cast<const T*>(w);
  auto* bp = static_cast<const T*>(bias);
  auto* op = static_cast<T*>(out);
  auto* wo = static_cast<T*>(window);
  if (vec)
    hipLaunchKernelGGL((causal_conv1d_fwd_kernel<T, K, true>), grid, dim3(kConvThreads), 0, st, xp,
                       xbs, wp, bp, op, dim, L, silu, lengths, wo);
  else
    hipLaunchKernelGGL((causal_conv1d_fwd_kernel<T, K, false>), grid, dim3(kConvThreads), 0, st, xp,
                       xbs, wp, bp, op, dim, L, silu, lengths, wo);
  return hipGetLastError();
}

template <typename T, int K>
hipError_t launch_bwd_k(int batch, int dim, int L, const void* x, const void* w, const void* bias,
                        const void* dout, int silu, void* dx, void* dw, void* dbias, float* part,
                        bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((size_t)batch * dim));
  auto* xp = static_cast<const T*>(x);
  auto* wp = static_cast<const T*>(w);
  auto* bp = static_cast<const T*>(bias);
  auto* gp = static_cast<const T*>(dout);
  auto* dxp = static_cast<T*>(dx);
  {
    ProfScope prof("causal_conv1d_bwd", st);
    if (vec)
      hipLaunchKernelGGL((causal_conv1d_bwd_kernel<T, K, true>), grid, dim3(kConvThreads), 0, st,
                         xp, wp, bp, gp, dxp, part, dim, L, silu);
    else
      hipLaunchKernelGGL((causal_conv1d_bwd_kernel<T, K, false>), grid, dim3(kConvThreads), 0, st,
                         xp, wp, bp, gp, dxp, part, dim, L, silu);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  ProfScope prof("causal_conv1d_wgrad", st);
  const int n = dim * (K + 1);
  hipLaunchKernelGGL((causal_conv1d_wgrad_kernel<T>), dim3((n + 255) / 256), dim3(256), 0, st,
                     part, static_cast<T*>(dw), static_cast<T*>(dbias), batch, dim, K);
  return hipGetLastError();
}

template <typename T>
hipError_t dispatch_fwd(int batch, int dim, int L, int K, const void* x, int64_t xbs, const void* w,
                        const void* bias, int silu, void* out, const int64_t* lengths,
                        void* window, bool vec, hipStream_t st) {
  switch (K) {
    case 1: return launch_fwd_k<T, 1>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    case 2: return launch_fwd_k<T, 2>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    case 3: return launch_fwd_k<T, 3>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    case 4: return launch_fwd_k<T, 4>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    case 5: return launch_fwd_k<T, 5>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    case 6: return launch_fwd_k<T, 6>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    case 7: return launch_fwd_k<T, 7>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    case 8: return launch_fwd_k<T, 8>(batch, dim, L, x, xbs, w, bias, silu, out, lengths, window, vec, st);
    default: return hipErrorInvalidValue;
  }
}

template <typename T>
hipError_t dispatch_bwd(int batch, int dim, int L, int K, const void* x, const void* w,
                        const void* bias, const void* dout, int silu, void* dx, void* dw,
                        void* dbias, float* part, bool vec, hipStream_t st) {
  switch (K) {
#define SSM_CONV_BWD_CASE(k)                                                                 \
  case k:                                                                                    \
    return launch_bwd_k<T, k>(batch, dim, L, x, w, bias, dout, silu, dx, dw, dbias, part, vec, \
                              st);
    SSM_CONV_BWD_CASE(1)
    SSM_CONV_BWD_CASE(2)
    SSM_CONV_BWD_CASE(3)
    SSM_CONV_BWD_CASE(4)
    SSM_CONV_BWD_CASE(5)
    SSM_CONV_BWD_CASE(6)
    SSM_CONV_BWD_CASE(7)
    SSM_CONV_BWD_CASE(8)
#undef SSM_CONV_BWD_CASE
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int conv1d_max_width() { return kMaxWidth; }

hipError_t launch_causal_conv1d_fwd(int batch, int dim, int L, int K, int dtype_bf16,
                                    const void* x, int64_t xbs, const void* w, const void* bias,
                                    int silu, void* out, const int64_t* lengths, void* window,
                                    bool vec, hipStream_t st) {
  return dtype_bf16 ? dispatch_fwd<__hip_bfloat16>(batch, dim, L, K, x, xbs, w, bias, silu, out,
                                                   lengths, window, vec, st)
                    : dispatch_fwd<float>(batch, dim, L, K, x, xbs, w, bias, silu, out, lengths,
                                          window, vec, st);
}

hipError_t launch_causal_conv1d_bwd(int batch, int dim, int L, int K, int dtype_bf16,
                                    const void* x, const void* w, const void* bias,
                                    const void* dout, int silu, void* dx, void* dw, void* dbias,
                                    float* part, bool vec, hipStream_t st) {
  return dtype_bf16 ? dispatch_bwd<__hip_bfloat16>(batch, dim, L, K, x, w, bias, dout, silu, dx, dw,
                                                   dbias, part, vec, st)
                    : dispatch_bwd<float>(batch, dim, L, K, x, w, bias, dout, silu, dx, dw, dbias,
                                          part, vec, st);
}

}  // namespace ssm
