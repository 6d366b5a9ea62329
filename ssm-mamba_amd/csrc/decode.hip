// Fused decode step of the Mamba block for gfx950: the per-token work of
// Block.step / Mamba.step (modules/block.py:80-86, modules/mamba.py:189-243 of
// the reference) as four kernels per layer instead of a score of torch ops:
//
//   gemv_kernel (norm, conv epilogue)  xz = W_in @ rmsnorm(x); for the x half
//                                      xc = silu(window . w + xs w_last + b),
//                                      window roll
//   gemv_kernel                        p = W_x @ xc                    (B, R+2N)
//   ssm_step_kernel                    delta = W_dt @ p[:R];
//                                      state update with B = p[R:R+N],
//                                      C = p[R+N:]; y = (C.h + D*xc) * silu(z)
//   gemv_kernel (residual)             x' = x + W_out @ y
//
// and the LM head as gemv_kernel with the final norm.  Batch is small (one
// token per sequence), so every kernel is a weight stream: a wave owns a few
// weight rows, each lane issues all of its 16-byte row loads before any
// arithmetic, the workgroup stages the (tiny) activation rows in LDS meanwhile,
// and every weight chunk is applied to all batch rows.  Activations, weights and norm/conv/dt
// parameters share the element type T; accumulation is fp32; the SSM state
// stays fp32.
#include "ss_common.cuh"
#include "ss_io.cuh"
#include "ss_prof.h"

namespace ssm {

namespace {

constexpr int kDecThreads = 256;
constexpr int kGemvPass = 4;     // 16-byte chunks per lane per row per pass
constexpr int kMaxDecBatch = 8;  // batch rows per launch

template <typename T>
struct Chunk;  // 16 bytes of T

template <>
struct Chunk<float> {
  static constexpr int E = 4;
  using Raw = float4;
  __device__ static __forceinline__ void cvt(const Raw& r, float* v) {
    v[0] = r.x; v[1] = r.y; v[2] = r.z; v[3] = r.w;
  }
  __device__ static __forceinline__ Raw zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
};

template <>
struct Chunk<__hip_bfloat16> {
  static constexpr int E = 8;
  using Raw = uint4;
  __device__ static __forceinline__ void cvt(const Raw& r, float* v) {
    v[0] = bf16_lo(r.x); v[1] = bf16_hi(r.x); v[2] = bf16_lo(r.y); v[3] = bf16_hi(r.y);
    v[4] = bf16_lo(r.z); v[5] = bf16_hi(r.z); v[6] = bf16_lo(r.w); v[7] = bf16_hi(r.w);
  }
  __device__ static __forceinline__ Raw zero() { return make_uint4(0u, 0u, 0u, 0u); }
};

template <typename T>
__device__ __forceinline__ typename Chunk<T>::Raw ldchunk(const T* __restrict__ p) {
  return *reinterpret_cast<const typename Chunk<T>::Raw*>(p);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Totals over the wave of NV per-lane values: afterwards out[g] of lane l is
// the sum over all lanes of v[g * 16 + (l >> 2)] (zero past NV); the four
// lanes of a quad agree.  permlane/DPP reduce-scatter, no LDS round trips.
template <int NV>
__device__ __forceinline__ void wave_totals(const float (&v)[NV], float (&out)[(NV + 15) / 16],
                                            int lane) {
#pragma unroll
  for (int g = 0; g < (NV + 15) / 16; ++g) {
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = g * 16 + i < NV ? v[g * 16 + i] : 0.0f;
    wave_reduce16(t, lane);
    out[g] = t[0];
  }
}

// value rounded to T and back (the reference keeps these intermediates as T tensors)
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  T t;
  Elem<T>::store1(&t, v);
  return Elem<T>::load1(&t);
}

enum GemvEpi { kEpiPlain = 0, kEpiConv = 1 };

struct GemvArgs {
  const void* W;     // (O, K)
  const void* x;     // (B, K)
  const void* nw;    // (K) RMSNorm weight (kNorm)
  float eps;
  const void* bias;  // (O) nullable
  const void* res;   // (B, O) nullable (plain epilogue)
  void* y;           // (B, O)
  int B, O, K;
  // conv epilogue: rows o < dim are xs; window (B, dim, width-1), weight (dim, width)
  int dim, width;
  void* ctx;
  const void* cw;
  const void* cb;    // nullable
  void* xc;          // (B, dim)
};

// y[b, o] = scale_b * sum_k W[o, k] * (1 + nw[k])^[kNorm] * x[b, k] (+ bias[o]) (+ res[b, o]),
// scale_b = rsqrt(mean_k x[b, k]^2 + eps) with kNorm, else 1 -- i.e. W @ rmsnorm(x).
//
// Per pass of PK = 64 * E * kGemvPass columns: each lane issues all of its
// weight loads (kRows rows x kGemvPass 16-byte chunks), then the workgroup
// stages x[:, pass] in LDS (and accumulates x^2 for the norm), then the
// weights meet the staged activations.  kEpiConv adds the Mamba conv step for
// the x half of the in-projection (rows o < dim): xc = silu(window . w + xs w
// + cb), and the window rolls by one.
template <typename T, int kMB, int kRows, bool kNorm, int kEpi>
__global__ __launch_bounds__(kDecThreads) void gemv_kernel(const GemvArgs a) {
  constexpr int E = Chunk<T>::E;
  constexpr int span = 64 * E;            // columns of one chunk step of a wave
  constexpr int PK = span * kGemvPass;    // columns per pass
  using Raw = typename Chunk<T>::Raw;
  __shared__ __align__(16) T sx[kMB][PK];
  __shared__ float s_red[4][kMB];
  __shared__ float s_scale[kMB];
  const T* __restrict__ W = static_cast<const T*>(a.W);
  const T* __restrict__ x = static_cast<const T*>(a.x);
  const T* __restrict__ nw = static_cast<const T*>(a.nw);
  const int B = a.B, O = a.O, K = a.K;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * (kDecThreads / 64) + wave) * kRows;
  float acc[kRows][kMB];
  float ssq[kMB];
#pragma unroll
  for (int b = 0; b < kMB; ++b) {
    ssq[b] = 0.0f;
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r][b] = 0.0f;
  }

  // epilogue operands (bias, residual, conv taps and window) of this lane's
  // outputs, fetched before the weight stream so their latency overlaps it
  constexpr int kNV = kRows * kMB;
  constexpr int kNG = (kNV + 15) / 16;
  constexpr int kMaxTaps = 8;
  int e_row[kNG], e_b[kNG];
  bool e_ok[kNG];
  float e_bias[kNG], e_res[kNG], e_cb[kNG];
  float e_cw[kNG][kMaxTaps], e_win[kNG][kMaxTaps - 1];
#pragma unroll
  for (int g = 0; g < kNG; ++g) {
    const int i = g * 16 + (lane >> 2);
    const int rl = i / kMB;
    e_row[g] = row0 + rl;
    e_b[g] = i - rl * kMB;
    e_ok[g] = (lane & 3) == 0 && i < kNV && e_row[g] < O && e_b[g] < B;
    const bool ok = e_ok[g];
    e_bias[g] = ok && a.bias ? Elem<T>::load1(static_cast<const T*>(a.bias) + e_row[g]) : 0.0f;
    e_res[g] = 0.0f;
    e_cb[g] = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTaps; ++j) e_cw[g][j] = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTaps - 1; ++j) e_win[g][j] = 0.0f;
    if constexpr (kEpi == kEpiPlain) {
      if (ok && a.res)
        e_res[g] = Elem<T>::load1(static_cast<const T*>(a.res) + (size_t)e_b[g] * O + e_row[g]);
    } else {
      if (ok && e_row[g] < a.dim) {
        const int wd = a.width;
        const T* __restrict__ cw = static_cast<const T*>(a.cw) + (size_t)e_row[g] * wd;
        const T* __restrict__ win =
            static_cast<const T*>(a.ctx) + ((size_t)e_b[g] * a.dim + e_row[g]) * (wd - 1);
#pragma unroll
        for (int j = 0; j < kMaxTaps; ++j) e_cw[g][j] = Elem<T>::load1(cw + min(j, wd - 1));
#pragma unroll
        for (int j = 0; j < kMaxTaps - 1; ++j) e_win[g][j] = Elem<T>::load1(win + min(j, wd - 2));
        e_cb[g] = a.cb ? Elem<T>::load1(static_cast<const T*>(a.cb) + e_row[g]) : 0.0f;
      }
    }
  }
  for (int kb = 0; kb < K; kb += PK) {
    Raw wr[kRows][kGemvPass];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int row = min(row0 + r, O - 1);
#pragma unroll
      for (int c = 0; c < kGemvPass; ++c) {
        if (kb + c * span < K) {  // wave-uniform: whole chunks past K are not loaded
          const int k0 = min(kb + c * span + lane * E, K - E);
          wr[r][c] = ldchunk(W + (size_t)row * K + k0);
        } else {
          wr[r][c] = Chunk<T>::zero();
        }
      }
    }
    // stage x[:, kb:kb+PK]: thread t owns chunk t of every batch row (PK / E == 256)
    static_assert(PK / E == kDecThreads, "one staged chunk per thread and batch row");
    {
      const int k = kb + threadIdx.x * E;
#pragma unroll
      for (int b = 0; b < kMB; ++b) {
        if (b < B) {
          const Raw v = k < K ? ldchunk(x + (size_t)b * K + k) : Chunk<T>::zero();
          *reinterpret_cast<Raw*>(&sx[b][threadIdx.x * E]) = v;
          if constexpr (kNorm) {
            float f[E];
            Chunk<T>::cvt(v, f);
#pragma unroll
            for (int i = 0; i < E; ++i) ssq[b] = fmaf(f[i], f[i], ssq[b]);
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < kGemvPass; ++c) {
      const int kl = c * span + lane * E;
      if (kb + kl < K) {
        float wf[kRows][E];
#pragma unroll
        for (int r = 0; r < kRows; ++r) Chunk<T>::cvt(wr[r][c], wf[r]);
        if constexpr (kNorm) {
          float nv[E];
          Chunk<T>::cvt(ldchunk(nw + kb + kl), nv);
#pragma unroll
          for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int i = 0; i < E; ++i) wf[r][i] *= 1.0f + nv[i];
        }
#pragma unroll
        for (int b = 0; b < kMB; ++b) {
          if (b < B) {
            float v[E];
            Chunk<T>::cvt(*reinterpret_cast<const Raw*>(&sx[b][kl]), v);
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
              float s = acc[r][b];
#pragma unroll
              for (int i = 0; i < E; ++i) s = fmaf(wf[r][i], v[i], s);
              acc[r][b] = s;
            }
          }
        }
      }
    }
    __syncthreads();
  }

  if constexpr (kNorm) {
    float st[(kMB + 15) / 16];
    wave_totals<kMB>(ssq, st, lane);
    if ((lane & 3) == 0 && (lane >> 2) < kMB) s_red[wave][lane >> 2] = st[0];
    __syncthreads();
    if (threadIdx.x < kMB) {
      const int b = threadIdx.x;
      const float t = s_red[0][b] + s_red[1][b] + s_red[2][b] + s_red[3][b];
      s_scale[b] = rsqrtf(t / (float)K + a.eps);
    }
    __syncthreads();
  }
  // wave totals: lane 4i (+0..3) of group g finishes output i = g * 16 + (lane >> 2),
  // i = r * kMB + b; its operands were fetched before the weight stream (below)
  float tot[kNG];
  {
    float flat[kNV];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
#pragma unroll
      for (int b = 0; b < kMB; ++b) flat[r * kMB + b] = acc[r][b];
    wave_totals<kNV>(flat, tot, lane);
  }
  T* __restrict__ y = static_cast<T*>(a.y);
#pragma unroll
  for (int g = 0; g < kNG; ++g) {
    if (!e_ok[g]) continue;
    const int row = e_row[g], bl = e_b[g];
    float s = tot[g];
    if constexpr (kNorm) s *= s_scale[bl];
    s += e_bias[g];
    if constexpr (kEpi == kEpiPlain) {
      Elem<T>::store1(y + (size_t)bl * O + row, s + e_res[g]);
    } else {
      Elem<T>::store1(y + (size_t)bl * O + row, s);
      if (row < a.dim) {
        const int wd = a.width;
        const float xs = round_to<T>(s);
        float cv = e_cb[g];
        float wlast = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxTaps; ++j) {
          if (j < wd - 1) cv = fmaf(e_cw[g][j], e_win[g][j], cv);
          if (j == wd - 1) wlast = e_cw[g][j];
        }
        cv = fmaf(wlast, xs, cv);
        const float xcv = round_to<T>(silu_f(cv));
        Elem<T>::store1(static_cast<T*>(a.xc) + (size_t)bl * a.dim + row, xcv);
        T* __restrict__ win = static_cast<T*>(a.ctx) + ((size_t)bl * a.dim + row) * (wd - 1);
#pragma unroll
        for (int j = 0; j + 1 < kMaxTaps - 1; ++j)
          if (j + 1 < wd - 1) Elem<T>::store1(win + j, e_win[g][j + 1]);
        Elem<T>::store1(win + wd - 2, xs);
      }
    }
  }
}

// Step-size projection, state update and gate, one thread per (b, d):
//   delta = round_T(W_dt[d, :R] . p[b, :R]); delta' = softplus(delta + dt_bias[d])
//   h' = exp(delta' A) h + delta' xc B,  A = -exp(log_A), B = p[b, R:R+N]
//   y = (sum_n C h' + D xc) * silu(z),   C = p[b, R+N:R+2N], z = xz[b, dim + d]
// (modules/mamba.py:216-240 with selective_update/kernel.cu:39-71; the T
// roundings mirror the reference's intermediate T tensors).
template <typename T, int kN, bool kVecR>
__global__ __launch_bounds__(kDecThreads) void ssm_step_kernel(
    const T* __restrict__ p, int nout, int R, const T* __restrict__ Wdt,
    const T* __restrict__ dt_bias, const T* __restrict__ logA, const T* __restrict__ Dv,
    const T* __restrict__ xc, const T* __restrict__ xz, int ld_xz, float* __restrict__ state,
    T* __restrict__ y, int dim) {
  constexpr int E = Chunk<T>::E;
  constexpr int kMaxRC = 16;  // dt-projection chunks held in registers (R <= 16 E)
  extern __shared__ float s_p[];  // [nout]
  const int b = blockIdx.y;
  const int d = blockIdx.x * kDecThreads + threadIdx.x;
  const int dc = min(d, dim - 1);
  // this thread's operands first (none depends on p), so their latency
  // overlaps the staging of p and the barrier
  typename Chunk<T>::Raw wv[kVecR ? kMaxRC : 1];
  const T* __restrict__ wrow = Wdt + (size_t)dc * R;
  if constexpr (kVecR) {
#pragma unroll
    for (int c = 0; c < kMaxRC; ++c) wv[c] = c * E < R ? ldchunk(wrow + c * E) : Chunk<T>::zero();
  }
  float* __restrict__ h = state + ((size_t)b * dim + dc) * kN;
  float4 hv[kN / 4];
#pragma unroll
  for (int q = 0; q < kN / 4; ++q) hv[q] = *reinterpret_cast<const float4*>(h + 4 * q);
  float la[kN];
#pragma unroll
  for (int n = 0; n < kN; ++n) la[n] = Elem<T>::load1(logA + (size_t)dc * kN + n);
  const float bias = dt_bias ? Elem<T>::load1(dt_bias + dc) : 0.0f;
  const float dv = Dv ? Elem<T>::load1(Dv + dc) : 0.0f;
  const float u = Elem<T>::load1(xc + (size_t)b * dim + dc);
  const float z = Elem<T>::load1(xz + (size_t)b * ld_xz + dim + dc);

  for (int i = threadIdx.x; i < nout; i += kDecThreads) s_p[i] = Elem<T>::load1(p + (size_t)b * nout + i);
  __syncthreads();
  if (d >= dim) return;

  float dl = 0.0f;
  if constexpr (kVecR) {
#pragma unroll
    for (int c = 0; c < kMaxRC; ++c) {
      if (c * E < R) {
        float w[E];
        Chunk<T>::cvt(wv[c], w);
#pragma unroll
        for (int i = 0; i < E; ++i) dl = fmaf(w[i], s_p[c * E + i], dl);
      }
    }
  } else {
    for (int r = 0; r < R; ++r) dl = fmaf(Elem<T>::load1(wrow + r), s_p[r], dl);
  }
  dl = round_to<T>(dl);
  const float dt = softplus_t20(dl + bias);
  const float du = dt * u;
  float out = 0.0f;
#pragma unroll
  for (int q = 0; q < kN / 4; ++q) {
    float hn[4] = {hv[q].x, hv[q].y, hv[q].z, hv[q].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = 4 * q + i;
      const float a = fast_exp2(-dt * fast_exp2(la[n] * kLog2e) * kLog2e);  // exp(dt * A), A = -exp(log_A)
      hn[i] = fmaf(a, hn[i], du * s_p[R + n]);
      out = fmaf(s_p[R + kN + n], hn[i], out);
    }
    *reinterpret_cast<float4*>(h + 4 * q) = make_float4(hn[0], hn[1], hn[2], hn[3]);
  }
  out = fmaf(dv, u, out);
  Elem<T>::store1(y + (size_t)b * dim + d, out * silu_f(z));
}

template <typename T, int kMB, int kRows>
hipError_t launch_gemv_r(const GemvArgs& a, bool norm, bool conv, hipStream_t st) {
  const int rows_per_block = (kDecThreads / 64) * kRows;
  const dim3 grid((a.O + rows_per_block - 1) / rows_per_block);
  if (conv) {
    if (norm)
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, true, kEpiConv>), grid, dim3(kDecThreads), 0, st, a);
    else
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, false, kEpiConv>), grid, dim3(kDecThreads), 0, st, a);
  } else {
    if (norm)
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, true, kEpiPlain>), grid, dim3(kDecThreads), 0, st, a);
    else
      hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, false, kEpiPlain>), grid, dim3(kDecThreads), 0, st, a);
  }
  return hipGetLastError();
}

template <typename T, int kMB>
hipError_t launch_gemv_b(const GemvArgs& a, bool norm, bool conv, hipStream_t st) {
  // rows per wave: four for tall matrices (the LM head), one for short ones
  // (more workgroups in flight), two otherwise
  if (a.O >= 16384) return launch_gemv_r<T, kMB, 4>(a, norm, conv, st);
  if (a.O <= 2048 && !conv) return launch_gemv_r<T, kMB, 1>(a, norm, conv, st);
  return launch_gemv_r<T, kMB, 2>(a, norm, conv, st);
}

template <typename T>
hipError_t launch_gemv_t(const GemvArgs& a, bool norm, bool conv, hipStream_t st) {
  if (a.B <= 1) return launch_gemv_b<T, 1>(a, norm, conv, st);
  if (a.B <= 2) return launch_gemv_b<T, 2>(a, norm, conv, st);
  if (a.B <= 4) return launch_gemv_b<T, 4>(a, norm, conv, st);
  return launch_gemv_b<T, 8>(a, norm, conv, st);
}

template <typename T, int kN>
hipError_t launch_ssm_step_n(const void* p, int nout, int R, const void* Wdt, const void* dtb,
                             const void* logA, const void* D, const void* xc, const void* xz,
                             int ld, float* state, void* y, int B, int dim, bool vecR,
                             hipStream_t st) {
  const dim3 grid((dim + kDecThreads - 1) / kDecThreads, B);
  const size_t lds = (size_t)nout * sizeof(float);
  auto* pp = static_cast<const T*>(p);
  auto* wdt = static_cast<const T*>(Wdt);
  auto* bb = static_cast<const T*>(dtb);
  auto* la = static_cast<const T*>(logA);
  auto* dv = static_cast<const T*>(D);
  auto* u = static_cast<const T*>(xc);
  auto* zz = static_cast<const T*>(xz);
  auto* o = static_cast<T*>(y);
  if (vecR)
    hipLaunchKernelGGL((ssm_step_kernel<T, kN, true>), grid, dim3(kDecThreads), lds, st, pp, nout,
                       R, wdt, bb, la, dv, u, zz, ld, state, o, dim);
  else
    hipLaunchKernelGGL((ssm_step_kernel<T, kN, false>), grid, dim3(kDecThreads), lds, st, pp, nout,
                       R, wdt, bb, la, dv, u, zz, ld, state, o, dim);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_ssm_step_t(const void* p, int nout, int R, const void* Wdt, const void* dtb,
                             const void* logA, const void* D, const void* xc, const void* xz,
                             int ld, float* state, void* y, int B, int dim, int nstate, bool vecR,
                             hipStream_t st) {
  switch (nstate) {
#define SSM_DEC_N(n)                                                                               \
  case n:                                                                                          \
    return launch_ssm_step_n<T, n>(p, nout, R, Wdt, dtb, logA, D, xc, xz, ld, state, y, B, dim,    \
                                   vecR, st);
    SSM_DEC_N(4)
    SSM_DEC_N(8)
    SSM_DEC_N(16)
    SSM_DEC_N(32)
    SSM_DEC_N(64)
#undef SSM_DEC_N
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int decode_max_batch() { return kMaxDecBatch; }

hipError_t launch_decode_gemv(int bf16, const void* W, const void* x, const void* nw, float eps,
                              const void* bias, const void* res, void* y, int B, int O, int K,
                              hipStream_t st) {
  ProfScope prof("decode_gemv", st);
  GemvArgs a{};
  a.W = W; a.x = x; a.nw = nw; a.eps = eps; a.bias = bias; a.res = res; a.y = y;
  a.B = B; a.O = O; a.K = K;
  return bf16 ? launch_gemv_t<__hip_bfloat16>(a, nw != nullptr, false, st)
              : launch_gemv_t<float>(a, nw != nullptr, false, st);
}

hipError_t launch_decode_in_proj_conv(int bf16, const void* W, const void* x, const void* nw,
                                      float eps, const void* bias, void* xz, int B, int dim, int K,
                                      int width, void* ctx, const void* cw, const void* cb,
                                      void* xc, hipStream_t st) {
  ProfScope prof("decode_in_proj_conv", st);
  GemvArgs a{};
  a.W = W; a.x = x; a.nw = nw; a.eps = eps; a.bias = bias; a.res = nullptr; a.y = xz;
  a.B = B; a.O = 2 * dim; a.K = K;
  a.dim = dim; a.width = width; a.ctx = ctx; a.cw = cw; a.cb = cb; a.xc = xc;
  return bf16 ? launch_gemv_t<__hip_bfloat16>(a, nw != nullptr, true, st)
              : launch_gemv_t<float>(a, nw != nullptr, true, st);
}

hipError_t launch_decode_ssm_step(int bf16, const void* p, int nout, int R, const void* Wdt,
                                  const void* dtb, const void* logA, const void* D, const void* xc,
                                  const void* xz, int ld, float* state, void* y, int B, int dim,
                                  int nstate, bool vecR, hipStream_t st) {
  ProfScope prof("decode_ssm_step", st);
  return bf16 ? launch_ssm_step_t<__hip_bfloat16>(p, nout, R, Wdt, dtb, logA, D, xc, xz, ld, state,
                                                  y, B, dim, nstate, vecR, st)
              : launch_ssm_step_t<float>(p, nout, R, Wdt, dtb, logA, D, xc, xz, ld, state, y, B,
                                         dim, nstate, vecR, st);
}

}  // namespace ssm
