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
// or in three, with p = W_x @ xc folded into the other two: each in-projection
// workgroup of the x half writes the fp32 partial W_x[:, its channels] @ xc,
// and every ssm_step workgroup adds the partials of its batch row in a fixed
// order (kEpiConvX / kParts below).
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

enum GemvEpi { kEpiPlain = 0, kEpiConv = 1, kEpiConvX = 2 };

// x-projection partials: the in-projection with them runs kXRows weight rows
// per wave, so each workgroup covers kXBlock channels of the x half
constexpr int kXRows = 4;
constexpr int kXBlock = (kDecThreads / 64) * kXRows;
constexpr int kMaxXOut = 256;    // R + 2N limit of the folded x-projection
constexpr int kPartLoads = 16;   // partial float4 loads in flight per thread

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
  // kEpiConvX: part (dim / kXBlock, B, nout4) fp32 = W_x (nout, dim) partials
  const void* Wx;
  int nout, nout4;
  float* part;
};

// y[b, o] = scale_b * sum_k W[o, k] * (1 + nw[k])^[kNorm] * x[b, k] (+ bias[o]) (+ res[b, o]),
// scale_b = rsqrt(mean_k x[b, k]^2 + eps) with kNorm, else 1 -- i.e. W @ rmsnorm(x).
//
// Per pass of PK = 64 * E * kGemvPass columns: each lane issues all of its
// weight loads (kRows rows x kGemvPass 16-byte chunks), then the workgroup
// stages x[:, pass] in LDS (and accumulates x^2 for the norm), then the
// weights meet the staged activations.  kEpiConv adds the Mamba conv step for
// the x half of the in-projection (rows o < dim): xc = silu(window . w + xs w
// + cb), and the window rolls by one.  kEpiConvX also writes this workgroup's
// x-projection partial part[blk, b, j] = sum_{c in blk} W_x[j, c] xc[b, c].
template <typename T, int kMB, int kRows, bool kNorm, int kEpi>
__global__ __launch_bounds__(kDecThreads) void gemv_kernel(const GemvArgs a) {
  constexpr int E = Chunk<T>::E;
  constexpr bool kXP = kEpi == kEpiConvX;
  static_assert(!kXP || kRows == kXRows, "x-projection partials need kXRows rows per wave");
  constexpr int kXC = kXP ? kXBlock / E : 1;  // 16-byte chunks of one W_x row slice
  constexpr int span = 64 * E;            // columns of one chunk step of a wave
  constexpr int PK = span * kGemvPass;    // columns per pass
  using Raw = typename Chunk<T>::Raw;
  __shared__ __align__(16) T sx[kMB][PK];
  __shared__ float s_red[4][kMB];
  __shared__ float s_scale[kMB];
  __shared__ float s_xc[kXP ? kMB : 1][kXP ? kXBlock : 1];
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
  // outputs, fetched before the weight stream so their latency overlaps it.
  // Every lane loads, from clamped addresses (absent operands from a valid
  // stand-in), so no load sits in a branch: a load inside a branch is waited
  // for inside it, which would serialise these round trips.
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
    const int rc = min(e_row[g], O - 1), bc = min(e_b[g], B - 1);
    e_bias[g] = Elem<T>::load1((a.bias ? static_cast<const T*>(a.bias) : W) + rc);
    e_res[g] = 0.0f;
    e_cb[g] = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTaps; ++j) e_cw[g][j] = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTaps - 1; ++j) e_win[g][j] = 0.0f;
    if constexpr (kEpi == kEpiPlain) {
      e_res[g] = Elem<T>::load1(a.res ? static_cast<const T*>(a.res) + (size_t)bc * O + rc : W + rc);
    } else {
      const int wd = a.width;
      const int rx = min(rc, a.dim - 1);  // x-half row (rows past dim use none of these)
      const T* __restrict__ cw = static_cast<const T*>(a.cw) + (size_t)rx * wd;
      const T* __restrict__ win =
          static_cast<const T*>(a.ctx) + ((size_t)bc * a.dim + rx) * (wd - 1);
#pragma unroll
      for (int j = 0; j < kMaxTaps; ++j) e_cw[g][j] = Elem<T>::load1(cw + min(j, wd - 1));
#pragma unroll
      for (int j = 0; j < kMaxTaps - 1; ++j) e_win[g][j] = Elem<T>::load1(win + min(j, wd - 2));
      e_cb[g] = Elem<T>::load1(a.cb ? static_cast<const T*>(a.cb) + rx : cw);
    }
  }
  // the W_x slice of output j = threadIdx.x, ahead of the weight stream; xc
  // slots of rows this workgroup does not finish stay zero
  const int xblk0 = blockIdx.x * kXBlock;
  const bool xblk = kXP && xblk0 < a.dim;
  Raw xw[kXC];
#pragma unroll
  for (int c = 0; c < kXC; ++c) xw[c] = Chunk<T>::zero();
  if constexpr (kXP) {
    if (threadIdx.x < kMB * kXBlock) s_xc[threadIdx.x / kXBlock][threadIdx.x % kXBlock] = 0.0f;
    // clamped row and block (dim >= kXBlock); rows past nout are zeroed at use
    const int jr = min((int)threadIdx.x, a.nout - 1);
    const T* __restrict__ wx =
        static_cast<const T*>(a.Wx) + (size_t)jr * a.dim + min(xblk0, a.dim - kXBlock);
#pragma unroll
    for (int c = 0; c < kXC; ++c) xw[c] = ldchunk(wx + c * E);
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
    // the norm weight of this lane's columns, with the weight stream (clamped
    // past K, where the chunk is not used)
    Raw nwr[kNorm ? kGemvPass : 1];
    if constexpr (kNorm) {
#pragma unroll
      for (int c = 0; c < kGemvPass; ++c) nwr[c] = ldchunk(nw + min(kb + c * span + lane * E, K - E));
    }
    // stage x[:, kb:kb+PK]: thread t owns chunk t of every batch row (PK / E == 256).
    // Loads from clamped addresses, zeroed past K by a select (no load in a
    // branch); slots of rows b >= B hold row B-1 and are never read.
    static_assert(PK / E == kDecThreads, "one staged chunk per thread and batch row");
    {
      const int k = kb + threadIdx.x * E;
      const int kc = min(k, K - E);
      Raw xr[kMB];
#pragma unroll
      for (int b = 0; b < kMB; ++b) xr[b] = ldchunk(x + (size_t)min(b, B - 1) * K + kc);
#pragma unroll
      for (int b = 0; b < kMB; ++b) {
        Raw v = xr[b];
        if (k >= K) v = Chunk<T>::zero();
        *reinterpret_cast<Raw*>(&sx[b][threadIdx.x * E]) = v;
        if constexpr (kNorm) {
          if (b < B) {
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
          Chunk<T>::cvt(nwr[c], nv);
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
  // the W_x slice as floats now, while its (oldest) loads are known complete:
  // converted after the epilogue's stores, it would wait for those too
  float xwf[kXP ? kXBlock : 1];
  if constexpr (kXP) {
#pragma unroll
    for (int c = 0; c < kXC; ++c) Chunk<T>::cvt(xw[c], xwf + c * E);
    if ((int)threadIdx.x >= a.nout) {  // padding columns of the partial
#pragma unroll
      for (int c = 0; c < kXBlock; ++c) xwf[c] = 0.0f;
    }
    // keep the conversion here (the compiler would sink it to its use)
#pragma unroll
    for (int c = 0; c < kXBlock; ++c) asm volatile("" : "+v"(xwf[c]));
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
    if (a.bias) s += e_bias[g];
    if constexpr (kEpi == kEpiPlain) {
      Elem<T>::store1(y + (size_t)bl * O + row, a.res ? s + e_res[g] : s);
    } else {
      Elem<T>::store1(y + (size_t)bl * O + row, s);
      if (row < a.dim) {
        const int wd = a.width;
        const float xs = round_to<T>(s);
        float cv = a.cb ? e_cb[g] : 0.0f;
        float wlast = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxTaps; ++j) {
          if (j < wd - 1) cv = fmaf(e_cw[g][j], e_win[g][j], cv);
          if (j == wd - 1) wlast = e_cw[g][j];
        }
        cv = fmaf(wlast, xs, cv);
        const float xcv = round_to<T>(silu_f(cv));
        Elem<T>::store1(static_cast<T*>(a.xc) + (size_t)bl * a.dim + row, xcv);
        if constexpr (kXP) s_xc[bl][row - xblk0] = xcv;
        T* __restrict__ win = static_cast<T*>(a.ctx) + ((size_t)bl * a.dim + row) * (wd - 1);
#pragma unroll
        for (int j = 0; j + 1 < kMaxTaps - 1; ++j)
          if (j + 1 < wd - 1) Elem<T>::store1(win + j, e_win[g][j + 1]);
        Elem<T>::store1(win + wd - 2, xs);
      }
    }
  }
  if constexpr (kXP) {
    __syncthreads();
    if (xblk && (int)threadIdx.x < a.nout4) {
      float* __restrict__ part = a.part + (size_t)blockIdx.x * a.B * a.nout4 + threadIdx.x;
#pragma unroll
      for (int b = 0; b < kMB; ++b) {
        if (b < a.B) {
          float s = 0.0f;
#pragma unroll
          for (int c = 0; c < kXBlock; ++c) s = fmaf(xwf[c], s_xc[b][c], s);
          part[(size_t)b * a.nout4] = s;
        }
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
//
// kParts: p is not given; pp holds the in-projection's fp32 x-projection
// partials (nparts, batch, nout4) and p[b] = round_T(sum over the partials),
// added in a fixed order: thread group s of S = 256 / (nout4 / 4) sums
// partials [s nparts / S, (s+1) nparts / S) in turn, then the S group sums in
// turn.
template <typename T, int kN, bool kVecR, bool kParts>
__global__ __launch_bounds__(kDecThreads) void ssm_step_kernel(
    const void* __restrict__ pp, int nout, int nout4, int nparts, int R,
    const T* __restrict__ Wdt, const T* __restrict__ dt_bias, const T* __restrict__ logA,
    const T* __restrict__ Dv, const T* __restrict__ xc, const T* __restrict__ xz, int ld_xz,
    float* __restrict__ state, T* __restrict__ y, int dim) {
  constexpr int E = Chunk<T>::E;
  constexpr int kMaxRC = 16;  // dt-projection chunks held in registers (R <= 16 E)
  extern __shared__ __align__(16) float s_p[];  // [nout4] (+ [S][nout4 / 4] float4 with kParts)
  const int b = blockIdx.y;
  const int d = blockIdx.x * kDecThreads + threadIdx.x;
  const int dc = min(d, dim - 1);
  // partial loads first: they are the longest chain
  const int ng = nout4 >> 2;
  const int S = kParts ? kDecThreads / ng : 1;
  const int sg = threadIdx.x / ng, gi = threadIdx.x - sg * ng;
  const int w0 = sg * nparts / S, w1 = (sg + 1) * nparts / S;
  const float4* __restrict__ p4 =
      reinterpret_cast<const float4*>(pp) + (size_t)b * ng + gi;
  const size_t wstride = (size_t)gridDim.y * ng;
  float4 pacc = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 pv[kParts ? kPartLoads : 1];
  if constexpr (kParts) {
    // clamped (always valid) partial indexes, unused ones skipped in the sum:
    // no load in a branch, so all of them are in flight at once
#pragma unroll
    for (int j = 0; j < kPartLoads; ++j) pv[j] = p4[min(w0 + j, nparts - 1) * wstride];
  }
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
  // absent dt_bias / D read a valid stand-in (log_A) and are dropped at use:
  // loads in a branch would be waited for there
  const float bias_v = Elem<T>::load1((dt_bias ? dt_bias : logA) + dc);
  const float dv_v = Elem<T>::load1((Dv ? Dv : logA) + dc);
  const float u = Elem<T>::load1(xc + (size_t)b * dim + dc);
  const float z = Elem<T>::load1(xz + (size_t)b * ld_xz + dim + dc);

  if constexpr (kParts) {
    float4* s_red = reinterpret_cast<float4*>(s_p + nout4);  // [S][ng]
    if (sg < S) {
      for (int wb = w0;; wb += kPartLoads) {
#pragma unroll
        for (int j = 0; j < kPartLoads; ++j) {
          if (wb + j < w1) {
            pacc.x += pv[j].x; pacc.y += pv[j].y; pacc.z += pv[j].z; pacc.w += pv[j].w;
          }
        }
        if (wb + kPartLoads >= w1) break;
#pragma unroll
        for (int j = 0; j < kPartLoads; ++j)
          pv[j] = p4[min(wb + kPartLoads + j, nparts - 1) * wstride];
      }
      s_red[sg * ng + gi] = pacc;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nout; i += kDecThreads) {
      const float* r = reinterpret_cast<const float*>(s_red) + i;
      float t = 0.0f;
      for (int g = 0; g < S; ++g) t += r[g * nout4];
      s_p[i] = round_to<T>(t);
    }
  } else {
    const T* __restrict__ p = static_cast<const T*>(pp);
    for (int i = threadIdx.x; i < nout; i += kDecThreads) s_p[i] = Elem<T>::load1(p + (size_t)b * nout + i);
  }
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
  const float dt = softplus_t20(dl + (dt_bias ? bias_v : 0.0f));
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
  out = fmaf(Dv ? dv_v : 0.0f, u, out);
  Elem<T>::store1(y + (size_t)b * dim + d, out * silu_f(z));
}

template <typename T, int kMB, int kRows>
hipError_t launch_gemv_r(const GemvArgs& a, bool norm, bool conv, hipStream_t st) {
  const int rows_per_block = (kDecThreads / 64) * kRows;
  const dim3 grid((a.O + rows_per_block - 1) / rows_per_block);
  if (conv && a.Wx) {
    if constexpr (kRows == kXRows) {
      if (norm)
        hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, true, kEpiConvX>), grid, dim3(kDecThreads), 0, st, a);
      else
        hipLaunchKernelGGL((gemv_kernel<T, kMB, kRows, false, kEpiConvX>), grid, dim3(kDecThreads), 0, st, a);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (conv) {
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
  // rows per wave: four for tall matrices (the LM head) and with the
  // x-projection partials, one for short ones (more workgroups in flight),
  // two otherwise
  if (a.O >= 16384 || (conv && a.Wx)) return launch_gemv_r<T, kMB, 4>(a, norm, conv, st);
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
hipError_t launch_ssm_step_n(const void* p, int nout, int nparts, int R, const void* Wdt,
                             const void* dtb, const void* logA, const void* D, const void* xc,
                             const void* xz, int ld, float* state, void* y, int B, int dim,
                             bool vecR, hipStream_t st) {
  const dim3 grid((dim + kDecThreads - 1) / kDecThreads, B);
  const int nout4 = (nout + 3) & ~3;
  // s_p, plus the partial sums' [S][nout4 / 4] float4 with partials (S * nout4 <= 4 * 256)
  const size_t lds = (size_t)nout4 * sizeof(float) +
                     (nparts ? (size_t)(kDecThreads / (nout4 / 4)) * nout4 * sizeof(float) : 0);
  auto* wdt = static_cast<const T*>(Wdt);
  auto* bb = static_cast<const T*>(dtb);
  auto* la = static_cast<const T*>(logA);
  auto* dv = static_cast<const T*>(D);
  auto* u = static_cast<const T*>(xc);
  auto* zz = static_cast<const T*>(xz);
  auto* o = static_cast<T*>(y);
#define SSM_STEP_LAUNCH(vr, pt)                                                                    \
  hipLaunchKernelGGL((ssm_step_kernel<T, kN, vr, pt>), grid, dim3(kDecThreads), lds, st, p, nout, \
                     nout4, nparts, R, wdt, bb, la, dv, u, zz, ld, state, o, dim)
  if (nparts) {
    if (vecR) SSM_STEP_LAUNCH(true, true);
    else SSM_STEP_LAUNCH(false, true);
  } else {
    if (vecR) SSM_STEP_LAUNCH(true, false);
    else SSM_STEP_LAUNCH(false, false);
  }
#undef SSM_STEP_LAUNCH
  return hipGetLastError();
}

template <typename T>
hipError_t launch_ssm_step_t(const void* p, int nout, int nparts, int R, const void* Wdt,
                             const void* dtb, const void* logA, const void* D, const void* xc,
                             const void* xz, int ld, float* state, void* y, int B, int dim,
                             int nstate, bool vecR, hipStream_t st) {
  switch (nstate) {
#define SSM_DEC_N(n)                                                                               \
  case n:                                                                                          \
    return launch_ssm_step_n<T, n>(p, nout, nparts, R, Wdt, dtb, logA, D, xc, xz, ld, state, y, B, \
                                   dim, vecR, st);
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

int decode_xproj_blocks(int64_t dim, int64_t nout) {
  if (dim < kXBlock || dim % kXBlock || nout < 1 || nout > kMaxXOut) return 0;
  return (int)(dim / kXBlock);
}

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
                                      void* xc, const void* Wx, int nout, float* part,
                                      hipStream_t st) {
  ProfScope prof("decode_in_proj_conv", st);
  GemvArgs a{};
  a.W = W; a.x = x; a.nw = nw; a.eps = eps; a.bias = bias; a.res = nullptr; a.y = xz;
  a.B = B; a.O = 2 * dim; a.K = K;
  a.dim = dim; a.width = width; a.ctx = ctx; a.cw = cw; a.cb = cb; a.xc = xc;
  a.Wx = Wx; a.nout = nout; a.nout4 = (nout + 3) & ~3; a.part = part;
  return bf16 ? launch_gemv_t<__hip_bfloat16>(a, nw != nullptr, true, st)
              : launch_gemv_t<float>(a, nw != nullptr, true, st);
}

hipError_t launch_decode_ssm_step(int bf16, const void* p, int nout, int nparts, int R,
                                  const void* Wdt, const void* dtb, const void* logA, const void* D,
                                  const void* xc, const void* xz, int ld, float* state, void* y,
                                  int B, int dim, int nstate, bool vecR, hipStream_t st) {
  ProfScope prof("decode_ssm_step", st);
  return bf16 ? launch_ssm_step_t<__hip_bfloat16>(p, nout, nparts, R, Wdt, dtb, logA, D, xc, xz,
                                                  ld, state, y, B, dim, nstate, vecR, st)
              : launch_ssm_step_t<float>(p, nout, nparts, R, Wdt, dtb, logA, D, xc, xz, ld, state,
                                         y, B, dim, nstate, vecR, st);
}

}  // namespace ssm
