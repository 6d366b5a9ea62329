// Single-step selective state update (decode) for gfx950.
//
// Per (b, d) (reference semantics: csrc/selective_update/kernel.cu:39-71):
//   delta = softplus(dt + bias_d);  h'_n = exp(delta * A_dn) * h_n + delta * x * B_n
//   out   = D_d * x + sum_n C_n h'_n            (* silu(z) when z is given)
// The step is a pure stream over the fp32 state (64 B in and 64 B out per
// (b, d) at N = 16), so one thread owns one (b, d) row and all its states:
// consecutive lanes own consecutive rows, a wave streams 64 contiguous state
// rows (4 KB at N = 16) with 128-bit accesses, the sum over states stays in
// registers and x / dt / z / out are coalesced 16-bit accesses.  A and the
// per-batch B, C rows are small and cache-resident.  The new state may alias
// the old one (in-place update): each thread reads its whole row before
// writing it.
#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"

namespace ssm {

// kN4: number of float4 state groups handled per thread when N % 4 == 0
// (N = 4 * kN4); kN4 = 0 selects the generic scalar path for any N.
template <typename T, int kN4>
__global__ __launch_bounds__(256) void state_update_kernel(
    const int batch, const int dim, const int N, const int softplus,
    const float* __restrict__ state, float* new_state, const T* __restrict__ xp,
    const T* __restrict__ dtp, const float* __restrict__ Ap, const T* __restrict__ Bp,
    const T* __restrict__ Cp, const float* __restrict__ Dp, const float* __restrict__ biasp,
    const T* __restrict__ zp, T* __restrict__ out) {
  const size_t bd = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (bd >= (size_t)batch * dim) return;
  const int d = (int)(bd % dim);
  const int b = (int)(bd / dim);

  const float x = Elem<T>::load1(xp + bd);
  const float v = Elem<T>::load1(dtp + bd) + (biasp ? biasp[d] : 0.0f);
  const float zv = zp ? Elem<T>::load1(zp + bd) : 0.0f;
  const float delta = softplus ? softplus_t20(v) : v;
  const float dx = delta * x;
  const float dl2 = delta * kLog2e;

  float part = 0.0f;
  if constexpr (kN4 > 0) {
    const float4* __restrict__ hs = reinterpret_cast<const float4*>(state + bd * (4 * kN4));
    const float4* __restrict__ as = reinterpret_cast<const float4*>(Ap + (size_t)d * (4 * kN4));
    float4 h4[kN4];
#pragma unroll
    for (int q = 0; q < kN4; ++q) h4[q] = hs[q];
#pragma unroll
    for (int q = 0; q < kN4; ++q) {
      const float4 a4 = as[q];
      float Bv[4], Cv[4];
      Elem<T>::load4(Bp + (size_t)b * (4 * kN4) + 4 * q, Bv);
      Elem<T>::load4(Cp + (size_t)b * (4 * kN4) + 4 * q, Cv);
      float hv[4] = {h4[q].x, h4[q].y, h4[q].z, h4[q].w};
      const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        hv[s] = fmaf(fast_exp2(dl2 * av[s]), hv[s], dx * Bv[s]);
        part = fmaf(Cv[s], hv[s], part);
      }
      h4[q] = make_float4(hv[0], hv[1], hv[2], hv[3]);
    }
    float4* hn = reinterpret_cast<float4*>(new_state + bd * (4 * kN4));
#pragma unroll
    for (int q = 0; q < kN4; ++q) hn[q] = h4[q];
  } else {
    for (int n = 0; n < N; ++n) {
      const float hn = fmaf(fast_exp2(dl2 * Ap[(size_t)d * N + n]), state[bd * N + n],
                            dx * Elem<T>::load1(Bp + (size_t)b * N + n));
      new_state[bd * N + n] = hn;
      part = fmaf(Elem<T>::load1(Cp + (size_t)b * N + n), hn, part);
    }
  }
  float y = fmaf(Dp ? Dp[d] : 0.0f, x, part);
  if (zp) y *= silu_f(zv);
  Elem<T>::store1(out + bd, y);
}

template <typename T, int kN4>
static hipError_t launch_upd2(const UpdateParams& p, hipStream_t st) {
  const size_t threads = (size_t)p.batch * p.dim;
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  ProfScope prof("state_update", st);
  hipLaunchKernelGGL((state_update_kernel<T, kN4>), dim3(blocks), dim3(256), 0, st, p.batch,
                     p.dim, p.nstate, p.softplus, p.state, p.new_state, (const T*)p.x,
                     (const T*)p.dt, p.A, (const T*)p.B, (const T*)p.C, p.D, p.bias,
                     (const T*)p.z, (T*)p.out);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_upd1(const UpdateParams& p, bool vecN, hipStream_t st) {
  if (vecN) {
    switch (p.nstate) {
      case 4: return launch_upd2<T, 1>(p, st);
      case 8: return launch_upd2<T, 2>(p, st);
      case 16: return launch_upd2<T, 4>(p, st);
      case 32: return launch_upd2<T, 8>(p, st);
      case 64: return launch_upd2<T, 16>(p, st);
      default: break;
    }
  }
  return launch_upd2<T, 0>(p, st);
}

hipError_t launch_state_update(const UpdateParams& p, int dtype, bool vecN, hipStream_t st) {
  if (dtype == 1) return launch_upd1<__hip_bfloat16>(p, vecN, st);
  return launch_upd1<float>(p, vecN, st);
}

}  // namespace ssm
