// Single-step selective state update (decode) for gfx950.
//
// Per (b, d) (reference semantics: csrc/selective_update/kernel.cu:39-71):
//   delta = softplus(dt + bias_d);  h'_n = exp(delta * A_dn) * h_n + delta * x * B_n
//   out   = D_d * x + sum_n C_n h'_n            (* silu(z) when z is given)
// The step is a pure stream over the fp32 state (64 B in, 64 B out per (b, d)
// at N = 16), so the layout is chosen for 128-bit coalesced access: kQ lanes
// per (b, d), each owning 4 consecutive states (one float4 of h, A, and of the
// new state), the out-sum over states is a kQ-lane shuffle reduction.  The new
// state may alias the old one (in-place update): every lane reads its float4
// before writing it.
#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"

namespace ssm {

template <typename T, int kQ, bool kVecN>
__global__ __launch_bounds__(256) void state_update_kernel(
    const int batch, const int dim, const int N, const int softplus,
    const float* __restrict__ state, float* new_state, const T* __restrict__ xp,
    const T* __restrict__ dtp, const float* __restrict__ Ap, const T* __restrict__ Bp,
    const T* __restrict__ Cp, const float* __restrict__ Dp, const float* __restrict__ biasp,
    const T* __restrict__ zp, T* __restrict__ out) {
  const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const int q = (int)(gid % kQ);
  const size_t bd = gid / kQ;
  // groups of kQ lanes are aligned inside a wave and are either all in range
  // or all out of range, so the shuffle reduction below sees full groups
  if (bd >= (size_t)batch * dim) return;
  const int d = (int)(bd % dim);
  const int b = (int)(bd / dim);

  const float x = Elem<T>::load1(xp + bd);
  const float v = Elem<T>::load1(dtp + bd) + (biasp ? biasp[d] : 0.0f);
  const float delta = softplus ? softplus_t20(v) : v;
  const float dx = delta * x;
  const int n0 = q * 4;

  float part = 0.0f;
  if (kVecN) {
    // N % 4 == 0: 128-bit state / A access
    const float4 h4 = *reinterpret_cast<const float4*>(state + bd * N + n0);
    const float4 a4 = *reinterpret_cast<const float4*>(Ap + (size_t)d * N + n0);
    float Bv[4], Cv[4];
    Elem<T>::load4(Bp + (size_t)b * N + n0, Bv);
    Elem<T>::load4(Cp + (size_t)b * N + n0, Cv);
    float hv[4] = {h4.x, h4.y, h4.z, h4.w};
    const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      hv[s] = fmaf(fast_exp2(delta * av[s] * kLog2e), hv[s], dx * Bv[s]);
      part = fmaf(Cv[s], hv[s], part);
    }
    *reinterpret_cast<float4*>(new_state + bd * N + n0) = make_float4(hv[0], hv[1], hv[2], hv[3]);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int n = n0 + s;
      if (n < N) {
        const float hn = fmaf(fast_exp2(delta * Ap[(size_t)d * N + n] * kLog2e), state[bd * N + n],
                              dx * Elem<T>::load1(Bp + (size_t)b * N + n));
        new_state[bd * N + n] = hn;
        part = fmaf(Elem<T>::load1(Cp + (size_t)b * N + n), hn, part);
      }
    }
  }
  part = group_sum<kQ>(part);
  if (q == 0) {
    float y = fmaf(Dp ? Dp[d] : 0.0f, x, part);
    if (zp) y *= silu_f(Elem<T>::load1(zp + bd));
    Elem<T>::store1(out + bd, y);
  }
}

template <typename T, int kQ>
static hipError_t launch_upd2(const UpdateParams& p, bool vecN, hipStream_t st) {
  const size_t threads = (size_t)p.batch * p.dim * kQ;
  const unsigned blocks = (unsigned)((threads + 255) / 256);
  ProfScope prof("state_update", st);
  if (vecN)
    hipLaunchKernelGGL((state_update_kernel<T, kQ, true>), dim3(blocks), dim3(256), 0, st, p.batch,
                       p.dim, p.nstate, p.softplus, p.state, p.new_state, (const T*)p.x,
                       (const T*)p.dt, p.A, (const T*)p.B, (const T*)p.C, p.D, p.bias,
                       (const T*)p.z, (T*)p.out);
  else
    hipLaunchKernelGGL((state_update_kernel<T, kQ, false>), dim3(blocks), dim3(256), 0, st,
                       p.batch, p.dim, p.nstate, p.softplus, p.state, p.new_state, (const T*)p.x,
                       (const T*)p.dt, p.A, (const T*)p.B, (const T*)p.C, p.D, p.bias,
                       (const T*)p.z, (T*)p.out);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_upd1(const UpdateParams& p, bool vecN, hipStream_t st) {
  const int nq = (p.nstate + 3) / 4;
  if (nq <= 1) return launch_upd2<T, 1>(p, vecN, st);
  if (nq <= 2) return launch_upd2<T, 2>(p, vecN, st);
  if (nq <= 4) return launch_upd2<T, 4>(p, vecN, st);
  if (nq <= 8) return launch_upd2<T, 8>(p, vecN, st);
  if (nq <= 16) return launch_upd2<T, 16>(p, vecN, st);
  if (nq <= 32) return launch_upd2<T, 32>(p, vecN, st);
  return launch_upd2<T, 64>(p, vecN, st);
}

hipError_t launch_state_update(const UpdateParams& p, int dtype, bool vecN, hipStream_t st) {
  if (dtype == 1) return launch_upd1<__hip_bfloat16>(p, vecN, st);
  return launch_upd1<float>(p, vecN, st);
}

}  // namespace ssm
