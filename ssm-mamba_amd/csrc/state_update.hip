// Single-step selective state update (decode) for gfx950.
//
// Per (b, d) (reference semantics: csrc/selective_update/kernel.cu:39-71):
//   delta = softplus(dt + bias_d);  h'_n = exp(delta * A_dn) * h_n + delta * x * B_n
//   out   = D_d * x + sum_n C_n h'_n            (* silu(z) when z is given)
// The step is a pure stream over the fp32 state (64 B in and 64 B out per
// (b, d) at N = 16), so the layout is chosen for contiguous 128-bit access:
// kQ lanes per (b, d) row, each owning 4 consecutive states (one float4 of h,
// of A and of the new state), so a wave's state access is one contiguous
// 1 KB stretch; the out-sum over states is a kQ-lane DPP/shuffle reduction.
// Measured on MI355X this runs at ~1.27x the time of a plain copy of the
// state, where one thread per row (64 B per lane, 64 lines per wave access)
// runs at ~1.6x.  The new state may alias the old one (in-place update): every
// lane reads its float4 before writing it.
#include "ss_io.cuh"
#include "ss_params.h"
#include "ss_prof.h"

namespace ssm {

typedef float f4v __attribute__((ext_vector_type(4)));

// Sum over aligned groups of kW lanes (every lane gets its group's sum); DPP
// quad permutes for the 2- and 4-lane levels, shuffles above.
template <int kW>
__device__ __forceinline__ float lane_group_sum(float v) {
  if constexpr (kW >= 2) v += dpp_mov<kDppQuadXor1>(v);
  if constexpr (kW >= 4) v += dpp_mov<kDppQuadXor2>(v);
#pragma unroll
  for (int m = 4; m < kW; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Vector path (N == 4 * kQ, 16-byte aligned state and A): kQ lanes per
// (b, d) row and kRows rows per thread.  A wave covers 64 / kQ rows per slice
// and kRows slices, each slice one contiguous 1 KB stretch of state; all of a
// thread's loads are issued before any arithmetic, so a wave has kRows KB of
// state in flight and the whole grid fits the machine in about one round.
// Rows past `dim` load a clamped row and skip their stores.
//
// kNT: the new state is written with nontemporal stores.  Measured at
// config 2 (21 MB of state): 3-6% faster when the state streams from HBM
// (the 256 MB Infinity Cache flushed between steps, or 16 states in
// rotation), 27% slower when the same state stays in that cache from step to
// step.  A model of a dozen layers with states that size already exceeds the
// cache, so the launch takes nontemporal stores from 16 MB of state up.
template <typename T, int kQ, int kRows, bool kNT>
__global__ __launch_bounds__(256) void state_update_vec_kernel(
    const int dim, const int N, const int softplus, const float* __restrict__ state,
    float* new_state, const T* __restrict__ xp, const T* __restrict__ dtp,
    const float* __restrict__ Ap, const T* __restrict__ Bp, const T* __restrict__ Cp,
    const float* __restrict__ Dp, const float* __restrict__ biasp, const T* __restrict__ zp,
    T* __restrict__ out) {
  constexpr int kRW = 64 / kQ;  // rows per wave slice
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q = lane % kQ;
  const int b = blockIdx.y;
  const int dbase = (blockIdx.x * 4 + wave) * (kRows * kRW) + lane / kQ;
  const int n0 = q * 4;
  const unsigned bo = (unsigned)b * N + n0;
  float Bv[4], Cv[4];
  Elem<T>::load4(Bp + bo, Bv);
  Elem<T>::load4(Cp + bo, Cv);
  float4 h4[kRows], a4[kRows];
  float xv[kRows], dtv[kRows], bias[kRows], dv[kRows], zv[kRows];
  // optional operands are read from a valid stand-in address when absent, so
  // every load of the thread issues here, unconditionally, and the waits are
  // counted (a load inside a branch is waited for inside it)
  const float* __restrict__ bq = biasp ? biasp : Ap;
  const float* __restrict__ dq = Dp ? Dp : Ap;
  const T* __restrict__ zq = zp ? zp : xp;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int d = min(dbase + r * kRW, dim - 1);
    const unsigned bd = (unsigned)b * dim + d;
    // the state is read once per step: a nontemporal load (measured 10% faster
    // for a state that does not fit the last-level cache)
    const f4v t = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(state + bd * (unsigned)N + n0));
    h4[r] = make_float4(t.x, t.y, t.z, t.w);
    a4[r] = *reinterpret_cast<const float4*>(Ap + (unsigned)d * N + n0);
    xv[r] = Elem<T>::load1(xp + bd);
    dtv[r] = Elem<T>::load1(dtp + bd);
    bias[r] = bq[d];
    dv[r] = dq[d];
    zv[r] = Elem<T>::load1(zq + bd);
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int dr = dbase + r * kRW;
    const int d = min(dr, dim - 1);
    const unsigned bd = (unsigned)b * dim + d;
    const float v = dtv[r] + (biasp ? bias[r] : 0.0f);
    const float delta = softplus ? softplus_t20(v) : v;
    const float dx = delta * xv[r], dl2 = delta * kLog2e;
    float hv[4] = {h4[r].x, h4[r].y, h4[r].z, h4[r].w};
    const float av[4] = {a4[r].x, a4[r].y, a4[r].z, a4[r].w};
    float part = 0.0f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      hv[s] = fmaf(fast_exp2(dl2 * av[s]), hv[s], dx * Bv[s]);
      part = fmaf(Cv[s], hv[s], part);
    }
    // a row's kQ lanes are aligned in the wave and share `dr`, so the group
    // reduction always sees whole rows
    part = lane_group_sum<kQ>(part);
    if (dr < dim) {
      const f4v nv = {hv[0], hv[1], hv[2], hv[3]};
      f4v* const dst = reinterpret_cast<f4v*>(new_state + bd * (unsigned)N + n0);
      if constexpr (kNT) __builtin_nontemporal_store(nv, dst);
      else *dst = nv;
      if (q == 0) {
        float y = fmaf(Dp ? dv[r] : 0.0f, xv[r], part);
        if (zp) y *= silu_f(zv[r]);
        Elem<T>::store1(out + bd, y);
      }
    }
  }
}

// Scalar path (any N, any alignment): kQ lanes per (b, d) row, each owning
// up to 4 consecutive states.
template <typename T, int kQ>
__global__ __launch_bounds__(256) void state_update_kernel(
    const int batch, const int dim, const int N, const int softplus,
    const float* __restrict__ state, float* new_state, const T* __restrict__ xp,
    const T* __restrict__ dtp, const float* __restrict__ Ap, const T* __restrict__ Bp,
    const T* __restrict__ Cp, const float* __restrict__ Dp, const float* __restrict__ biasp,
    const T* __restrict__ zp, T* __restrict__ out) {
  // grid: x covers dim * kQ lanes of one batch row, y = batch row (no
  // integer division by runtime sizes); offsets are 32-bit (the host checks
  // batch * dim * nstate < 2^31)
  const int gx = blockIdx.x * blockDim.x + threadIdx.x;
  const int q = gx % kQ;
  const int d = gx / kQ;
  // groups of kQ lanes are aligned inside a wave and are either all in range
  // or all out of range, so the group reduction below sees whole groups
  if (d >= dim) return;
  const int b = blockIdx.y;
  const unsigned bd = (unsigned)b * dim + d;
  const int n0 = q * 4;
  const unsigned so = bd * (unsigned)N + n0;        // state offset
  const unsigned ao = (unsigned)d * N + n0;         // A offset
  const unsigned bo = (unsigned)b * N + n0;         // B / C offset

  float part = 0.0f;
  // optional operands from a valid stand-in address when absent (all loads
  // issue up front)
  const float x = Elem<T>::load1(xp + bd);
  const float bv = (biasp ? biasp : Ap)[d];
  const float dv = (Dp ? Dp : Ap)[d];
  const float zv = Elem<T>::load1((zp ? zp : xp) + bd);
  const float v = Elem<T>::load1(dtp + bd) + (biasp ? bv : 0.0f);
  const float delta = softplus ? softplus_t20(v) : v;
  const float dx = delta * x, dl2 = delta * kLog2e;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (n0 + s < N) {
      const float hn = fmaf(fast_exp2(dl2 * Ap[ao + s]), state[so + s], dx * Elem<T>::load1(Bp + bo + s));
      new_state[so + s] = hn;
      part = fmaf(Elem<T>::load1(Cp + bo + s), hn, part);
    }
  }
  part = lane_group_sum<kQ>(part);
  if (q == 0) {
    float y = fmaf(Dp ? dv : 0.0f, x, part);
    if (zp) y *= silu_f(zv);
    Elem<T>::store1(out + bd, y);
  }
}

constexpr int kUpdRows = 4;  // rows per thread on the vector path
// states of at least this many bytes take nontemporal stores (see kNT)
constexpr size_t kUpdNtBytes = size_t(16) << 20;

template <typename T, int kQ>
static hipError_t launch_upd2(const UpdateParams& p, bool vecN, hipStream_t st) {
  ProfScope prof("state_update", st);
  if (vecN) {
    const int per_block = 4 * kUpdRows * (64 / kQ);  // rows per 256-thread block
    const dim3 grid((unsigned)((p.dim + per_block - 1) / per_block), (unsigned)p.batch);
    const bool nt = (size_t)p.batch * p.dim * p.nstate * sizeof(float) >= kUpdNtBytes;
    if (nt)
      hipLaunchKernelGGL((state_update_vec_kernel<T, kQ, kUpdRows, true>), grid, dim3(256), 0, st,
                         p.dim, p.nstate, p.softplus, p.state, p.new_state, (const T*)p.x,
                         (const T*)p.dt, p.A, (const T*)p.B, (const T*)p.C, p.D, p.bias,
                         (const T*)p.z, (T*)p.out);
    else
      hipLaunchKernelGGL((state_update_vec_kernel<T, kQ, kUpdRows, false>), grid, dim3(256), 0, st,
                         p.dim, p.nstate, p.softplus, p.state, p.new_state, (const T*)p.x,
                         (const T*)p.dt, p.A, (const T*)p.B, (const T*)p.C, p.D, p.bias,
                         (const T*)p.z, (T*)p.out);
  } else {
    const size_t lanes = (size_t)p.dim * kQ;
    const dim3 grid((unsigned)((lanes + 255) / 256), (unsigned)p.batch);
    hipLaunchKernelGGL((state_update_kernel<T, kQ>), grid, dim3(256), 0, st, p.batch, p.dim,
                       p.nstate, p.softplus, p.state, p.new_state, (const T*)p.x, (const T*)p.dt,
                       p.A, (const T*)p.B, (const T*)p.C, p.D, p.bias, (const T*)p.z,
                       (T*)p.out);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_upd1(const UpdateParams& p, bool vecN, hipStream_t st) {
  const int nq = (p.nstate + 3) / 4;
  // the vector path needs N == 4 * kQ exactly
  auto vec = [&](int kq) { return vecN && p.nstate == 4 * kq; };
  if (nq <= 1) return launch_upd2<T, 1>(p, vec(1), st);
  if (nq <= 2) return launch_upd2<T, 2>(p, vec(2), st);
  if (nq <= 4) return launch_upd2<T, 4>(p, vec(4), st);
  if (nq <= 8) return launch_upd2<T, 8>(p, vec(8), st);
  if (nq <= 16) return launch_upd2<T, 16>(p, vec(16), st);
  if (nq <= 32) return launch_upd2<T, 32>(p, vec(32), st);
  return launch_upd2<T, 64>(p, vec(64), st);
}

hipError_t launch_state_update(const UpdateParams& p, int dtype, bool vecN, hipStream_t st) {
  if (dtype == 1) return launch_upd1<__hip_bfloat16>(p, vecN, st);
  return launch_upd1<float>(p, vecN, st);
}

}  // namespace ssm
