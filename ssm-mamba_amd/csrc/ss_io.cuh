// Predicated row loads/stores used by the tile phases of the scan kernels.
#pragma once

#include "ss_common.cuh"

namespace ssm {

// Load Elem<T>::kVec consecutive elements starting at column t of a row of
// length L.  kAligned: L is a multiple of kVec and the row is 16-byte aligned,
// so a vector is either fully inside or fully outside [0, L).
template <typename T, bool kAligned>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int t, int L, bool ok,
                                         float (&v)[Elem<T>::kVec]) {
  constexpr int kV = Elem<T>::kVec;
  if constexpr (kAligned) {
    if (ok && t < L) {
      Elem<T>::loadv(row + t, v);
    } else {
#pragma unroll
      for (int j = 0; j < kV; ++j) v[j] = 0.0f;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kV; ++j) v[j] = (ok && t + j < L) ? Elem<T>::load1(row + t + j) : 0.0f;
  }
}

template <typename T, bool kAligned>
__device__ __forceinline__ void store_row(T* __restrict__ row, int t, int L,
                                          const float (&v)[Elem<T>::kVec]) {
  constexpr int kV = Elem<T>::kVec;
  if constexpr (kAligned) {
    if (t < L) Elem<T>::storev(row + t, v);
  } else {
#pragma unroll
    for (int j = 0; j < kV; ++j)
      if (t + j < L) Elem<T>::store1(row + t + j, v[j]);
  }
}

// B and C re-laid out for the scan kernels by bc_prep_kernel: fp32,
// [b][state group G = n/4][t (padded to a multiple of 4)][s = n%4][B, C].
// One 4-step block of one state group is 32 contiguous floats, which a wave
// (whose group, batch row and steps are uniform) reads with two scalar
// s_load_dwordx16 -- no VALU or LDS work for B/C.
struct BC4 {
  float v[32];  // [j (step)][s (state)][0: B, 1: C]
  __device__ __forceinline__ float B(int j, int s) const { return v[j * 8 + s * 2]; }
  __device__ __forceinline__ float C(int j, int s) const { return v[j * 8 + s * 2 + 1]; }
};

__device__ __forceinline__ void load_bc_block(const float* __restrict__ bc, size_t off, BC4& r) {
  // off is wave-uniform; the __restrict__ kernel argument lets these be s_loads
#pragma unroll
  for (int i = 0; i < 32; ++i) r.v[i] = bc[off + i];
}

// Row length of the prepped layout: whole 16-step chunks, so every 4-step
// block the kernels touch (up to the end of the last chunk) is inside the row.
__host__ __device__ inline int bc_row_len(int L) { return (L + 15) & ~15; }

__device__ __forceinline__ size_t bc_offset(int b, int G, int ngroups, int Lp, int t) {
  return (((size_t)b * ngroups + G) * Lp + t) * 8;
}

__device__ __forceinline__ void f4_to(const float4 x, float (&v)[4]) {
  v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
}

__device__ __forceinline__ float silu_f(float z) { return z * sigmoidf_fast(z); }

// d silu(z)/dz = s * (1 + z * (1 - s)), s = sigmoid(z)
__device__ __forceinline__ float silu_grad_f(float z) {
  float s = sigmoidf_fast(z);
  return s * (1.0f + z * (1.0f - s));
}

// Valid window [vlo, vhi) of batch row b from the optional lengths.
__device__ __forceinline__ void valid_window(const int64_t* __restrict__ length, int pad_right,
                                             int b, int L, int& vlo, int& vhi) {
  vlo = 0;
  vhi = L;
  if (length) {
    long long ln = length[b];
    ln = ln < 0 ? 0 : (ln > L ? L : ln);
    if (pad_right) vhi = (int)ln;
    else vlo = L - (int)ln;
  }
}

}  // namespace ssm
