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
// [b][state pair G = n/2][t (rows padded to whole 16-step chunks)][s = n%2][B, C].
// One 4-step block of one state pair is 16 contiguous floats, which a wave
// (whose pair, batch row and steps are uniform) reads with one scalar
// s_load_dwordx16 -- no VALU, LDS or vector-memory work for B and C.
struct BC2 {
  float v[16];  // [j (step)][s (state)][0: B, 1: C]
  __device__ __forceinline__ float B(int j, int s) const { return v[j * 4 + s * 2]; }
  __device__ __forceinline__ float C(int j, int s) const { return v[j * 4 + s * 2 + 1]; }
};

__device__ __forceinline__ void load_bc_block(const float* __restrict__ bc, size_t off, BC2& r) {
  // off is wave-uniform; the __restrict__ kernel argument lets these be s_loads
#pragma unroll
  for (int i = 0; i < 16; ++i) r.v[i] = bc[off + i];
}

// Row length of the prepped layout: whole 16-step chunks, so every 4-step
// block the kernels touch (up to the end of the last chunk) is inside the row.
__host__ __device__ inline int bc_row_len(int L) { return (L + 15) & ~15; }

// State pairs in the prepped layout: ceil(N / 2) rounded up to a multiple of
// the 8 waves of a workgroup; pairs past N hold zeros, so every wave of a
// dispatch bucket can read a (zero) block without a branch.
__host__ __device__ inline int bc_pairs(int N) { return (((N + 1) / 2) + 7) & ~7; }

__device__ __forceinline__ size_t bc_offset(int b, int G, int npair, int Lp, int t) {
  return (((size_t)b * npair + G) * Lp + t) * 4;
}

// 4 consecutive elements of a row as raw bits (8 B of bf16 or 16 B of fp32).
template <typename T> struct Raw4;
template <> struct Raw4<float> { using type = uint4; };
template <> struct Raw4<__hip_bfloat16> { using type = uint2; };

// kAligned: L % 4 == 0 and rows 16-byte aligned, so a 4-element group is
// either wholly inside or wholly outside [0, L).
template <typename T, bool kAligned>
__device__ __forceinline__ typename Raw4<T>::type load_raw4(const T* __restrict__ row, int t, int L,
                                                            bool ok) {
  using R = typename Raw4<T>::type;
  if constexpr (kAligned) {
    if (ok && t < L) return *reinterpret_cast<const R*>(row + t);
    R z{};
    return z;
  } else {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (ok && t + j < L) ? Elem<T>::load1(row + t + j) : 0.0f;
    if constexpr (sizeof(T) == 4) {
      return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                        __float_as_uint(v[3]));
    } else {
      return make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  }
}

__device__ __forceinline__ void decode4(const uint4 r, float (&v)[4]) {
  v[0] = __uint_as_float(r.x); v[1] = __uint_as_float(r.y);
  v[2] = __uint_as_float(r.z); v[3] = __uint_as_float(r.w);
}
__device__ __forceinline__ void decode4(const uint2 r, float (&v)[4]) {
  v[0] = bf16_lo(r.x); v[1] = bf16_hi(r.x); v[2] = bf16_lo(r.y); v[3] = bf16_hi(r.y);
}

// Branch-free variants for the kernels' steady-state loops.  A branch around
// a memory operation leaves a path without it, and the compiler then waits for
// every outstanding load and store wherever it needs a loaded value; without
// branches it can wait for exactly the loads it needs.
//  load_raw4_nb: the row pointer must be valid (callers clamp the channel)
//    and the step is clamped into the row; past the row end or the last
//    channel the value is other data of the same tensor, which the callers
//    must mask (steps outside the valid window or past the last channel get
//    delta = 0 and dout = 0, so they add nothing to any sum) or never store.  No
//    select on the loaded value: it would make the compiler wait for the
//    load right where it is issued.
//  store4_nb: lanes with !(ok && t < L) write to `dummy` (16 bytes, aligned,
//    never read) instead.
// The unaligned path keeps per-element bounds branches.
template <typename T, bool kAligned>
__device__ __forceinline__ typename Raw4<T>::type load_raw4_nb(const T* __restrict__ row, int t, int L,
                                                               bool ok) {
  using R = typename Raw4<T>::type;
  if constexpr (kAligned) {
    (void)ok;
    return *reinterpret_cast<const R*>(row + min(t, L - 4));
  } else {
    return load_raw4<T, false>(row, t, L, ok);
  }
}

template <typename T, bool kAligned>
__device__ __forceinline__ void store4_nb(T* __restrict__ row, int t, int L, bool ok,
                                          void* __restrict__ dummy, const float (&v)[4]) {
  if constexpr (kAligned) {
    T* dst = (ok && t < L) ? row + t : static_cast<T*>(dummy);
    if constexpr (sizeof(T) == 4) {
      *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  } else {
    if (ok) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (t + j < L) Elem<T>::store1(row + t + j, v[j]);
    }
  }
}

template <typename T, bool kAligned>
__device__ __forceinline__ void store4(T* __restrict__ row, int t, int L, const float (&v)[4]) {
  if constexpr (kAligned) {
    if (t < L) {
      if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(row + t) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        *reinterpret_cast<uint2*>(row + t) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (t + j < L) Elem<T>::store1(row + t + j, v[j]);
  }
}

// ---------------------------------------------------------------- raw buffer stores

// A raw (untyped) buffer descriptor over `bytes` bytes at `base`, held in
// scalar registers.  The hardware checks every access against `bytes`: a store
// at a larger offset is dropped, so a masked lane needs no separate address.
// Dword 3 = 0x00020000 selects a 32-bit data format (the gfx9-family value; an
// untyped access ignores the format, but a zero format disables the buffer).
// base and bytes must be wave-uniform; they are passed through readfirstlane
// so that the descriptor is built in scalar registers (a descriptor the
// compiler cannot prove uniform is used one lane value at a time instead).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* const ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}
constexpr uint32_t kOffDrop = 0x80000000u;  // past every range built here (bytes < 2^31)

typedef unsigned int u32x2_v __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

// 4 consecutive elements at byte offset `off` of the buffer, as loaded; zero
// when off is past its range.
template <typename T>
__device__ __forceinline__ typename Raw4<T>::type buffer_load_raw4(__amdgpu_buffer_rsrc_t r,
                                                                   uint32_t off) {
  if constexpr (sizeof(T) == 4) {
    const u32x4_v v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return uint4{v.x, v.y, v.z, v.w};
  } else {
    const u32x2_v v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
    return uint2{v.x, v.y};
  }
}

// The bits of one element at byte offset `off` (zero past the range).
template <typename T>
__device__ __forceinline__ uint32_t buffer_load_bits1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 4) return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
  else return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// The bits of one element as held in memory, and those bits as a float.
template <typename T>
__device__ __forceinline__ uint32_t elem_bits(T x) {
  if constexpr (sizeof(T) == 4) {
    return __float_as_uint(x);
  } else {
    unsigned short s;
    __builtin_memcpy(&s, &x, sizeof(s));
    return s;
  }
}
template <typename T>
__device__ __forceinline__ float bits_to_f32(uint32_t v) {
  if constexpr (sizeof(T) == 4) return __uint_as_float(v);
  else return __uint_as_float(v << 16);
}

// 4 consecutive elements at byte offset `off` of the buffer (dropped when off
// is past its range).
template <typename T>
__device__ __forceinline__ void buffer_store4(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                              const float (&v)[4]) {
  if constexpr (sizeof(T) == 4) {
    const u32x4_v x = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                       __float_as_uint(v[3])};
    __builtin_amdgcn_raw_buffer_store_b128(x, r, (int)off, 0, 0);
  } else {
    const u32x2_v x = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    __builtin_amdgcn_raw_buffer_store_b64(x, r, (int)off, 0, 0);
  }
}

// Wait until every outstanding LDS and scalar-memory load of this wave has
// returned (s_waitcnt lgkmcnt(0)) and keep the scheduler from moving
// instructions across this point.  Orders "consume block k" before "issue
// block k+1", so one block of work hides the latency of the next block's loads
// (scalar loads may return out of order, so lgkmcnt can only be waited to 0).
__device__ __forceinline__ void wait_lgkm_fence() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt=63, expcnt=7, lgkmcnt=0 (gfx9 encoding)
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

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
